"""Slot-cache / gap oracle (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

A CPU restatement of the reference's per-layer slot cache and the
router-split gap's bookkeeping, kept in the reference's own data structures
(OrderedDict segments, a list free stack) so that slot assignment can be
compared bit for bit with the native implementation:

  install          src/sluice/offloader.py:936-947, 974-989 (num_slots,
                   protected_cap, free list [S-1..0], local_of / global_of_local,
                   map all -1), 1000-1010 (full-residency pre-fill)
  touch            src/sluice/offloader.py:2009-2021
  coldest          src/sluice/offloader.py:2023-2034 (LRU; with SLUICE_LFU the
                   least frequently used, LRU among equals)
  acquire_slot     src/sluice/offloader.py:2036-2074 (with SLUICE_LFU the
                   protected segment is walked coldest-first)
  LFU frequency    src/sluice/offloader.py:1993-2007 (per-local counts bumped
                   by real classic steps, halved every 256 of them)
  expert counts    src/sluice/offloader.py:1026-1034, 1664-1671 (per-global
                   decode / scan selection counts of real classic steps)
  evict_to         src/sluice/offloader.py:2076-2081
  standing map     src/sluice/offloader.py:2083-2123 (map contents only)
  gap              src/sluice/offloader.py:2405-2467 (fast-hit, sorted unique,
                   hit touches, miss acquisition with the claimed set seeded by
                   the step's hit slots, overflow, standing-map refresh)
  pins             src/sluice/offloader.py:1046-1083
  classic step     src/sluice/offloader.py:1452-1765 (run_moe with the
                   defaults: no lazy/hook-lite/prefill-block modes) and
                   1846-1933 (_run_waves): decode/scan classification from the
                   step's decode counts, class-aware touches and acquisition,
                   wave 0 = hits + the fills that fit, the rest rotated through
                   the probation slots in two ping-pong groups, one sparse map
                   per wave
"""

from __future__ import annotations

from collections import OrderedDict


class GapOverflow(RuntimeError):
    pass


LFU_AGE_STEPS = 256


class LayerCache:
    def __init__(self, global_n: int, local_n: int, slots: int, protect_frac: float = 0.5,
                 local_of=None, lfu: bool = False, counts: bool = False):
        self.global_n = global_n
        self.local_n = local_n
        self.num_slots = min(slots, local_n)
        frac = min(max(float(protect_frac), 0.0), 0.9)
        self.protected_cap = max(min(int(self.num_slots * frac), self.num_slots - 1), 0)
        self.local_of = list(range(global_n)) if local_of is None else [int(v) for v in local_of]
        self.global_of_local = [-1] * local_n
        for g, loc in enumerate(self.local_of):
            if 0 <= loc < local_n:
                self.global_of_local[loc] = g
        self.slot_of: dict[int, int] = {}
        self.expert_in_slot: list[int | None] = [None] * self.num_slots
        self.free_slots = list(range(self.num_slots - 1, -1, -1))
        self.protected: OrderedDict = OrderedDict()
        self.probation: OrderedDict = OrderedDict()
        self.pinned_slots: set = set()
        self.map = [-1] * global_n
        self.map_is_standing = False
        self.gaps = 0
        self.misses = 0
        self.fast_hits = 0
        self.map_writes = 0
        self.lfu = lfu
        self.freq: dict = {}
        self.lfu_steps = 0
        self.counts = ([0] * global_n, [0] * global_n) if counts else None
        self.steps_small = 0
        self.steps_scan = 0

    # -- SLRU core -------------------------------------------------------
    def touch(self, slot: int, friendly: bool = True) -> None:
        if slot in self.protected:
            self.protected.move_to_end(slot)
        elif slot in self.probation:
            if friendly and self.protected_cap > 0:
                del self.probation[slot]
                self.protected[slot] = None
                while len(self.protected) > self.protected_cap:
                    victim = self.coldest_protected()
                    del self.protected[victim]
                    self.probation[victim] = None
            else:
                self.probation.move_to_end(slot)

    def _heat(self, slot: int) -> int:
        return self.freq.get(self.expert_in_slot[slot], 0)

    def coldest_protected(self) -> int:
        if self.lfu and self.freq:
            return min(self.protected, key=self._heat)  # min keeps the first (LRU) of equals
        return next(iter(self.protected))

    def bump_freq(self, locals_) -> None:
        for loc in locals_:
            self.freq[loc] = self.freq.get(loc, 0) + 1
        self.lfu_steps += 1
        if self.lfu_steps >= LFU_AGE_STEPS:
            self.lfu_steps = 0
            for loc in list(self.freq):
                v = self.freq[loc] >> 1
                if v:
                    self.freq[loc] = v
                else:
                    del self.freq[loc]

    def evict_to(self, slot: int, local: int) -> None:
        prev = self.expert_in_slot[slot]
        if prev is not None:
            self.slot_of.pop(prev, None)
        self.expert_in_slot[slot] = local
        self.slot_of[local] = slot

    def acquire_slot(self, local: int, claimed: set, allow_protected: bool = True):
        chosen = None
        if self.free_slots:
            chosen = self.free_slots.pop()
        else:
            for cand in self.probation:
                if cand not in claimed:
                    chosen = cand
                    break
            if chosen is not None:
                del self.probation[chosen]
            elif allow_protected:
                order = list(self.protected)
                if self.lfu and self.freq:
                    order = sorted(order, key=self._heat)  # stable: LRU among equals
                for cand in order:
                    if cand not in claimed:
                        chosen = cand
                        break
                if chosen is not None:
                    del self.protected[chosen]
        if chosen is None:
            return None
        self.evict_to(chosen, local)
        self.probation[chosen] = None
        return chosen

    def pin(self, local: int, debit_protected: bool = True):
        if local in self.slot_of or not self.free_slots:
            return None
        slot = self.free_slots.pop()
        self.expert_in_slot[slot] = local
        self.slot_of[local] = slot
        self.pinned_slots.add(slot)
        if debit_protected:
            self.protected_cap -= 1
        return slot

    def unfill(self, slot: int) -> bool:
        """Recovery after a fill whose rows did not land (a failed copy): the
        slot's expert leaves the cache and the slot goes back on the free list
        (popped next); the map stops being standing.  No reference
        counterpart (the reference's copy errors end the engine): these are
        this build's recovery semantics, stated here so the native cache can
        be checked against them."""
        local = self.expert_in_slot[slot]
        if local is None or slot in self.pinned_slots:
            return False
        self.probation.pop(slot, None)
        self.protected.pop(slot, None)
        self.slot_of.pop(local, None)
        self.expert_in_slot[slot] = None
        self.free_slots.append(slot)
        self.map_is_standing = False
        return True

    # -- maps ------------------------------------------------------------
    def standing_map(self) -> list[int]:
        m = [-1] * self.global_n
        for slot, local in enumerate(self.expert_in_slot):
            if local is not None:
                m[self.global_of_local[local]] = slot
        return m

    def write_standing_map(self) -> None:
        self.map = self.standing_map()
        self.map_is_standing = True
        self.map_writes += 1

    # -- the gap ---------------------------------------------------------
    def gap(self, ids, fast_hit: bool = False):
        """One router-split gap on the flat list of selected global ids.

        Returns the (local, slot) stream-ins in issue order.  Raises
        GapOverflow where the reference raises RuntimeError."""
        self.gaps += 1
        ids_list = [int(v) for v in ids]
        n_global = len(self.local_of)
        if fast_hit and self.map_is_standing:
            all_hit = True
            for g in ids_list:
                if 0 <= g < n_global:
                    loc = self.local_of[g]
                    if loc >= 0 and loc not in self.slot_of:
                        all_hit = False
                        break
            if all_hit:
                self.fast_hits += 1
                return []
        missing = []
        hit_slots = set()
        for g in sorted(set(ids_list)):
            if not (0 <= g < n_global):
                continue
            loc = self.local_of[g]
            if loc < 0:
                continue
            slot = self.slot_of.get(loc)
            if slot is None:
                missing.append(loc)
            else:
                hit_slots.add(slot)
                self.touch(slot, True)
        streams = []
        changed = False
        if missing:
            claimed = set(hit_slots)
            for loc in missing:
                slot = self.acquire_slot(loc, claimed, True)
                if slot is None:
                    raise GapOverflow(
                        "Sluice router-split: working set exceeds slots on a decode-sized "
                        "step; raise SLUICE_SLOTS.")
                streams.append((loc, slot))
                claimed.add(slot)
            self.misses += len(missing)
            changed = True
        if changed or not self.map_is_standing:
            self.write_standing_map()
        return streams

    # -- the classic (wave) step ---------------------------------------------
    def classic(self, ids, T: int, nd=None, ndec=None, real_step: bool = True,
                spec_tokens: int = 0):
        """One classic step on the flat row-major [T, k] list of selected
        global ids; nd / ndec: the step's decode-token / decode-request counts
        (None when the engine publishes none), real_step False for dummy runs.

        Returns the waves in execution order, each a dict with "pairs"
        ([(global, slot)] written as that wave's map, every other entry -1)
        and "streams" ([(local, slot)] copied before that wave runs)."""
        ids_list = [int(v) for v in ids]
        k = len(ids_list) // T if T else 0
        selected = sorted(set(ids_list))
        decode_span = ndec * (1 + spec_tokens) if ndec is not None else None
        pure_decode_region = (real_step and nd is not None and decode_span is not None
                              and nd == decode_span)
        if pure_decode_region and 0 < nd <= T:
            decode_ids = set(selected) if nd == T else set(ids_list[:nd * k])
        else:
            decode_ids = None
        n_global = len(self.local_of)
        pairs = []
        for g in selected:
            if 0 <= g < n_global:
                loc = self.local_of[g]
                if loc >= 0:
                    pairs.append((g, loc, decode_ids is not None and g in decode_ids))
        ws = len(pairs)
        mla_forced_scan = real_step and nd is not None and not pure_decode_region
        heuristic_friendly = None
        if decode_ids is None and not mla_forced_scan:
            decode_cap = self.protected_cap + len(self.pinned_slots)
            heuristic_friendly = real_step and ws <= max(decode_cap, 1)
            if heuristic_friendly:
                pairs = [(g, loc, True) for g, loc, _ in pairs]
        if ws == 0:
            self.map = [-1] * self.global_n
            self.map_is_standing = False
            return [{"pairs": [], "streams": []}]
        if real_step:
            pure_decode = (nd == T) if decode_ids is not None else heuristic_friendly
            if pure_decode:
                self.steps_small += 1
            else:
                self.steps_scan += 1
            if self.lfu:
                self.bump_freq(loc for _, loc, _ in pairs)
            if self.counts is not None:
                for g, _, dcls in pairs:
                    self.counts[0 if dcls else 1][g] += 1
        hits, missing = [], []
        for g, loc, dcls in pairs:
            slot = self.slot_of.get(loc)
            if slot is None:
                missing.append((g, loc, dcls))
            else:
                self.touch(slot, dcls)
                hits.append((g, slot))
        missing.sort(key=lambda t: not t[2])
        claimed = {slot for _, slot in hits}
        wave0 = list(hits)
        streams0 = []
        taken = len(missing)
        for i, (g, loc, dcls) in enumerate(missing):
            slot = self.acquire_slot(loc, claimed, allow_protected=dcls)
            if slot is None:
                taken = i
                break
            streams0.append((loc, slot))
            wave0.append((g, slot))
            claimed.add(slot)
        self.misses += len(missing)
        leftover = [(g, loc) for g, loc, _ in missing[taken:]]
        waves = [{"pairs": wave0, "streams": streams0}]
        if leftover:
            rot = list(self.probation.keys())
            if not rot:
                rot = [s for s in range(self.num_slots)
                       if s not in self.pinned_slots][-max(1, self.num_slots // 4):]
            half = (len(rot) + 1) // 2
            group_a, group_b = rot[:half], rot[half:]
            groups = (group_a, group_b if group_b else group_a)
            i = 0
            gi = 0
            while i < len(leftover):
                group = groups[gi % 2]
                chunk = []
                for (g, loc), slot in zip(leftover[i:i + len(group)], group):
                    self.evict_to(slot, loc)
                    chunk.append((g, loc, slot))
                waves.append({"pairs": [(g, slot) for g, _, slot in chunk],
                              "streams": [(loc, slot) for _, loc, slot in chunk]})
                i += len(chunk)
                gi += 1
        last = [-1] * self.global_n
        for g, slot in waves[-1]["pairs"]:
            last[g] = slot
        self.map = last
        self.map_is_standing = False
        return waves

    def snapshot(self) -> dict:
        return {
            "slot_of": [self.slot_of.get(l, -1) for l in range(self.local_n)],
            "expert_in_slot": [-1 if v is None else v for v in self.expert_in_slot],
            "probation": list(self.probation.keys()),
            "protected": list(self.protected.keys()),
            "free_slots": list(self.free_slots),
            "map": list(self.map),
            "map_is_standing": self.map_is_standing,
        }
