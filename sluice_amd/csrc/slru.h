// Host-side slot cache: the per-layer SLRU state machine of the streaming gap.
//
// Follows the reference's Python state machine step for step:
//   _ExpertLayerCache fields      src/sluice/offloader.py:121-169
//   free list / caps at install   src/sluice/offloader.py:936-947
//   _touch                        src/sluice/offloader.py:2009-2021
//   _coldest_protected (LRU)      src/sluice/offloader.py:2023-2034
//   _acquire_slot / _evict_to     src/sluice/offloader.py:2036-2081
//   _router_split_gap bookkeeping src/sluice/offloader.py:2405-2467
// The reference keeps its two segments in OrderedDicts keyed by slot
// (insertion order = recency, first = LRU).  Here each segment is an
// intrusive doubly-linked list over slot indices with O(1) unlink and
// append, which reproduces OrderedDict order exactly: `d[s] = None` for a
// new key appends, `move_to_end` relinks at the tail, `del` unlinks, and
// iteration walks from the head.
#pragma once

#include <stdint.h>

#include <vector>

namespace slru {

enum Seg : uint8_t { kNone = 0, kProbation = 1, kProtected = 2, kPinned = 3 };

struct List {
  int head = -1, tail = -1, size = 0;
};

struct Cache {
  int E = 0, local_n = 0, S = 0, protected_cap = 0;
  std::vector<int> local_of;         // [E] global -> local or -1
  std::vector<int> global_of_local;  // [local_n] local -> global or -1
  std::vector<int> slot_of;          // [local_n] local -> slot or -1
  std::vector<int> expert_in_slot;   // [S] slot -> local or -1
  std::vector<int> free_slots;       // stack; back() is popped next
  std::vector<int> prev, next;       // intrusive links, [S]
  std::vector<uint8_t> seg;          // [S] which segment holds the slot
  List lists[3];                     // indexed by kProbation / kProtected
  bool map_is_standing = false;
  int64_t gaps = 0, misses = 0, fast_hits = 0, map_writes = 0;

  // scratch reused across gaps
  std::vector<uint8_t> claimed;
  std::vector<int> missing;

  void init(int E_, int local_n_, int S_, int cap, const int32_t* lof) {
    E = E_;
    local_n = local_n_;
    S = S_;
    protected_cap = cap;
    local_of.assign(E, -1);
    global_of_local.assign(local_n, -1);
    for (int g = 0; g < E; ++g) {
      const int l = lof != nullptr ? lof[g] : (g < local_n ? g : -1);
      local_of[g] = l;
      if (l >= 0 && l < local_n) global_of_local[l] = g;
    }
    slot_of.assign(local_n, -1);
    expert_in_slot.assign(S, -1);
    free_slots.clear();
    for (int s = S - 1; s >= 0; --s) free_slots.push_back(s);  // [S-1 .. 0]
    prev.assign(S, -1);
    next.assign(S, -1);
    seg.assign(S, kNone);
    lists[1] = List();
    lists[2] = List();
    claimed.assign(S, 0);
  }

  void push_back(Seg sg, int s) {
    List& L = lists[sg];
    prev[s] = L.tail;
    next[s] = -1;
    if (L.tail >= 0) next[L.tail] = s;
    else L.head = s;
    L.tail = s;
    ++L.size;
    seg[s] = sg;
  }

  void unlink(int s) {
    List& L = lists[seg[s]];
    if (prev[s] >= 0) next[prev[s]] = next[s];
    else L.head = next[s];
    if (next[s] >= 0) prev[next[s]] = prev[s];
    else L.tail = prev[s];
    prev[s] = next[s] = -1;
    --L.size;
    seg[s] = kNone;
  }

  void move_to_end(int s) {
    const Seg sg = (Seg)seg[s];
    unlink(s);
    push_back(sg, s);
  }

  // _touch(cache, slot, friendly)
  void touch(int slot, bool friendly) {
    if (seg[slot] == kProtected) {
      move_to_end(slot);
    } else if (seg[slot] == kProbation) {
      if (friendly && protected_cap > 0) {
        unlink(slot);
        push_back(kProtected, slot);
        while (lists[kProtected].size > protected_cap) {
          const int demoted = lists[kProtected].head;  // _coldest_protected (LRU)
          unlink(demoted);
          push_back(kProbation, demoted);
        }
      } else {
        move_to_end(slot);
      }
    }
  }

  void evict_to(int slot, int local) {
    const int old = expert_in_slot[slot];
    if (old >= 0) slot_of[old] = -1;
    expert_in_slot[slot] = local;
    slot_of[local] = slot;
  }

  // _acquire_slot(cache, local, claimed, allow_protected); -1 = none.
  int acquire(int local, bool allow_protected) {
    int slot = -1;
    if (!free_slots.empty()) {
      slot = free_slots.back();
      free_slots.pop_back();
    } else {
      for (int c = lists[kProbation].head; c >= 0; c = next[c]) {
        if (!claimed[c]) {
          slot = c;
          unlink(c);
          break;
        }
      }
      if (slot < 0 && allow_protected) {
        for (int c = lists[kProtected].head; c >= 0; c = next[c]) {
          if (!claimed[c]) {
            slot = c;
            unlink(c);
            break;
          }
        }
      }
    }
    if (slot < 0) return -1;
    evict_to(slot, local);
    push_back(kProbation, slot);  // new entries start probationary
    return slot;
  }

  // Static pin / full-residency pre-fill: take the next free slot outside
  // both segments (src/sluice/offloader.py:1046-1083, 1000-1010).
  int pin(int local, bool debit_protected) {
    if (local < 0 || local >= local_n || slot_of[local] >= 0 || free_slots.empty()) return -1;
    const int slot = free_slots.back();
    free_slots.pop_back();
    expert_in_slot[slot] = local;
    slot_of[local] = slot;
    seg[slot] = kPinned;
    if (debit_protected && protected_cap > 0) --protected_cap;
    return slot;
  }

  // Gap bookkeeping for one step.  uniq: the step's selected ids, sorted
  // ascending, unique, all in [0, E).  Appends (local, slot) stream-ins in
  // issue order.  Returns 0, or -2 on overflow (state then matches the
  // reference at the point it raises).
  int gap(const int32_t* uniq, int n_uniq, bool fast_hit, std::vector<int>& streams,
          bool& map_write) {
    map_write = false;
    ++gaps;
    if (fast_hit && map_is_standing) {
      bool all_hit = true;
      for (int i = 0; i < n_uniq; ++i) {
        const int l = local_of[uniq[i]];
        if (l >= 0 && slot_of[l] < 0) {
          all_hit = false;
          break;
        }
      }
      if (all_hit) {
        ++fast_hits;
        return 0;
      }
    }
    missing.clear();
    for (int s = 0; s < S; ++s) claimed[s] = 0;
    for (int i = 0; i < n_uniq; ++i) {
      const int l = local_of[uniq[i]];
      if (l < 0) continue;
      const int slot = slot_of[l];
      if (slot < 0) {
        missing.push_back(l);
      } else {
        claimed[slot] = 1;  // hit_slots
        touch(slot, true);
      }
    }
    bool changed = false;
    if (!missing.empty()) {
      for (int l : missing) {
        const int slot = acquire(l, true);
        if (slot < 0) return -2;
        streams.push_back(l);
        streams.push_back(slot);
        claimed[slot] = 1;
      }
      misses += (int64_t)missing.size();
      changed = true;
    }
    if (changed || !map_is_standing) {
      map_write = true;
      ++map_writes;
      map_is_standing = true;
    }
    return 0;
  }

  // slot -> global id table of the standing map (-1 = empty slot).
  void slot_globals(int32_t* out) const {
    for (int s = 0; s < S; ++s) {
      const int l = expert_in_slot[s];
      out[s] = l >= 0 ? global_of_local[l] : -1;
    }
  }

  void standing_map(int32_t* map) const {
    for (int g = 0; g < E; ++g) map[g] = -1;
    for (int s = 0; s < S; ++s) {
      const int l = expert_in_slot[s];
      if (l < 0) continue;
      const int g = global_of_local[l];
      if (g >= 0 && g < E) map[g] = s;
    }
  }
};

}  // namespace slru
