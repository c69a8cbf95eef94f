// Host-side slot cache: the per-layer SLRU state machine of the streaming gap.
//
// Follows the reference's Python state machine step for step:
//   _ExpertLayerCache fields      src/sluice/offloader.py:121-169
//   free list / caps at install   src/sluice/offloader.py:936-947
//   _touch                        src/sluice/offloader.py:2009-2021
//   _coldest_protected (LRU)      src/sluice/offloader.py:2023-2034
//   _acquire_slot / _evict_to     src/sluice/offloader.py:2036-2081
//   _router_split_gap bookkeeping src/sluice/offloader.py:2405-2467
//   run_moe / _run_waves planning src/sluice/offloader.py:1540-1765, 1846-1890
//   opt-in LFU (SLUICE_LFU)       src/sluice/offloader.py:1993-2007, 2023-2034, 2057-2068
//   opt-in expert counts          src/sluice/offloader.py:1026-1034, 1664-1671
// The reference keeps its two segments in OrderedDicts keyed by slot
// (insertion order = recency, first = LRU).  Here each segment is an
// intrusive doubly-linked list over slot indices with O(1) unlink and
// append, which reproduces OrderedDict order exactly: `d[s] = None` for a
// new key appends, `move_to_end` relinks at the tail, `del` unlinks, and
// iteration walks from the head.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <vector>

namespace slru {

enum Seg : uint8_t { kNone = 0, kProbation = 1, kProtected = 2, kPinned = 3 };

struct List {
  int head = -1, tail = -1, size = 0;
};

// One wave of a classic step: pairs [p0, p0 + np) of Plan::pairs are the
// (global, slot) entries of the map the wave runs with (every other entry
// -1); streams [s0, s0 + ns) of Plan::streams are the (local, slot) rows
// copied in before it runs.
struct Wave {
  int p0, np, s0, ns;
};

struct Plan {
  std::vector<Wave> waves;
  std::vector<int32_t> pairs;    // (global, slot) flattened
  std::vector<int32_t> streams;  // (local, slot) flattened
  bool pipelined = false;        // waves >= 1 alternate between two slot groups
  void clear() {
    waves.clear();
    pairs.clear();
    streams.clear();
    pipelined = false;
  }
  void open_wave() {
    waves.push_back({(int)pairs.size() / 2, 0, (int)streams.size() / 2, 0});
  }
  void add_pair(int g, int slot) {
    pairs.push_back(g);
    pairs.push_back(slot);
    ++waves.back().np;
  }
  void add_stream(int local, int slot) {
    streams.push_back(local);
    streams.push_back(slot);
    ++waves.back().ns;
  }
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
  // Opt-in policies.  LFU: per-local selection frequency of real classic
  // steps, halved every kLfuAgeSteps of them; while any is nonzero, protected
  // victims are taken least frequent first (LRU among equals).  Counts: per-
  // global decode-class / scan-class selections of real classic steps.
  static constexpr int kLfuAgeSteps = 256;
  bool lfu = false, count = false;
  std::vector<int64_t> freq;       // [local_n]
  int freq_nonzero = 0;            // entries of freq above zero
  int lfu_steps = 0;
  std::vector<int64_t> cnt_decode, cnt_scan;  // [E]
  int64_t steps_small = 0, steps_scan = 0;
  // Real classic steps by class (0 = pure decode "small", 1 = "scan"): hit
  // and missed local experts and waves run, as the reference's per-class
  // step stats count them (src/sluice/offloader.py:1656-1684, 1711-1713, 1887).
  int64_t cls_hits[2] = {0, 0}, cls_misses[2] = {0, 0}, cls_waves[2] = {0, 0};

  // scratch reused across gaps and classic steps
  struct Pair {
    int g, local;
    bool dcls;
  };
  std::vector<uint8_t> claimed;
  std::vector<int> missing;
  std::vector<uint8_t> present, decode;
  std::vector<Pair> cl_pairs, cl_missing;
  std::vector<int> rot, order;

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
    freq.assign(local_n, 0);
    freq_nonzero = 0;
    lfu_steps = 0;
    cnt_decode.assign(E, 0);
    cnt_scan.assign(E, 0);
  }

  bool lfu_active() const { return lfu && freq_nonzero > 0; }
  int64_t heat(int slot) const {
    const int l = expert_in_slot[slot];
    return l >= 0 ? freq[l] : 0;
  }

  // _coldest_protected: LRU, or under LFU the least frequent (first of equals)
  int coldest_protected() const {
    int best = lists[kProtected].head;
    if (!lfu_active()) return best;
    for (int c = best; c >= 0; c = next[c])
      if (heat(c) < heat(best)) best = c;
    return best;
  }

  // _bump_freq
  void bump_freq(int local) {
    if (freq[local]++ == 0) ++freq_nonzero;
  }
  void age_freq() {
    if (++lfu_steps < kLfuAgeSteps) return;
    lfu_steps = 0;
    freq_nonzero = 0;
    for (int64_t& f : freq) {
      f >>= 1;
      freq_nonzero += f > 0;
    }
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
          const int demoted = coldest_protected();
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
        if (lfu_active()) {
          // protected walked coldest first, LRU among equals
          order.clear();
          for (int c = lists[kProtected].head; c >= 0; c = next[c]) order.push_back(c);
          std::stable_sort(order.begin(), order.end(),
                           [this](int a, int b) { return heat(a) < heat(b); });
          for (int c : order) {
            if (!claimed[c]) {
              slot = c;
              unlink(c);
              break;
            }
          }
        } else {
          for (int c = lists[kProtected].head; c >= 0; c = next[c]) {
            if (!claimed[c]) {
              slot = c;
              unlink(c);
              break;
            }
          }
        }
      }
    }
    if (slot < 0) return -1;
    evict_to(slot, local);
    push_back(kProbation, slot);  // new entries start probationary
    return slot;
  }

  // Recovery after a fill whose rows did not land (a failed copy): the
  // slot's expert leaves the cache -- its segment, slot_of, expert_in_slot
  // -- and the slot goes back on the free list (popped next), so the next
  // gap that selects the expert misses and streams it again.  The map stops
  // being the standing map.  No counterpart in the reference, whose copy
  // errors end the engine.  Returns false for a slot holding nothing or a
  // pinned expert (pins are loaded once, at install).
  bool unfill(int slot) {
    if (slot < 0 || slot >= S) return false;
    const int l = expert_in_slot[slot];
    if (l < 0 || seg[slot] == kPinned) return false;
    if (seg[slot] != kNone) unlink(slot);
    slot_of[l] = -1;
    expert_in_slot[slot] = -1;
    free_slots.push_back(slot);
    map_is_standing = false;
    return true;
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

  // Classic step (run_moe, src/sluice/offloader.py:1540-1765, and the
  // planning half of _run_waves, 1855-1890) on the flat row-major [T, k]
  // ids.  nd / ndec: the step's decode-token / decode-request counts, < 0
  // when the engine publishes none; real_step false for dummy runs.  Fills
  // `plan` with the waves in execution order.  Returns 0, or -1 when the
  // leftover misses have no slot to rotate through (every slot pinned;
  // the reference would loop forever).
  int classic(const int32_t* ids, int n, int T, int nd, int ndec, bool real_step,
              int spec_tokens, Plan& plan) {
    plan.clear();
    const int k = T > 0 ? n / T : 0;
    present.assign(E, 0);
    for (int i = 0; i < n; ++i)
      if ((unsigned)ids[i] < (unsigned)E) present[ids[i]] = 1;
    // Decode-hot rows [0, nd) only when they are all one-token decodes:
    // nd == ndec * (1 + spec_tokens) (1568-1576).
    const bool has_nd = nd >= 0, has_ndec = ndec >= 0;
    const long long span = has_ndec ? (long long)ndec * (1 + spec_tokens) : -1;
    const bool pure_region = real_step && has_nd && has_ndec && (long long)nd == span;
    const bool have_dec = pure_region && nd > 0 && nd <= T;
    decode.assign(E, 0);
    if (have_dec) {
      if (nd == T) {
        decode = present;
      } else {
        const int m = nd * k < n ? nd * k : n;
        for (int i = 0; i < m; ++i)
          if ((unsigned)ids[i] < (unsigned)E) decode[ids[i]] = 1;
      }
    }
    cl_pairs.clear();  // (global, local, decode class) in ascending global id
    for (int g = 0; g < E; ++g)
      if (present[g] && local_of[g] >= 0) cl_pairs.push_back({g, local_of[g], decode[g] != 0});
    const int ws = (int)cl_pairs.size();
    // No per-token signal: real steps whose working set fits the decode
    // capacity (pinned + protected) count as decode-class (1620-1637).
    const bool forced_scan = real_step && has_nd && !pure_region;
    bool friendly = false;  // the working-set heuristic classified the step decode
    if (!have_dec && !forced_scan) {
      int n_pinned = 0;
      for (int s = 0; s < S; ++s) n_pinned += seg[s] == kPinned;
      const int cap = protected_cap + n_pinned;
      friendly = real_step && ws <= (cap > 1 ? cap : 1);
      if (friendly)
        for (Pair& p : cl_pairs) p.dcls = true;
    }
    map_is_standing = false;
    plan.open_wave();
    if (ws == 0) return 0;
    int cls = -1;  // the step's stats class; dummy runs have none
    if (real_step) {
      const bool pure_decode = have_dec ? nd == T : friendly;
      ++(pure_decode ? steps_small : steps_scan);
      cls = pure_decode ? 0 : 1;
      if (lfu) {
        for (const Pair& p : cl_pairs) bump_freq(p.local);
        age_freq();
      }
      if (count)
        for (const Pair& p : cl_pairs) ++(p.dcls ? cnt_decode : cnt_scan)[p.g];
    }
    cl_missing.clear();
    for (int s = 0; s < S; ++s) claimed[s] = 0;
    for (const Pair& p : cl_pairs) {
      const int slot = slot_of[p.local];
      if (slot < 0) {
        cl_missing.push_back(p);
      } else {
        touch(slot, p.dcls);
        plan.add_pair(p.g, slot);
        claimed[slot] = 1;
      }
    }
    // decode-class misses take slots first (stable)
    std::stable_partition(cl_missing.begin(), cl_missing.end(),
                          [](const Pair& p) { return p.dcls; });
    size_t taken = cl_missing.size();
    for (size_t i = 0; i < cl_missing.size(); ++i) {
      const Pair& p = cl_missing[i];
      const int slot = acquire(p.local, p.dcls);
      if (slot < 0) {
        taken = i;
        break;
      }
      plan.add_stream(p.local, slot);
      plan.add_pair(p.g, slot);
      claimed[slot] = 1;
    }
    misses += (int64_t)cl_missing.size();
    if (cls >= 0) {
      cls_hits[cls] += (int64_t)(cl_pairs.size() - cl_missing.size());
      cls_misses[cls] += (int64_t)cl_missing.size();
    }
    if (taken == cl_missing.size()) {
      if (cls >= 0) ++cls_waves[cls];
      return 0;
    }
    // Leftover misses rotate through the probation slots split in two
    // groups (ping-pong); with no probation slot, through the last S/4
    // unpinned slots.  Protected slots are never rotated (1855-1890).
    rot.clear();
    for (int s = lists[kProbation].head; s >= 0; s = next[s]) rot.push_back(s);
    if (rot.empty()) {
      for (int s = 0; s < S; ++s)
        if (seg[s] != kPinned) rot.push_back(s);
      const size_t keep = S / 4 > 1 ? (size_t)(S / 4) : 1;
      if (rot.size() > keep) rot.erase(rot.begin(), rot.end() - keep);
    }
    if (rot.empty()) return -1;
    const size_t half = (rot.size() + 1) / 2;
    plan.pipelined = rot.size() > half;
    size_t i = taken;
    for (int gi = 0; i < cl_missing.size(); ++gi) {
      const bool b = (gi & 1) && plan.pipelined;
      const size_t g0 = b ? half : 0, g1 = b ? rot.size() : half;
      plan.open_wave();
      for (size_t j = g0; j < g1 && i < cl_missing.size(); ++j, ++i) {
        const Pair& p = cl_missing[i];
        const int slot = rot[j];
        evict_to(slot, p.local);
        plan.add_pair(p.g, slot);
        plan.add_stream(p.local, slot);
      }
    }
    if (cls >= 0) cls_waves[cls] += (int64_t)plan.waves.size();
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
