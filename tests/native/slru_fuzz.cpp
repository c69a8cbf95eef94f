// Host-only stress of the native slot cache (sluice_amd/csrc/slru.h), built
// with AddressSanitizer and UndefinedBehaviorSanitizer: random layer shapes
// (full and expert-parallel ownership, pins, LFU and expert counts on or
// off) driven through random router-split gaps and classic steps, with the
// cache's structural invariants checked after every operation.  Prints "ok"
// and exits 0, or names the first broken invariant and exits 1.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <random>
#include <vector>

#include "slru.h"

namespace {

int fail(const char* what, int cfg, int step, int a, int b) {
  printf("FAIL %s (config %d, step %d: %d, %d)\n", what, cfg, step, a, b);
  return 1;
}

// Every slot is in exactly one place (free list, probation, protected,
// pinned), the two maps agree, the lists are well linked, protected stays
// within its cap.
int check(const slru::Cache& c, int cfg, int step) {
  const int S = c.S;
  std::vector<int> where(S, 0);
  for (int s : c.free_slots) {
    if (s < 0 || s >= S) return fail("free slot out of range", cfg, step, s, S);
    if (where[s]++) return fail("slot listed twice", cfg, step, s, 0);
    if (c.expert_in_slot[s] != -1) return fail("free slot holds an expert", cfg, step, s,
                                               c.expert_in_slot[s]);
    if (c.seg[s] != slru::kNone) return fail("free slot in a segment", cfg, step, s, c.seg[s]);
  }
  for (int sg = slru::kProbation; sg <= slru::kProtected; ++sg) {
    const slru::List& L = c.lists[sg];
    int n = 0, prev = -1;
    for (int s = L.head; s >= 0; s = c.next[s]) {
      if (s >= S) return fail("list link out of range", cfg, step, s, S);
      if (++n > S) return fail("list cycle", cfg, step, sg, n);
      if (where[s]++) return fail("slot listed twice", cfg, step, s, sg);
      if (c.seg[s] != sg) return fail("segment tag", cfg, step, s, c.seg[s]);
      if (c.prev[s] != prev) return fail("back link", cfg, step, s, c.prev[s]);
      if (c.expert_in_slot[s] < 0) return fail("listed slot empty", cfg, step, s, sg);
      prev = s;
    }
    if (n != L.size || prev != L.tail) return fail("list size or tail", cfg, step, n, L.size);
  }
  if (c.lists[slru::kProtected].size > c.protected_cap)
    return fail("protected over cap", cfg, step, c.lists[slru::kProtected].size, c.protected_cap);
  for (int s = 0; s < S; ++s) {
    if (c.seg[s] == slru::kPinned) {
      if (where[s]++) return fail("pinned slot listed", cfg, step, s, 0);
      if (c.expert_in_slot[s] < 0) return fail("pinned slot empty", cfg, step, s, 0);
    }
    if (where[s] != 1) return fail("slot not accounted for", cfg, step, s, where[s]);
    const int l = c.expert_in_slot[s];
    if (l >= 0 && (l >= c.local_n || c.slot_of[l] != s))
      return fail("slot -> expert -> slot", cfg, step, s, l);
  }
  for (int l = 0; l < c.local_n; ++l) {
    const int s = c.slot_of[l];
    if (s >= 0 && (s >= S || c.expert_in_slot[s] != l))
      return fail("expert -> slot -> expert", cfg, step, l, s);
  }
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  const int configs = argc > 1 ? atoi(argv[1]) : 120;
  const int steps = argc > 2 ? atoi(argv[2]) : 300;
  std::mt19937 rng(12345);
  auto uni = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
  for (int cfg = 0; cfg < configs; ++cfg) {
    const int E = uni(2, 300);
    const bool ep = uni(0, 3) == 0;
    std::vector<int32_t> lof(E);
    int local_n = 0;
    for (int g = 0; g < E; ++g) lof[g] = (!ep || uni(0, 1) == 0) ? local_n++ : -1;
    if (local_n == 0) {
      lof[0] = 0;
      local_n = 1;
    }
    const int S = uni(1, std::min(local_n, 128));
    const int cap = std::max(std::min(S * uni(0, 9) / 10, S - 1), 0);
    slru::Cache c;
    c.init(E, local_n, S, cap, lof.data());
    c.lfu = uni(0, 1) == 1;
    c.count = uni(0, 1) == 1;
    if (int rc = check(c, cfg, -1)) return rc;
    for (int p = uni(0, 3); p > 0; --p) {
      c.pin(uni(-1, local_n), uni(0, 1) == 1);
      if (int rc = check(c, cfg, -1)) return rc;
    }
    std::vector<int32_t> ids, uniq;
    std::vector<int> streams;
    slru::Plan plan;
    for (int step = 0; step < steps; ++step) {
      const int T = uni(1, 24), k = uni(1, std::min(8, E));
      ids.clear();
      // a hot set the steps revisit, plus fresh picks: hits, misses, evictions
      for (int i = 0; i < T * k; ++i)
        ids.push_back(uni(0, 3) ? uni(0, std::min(E - 1, S + 4)) : uni(0, E - 1));
      if (uni(0, 2)) {
        uniq = ids;
        std::sort(uniq.begin(), uniq.end());
        uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
        streams.clear();
        bool map_write = false;
        const int rc = c.gap(uniq.data(), (int)uniq.size(), uni(0, 1) == 1, streams, map_write);
        if (rc != 0 && rc != -2) return fail("gap status", cfg, step, rc, 0);
        for (size_t i = 0; i + 1 < streams.size(); i += 2)
          if (streams[i] < 0 || streams[i] >= local_n || streams[i + 1] < 0 || streams[i + 1] >= S)
            return fail("gap stream out of range", cfg, step, streams[i], streams[i + 1]);
        if (rc == 0)
          for (int g : uniq)
            if (lof[g] >= 0 && c.slot_of[lof[g]] < 0)
              return fail("selected expert not resident after gap", cfg, step, g, 0);
        // now and then the fills' copies fail: the tail of the streams leaves
        // the cache again (recovery), and a random slot is asked to as well
        if (!streams.empty() && uni(0, 4) == 0) {
          const int ns = (int)streams.size() / 2, landed = uni(0, ns - 1);
          for (int i = landed; i < ns; ++i) {
            const int slot = streams[2 * i + 1];
            const bool pinned = c.seg[slot] == slru::kPinned;
            if (c.unfill(slot) == pinned) return fail("unfill of a fill", cfg, step, slot, 0);
          }
          const int s = uni(0, S - 1);
          const bool had = c.expert_in_slot[s] >= 0 && c.seg[s] != slru::kPinned;
          if (c.unfill(s) != had) return fail("unfill of a random slot", cfg, step, s, 0);
        }
      } else {
        const int n = (int)ids.size();
        if (uni(0, 9) == 0) ids[uni(0, n - 1)] = E + uni(0, 5);  // out-of-range ids are ignored
        const int nd = uni(-1, T), ndec = uni(-1, T);
        const int rc = c.classic(ids.data(), n, T, nd, ndec, uni(0, 4) != 0, uni(0, 1), plan);
        if (rc != 0) {
          // the one refusal: misses left over and every slot pinned (nothing
          // to rotate them through; the reference has no answer either)
          bool all_pinned = true;
          for (int s = 0; s < S; ++s) all_pinned = all_pinned && c.seg[s] == slru::kPinned;
          if (rc != -1 || !all_pinned) return fail("classic status", cfg, step, rc, 0);
        }
        for (const slru::Wave& w : plan.waves) {
          for (int i = w.p0; i < w.p0 + w.np; ++i)
            if (plan.pairs[2 * i + 1] < 0 || plan.pairs[2 * i + 1] >= S)
              return fail("wave pair slot out of range", cfg, step, plan.pairs[2 * i + 1], S);
          for (int i = w.s0; i < w.s0 + w.ns; ++i)
            if (plan.streams[2 * i + 1] < 0 || plan.streams[2 * i + 1] >= S)
              return fail("wave stream slot out of range", cfg, step, plan.streams[2 * i + 1], S);
        }
      }
      if (int rc = check(c, cfg, step)) return rc;
    }
  }
  printf("ok\n");
  return 0;
}
