// Host-only check of the gap mailbox stamps (sluice_amd/csrc/stamp.h):
// a ring writer and reader driven across the stamp wrap.  Prints "ok" and
// exits 0, or names the first broken property and exits 1.
#include <stdio.h>

#include "stamp.h"

namespace st = sluice_stamp;

static int fail(const char* what, long long a, long long b) {
  printf("FAIL %s (%lld, %lld)\n", what, a, b);
  return 1;
}

int main() {
  if (st::next(0) != 1) return fail("next(0)", st::next(0), 1);
  if (st::next(st::kStampMax) != 1) return fail("next(max)", st::next(st::kStampMax), 1);
  if (st::dist(1, 0) != 1) return fail("dist(1,0)", st::dist(1, 0), 1);
  if (st::dist(1, st::kStampMax) != 1) return fail("dist(1,max)", st::dist(1, st::kStampMax), 1);
  // Walk 64 stamps across the wrap.  The slot a stamp writes must be the one
  // the stamp kRing records earlier wrote, and no other stamp of the last
  // kRing - 1 records may hold it.
  int32_t hist[64];
  int32_t s = st::kStampMax - 20;
  for (int i = 0; i < 64; ++i) {
    hist[i] = s;
    if (i > 0) {
      if (st::dist(s, hist[i - 1]) != 1) return fail("dist(next, prev)", s, hist[i - 1]);
      if (st::slot(s) != (st::slot(hist[i - 1]) + 1) % st::kRing)
        return fail("consecutive slots", s, hist[i - 1]);
    }
    for (int j = 1; j < st::kRing && i - j >= 0; ++j)
      if (st::slot(hist[i - j]) == st::slot(s)) return fail("slot reused early", s, hist[i - j]);
    if (i >= st::kRing) {
      if (st::slot(hist[i - st::kRing]) != st::slot(s)) return fail("ring period", s, hist[i - st::kRing]);
      if (st::dist(s, hist[i - st::kRing]) != st::kRing)
        return fail("dist over the ring", s, hist[i - st::kRing]);
    }
    const int32_t n = st::next(s);
    if (n <= 0 || n > st::kStampMax) return fail("next out of range", s, n);
    s = n;
  }
  printf("ok\n");
  return 0;
}
