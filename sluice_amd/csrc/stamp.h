// Stamps of the gap mailbox records (host and device).
//
// Records of a layer are numbered 1, 2, ..., kStampMax, 1, ... (0 is "none
// yet", the stamp before 1) and record s lives in ring slot s % kRing.  The
// period kStampMax is a multiple of kRing, so consecutive stamps always take
// consecutive slots, also across the wrap: a slot is reused exactly kRing
// records later, which is what the device's free-slot test assumes.  Nothing
// here overflows a signed int.
//
// Plain C++ (no HIP headers), so a host-only build can test it.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define SLUICE_STAMP_HD __host__ __device__
#else
#define SLUICE_STAMP_HD
#endif

namespace sluice_stamp {

constexpr int kRing = 4;
constexpr int32_t kStampMax = (INT32_MAX / kRing) * kRing;
static_assert(kStampMax % kRing == 0, "stamp period must be a multiple of the ring");

// The stamp after s (s = 0 or any value outside 1..kStampMax starts at 1).
SLUICE_STAMP_HD inline int32_t next(int32_t s) {
  return (s <= 0 || s >= kStampMax) ? 1 : s + 1;
}

// Records from stamp b forward to stamp a (0 <= result < kStampMax); b = 0
// counts as kStampMax, the stamp before 1.
SLUICE_STAMP_HD inline int32_t dist(int32_t a, int32_t b) {
  int64_t d = (int64_t)a - (int64_t)b;
  if (d < 0) d += kStampMax;
  if (d >= kStampMax) d -= kStampMax;
  return (int32_t)d;
}

// Ring slot of record s.
SLUICE_STAMP_HD inline int slot(int32_t s) { return (int)(s % kRing); }

}  // namespace sluice_stamp
