// Weight streaming for decode-sized products (gfx950, wave64).
//
// The expert GEMMs and the decoder's skinny GEMMs are weight streams: a few
// (<= 16) token columns against matrices read once from HBM.  Here a wave
// multiplies two 16-row weight tiles by the token columns over a range of
// 64-element K chunks:
//
//   * weights are read as whole 128-byte row segments: one 16-byte load per
//     lane covers 8 rows x 128 B (row lane >> 3, segment lane & 7) -- loads
//     of 16 rows x 64 B each ran ~15% slower on MI355X;
//   * each wave stages its segments through 4 KB of LDS, XOR-swizzled
//     (segment s of row r at s ^ (r & 7)) so that the row-major writes and
//     the MFMA-order reads are both free of bank conflicts, and reads them
//     back in the A layout of v_mfma_f32_16x16x32_bf16 (row lane & 15, K
//     group lane >> 4);
//   * the K groups of a segment go to (MFMA m, K group kb) as group
//     2*kb + m; the token operand is loaded in the same order, so every dot
//     product is the same sum of the same products;
//   * D chunks are in flight; the steady loop issues its loads
//     unconditionally, so the compiler waits for exactly the chunk it
//     consumes (a conditional reload made it drain every load in flight each
//     round).
#pragma once

#include "common.h"

// Device-coherent (sc1) 16-byte load / 8-byte store: values handed between
// workgroups on different XCDs go through these instead of writing back /
// invalidating whole L2 caches.
__device__ __forceinline__ u32x4_t ld16_coh(const void* p) {
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return u32x4_t{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}
__device__ __forceinline__ void st8_coh(void* p, uint32_t lo, uint32_t hi) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), (uint64_t)lo | ((uint64_t)hi << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave's LDS stage: 2 tiles x 16 rows x 8 segments of 16 bytes.
constexpr int kStageVecs = 256;

// How the token operand is read.
enum TokMode {
  kTokPlain = 0,  // bf16 rows, ordinary loads
  kTokCoh = 1     // bf16 rows written by other workgroups of the same launch
};

// acc0 / acc1 += tile 0 / tile 1 [16 rows, K chunks c0 .. c0+n) . tokens^T.
// a0, a1: row 0 of each tile (row stride ld elements); b: this lane's token
// row (column lane & 15) at K offset 0; st: this wave's stage.  n <= 0 is a
// no-op.  Every lane of the wave must call it (it uses the whole wave).
template <int TM, int D>
__device__ __forceinline__ void stream_bf16(const uint16_t* __restrict__ a0,
                                            const uint16_t* __restrict__ a1, size_t ld,
                                            const uint16_t* __restrict__ b, int c0, int n,
                                            u32x4_t* st, f32x4_t& acc0, f32x4_t& acc1) {
  if (n <= 0) return;
  const int lane = threadIdx.x & 63;
  const int r = lane >> 3, s = lane & 7;
  const int R = lane & 15, kb = lane >> 4;
  const uint16_t* p0 = a0 + (size_t)r * ld + (size_t)c0 * 64 + s * 8;
  const uint16_t* p1 = a1 + (size_t)r * ld + (size_t)c0 * 64 + s * 8;
  const size_t ld8 = 8 * ld;
  const uint16_t* pb = b + (size_t)c0 * 64 + kb * 16;
  const int wl = r * 8 + (s ^ r), wh = wl + 64;
  const int rd0 = R * 8 + ((2 * kb) ^ (R & 7)), rd1 = R * 8 + ((2 * kb + 1) ^ (R & 7));
  u32x4_t q0l[D], q0h[D], q1l[D], q1h[D], xb[D][2];
  auto ldb = [&](const uint16_t* p) { return TM == kTokCoh ? ld16_coh(p) : ldg16(p); };
  auto issue = [&](int d, int c) {
    const size_t o = (size_t)c * 64;
    q0l[d] = ldg16_stream(p0 + o);
    q0h[d] = ldg16_stream(p0 + ld8 + o);
    q1l[d] = ldg16_stream(p1 + o);
    q1h[d] = ldg16_stream(p1 + ld8 + o);
    xb[d][0] = ldb(pb + o);
    xb[d][1] = ldb(pb + o + 8);
  };
  auto consume = [&](int d) {
    st[wl] = q0l[d];
    st[wh] = q0h[d];
    st[128 + wl] = q1l[d];
    st[128 + wh] = q1h[d];
    __builtin_amdgcn_wave_barrier();
    const u32x4_t g0 = st[rd0], g1 = st[rd1], u0 = st[128 + rd0], u1 = st[128 + rd1];
    __builtin_amdgcn_wave_barrier();
    const u32x4_t x0 = xb[d][0], x1 = xb[d][1];
    acc0 = mfma16x16x32_bf16(g0, x0, acc0);
    acc0 = mfma16x16x32_bf16(g1, x1, acc0);
    acc1 = mfma16x16x32_bf16(u0, x0, acc1);
    acc1 = mfma16x16x32_bf16(u1, x1, acc1);
  };
  // The prologue issues every group (a wave with n < D re-reads its last
  // chunk) so that the load count at the loop head does not depend on n.
#pragma unroll
  for (int d = 0; d < D; ++d) {
    issue(d, d < n ? d : n - 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  int base = 0;
  for (; base + 2 * D <= n; base += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      consume(d);
      issue(d, base + D + d);
      __builtin_amdgcn_sched_barrier(0);  // keep the load groups in issue order
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    if (base + d < n) {
      consume(d);
      if (base + D + d < n) issue(d, base + D + d);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (base + D + d < n) consume(d);
}
