// a9/a10: grouped SwiGLU expert product over slot buffers + weighted combine.
//
// Replaces torch.ops.vllm.fused_experts(h, w13, w2, tw, ti, activation="silu",
// global_num_experts=E, expert_map=map) as called by the router-split entry
// (src/sluice/offloader.py:2590-2599) and vLLM's moe_sum.  The arithmetic is
// the textbook per-expert SwiGLU: gate/up = W13[s]·x (gate rows first, then
// up rows), act = silu(gate)*up, y = W2[s]·act, out[t] = sum_j w[t,j]*y[t,j];
// a pair whose expert maps to slot -1 contributes nothing.
//
// At decode (T <= 16 tokens, k <= 8) every expert sees 1..16 tokens, so the
// product is a weight stream: each (expert, 16-row tile) is read once from
// HBM and multiplied against the expert's token block on MFMA
// v_mfma_f32_16x16x32_bf16 -- weight rows on the MFMA M side (one 16-byte
// load per lane per 32-wide K chunk), tokens on the N side.  A workgroup is
// 4 waves that split K and reduce through LDS.
//
// Launch shape: align (1 WG) -> gemm1 (+silu*up) -> gemm2 (*w) -> combine,
// grid-stride kernels over a plan in global memory; the align launch is
// skipped when the caller hands in the plan its router-split gap kernel
// built.  (A single persistent kernel with cross-workgroup hand-offs was
// measured 1.6-1.8x slower than these launches and is not kept.)
#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "common.h"
#include "plan.h"
#include "trace.h"
#include "slotwait.h"
#include "stream.h"

// Scratch of sluice_fused_experts_bf16_noalloc (align plan, activations, fp32
// partials), for callers that cannot allocate.  Every GPU the library runs on
// holds its own copy until the process ends; host code reaches it only
// through the per-device address hipGetSymbolAddress returns (the name
// itself is not a device address in host code).
static __device__ __align__(256) uint8_t scratch[SLUICE_NOALLOC_SCRATCH_BYTES];

namespace {

using sluice_plan::kBM;          // tokens per block (MFMA N)
using sluice_plan::kBlockInts;   // {slot field, count, pair[16]}
// A block's slot field carries kPendingBit when the slot's rows may still be
// streaming in (a pending slot of the layer's last gap): its work items
// wait for the slot before they read its weights.
using sluice_plan::kPendingBit;
using sluice_plan::kSlotMask;
using sluice_plan::plan_ints;
constexpr int kPlanHeader = sluice_plan::kHeader;
constexpr int kKS = 4;                   // waves per workgroup (K split)
constexpr int kThreads = 64 * kKS;
static_assert(kThreads == sluice_plan::kPlanThreads, "the align kernel builds the plan");
constexpr int kG2T = 2;                  // 16-row hidden tiles per gemm2 item
constexpr int kFp8Blk = 128;

// Chunks in flight per wave.  Deeper pipelines measured no faster for
// gemm1 and slower for gemm2 and fp8 (fewer resident waves per CU).
#ifndef SLUICE_G1_D
#define SLUICE_G1_D 2
#endif
#ifndef SLUICE_G2_D
#define SLUICE_G2_D 2
#endif
#ifndef SLUICE_F8_D
#define SLUICE_F8_D 1
#endif
constexpr int kG1D = SLUICE_G1_D;  // bf16 gemm1: 64-wide K chunks in flight per wave
constexpr int kG2D = SLUICE_G2_D;  // bf16 gemm2
constexpr int kF8D = SLUICE_F8_D;  // fp8: 128-wide K chunks in flight per wave


// Align: the plan of the P routed pairs (sluice_plan::plan_build).
__global__ __launch_bounds__(kThreads) void moe_align_kernel(
    const int32_t* __restrict__ ids, int P, const int32_t* __restrict__ map, int E, int S,
    const int32_t* __restrict__ pending, int32_t* __restrict__ plan) {
  __shared__ sluice_plan::Scratch sc;
  (void)sluice_plan::plan_build(ids, P, map, E, S, pending, sc, plan);
}

typedef f32x4_t RedBuf[kKS][2][64];

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}

// Wave 0 reduces the 4 K-split partial accumulators and writes
// act[pair, tile*16 + kg*4 .. +4] = bf16(silu(g) * u).  COH: the row is read
// by other workgroups of the same launch, so it is stored device-coherent
// and written through before the closing barrier.
template <bool COH>
__device__ __forceinline__ void g1_epilogue(RedBuf& red, int pair, int tile, int I,
                                            uint16_t* __restrict__ act) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, kg = lane >> 4;
  __syncthreads();
  if (wave == 0 && pair >= 0) {
    f32x4_t g = red[0][0][lane], u = red[0][1][lane];
#pragma unroll
    for (int w = 1; w < kKS; ++w) {
      g += red[w][0][lane];
      u += red[w][1][lane];
    }
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = g[r] / (1.0f + expf(-g[r])) * u[r];
    uint16_t* dst = act + (size_t)pair * I + tile * 16 + kg * 4;
    if (COH) {
      st8_coh(dst, pack2_bf16(o[0], o[1]), pack2_bf16(o[2], o[3]));
      __builtin_amdgcn_s_waitcnt(0);
    } else {
      *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{pack2_bf16(o[0], o[1]), pack2_bf16(o[2], o[3])};
    }
  }
  __syncthreads();
}

// gemm2 work items: R row groups x kKS / R K parts per workgroup.  Wave w
// takes the 32-row tile group*R + w % R and K part w / R; the K parts of a
// tile reduce through LDS.  Measured over recorded decode routing (fraction
// of 8 TB/s for R = 1 / 2 / 4): bf16 V2-Lite (K = 1408, 22 chunks: 5+6+5+6
// at R = 1) 0.732 / 0.696 / 0.614, bf16 Qwen3 0.687 / 0.658 / 0.654, fp8
// DeepSeek-V3 0.778 / 0.811 / 0.786.  Smaller items (R = 1) balance the
// short bf16 launches best, despite uneven K parts; fp8 streams one chunk
// in flight per wave, so its waves gain from the longer streams of R = 2.
template <bool FP8>
struct G2Shape {
  static constexpr int R = FP8 ? 2 : 1;
  static constexpr int K = kKS / R;
  static_assert(R * K == kKS, "gemm2 waves");
};

// The first K part of each tile sums the tile's K parts and writes
// partial[pair, tile2*32 + t*16 + kg*4 .. +4] = w * sum.
template <int R>
__device__ __forceinline__ void g2_epilogue(RedBuf& red, int pair, int tile2, int n_tiles,
                                            int H, float wv, float* __restrict__ partial) {
  constexpr int K = kKS / R;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, kg = lane >> 4;
  if (K > 1) __syncthreads();
  if (wave < R && pair >= 0 && tile2 < n_tiles) {
#pragma unroll
    for (int t = 0; t < kG2T; ++t) {
      f32x4_t v = red[wave][t][lane];
#pragma unroll
      for (int q = 1; q < K; ++q) v += red[wave + q * R][t][lane];
      float* dst = partial + (size_t)pair * H + (tile2 * kG2T + t) * 16 + kg * 4;
      *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{wv * v[0], wv * v[1], wv * v[2], wv * v[3]};
    }
  }
  if (K > 1) __syncthreads();
}

// ---------------------------------------------------------------------------
// Work items stream their weights with stream_bf16 / stream_fp8: two 16-row
// tiles (the gate and up rows of an intermediate tile for gemm1; 32
// consecutive hidden rows for gemm2) against the block's token columns.
// ---------------------------------------------------------------------------
typedef u32x4_t StageBuf[kKS][kStageVecs];

struct ItemLds {
  RedBuf red;
  StageBuf stage;
};

// ---------------------------------------------------------------------------
// fp8 e4m3fn weights with 128x128 fp32 block scales, bf16 activations.  A
// chunk is 128 K elements (one scale block, one 128-byte segment per row).
// Lane (row R, K group kb) reads the 32 fp8 bytes kb*32 .. +32 of its row
// from LDS, widens them exactly to bf16 and issues four MFMAs against the
// token elements loaded in the same order; the fp32 sum over the chunk is
// multiplied by its scale before it joins the accumulator.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t pack_bf16_hi(float a, float b) {
  // fp8 values are exact in bf16: keep the top 16 bits of each fp32.
  return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
}

// 4 fp8 bytes -> 4 bf16 (two dwords).
__device__ __forceinline__ u32x2_t fp8x4_to_bf16x4(uint32_t v) {
  const f32x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(v, 1.0f, false);
  const f32x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(v, 1.0f, true);
  return u32x2_t{pack_bf16_hi(lo.x, lo.y), pack_bf16_hi(hi.x, hi.y)};
}

__device__ __forceinline__ void fp8x16_to_bf16(u32x4_t q, u32x4_t& lo, u32x4_t& hi) {
  const u32x2_t a = fp8x4_to_bf16x4(q[0]);
  const u32x2_t b = fp8x4_to_bf16x4(q[1]);
  const u32x2_t c = fp8x4_to_bf16x4(q[2]);
  const u32x2_t d = fp8x4_to_bf16x4(q[3]);
  lo = u32x4_t{a[0], a[1], b[0], b[1]};
  hi = u32x4_t{c[0], c[1], d[0], d[1]};
}

// As stream_bf16 for fp8 weights; s0 / s1: the tiles' scales, one per chunk
// (absolute chunk index).
template <int TM, int D>
__device__ __forceinline__ void stream_fp8(const uint8_t* __restrict__ a0,
                                           const uint8_t* __restrict__ a1, size_t ld,
                                           const float* __restrict__ s0,
                                           const float* __restrict__ s1,
                                           const uint16_t* __restrict__ b, int c0, int n,
                                           u32x4_t* st, f32x4_t& acc0, f32x4_t& acc1) {
  const int lane = threadIdx.x & 63;
  const int r = lane >> 3, s = lane & 7;
  const int R = lane & 15, kb = lane >> 4;
  const uint8_t* p0 = a0 + (size_t)r * ld + (size_t)c0 * 128 + s * 16;
  const uint8_t* p1 = a1 + (size_t)r * ld + (size_t)c0 * 128 + s * 16;
  const size_t ld8 = 8 * ld;
  const uint16_t* pb = b + (size_t)c0 * 128 + kb * 32;
  const int wl = r * 8 + (s ^ r), wh = wl + 64;
  const int rd0 = R * 8 + ((2 * kb) ^ (R & 7)), rd1 = R * 8 + ((2 * kb + 1) ^ (R & 7));
  u32x4_t q0l[D], q0h[D], q1l[D], q1h[D], xb[D][4];
  auto issue = [&](int d, int c) {
    const size_t o = (size_t)c * 128;
    q0l[d] = ldg16_stream(p0 + o);
    q0h[d] = ldg16_stream(p0 + ld8 + o);
    q1l[d] = ldg16_stream(p1 + o);
    q1h[d] = ldg16_stream(p1 + ld8 + o);
#pragma unroll
    for (int m = 0; m < 4; ++m)
      xb[d][m] = TM == kTokCoh ? ld16_coh(pb + o + m * 8) : ldg16(pb + o + m * 8);
  };
  auto consume = [&](int d, int c) {
    st[wl] = q0l[d];
    st[wh] = q0h[d];
    st[128 + wl] = q1l[d];
    st[128 + wh] = q1h[d];
    __builtin_amdgcn_wave_barrier();
    const u32x4_t g0 = st[rd0], g1 = st[rd1], u0 = st[128 + rd0], u1 = st[128 + rd1];
    __builtin_amdgcn_wave_barrier();
    u32x4_t w0, w1, w2, w3;
    f32x4_t t0 = {0.f, 0.f, 0.f, 0.f}, t1 = t0;
    fp8x16_to_bf16(g0, w0, w1);
    fp8x16_to_bf16(g1, w2, w3);
    t0 = mfma16x16x32_bf16(w0, xb[d][0], t0);
    t0 = mfma16x16x32_bf16(w1, xb[d][1], t0);
    t0 = mfma16x16x32_bf16(w2, xb[d][2], t0);
    t0 = mfma16x16x32_bf16(w3, xb[d][3], t0);
    fp8x16_to_bf16(u0, w0, w1);
    fp8x16_to_bf16(u1, w2, w3);
    t1 = mfma16x16x32_bf16(w0, xb[d][0], t1);
    t1 = mfma16x16x32_bf16(w1, xb[d][1], t1);
    t1 = mfma16x16x32_bf16(w2, xb[d][2], t1);
    t1 = mfma16x16x32_bf16(w3, xb[d][3], t1);
    acc0 += s0[c0 + c] * t0;
    acc1 += s1[c0 + c] * t1;
  };
  if (n <= 0) return;
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
      consume(d, base + d);
      issue(d, base + D + d);
      __builtin_amdgcn_sched_barrier(0);  // keep the load groups in issue order
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    if (base + d < n) {
      consume(d, base + d);
      if (base + D + d < n) issue(d, base + D + d);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (base + D + d < n) consume(d, base + D + d);
}

// ---------------------------------------------------------------------------
// Expert weights of a call.  Slots 0..S-1 are the routed slot buffers; slots
// S..S+n_sh-1 are the shared experts' virtual experts: the shared MLP of
// intermediate I_s = n_sh * I split into n_sh column groups of width I
// (silu(g) * u is per channel and the down projection sums over channels, so
// the MLP is exactly the sum of its groups).  Virtual expert v takes gate rows
// v*I.. and up rows I_s + v*I.. of sh_w13 [2*I_s, H] and columns v*I.. of
// sh_w2 [H, I_s]; fp8 scales cover 128x128 blocks of both, like the slots'.
// ---------------------------------------------------------------------------
struct ExpertW {
  const uint8_t* w13;
  const uint8_t* w2;
  const float* s13;
  const float* s2;
  const uint8_t* sh_w13;
  const uint8_t* sh_w2;
  const float* sh_s13;
  const float* sh_s2;
  int S;      // routed slots
  int I_s;    // shared intermediate (n_sh * I), 0 = none
  SlotWait wait;  // slots whose rows may still stream (none for plain calls)
};

// A work item on a block flagged kPendingBit waits (bounded by the gap's
// timeout and the abort flag) until the slot's rows of the pending gap have
// landed.  The first workgroup to claim the slot for that gap polls the
// host-mapped ready mark (and, now and then, the abort flag) about every
// 0.4 us -- one read in flight at a time -- and publishes the stamp -- or
// kSeenFailed -- in device memory; the others poll that, reading no host
// memory (device reads of host memory share the link with the rows
// streaming in; a poll every ~3.4 us measured 0.3% slower decode steps at
// V2-Lite c=8).  Each then takes a system-scope acquire, so no
// cache returns the slot's previous expert -- the poller right after the
// relaxed load that saw the mark (a second, acquiring read of the mark cost
// a bus round trip, ~1.1 us of every streamed layer's tail) and before it
// publishes; the workgroup's loads follow the barrier.  A failed wait is recorded in the layer's status word (the host
// reports it) and the item computes on whatever the slot holds.
constexpr int32_t kSeenFailed = -1;

__device__ __forceinline__ void await_slot(const SlotWait& w, int slot_field) {
  if ((slot_field & kPendingBit) == 0 || w.pending == nullptr) return;
  if (threadIdx.x == 0) {
    const int slot = slot_field & kSlotMask;
    const int32_t p = w.pending[slot];
    bool acquired = false;  // this thread's system-scope acquire already taken
    if (p != 0 &&
        __hip_atomic_load(&w.seen[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != p) {
      const bool poller = atomicExch(&w.claim[slot], p) != p;
      const long long t0 = wall_clock64();
      const long long lim = w.bound != nullptr ? *w.bound : kDefaultWaitTicks;
      int st = 0;
      if (poller) {
        for (unsigned it = 1;; ++it) {
          if (__hip_atomic_load(w.ready + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == p)
            break;
          if ((it & 15u) == 0 &&
              __hip_atomic_load(w.abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != 0) {
            st = SLUICE_E_ABORTED;
            break;
          }
          if (wall_clock64() - t0 > lim) {
            st = SLUICE_E_TIMEOUT;
            break;
          }
          __builtin_amdgcn_s_sleep(16);
        }
        SLUICE_DTRACE(10, ((unsigned long long)slot << 24) | ((unsigned long long)p & 0xffffff));
        if (st != 0) {
          __hip_atomic_store(w.status, st, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          __hip_atomic_store(&w.seen[slot], kSeenFailed, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        } else {
          // The load that saw the mark, then a system-scope acquire fence
          // (no second read over the bus), before the release that the
          // others acquire through seen[].
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
          acquired = true;
          __hip_atomic_store(&w.seen[slot], p, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        for (;;) {
          const int32_t v =
              __hip_atomic_load(&w.seen[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (v == p || v == kSeenFailed) break;
          // the poller's own bound ends every wait; this one is a backstop
          if (wall_clock64() - t0 > lim) break;
          __builtin_amdgcn_s_sleep(32);
        }
      }
    }
    if (p != 0 && !acquired) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
  }
  __syncthreads();
}

// Call shape: T tokens, k routed pairs each (P = T*k routed pairs); shared
// pairs follow as P + v*T + t.
struct CallShape {
  int T, k, H, I;
};

__device__ __forceinline__ int pair_token(const CallShape& c, int pair) {
  const int P = c.T * c.k;
  return pair < P ? pair / c.k : (pair - P) % c.T;
}

// Where gemm1's gate and up tiles (16 rows at `tile`) of `slot` live.
struct G1Src {
  const uint8_t* gate;
  const uint8_t* up;
  const float* sg;  // fp8 scale rows of the tiles (chunk c at [c])
  const float* su;
};

template <int ESZ>
__device__ __forceinline__ G1Src g1_src(const ExpertW& W, const CallShape& c, int slot, int tile) {
  const int H = c.H, I = c.I;
  const int nkb = H / kFp8Blk;
  G1Src r;
  if (slot < W.S) {
    const size_t rg = (size_t)slot * 2 * I + (size_t)tile * 16, ru = rg + I;
    r.gate = W.w13 + rg * H * ESZ;
    r.up = W.w13 + ru * H * ESZ;
    const size_t nrb = (size_t)(2 * I) / kFp8Blk;
    r.sg = W.s13 + ((size_t)slot * nrb + (size_t)tile * 16 / kFp8Blk) * nkb;
    r.su = W.s13 + ((size_t)slot * nrb + (size_t)(I + tile * 16) / kFp8Blk) * nkb;
  } else {
    const size_t v = (size_t)(slot - W.S);
    const size_t rg = v * I + (size_t)tile * 16, ru = (size_t)W.I_s + rg;
    r.gate = W.sh_w13 + rg * H * ESZ;
    r.up = W.sh_w13 + ru * H * ESZ;
    r.sg = W.sh_s13 + rg / kFp8Blk * nkb;
    r.su = W.sh_s13 + ru / kFp8Blk * nkb;
  }
  return r;
}

// Where gemm2's 32 hidden rows at tile2 of `slot` live: row r0's first K
// element, the row stride, fp8 scales of the 128-row block (chunk c at [c]).
struct G2Src {
  const uint8_t* a0;
  size_t ld;
  const float* sr;
};

template <int ESZ>
__device__ __forceinline__ G2Src g2_src(const ExpertW& W, const CallShape& c, int slot,
                                        int tile2) {
  const int H = c.H, I = c.I;
  const size_t r0 = (size_t)tile2 * 16 * kG2T;
  G2Src r;
  if (slot < W.S) {
    r.a0 = W.w2 + ((size_t)slot * H + r0) * I * ESZ;
    r.ld = (size_t)I;
    r.sr = W.s2 + ((size_t)slot * (H / kFp8Blk) + r0 / kFp8Blk) * (I / kFp8Blk);
  } else {
    const size_t v = (size_t)(slot - W.S);
    r.a0 = W.sh_w2 + (r0 * W.I_s + v * I) * ESZ;
    r.ld = (size_t)W.I_s;
    r.sr = W.sh_s2 + r0 / kFp8Blk * (W.I_s / kFp8Blk) + v * I / kFp8Blk;
  }
  return r;
}

// ---------------------------------------------------------------------------
// Work items.  `pair` = this lane's pair (column lane & 15), -1 if none; a
// lane without a pair streams token row 0 (or act row 0) so every load is
// issued unconditionally, and its column is never written.
// gemm1: gate and up rows tile*16 .. +16 of `slot` -> act (silu(g) * u).
// gemm2: hidden rows tile2*32 .. +32 of `slot` against act -> w * partial,
// w = the routing weight of a routed pair, 1 for a shared pair.
// ---------------------------------------------------------------------------
template <bool COH>
__device__ __forceinline__ void g1_item_bf16(const uint16_t* __restrict__ x, const ExpertW& W,
                                             const CallShape& cs, int slot, int pair, int tile,
                                             uint16_t* __restrict__ act, ItemLds& l) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int H = cs.H;
  const int nc = H / 64;
  const int c0 = wave * nc / kKS, c1 = (wave + 1) * nc / kKS;
  const G1Src src = g1_src<2>(W, cs, slot, tile);
  const uint16_t* xr = x + (size_t)(pair >= 0 ? pair_token(cs, pair) : 0) * H;
  f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
  stream_bf16<kTokPlain, kG1D>((const uint16_t*)src.gate, (const uint16_t*)src.up, H, xr, c0,
                               c1 - c0, l.stage[wave], ag, au);
  l.red[wave][0][lane] = ag;
  l.red[wave][1][lane] = au;
  g1_epilogue<COH>(l.red, pair, tile, cs.I, act);
}

__device__ __forceinline__ float pair_weight(const CallShape& cs, const float* __restrict__ tw,
                                             int pair) {
  return pair < 0 ? 0.f : pair < cs.T * cs.k ? tw[pair] : 1.0f;
}

template <int TM>
__device__ __forceinline__ void g2_item_bf16(const uint16_t* __restrict__ act, const ExpertW& W,
                                             const CallShape& cs, int slot, int pair, int group,
                                             const float* __restrict__ topk_w,
                                             float* __restrict__ partial, ItemLds& l) {
  constexpr int R = G2Shape<false>::R, K = kKS / R;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int I = cs.I, n_tiles = cs.H / (16 * kG2T);
  const int tile2 = group * R + wave % R, kp = wave / R;
  f32x4_t a = {0.f, 0.f, 0.f, 0.f}, b = a;
  if (tile2 < n_tiles) {
    const int nc = I / 64;
    const int c0 = kp * nc / K, c1 = (kp + 1) * nc / K;
    const G2Src src = g2_src<2>(W, cs, slot, tile2);
    const uint16_t* a0 = (const uint16_t*)src.a0;
    const uint16_t* ar = act + (size_t)(pair >= 0 ? pair : 0) * I;
    stream_bf16<TM, kG2D>(a0, a0 + 16 * src.ld, src.ld, ar, c0, c1 - c0, l.stage[wave], a, b);
  }
  l.red[wave][0][lane] = a;
  l.red[wave][1][lane] = b;
  g2_epilogue<R>(l.red, pair, tile2, n_tiles, cs.H, pair_weight(cs, topk_w, pair), partial);
}

template <bool COH>
__device__ __forceinline__ void g1_item_fp8(const uint16_t* __restrict__ x, const ExpertW& W,
                                            const CallShape& cs, int slot, int pair, int tile,
                                            uint16_t* __restrict__ act, ItemLds& l) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int H = cs.H;
  const int nkb = H / kFp8Blk;
  const int c0 = wave * nkb / kKS, c1 = (wave + 1) * nkb / kKS;
  const G1Src src = g1_src<1>(W, cs, slot, tile);
  const uint16_t* xr = x + (size_t)(pair >= 0 ? pair_token(cs, pair) : 0) * H;
  f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
  stream_fp8<kTokPlain, kF8D>(src.gate, src.up, H, src.sg, src.su, xr, c0, c1 - c0,
                              l.stage[wave], ag, au);
  l.red[wave][0][lane] = ag;
  l.red[wave][1][lane] = au;
  g1_epilogue<COH>(l.red, pair, tile, cs.I, act);
}

template <int TM>
__device__ __forceinline__ void g2_item_fp8(const uint16_t* __restrict__ act, const ExpertW& W,
                                            const CallShape& cs, int slot, int pair, int group,
                                            const float* __restrict__ topk_w,
                                            float* __restrict__ partial, ItemLds& l) {
  constexpr int R = G2Shape<true>::R, K = kKS / R;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int I = cs.I, n_tiles = cs.H / (16 * kG2T);
  const int tile2 = group * R + wave % R, kp = wave / R;
  f32x4_t a = {0.f, 0.f, 0.f, 0.f}, b = a;
  if (tile2 < n_tiles) {
    const int nkb = I / kFp8Blk;
    const int c0 = kp * nkb / K, c1 = (kp + 1) * nkb / K;
    const G2Src src = g2_src<1>(W, cs, slot, tile2);
    const uint16_t* ar = act + (size_t)(pair >= 0 ? pair : 0) * I;
    stream_fp8<TM, kF8D>(src.a0, src.a0 + 16 * src.ld, src.ld, src.sr, src.sr, ar, c0, c1 - c0,
                         l.stage[wave], a, b);
  }
  l.red[wave][0][lane] = a;
  l.red[wave][1][lane] = b;
  g2_epilogue<R>(l.red, pair, tile2, n_tiles, cs.H, pair_weight(cs, topk_w, pair), partial);
}

// ---------------------------------------------------------------------------
// Staged kernels: grid-stride loops over a plan in global memory.
// ---------------------------------------------------------------------------
template <bool FP8, bool COH = false>
__device__ __forceinline__ void run_g1(const uint16_t* x, const ExpertW& W, const CallShape& cs,
                                       int slot, int pair, int tile, uint16_t* act, ItemLds& l) {
  if (FP8)
    g1_item_fp8<COH>(x, W, cs, slot, pair, tile, act, l);
  else
    g1_item_bf16<COH>(x, W, cs, slot, pair, tile, act, l);
}

template <bool FP8, int TM = kTokPlain>
__device__ __forceinline__ void run_g2(const uint16_t* act, const ExpertW& W, const CallShape& cs,
                                       int slot, int pair, int group, const float* tw,
                                       float* partial, ItemLds& l) {
  if (FP8)
    g2_item_fp8<TM>(act, W, cs, slot, pair, group, tw, partial, l);
  else
    g2_item_bf16<TM>(act, W, cs, slot, pair, group, tw, partial, l);
}

// The blocks of a call: the plan's routed blocks, then the shared experts'
// virtual experts (slot S + v, n_sh = I_s / I of them), each over every
// token in blocks of <= kBM, pairs P + v*T + t (P = T*k).  A plan handed in
// by the caller is only read within this call's bounds: a block count
// above P, a pair outside [0, P) or a slot outside [0, S) cannot send a
// load or store out of the call's buffers.
__device__ __forceinline__ int routed_blocks(const int32_t* __restrict__ plan,
                                             const CallShape& cs) {
  return min(max(plan[0], 0), cs.T * cs.k);
}

__device__ __forceinline__ int call_blocks(const int32_t* __restrict__ plan, const ExpertW& W,
                                           const CallShape& cs) {
  const int n_sh = W.I_s / cs.I;
  return routed_blocks(plan, cs) + n_sh * ((cs.T + kBM - 1) / kBM);
}

// Block b's slot field and the pair of token column `col` (-1 if none).
__device__ __forceinline__ void block_at(const int32_t* __restrict__ plan, const ExpertW& W,
                                         const CallShape& cs, int b, int col, int& slot_field,
                                         int& pair) {
  const int nr = routed_blocks(plan, cs);
  if (b < nr) {
    const int32_t* blk = plan + kPlanHeader + (size_t)b * kBlockInts;
    slot_field = blk[0];
    const int p = col < blk[1] ? blk[2 + col] : -1;
    const bool ok = (unsigned)(slot_field & kSlotMask) < (unsigned)W.S &&
                    (unsigned)p < (unsigned)(cs.T * cs.k);
    pair = ok ? p : -1;
    if ((unsigned)(slot_field & kSlotMask) >= (unsigned)W.S) slot_field = 0;
  } else {
    const int nbt = (cs.T + kBM - 1) / kBM;
    const int sb = b - nr, v = sb / nbt, c = sb - v * nbt;
    const int t = c * kBM + col;
    slot_field = W.S + v;
    pair = t < cs.T ? cs.T * cs.k + v * cs.T + t : -1;
  }
}

// A block record loaded before the plan header is known, so the first item's
// record and the header come back in one memory round trip (b is clamped
// into the plan's T*k records: the loads stay inside the plan buffer).
// Used by gemm1: 1.3-1.9% shorter launches over recorded decode routing
// (V2-Lite and Qwen3 c=8); gemm2 measured no change with it.
struct PreBlock {
  int b, field, count, pair;
};

__device__ __forceinline__ PreBlock block_pre(const int32_t* __restrict__ plan,
                                              const CallShape& cs, int b, int col) {
  const int bc = min(b, max(cs.T * cs.k - 1, 0));
  const int32_t* blk = plan + kPlanHeader + (size_t)bc * kBlockInts;
  PreBlock r;
  r.b = b;
  r.field = blk[0];
  r.count = blk[1];
  r.pair = blk[2 + col];
  // The empty asm makes the loads (and the header's) issue here, together;
  // otherwise the compiler sinks them into the item loop, behind the
  // header's round trip.
  const int h0 = plan[0], h2 = plan[2];
  asm volatile("" ::"s"(r.field), "s"(r.count), "v"(r.pair), "s"(h0), "s"(h2));
  return r;
}

// block_at, taking block pre.b's record from `pre`.
__device__ __forceinline__ void block_at_pre(const int32_t* __restrict__ plan, const ExpertW& W,
                                             const CallShape& cs, int b, int col,
                                             const PreBlock& pre, int& slot_field, int& pair) {
  if (b == pre.b && b < routed_blocks(plan, cs)) {
    slot_field = pre.field;
    const int p = col < pre.count ? pre.pair : -1;
    const bool ok = (unsigned)(slot_field & kSlotMask) < (unsigned)W.S &&
                    (unsigned)p < (unsigned)(cs.T * cs.k);
    pair = ok ? p : -1;
    if ((unsigned)(slot_field & kSlotMask) >= (unsigned)W.S) slot_field = 0;
  } else {
    block_at(plan, W, cs, b, col, slot_field, pair);
  }
}

// The plan's first routed blocks whose slots are not pending (plan[2],
// clamped to the routed blocks; any value gives the same product, only the
// order of the work changes).
__device__ __forceinline__ int resident_blocks(const int32_t* __restrict__ plan,
                                               const CallShape& cs) {
  return min(max(plan[2], 0), routed_blocks(plan, cs));
}

// gemm1 over the call's blocks.  With a hand-off area (the split launch
// below follows) it covers only the resident routed blocks and the shared
// ones, and workgroup 0 clears the area: [ticket counter | per pending
// block: gemm1 items done].
template <bool FP8>
__global__ __launch_bounds__(kThreads) void moe_gemm1_kernel(const uint16_t* __restrict__ x,
                                                             ExpertW W,
                                                             const int32_t* __restrict__ plan,
                                                             CallShape cs,
                                                             uint16_t* __restrict__ act,
                                                             int32_t* __restrict__ handoff) {
  __shared__ ItemLds lds;
  const int n_tiles = cs.I / 16;
  const PreBlock pre = block_pre(plan, cs, blockIdx.x / n_tiles, threadIdx.x & 15);
  const int nr = routed_blocks(plan, cs);
  const int n_res = handoff != nullptr ? resident_blocks(plan, cs) : nr;
  const int n_skip = nr - n_res;  // routed blocks [n_res, nr) are left to the split launch
  if (handoff != nullptr && blockIdx.x == 0)
    for (int i = threadIdx.x; i <= cs.T * cs.k; i += kThreads)
      __hip_atomic_store(handoff + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int total = (call_blocks(plan, W, cs) - n_skip) * n_tiles;
  const int col = threadIdx.x & 15;
  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int bb = item / n_tiles, tile = item - bb * n_tiles;
    int slot_field, pair;
    block_at_pre(plan, W, cs, bb < n_res ? bb : bb + n_skip, col, pre, slot_field, pair);
    await_slot(W.wait, slot_field);
    run_g1<FP8>(x, W, cs, slot_field & kSlotMask, pair, tile, act, lds);
  }
}

__host__ __device__ inline int g2_groups(int H, bool fp8) {
  const int n_tiles = H / (16 * kG2T);
  const int R = fp8 ? G2Shape<true>::R : G2Shape<false>::R;
  return (n_tiles + R - 1) / R;
}

template <bool FP8>
__global__ __launch_bounds__(kThreads) void moe_gemm2_kernel(const uint16_t* __restrict__ act,
                                                             ExpertW W,
                                                             const int32_t* __restrict__ plan,
                                                             const float* __restrict__ topk_w,
                                                             CallShape cs,
                                                             float* __restrict__ partial) {
  __shared__ ItemLds lds;
  const int n_groups = g2_groups(cs.H, FP8);
  const int total = call_blocks(plan, W, cs) * n_groups;
  const int col = threadIdx.x & 15;
  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int b = item / n_groups, g = item - b * n_groups;
    int slot_field, pair;
    block_at(plan, W, cs, b, col, slot_field, pair);
    await_slot(W.wait, slot_field);
    run_g2<FP8>(act, W, cs, slot_field & kSlotMask, pair, g, topk_w, partial, lds);
  }
}

// Bounded wait (thread 0) until *count reaches `want`; a bound reached is
// recorded as a timeout in the status word (when there is one).  The bound
// is twice the slot wait's: the items counted wait for their slot (bounded
// by it) and then compute.
__device__ __forceinline__ void wait_count(const int32_t* count, int want, const long long* bound,
                                           int32_t* status) {
  const long long t0 = wall_clock64();
  const long long ticks = 2 * (bound != nullptr ? *bound : kDefaultWaitTicks);
  while (__hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < want) {
    if (wall_clock64() - t0 > ticks) {
      if (status != nullptr)
        __hip_atomic_store(status, SLUICE_E_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      return;
    }
    __builtin_amdgcn_s_sleep(4);
  }
}

// The second launch of a product whose plan may hold pending blocks, one work
// item per workgroup, so that gemm2 of the resident experts runs while the
// pending slots' rows still stream in (with the single gemm2 launch it waited
// for gemm1 of the last pending expert).  Items:
//   [gemm2 of the resident and shared blocks | gemm1 of the pending blocks |
//    gemm2 of the pending blocks];
// a pending gemm1 item stores its act tile device-coherent and counts itself
// in its block's hand-off counter; a pending gemm2 item waits for its slot,
// then (bounded) for its block's count to reach the gemm1 tile count, and
// reads act coherently.
// The pending items take their order from a ticket counter, not from
// blockIdx: a workgroup holding a gemm2 ticket waits only on gemm1 tickets
// already taken, i.e. on running workgroups that wait for nothing but the
// host's ready marks, so the waits end whatever order the hardware
// dispatches workgroups in.  The grid must cover every item (the host sizes
// it for the largest plan of the call); workgroups beyond the items exit.
template <bool FP8>
__global__ __launch_bounds__(kThreads) void moe_gemm2_split_kernel(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ act, ExpertW W,
    const int32_t* __restrict__ plan, const float* __restrict__ topk_w, CallShape cs,
    float* __restrict__ partial, int32_t* __restrict__ handoff) {
  __shared__ ItemLds lds;
  __shared__ int s_ticket;
  const int n_groups = g2_groups(cs.H, FP8), n_tiles = cs.I / 16;
  const int nr = routed_blocks(plan, cs), n_res = resident_blocks(plan, cs);
  const int n_pend = nr - n_res;
  const int n_first = (call_blocks(plan, W, cs) - n_pend) * n_groups;
  const int n_g1 = n_pend * n_tiles, n_g2 = n_pend * n_groups;
  const int col = threadIdx.x & 15;
  const int item = blockIdx.x;
  if (item == 0 && threadIdx.x == 0) SLUICE_DTRACE(11, gridDim.x);
  int slot_field, pair;
  if (item < n_first) {
    const int bb = item / n_groups, g = item - bb * n_groups;
    block_at(plan, W, cs, bb < n_res ? bb : bb + n_pend, col, slot_field, pair);
    await_slot(W.wait, slot_field);
    run_g2<FP8>(act, W, cs, slot_field & kSlotMask, pair, g, topk_w, partial, lds);
    return;
  }
  if (item >= n_first + n_g1 + n_g2) return;
  if (threadIdx.x == 0) s_ticket = atomicAdd(handoff, 1);
  __syncthreads();
  const int t = s_ticket;
  int32_t* done = handoff + 1;
  if (t < n_g1) {
    const int pb = t / n_tiles, tile = t - pb * n_tiles;
    block_at(plan, W, cs, n_res + pb, col, slot_field, pair);
    await_slot(W.wait, slot_field);
    if (threadIdx.x == 0) SLUICE_DTRACE(14, t);
    run_g1<FP8, true>(x, W, cs, slot_field & kSlotMask, pair, tile, act, lds);
    if (threadIdx.x == 0) atomicAdd(done + pb, 1);
    if (threadIdx.x == 0) SLUICE_DTRACE(15, t);
  } else if (t < n_g1 + n_g2) {
    // First the slot (a gentle wait, like the gemm1 items'), then the few
    // microseconds of its gemm1 items (a tight one): a tight wait over the
    // whole stream-in would poll one word as hard as the copies write.
    const int pb = (t - n_g1) / n_groups, g = (t - n_g1) - pb * n_groups;
    block_at(plan, W, cs, n_res + pb, col, slot_field, pair);
    await_slot(W.wait, slot_field);
    if (threadIdx.x == 0) wait_count(done + pb, n_tiles, W.wait.bound, W.wait.status);
    if (threadIdx.x == 0) SLUICE_DTRACE(17, t);
    __syncthreads();
    run_g2<FP8, kTokCoh>(act, W, cs, slot_field & kSlotMask, pair, g, topk_w, partial, lds);
    if (threadIdx.x == 0) SLUICE_DTRACE(16, t);
  }
}

// out[t, h] = bf16(scale * sum_j valid ? partial[t*k+j, h] : 0
//                  + sum_v partial[T*k + v*T + t, h] + shared[t, h]),
// j and v ascending, for 4 consecutive columns at h: the routed pairs
// scaled, the shared experts' virtual experts (n_sh <= kMaxShared) and a
// precomputed shared output added unscaled.  Only rows that are added are
// loaded.  The shared groups present are known from the arguments; whether
// a routed pair is valid is a plan word.  SPEC (decode-sized calls, where
// every pair inside the router-split envelope is valid and the kernel is
// latency-bound): the valid words and the rows go out together and the
// thread waits on memory once; a row whose pair turns out invalid is read
// and not added.  !SPEC (large calls: prefill chunks, classic waves, where
// many pairs of a wave are invalid and the kernel is bandwidth-bound): the
// valid words first, then only the valid rows.
constexpr int kMaxShared = 4;
// partial bytes of a call above which the combine reads valid words first
constexpr long kCombineCheckFirstBytes = 2L << 20;

template <bool SPEC>
__device__ __forceinline__ void combine4(const float* __restrict__ partial,
                                         const int32_t* __restrict__ valid, int t, int T, int k,
                                         int n_sh, int H, int h, float scale,
                                         const uint16_t* __restrict__ shared,
                                         uint16_t* __restrict__ out) {
  auto ld = [&](int p) { return *reinterpret_cast<const f32x4_t*>(partial + (size_t)p * H + h); };
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  f32x4_t v[SLUICE_MAX_TOPK], vs[kMaxShared];
  bool ok[SLUICE_MAX_TOPK];
  u32x2_t sh = {0u, 0u};
  if (shared != nullptr) sh = *reinterpret_cast<const u32x2_t*>(shared + (size_t)t * H + h);
#pragma unroll
  for (int j = 0; j < SLUICE_MAX_TOPK; ++j) ok[j] = j < k && valid[t * k + j] != 0;
#pragma unroll
  for (int j = 0; j < SLUICE_MAX_TOPK; ++j) {
    if (SPEC)
      v[j] = j < k ? ld(t * k + j) : zero;
    else
      v[j] = ok[j] ? ld(t * k + j) : zero;
  }
  const int P = T * k;
#pragma unroll
  for (int u = 0; u < kMaxShared; ++u) vs[u] = u < n_sh ? ld(P + u * T + t) : zero;
  f32x4_t acc = zero, acs = zero;
#pragma unroll
  for (int j = 0; j < SLUICE_MAX_TOPK; ++j)
    if (ok[j]) acc += v[j];
#pragma unroll
  for (int u = 0; u < kMaxShared; ++u)
    if (u < n_sh) acs += vs[u];
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    o[r] = scale * acc[r] + acs[r];
    if (shared != nullptr)
      o[r] += __uint_as_float(r & 1 ? (sh[r >> 1] & 0xffff0000u) : (sh[r >> 1] << 16));
  }
  *reinterpret_cast<u32x2_t*>(out + (size_t)t * H + h) =
      u32x2_t{pack2_bf16(o[0], o[1]), pack2_bf16(o[2], o[3])};
}

template <bool SPEC>
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float* __restrict__ partial, const int32_t* __restrict__ valid, int T, int k, int n_sh,
    int H, float scale, const uint16_t* __restrict__ shared, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) SLUICE_DTRACE(13, T);
  if (h >= H) return;
  combine4<SPEC>(partial, valid, t, T, k, n_sh, H, h, scale, shared, out);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Workspace {
  int32_t* plan;
  int32_t* handoff;
  uint16_t* act;
  float* partial;
};

// [plan of the T*k routed pairs | hand-off counters (1 + T*k) | act [P2, I]
// bf16 | partial [P2, H] fp32], P2 = T*k routed + n_sh*T shared pairs.  Every
// call writes what it reads (align writes the whole plan, gemm1 clears the
// counters the split launch uses and writes the act rows of the planned
// pairs, gemm2 their partials; the combine adds only valid pairs), so the
// workspace needs no clearing and holds nothing between calls.
size_t workspace_bytes(int T, int H, int I, int k, int n_sh, Workspace* ws, void* base) {
  const int P2 = T * k + n_sh * T;
  const size_t plan_b = align_up(plan_ints(T * k) * sizeof(int32_t), 256);
  const size_t hand_b = align_up((size_t)(1 + T * k) * sizeof(int32_t), 256);
  const size_t act_b = align_up((size_t)P2 * I * sizeof(uint16_t), 256);
  const size_t part_b = align_up((size_t)P2 * H * sizeof(float), 256);
  if (ws != nullptr) {
    char* b = (char*)base;
    ws->plan = (int32_t*)b;
    ws->handoff = (int32_t*)(b + plan_b);
    ws->act = (uint16_t*)(b + plan_b + hand_b);
    ws->partial = (float*)(b + plan_b + hand_b + act_b);
  }
  return plan_b + hand_b + act_b + part_b;
}

#ifndef SLUICE_GRID_CAP
#define SLUICE_GRID_CAP 8192
#endif
int grid_for(int P, int n_tiles) {
  const long items = (long)P * n_tiles;  // upper bound on (block, tile) items
  const long cap = SLUICE_GRID_CAP;
  return (int)(items < cap ? (items > 0 ? items : 1) : cap);
}

// Grid of the split launch: one workgroup per item of the largest plan of
// the call (every routed block pending costs a gemm1 and a gemm2 item per
// block, P >= routed blocks, P2 >= all blocks), or 0 when that exceeds
// kSplitGridMax (prefill-sized calls keep the two grid-stride launches).
constexpr long kSplitGridMax = 1L << 15;
long split_grid_for(int P, int P2, int I, int n_groups) {
  const long g = (long)P2 * n_groups + (long)P * (I / 16);
  return g <= kSplitGridMax ? g : 0;
}

// Workgroups of a grid-stride launch over a map whose slots may stream, all
// of which may wait for slots at the same time.  The gap's row copies go to
// the SDMA engines; a host-to-device copy that runs as a kernel instead (a
// HIP-stream copy of small host rows, or any copy with SDMA switched off in
// the runtime) is one 512-thread workgroup at 16 VGPRs per lane, and if
// waiting workgroups held every CU, such a copy could not start and the
// waits it feeds would run to their bound.  So the grid leaves one of the
// kernel's workgroup places per CU free: (workgroups per CU at its occupancy
// - 1) x CUs, looked up once per device and kernel.  The split launch keeps
// one item per workgroup (a loop over tickets costs it a wave of occupancy);
// build.py checks instead that at full occupancy its waves leave that
// copy kernel's 32 VGPRs per SIMD free.
constexpr int kWaitDevices = 64;
enum WaitKernel { kWaitG1Bf16, kWaitG1Fp8, kWaitG2Bf16, kWaitG2Fp8, kWaitKinds };
std::atomic<int> g_wait_grid[kWaitDevices][kWaitKinds];

template <typename K>
int wait_grid(K kernel, WaitKernel kind, int* out) {
  int dev = 0;
  SLUICE_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kWaitDevices) return SLUICE_E_INVAL;
  int n = g_wait_grid[dev][kind].load(std::memory_order_relaxed);
  if (n == 0) {
    int per_cu = 0, cus = 0;
    SLUICE_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0));
    SLUICE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    n = std::max(per_cu - 1, 1) * std::max(cus, 1);
    g_wait_grid[dev][kind].store(n, std::memory_order_relaxed);
  }
  *out = n;
  return SLUICE_OK;
}

// The align kernel stages the map of all E experts in LDS.
int check_common(int T, int H, int I, int k, int E, int S, int n_sh, const void* x,
                 const void* w13, const void* w2, const float* tw, const int32_t* ti,
                 const void* shared, void* ws, size_t ws_bytes, void* out) {
  if (T < 0 || H <= 0 || I <= 0 || k <= 0 || k > SLUICE_MAX_TOPK || E <= 0 ||
      E > SLUICE_MAX_EXPERTS || S <= 0 || S > SLUICE_MAX_SLOTS)
    return SLUICE_E_INVAL;
  if ((long)T * k > SLUICE_MAX_PAIRS) return SLUICE_E_INVAL;
  if (n_sh < 0 || n_sh > kMaxShared || (long)T * (k + n_sh) > SLUICE_MAX_PAIRS)
    return SLUICE_E_INVAL;
  if (H % 64 != 0 || I % 64 != 0) return SLUICE_E_INVAL;
  if (T == 0) return SLUICE_OK;
  if (!x || !w13 || !w2 || !tw || !ti || !ws || !out) return SLUICE_E_INVAL;
  if (ws_bytes < workspace_bytes(T, H, I, k, n_sh, nullptr, nullptr)) return SLUICE_E_INVAL;
  if (((uintptr_t)x | (uintptr_t)w13 | (uintptr_t)w2 | (uintptr_t)ws | (uintptr_t)out) & 15)
    return SLUICE_E_INVAL;
  if ((uintptr_t)shared & 7) return SLUICE_E_INVAL;
  return SLUICE_OK;
}

int launch_combine(const float* partial, const int32_t* valid, int T, int k, int n_sh, int H,
                   float scale, const void* shared, void* out, hipStream_t st) {
  dim3 grid((H / 4 + 255) / 256, T);
  if ((long)T * k * H * (long)sizeof(float) > kCombineCheckFirstBytes)
    hipLaunchKernelGGL(moe_combine_kernel<false>, grid, dim3(256), 0, st, partial, valid, T, k,
                       n_sh, H, scale, (const uint16_t*)shared, (uint16_t*)out);
  else
    hipLaunchKernelGGL(moe_combine_kernel<true>, grid, dim3(256), 0, st, partial, valid, T, k,
                       n_sh, H, scale, (const uint16_t*)shared, (uint16_t*)out);
  return (int)hipGetLastError();
}

// plan: a plan of these ids over this map built on the stream before the
// call (by the layer's gap kernel), or nullptr: the align kernel builds one
// in the workspace.
template <bool FP8>
int run_experts(const void* x, const ExpertW& W, const float* tw, const int32_t* ti,
                const int32_t* map, int T, int H, int I, int k, int E, int S, int n_sh,
                float scale, const void* shared, void* workspace, const int32_t* plan,
                void* out, hipStream_t st) {
  Workspace w;
  workspace_bytes(T, H, I, k, n_sh, &w, workspace);
  const int P = T * k, P2 = P + n_sh * T;
  const CallShape cs{T, k, H, I};
  ExpertW Ww = W;
  if (map != nullptr) Ww.wait = slotwait_lookup(map);
  if (plan == nullptr) {
    hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kThreads), 0, st, ti, P, map, E, S,
                       Ww.wait.pending, w.plan);
    SLUICE_HIP_CHECK(hipGetLastError());
    plan = w.plan;
  }
  const long split_grid = split_grid_for(P, P2, I, g2_groups(H, FP8));
  if (Ww.wait.pending != nullptr && split_grid > 0) {
    // Slots of this map may stream: gemm1 of the resident blocks, then the
    // split launch (gemm2 of the resident blocks while the pending ones
    // stream, their gemm1 and gemm2 as their rows land).
    hipLaunchKernelGGL((moe_gemm1_kernel<FP8>), dim3(grid_for(P2, I / 16)), dim3(kThreads), 0, st,
                       (const uint16_t*)x, Ww, plan, cs, w.act, w.handoff);
    SLUICE_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL((moe_gemm2_split_kernel<FP8>), dim3((unsigned)split_grid), dim3(kThreads),
                       0, st, (const uint16_t*)x, w.act, Ww, plan, tw, cs, w.partial, w.handoff);
    SLUICE_HIP_CHECK(hipGetLastError());
  } else {
    // Grid-stride launches (any grid gives the same product): where slots
    // may stream, every workgroup may wait, so the grid stays within
    // wait_grid's bound.
    int g1 = grid_for(P2, I / 16), g2 = grid_for(P2, g2_groups(H, FP8));
    if (Ww.wait.pending != nullptr) {
      int c1 = 0, c2 = 0;
      int rc = wait_grid(moe_gemm1_kernel<FP8>, FP8 ? kWaitG1Fp8 : kWaitG1Bf16, &c1);
      if (rc == SLUICE_OK)
        rc = wait_grid(moe_gemm2_kernel<FP8>, FP8 ? kWaitG2Fp8 : kWaitG2Bf16, &c2);
      if (rc != SLUICE_OK) return rc;
      g1 = std::min(g1, c1);
      g2 = std::min(g2, c2);
    }
    hipLaunchKernelGGL((moe_gemm1_kernel<FP8>), dim3(g1), dim3(kThreads), 0, st,
                       (const uint16_t*)x, Ww, plan, cs, w.act, (int32_t*)nullptr);
    SLUICE_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL((moe_gemm2_kernel<FP8>), dim3(g2), dim3(kThreads), 0, st, w.act, Ww, plan,
                       tw, cs, w.partial);
    SLUICE_HIP_CHECK(hipGetLastError());
  }
  return launch_combine(w.partial, plan + kPlanHeader + (size_t)kBlockInts * P, T, k, n_sh, H,
                        scale, shared, out, st);
}

// Shared-expert weights: none (shared_I == 0), or n_sh = shared_I / I
// virtual experts (shared_I a multiple of I, n_sh <= kMaxShared).
int shared_groups(int shared_I, int I, const void* sw13, const void* sw2, int* n_sh) {
  *n_sh = 0;
  if (shared_I == 0) return SLUICE_OK;
  if (shared_I < 0 || I <= 0 || shared_I % I != 0 || shared_I / I > kMaxShared || !sw13 || !sw2 ||
      (((uintptr_t)sw13 | (uintptr_t)sw2) & 15))
    return SLUICE_E_INVAL;
  *n_sh = shared_I / I;
  return SLUICE_OK;
}

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_ptr(void** out) {
  int dev = 0;
  SLUICE_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    SLUICE_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (p == nullptr) return SLUICE_E_STATE;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SLUICE_OK;
}

// Weights of the per-stage entry points: every block's slot is routed.
ExpertW routed_only(const uint8_t* w13, const uint8_t* w2, const float* s13, const float* s2) {
  return ExpertW{w13, w2, s13, s2, nullptr, nullptr, nullptr, nullptr, 0x7fffffff, 0, SlotWait{}};
}

}  // namespace

extern "C" size_t sluice_moe_plan_ints(int T, int k) { return plan_ints(T * k); }

extern "C" size_t sluice_fused_experts_workspace(int T, int H, int I, int k, int shared_I) {
  if (T <= 0 || k <= 0) return 256;
  const int n_sh = (I > 0 && shared_I > 0) ? (shared_I + I - 1) / I : 0;
  return workspace_bytes(T, H, I, k, n_sh, nullptr, nullptr);
}

extern "C" int sluice_moe_align(const int32_t* topk_ids, int T, int k, const int32_t* expert_map,
                                int E, int S, int32_t* plan, sluice_stream_t stream) {
  if (T < 0 || k <= 0 || E <= 0 || E > SLUICE_MAX_EXPERTS || S <= 0 || S > SLUICE_MAX_SLOTS ||
      (long)T * k > SLUICE_MAX_PAIRS || plan == nullptr)
    return SLUICE_E_INVAL;
  const int32_t* pending =
      expert_map != nullptr ? slotwait_lookup(expert_map).pending : nullptr;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, topk_ids,
                     T * k, expert_map, E, S, pending, plan);
  return (int)hipGetLastError();
}

extern "C" int sluice_fused_experts_bf16(const void* x, const void* w13, const void* w2,
                                         const float* topk_w, const int32_t* topk_ids,
                                         const int32_t* expert_map, int T, int H, int I, int k,
                                         int E, int S, float scale, const void* shared_w13,
                                         const void* shared_w2, int shared_I, const void* shared,
                                         void* workspace, size_t workspace_bytes_, void* out,
                                         const int32_t* plan, sluice_stream_t stream) {
  int n_sh = 0;
  int rc = shared_groups(shared_I, I, shared_w13, shared_w2, &n_sh);
  if (rc != SLUICE_OK) return rc;
  rc = check_common(T, H, I, k, E, S, n_sh, x, w13, w2, topk_w, topk_ids, shared, workspace,
                    workspace_bytes_, out);
  if (rc != SLUICE_OK || T == 0) return rc;
  const ExpertW W{(const uint8_t*)w13, (const uint8_t*)w2, nullptr, nullptr,
                  (const uint8_t*)shared_w13, (const uint8_t*)shared_w2, nullptr, nullptr, S,
                  shared_I};
  return run_experts<false>(x, W, topk_w, topk_ids, expert_map, T, H, I, k, E, S, n_sh, scale,
                            shared, workspace, plan, out, (hipStream_t)stream);
}

extern "C" int sluice_fused_experts_bf16_noalloc(
    const void* x, const void* w13, const void* w2, const float* topk_w,
    const int32_t* topk_ids, const int32_t* expert_map, int T, int H, int I, int k, int E, int S,
    float scale, const void* shared_w13, const void* shared_w2, int shared_I, const void* shared,
    void* out, const int32_t* plan, sluice_stream_t stream) {
  int n_sh = 0;
  int rc = shared_groups(shared_I, I, shared_w13, shared_w2, &n_sh);
  if (rc != SLUICE_OK) return rc;
  // Every check runs before the scratch is looked up, so a refused call
  // touches no device state.
  if (T > 0 && H > 0 && I > 0 && k > 0 && (long)T * (k + n_sh) <= SLUICE_MAX_PAIRS &&
      workspace_bytes(T, H, I, k, n_sh, nullptr, nullptr) > SLUICE_NOALLOC_SCRATCH_BYTES)
    return SLUICE_E_SCRATCH;
  // (the workspace argument is an aligned stand-in for the scratch)
  rc = check_common(T, H, I, k, E, S, n_sh, x, w13, w2, topk_w, topk_ids, shared,
                    reinterpret_cast<void*>(uintptr_t{256}), SLUICE_NOALLOC_SCRATCH_BYTES, out);
  if (rc != SLUICE_OK || T == 0) return rc;
  void* ws = nullptr;
  rc = scratch_ptr(&ws);
  if (rc != SLUICE_OK) return rc;
  const ExpertW W{(const uint8_t*)w13, (const uint8_t*)w2, nullptr, nullptr,
                  (const uint8_t*)shared_w13, (const uint8_t*)shared_w2, nullptr, nullptr, S,
                  shared_I};
  return run_experts<false>(x, W, topk_w, topk_ids, expert_map, T, H, I, k, E, S, n_sh, scale,
                            shared, ws, plan, out, (hipStream_t)stream);
}

extern "C" int sluice_fused_experts_fp8(const void* x, const void* w13, const float* w13_scale,
                                        const void* w2, const float* w2_scale, int block_n,
                                        int block_k, const float* topk_w,
                                        const int32_t* topk_ids, const int32_t* expert_map, int T,
                                        int H, int I, int k, int E, int S, float scale,
                                        const void* shared_w13, const float* shared_w13_scale,
                                        const void* shared_w2, const float* shared_w2_scale,
                                        int shared_I, const void* shared, void* workspace,
                                        size_t workspace_bytes_, void* out,
                                        const int32_t* plan, sluice_stream_t stream) {
  if (block_n != kFp8Blk || block_k != kFp8Blk) return SLUICE_E_INVAL;
  if (H % kFp8Blk != 0 || I % kFp8Blk != 0) return SLUICE_E_INVAL;
  int n_sh = 0;
  int rc = shared_groups(shared_I, I, shared_w13, shared_w2, &n_sh);
  if (rc != SLUICE_OK) return rc;
  if (n_sh > 0 && (shared_w13_scale == nullptr || shared_w2_scale == nullptr))
    return SLUICE_E_INVAL;
  rc = check_common(T, H, I, k, E, S, n_sh, x, w13, w2, topk_w, topk_ids, shared, workspace,
                    workspace_bytes_, out);
  if (rc != SLUICE_OK || T == 0) return rc;
  if (w13_scale == nullptr || w2_scale == nullptr) return SLUICE_E_INVAL;
  const ExpertW W{(const uint8_t*)w13, (const uint8_t*)w2, w13_scale, w2_scale,
                  (const uint8_t*)shared_w13, (const uint8_t*)shared_w2, shared_w13_scale,
                  shared_w2_scale, S, shared_I};
  return run_experts<true>(x, W, topk_w, topk_ids, expert_map, T, H, I, k, E, S, n_sh, scale,
                           shared, workspace, plan, out, (hipStream_t)stream);
}

extern "C" int sluice_moe_gemm1_bf16(const void* x, const void* w13, const int32_t* plan, int T,
                                     int H, int I, int k, void* act, sluice_stream_t stream) {
  if (T <= 0 || k <= 0 || H <= 0 || I <= 0 || H % 64 || I % 64 || (long)T * k > SLUICE_MAX_PAIRS ||
      !x || !w13 || !plan || !act)
    return SLUICE_E_INVAL;
  const ExpertW W = routed_only((const uint8_t*)w13, nullptr, nullptr, nullptr);
  hipLaunchKernelGGL(moe_gemm1_kernel<false>, dim3(grid_for(T * k, I / 16)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const uint16_t*)x, W, plan, CallShape{T, k, H, I},
                     (uint16_t*)act, (int32_t*)nullptr);
  return (int)hipGetLastError();
}

extern "C" int sluice_moe_gemm2_bf16(const void* act, const void* w2, const int32_t* plan,
                                     const float* topk_w, int T, int H, int I, int k,
                                     float* partial, sluice_stream_t stream) {
  if (T <= 0 || k <= 0 || H <= 0 || I <= 0 || H % 64 || I % 64 ||
      (long)T * k > SLUICE_MAX_PAIRS || !act || !w2 || !plan || !topk_w || !partial)
    return SLUICE_E_INVAL;
  const ExpertW W = routed_only(nullptr, (const uint8_t*)w2, nullptr, nullptr);
  hipLaunchKernelGGL(moe_gemm2_kernel<false>, dim3(grid_for(T * k, g2_groups(H, false))),
                     dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)act, W, plan, topk_w,
                     CallShape{T, k, H, I}, partial);
  return (int)hipGetLastError();
}

extern "C" int sluice_moe_gemm1_fp8(const void* x, const void* w13, const float* w13_scale,
                                    const int32_t* plan, int T, int H, int I, int k, void* act,
                                    sluice_stream_t stream) {
  if (T <= 0 || k <= 0 || H <= 0 || I <= 0 || H % kFp8Blk || I % kFp8Blk ||
      (long)T * k > SLUICE_MAX_PAIRS || !x || !w13 || !w13_scale || !plan || !act)
    return SLUICE_E_INVAL;
  const ExpertW W = routed_only((const uint8_t*)w13, nullptr, w13_scale, nullptr);
  hipLaunchKernelGGL(moe_gemm1_kernel<true>, dim3(grid_for(T * k, I / 16)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const uint16_t*)x, W, plan, CallShape{T, k, H, I},
                     (uint16_t*)act, (int32_t*)nullptr);
  return (int)hipGetLastError();
}

extern "C" int sluice_moe_gemm2_fp8(const void* act, const void* w2, const float* w2_scale,
                                    const int32_t* plan, const float* topk_w, int T, int H, int I,
                                    int k, float* partial, sluice_stream_t stream) {
  if (T <= 0 || k <= 0 || H <= 0 || I <= 0 || H % kFp8Blk || I % kFp8Blk ||
      (long)T * k > SLUICE_MAX_PAIRS || !act || !w2 || !w2_scale || !plan || !topk_w || !partial)
    return SLUICE_E_INVAL;
  const ExpertW W = routed_only(nullptr, (const uint8_t*)w2, nullptr, w2_scale);
  hipLaunchKernelGGL(moe_gemm2_kernel<true>, dim3(grid_for(T * k, g2_groups(H, true))),
                     dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)act, W, plan, topk_w,
                     CallShape{T, k, H, I}, partial);
  return (int)hipGetLastError();
}

extern "C" int sluice_moe_combine(const float* partial, const int32_t* plan, int T, int k, int H,
                                  float scale, const void* shared, void* out,
                                  sluice_stream_t stream) {
  if (T <= 0 || k <= 0 || H <= 0 || H % 4 || (long)T * k > SLUICE_MAX_PAIRS || !partial || !plan ||
      !out || (((uintptr_t)shared | (uintptr_t)out | (uintptr_t)partial) & 7))
    return SLUICE_E_INVAL;
  return launch_combine(partial, plan + kPlanHeader + (size_t)kBlockInts * T * k, T, k, 0, H, scale,
                        shared, out, (hipStream_t)stream);
}

// Gap timeline tracing (trace.h): this translation unit's ring.
int trace_moe_read(unsigned long long* out, unsigned* n) {
#ifdef SLUICE_TRACE
  return trace_dev_read(out, n);
#else
  (void)out;
  (void)n;
  return SLUICE_E_STATE;
#endif
}
int trace_moe_reset() {
#ifdef SLUICE_TRACE
  return trace_dev_reset();
#else
  return SLUICE_E_STATE;
#endif
}
