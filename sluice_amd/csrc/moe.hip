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
// v_mfma_f32_16x16x32_bf16 — weight rows on the MFMA M side (one 16-byte
// load per lane per 32-wide K chunk), tokens on the N side.  A workgroup is
// KS waves that split K and reduce through LDS; the grid strides over
// (block, tile) items whose count is known only on the device.
//
// Kernels per call:  align (1 WG)  ->  gemm1 (+silu*up)  ->  gemm2 (*w)
//                    ->  combine (sum over k, *scale, +shared, -> bf16).
#include <math.h>

#include "common.h"

namespace {

constexpr int kBM = SLUICE_BLOCK_M;      // tokens per block (MFMA N)
constexpr int kBlockInts = 2 + kBM;      // {slot, count, pair[16]}
constexpr int kPlanHeader = 4;
constexpr int kKS = 4;                   // waves per workgroup (K split)
constexpr int kAlignThreads = 256;

__host__ __device__ inline size_t plan_ints(int P) {
  return (size_t)kPlanHeader + (size_t)kBlockInts * P + (size_t)P;
}

__device__ __forceinline__ int pair_slot(const int32_t* ids, const int32_t* map, int p, int E,
                                         int S) {
  const int g = ids[p];
  if ((unsigned)g >= (unsigned)E) return -1;
  const int s = map != nullptr ? map[g] : g;
  return ((unsigned)s < (unsigned)S) ? s : -1;
}

// ---------------------------------------------------------------------------
// Align: group the P = T*k pairs by slot into blocks of <= 16, slots
// ascending and pairs ascending inside a slot (deterministic).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(
    const int32_t* __restrict__ ids, int P, const int32_t* __restrict__ map, int E, int S,
    int32_t* __restrict__ plan) {
  __shared__ int cnt[SLUICE_MAX_SLOTS];
  __shared__ int boff[SLUICE_MAX_SLOTS];
  __shared__ int run[SLUICE_MAX_SLOTS];
  __shared__ int chunk_slot[kAlignThreads];
  __shared__ int wsum[kAlignThreads / SLUICE_WAVE];
  __shared__ int total_blocks;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  int32_t* blocks = plan + kPlanHeader;
  int32_t* valid = plan + kPlanHeader + (size_t)kBlockInts * P;

  for (int s = tid; s < S; s += kAlignThreads) {
    cnt[s] = 0;
    run[s] = 0;
  }
  __syncthreads();
  for (int p = tid; p < P; p += kAlignThreads) {
    const int s = pair_slot(ids, map, p, E, S);
    if (s >= 0) atomicAdd(&cnt[s], 1);
  }
  __syncthreads();

  // Exclusive scan of blocks-per-slot; thread t owns slots [t*per, t*per+per).
  const int per = (S + kAlignThreads - 1) / kAlignThreads;
  int mine = 0;
  for (int i = 0; i < per; ++i) {
    const int s = tid * per + i;
    if (s < S) mine += (cnt[s] + kBM - 1) / kBM;
  }
  int incl = mine;
#pragma unroll
  for (int off = 1; off < SLUICE_WAVE; off <<= 1) {
    const int v = __shfl_up(incl, off, SLUICE_WAVE);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int wbase = 0;
  for (int w = 0; w < wave; ++w) wbase += wsum[w];
  int acc = wbase + incl - mine;
  for (int i = 0; i < per; ++i) {
    const int s = tid * per + i;
    if (s < S) {
      boff[s] = acc;
      acc += (cnt[s] + kBM - 1) / kBM;
    }
  }
  if (tid == kAlignThreads - 1) total_blocks = wbase + incl;
  __syncthreads();

  // Ranks in pair order, one chunk of 256 pairs at a time.
  for (int c = 0; c < P; c += kAlignThreads) {
    const int p = c + tid;
    const int s = p < P ? pair_slot(ids, map, p, E, S) : -1;
    chunk_slot[tid] = s;
    __syncthreads();
    if (s >= 0) {
      int r = run[s];
      for (int q = 0; q < tid; ++q) r += (chunk_slot[q] == s) ? 1 : 0;
      const int b = boff[s] + r / kBM;
      const int pos = r % kBM;
      int32_t* blk = blocks + (size_t)b * kBlockInts;
      blk[2 + pos] = p;
      if (pos == 0) {
        blk[0] = s;
        const int left = cnt[s] - (r / kBM) * kBM;
        blk[1] = left < kBM ? left : kBM;
      }
    }
    if (p < P) valid[p] = s >= 0 ? 1 : 0;
    __syncthreads();
    if (s >= 0) atomicAdd(&run[s], 1);
    __syncthreads();
  }
  if (tid == 0) {
    plan[0] = total_blocks;
    plan[1] = P;
  }
}

// Tunables (compile-time): waves per workgroup splitting K, register
// prefetch depth in 32-wide K chunks, and hidden rows per GEMM2 item.
#ifndef SLUICE_G1_KS
#define SLUICE_G1_KS 4
#endif
#ifndef SLUICE_G1_D
#define SLUICE_G1_D 8
#endif
#ifndef SLUICE_G2_KS
#define SLUICE_G2_KS 4
#endif
#ifndef SLUICE_G2_D
#define SLUICE_G2_D 8
#endif
#ifndef SLUICE_G2_TILES
#define SLUICE_G2_TILES 2
#endif
constexpr int kG1KS = SLUICE_G1_KS, kG1D = SLUICE_G1_D;
constexpr int kG2KS = SLUICE_G2_KS, kG2D = SLUICE_G2_D, kG2T = SLUICE_G2_TILES;

// ---------------------------------------------------------------------------
// GEMM1: act[pair, i] = bf16(silu(gate) * up) for one 16-row intermediate
// tile of one block.  bf16 weights.  Each wave owns a contiguous K range and
// keeps kG1D chunks (3 x 16 B per lane each) in flight: the loads for chunk
// c + kG1D are issued as soon as chunk c has been consumed.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64 * kG1KS) void moe_gemm1_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w13,
    const int32_t* __restrict__ plan, int H, int I, int k, uint16_t* __restrict__ act) {
  __shared__ f32x4_t red[kG1KS][2][64];
  const int n_blocks = plan[0];
  const int n_tiles = I / 16;
  const int total = n_blocks * n_tiles;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kg = lane >> 4;
  const int nchunk = H / 32;
  const int c0 = wave * nchunk / kG1KS, c1 = (wave + 1) * nchunk / kG1KS;
  const int n = c1 - c0;
  const int32_t* blocks = plan + kPlanHeader;

  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int b = item / n_tiles, tile = item - b * n_tiles;
    const int32_t* blk = blocks + (size_t)b * kBlockInts;
    const int slot = blk[0], cnt = blk[1];
    const int pair = col < cnt ? blk[2 + col] : -1;
    const uint16_t* wg =
        w13 + ((size_t)slot * 2 * I + (size_t)tile * 16 + col) * H + kg * 8 + c0 * 32;
    const uint16_t* wu = wg + (size_t)I * H;
    const uint16_t* xr = x + (size_t)(pair >= 0 ? pair / k : 0) * H + kg * 8 + c0 * 32;
    const bool hx = pair >= 0;
    f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    u32x4_t rg[kG1D], ru[kG1D], rx[kG1D];
#pragma unroll
    for (int d = 0; d < kG1D; ++d) {
      rx[d] = u32x4_t{0u, 0u, 0u, 0u};
      if (d < n) {
        rg[d] = ldg16_stream(wg + d * 32);
        ru[d] = ldg16_stream(wu + d * 32);
        if (hx) rx[d] = ldg16(xr + d * 32);
      }
    }
    for (int base = 0; base < n; base += kG1D) {
#pragma unroll
      for (int d = 0; d < kG1D; ++d) {
        if (base + d < n) {
          ag = mfma16x16x32_bf16(rg[d], rx[d], ag);
          au = mfma16x16x32_bf16(ru[d], rx[d], au);
          const int nx = base + kG1D + d;
          if (nx < n) {
            rg[d] = ldg16_stream(wg + nx * 32);
            ru[d] = ldg16_stream(wu + nx * 32);
            if (hx) rx[d] = ldg16(xr + nx * 32);
          }
        }
      }
    }
    red[wave][0][lane] = ag;
    red[wave][1][lane] = au;
    __syncthreads();
    if (wave == 0 && pair >= 0) {
      f32x4_t g = red[0][0][lane], u = red[0][1][lane];
#pragma unroll
      for (int w = 1; w < kG1KS; ++w) {
        g += red[w][0][lane];
        u += red[w][1][lane];
      }
      uint16_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gv = g[r];
        o[r] = f32_to_bf16_bits(gv / (1.0f + expf(-gv)) * u[r]);
      }
      u32x2_t packed = {(uint32_t)o[0] | ((uint32_t)o[1] << 16),
                        (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
      *reinterpret_cast<u32x2_t*>(act + (size_t)pair * I + tile * 16 + kg * 4) = packed;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// GEMM2: partial[pair, h] = w[pair] * (W2[s] · act[pair])[h] for kG2T
// consecutive 16-row hidden tiles of one block (the act fragment is loaded
// once per K chunk and feeds kG2T MFMAs).  bf16 weights.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64 * kG2KS) void moe_gemm2_bf16_kernel(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ w2,
    const int32_t* __restrict__ plan, const float* __restrict__ topk_w, int H, int I,
    float* __restrict__ partial) {
  __shared__ f32x4_t red[kG2KS][kG2T][64];
  const int n_blocks = plan[0];
  const int n_tiles = H / (16 * kG2T);
  const int total = n_blocks * n_tiles;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kg = lane >> 4;
  const int nchunk = I / 32;
  const int c0 = wave * nchunk / kG2KS, c1 = (wave + 1) * nchunk / kG2KS;
  const int n = c1 - c0;
  const int32_t* blocks = plan + kPlanHeader;

  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int b = item / n_tiles, tile = item - b * n_tiles;
    const int32_t* blk = blocks + (size_t)b * kBlockInts;
    const int slot = blk[0], cnt = blk[1];
    const int pair = col < cnt ? blk[2 + col] : -1;
    const bool hx = pair >= 0;
    const uint16_t* wr =
        w2 + ((size_t)slot * H + (size_t)tile * 16 * kG2T + col) * I + kg * 8 + c0 * 32;
    const uint16_t* ar = act + (size_t)(hx ? pair : 0) * I + kg * 8 + c0 * 32;
    f32x4_t acc[kG2T];
#pragma unroll
    for (int t = 0; t < kG2T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    u32x4_t ra[kG2D][kG2T], rb[kG2D];
#pragma unroll
    for (int d = 0; d < kG2D; ++d) {
      rb[d] = u32x4_t{0u, 0u, 0u, 0u};
      if (d < n) {
#pragma unroll
        for (int t = 0; t < kG2T; ++t) ra[d][t] = ldg16_stream(wr + (size_t)t * 16 * I + d * 32);
        if (hx) rb[d] = ldg16(ar + d * 32);
      }
    }
    for (int base = 0; base < n; base += kG2D) {
#pragma unroll
      for (int d = 0; d < kG2D; ++d) {
        if (base + d < n) {
#pragma unroll
          for (int t = 0; t < kG2T; ++t) acc[t] = mfma16x16x32_bf16(ra[d][t], rb[d], acc[t]);
          const int nx = base + kG2D + d;
          if (nx < n) {
#pragma unroll
            for (int t = 0; t < kG2T; ++t)
              ra[d][t] = ldg16_stream(wr + (size_t)t * 16 * I + nx * 32);
            if (hx) rb[d] = ldg16(ar + nx * 32);
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kG2T; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    if (wave == 0 && pair >= 0) {
      const float wv = topk_w[pair];
#pragma unroll
      for (int t = 0; t < kG2T; ++t) {
        f32x4_t s = red[0][t][lane];
#pragma unroll
        for (int w = 1; w < kG2KS; ++w) s += red[w][t][lane];
        f32x4_t o = {wv * s[0], wv * s[1], wv * s[2], wv * s[3]};
        *reinterpret_cast<f32x4_t*>(partial + (size_t)pair * H + (tile * kG2T + t) * 16 +
                                    kg * 4) = o;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// fp8 e4m3fn weights with 128x128 fp32 block scales, bf16 activations.
// Each lane loads 16 fp8 (one 64-wide K chunk per lane group), widens them
// exactly to bf16 and issues two MFMAs; the fp32 sum of a 128-wide K block
// is multiplied by that block's scale before it joins the accumulator.
// ---------------------------------------------------------------------------
typedef __attribute__((ext_vector_type(2))) float f32x2_t;

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

constexpr int kFp8Blk = 128;

__global__ __launch_bounds__(64 * kKS) void moe_gemm1_fp8_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w13,
    const float* __restrict__ w13_scale, const int32_t* __restrict__ plan, int H, int I, int k,
    uint16_t* __restrict__ act) {
  __shared__ f32x4_t red[kKS][2][64];
  const int n_blocks = plan[0];
  const int n_tiles = I / 16;
  const int total = n_blocks * n_tiles;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kg = lane >> 4;
  const int nkb = H / kFp8Blk;                 // K scale blocks
  const int nrb = (2 * I) / kFp8Blk;           // row scale blocks per expert
  const int kb0 = wave * nkb / kKS, kb1 = (wave + 1) * nkb / kKS;
  const int32_t* blocks = plan + kPlanHeader;

  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int b = item / n_tiles, tile = item - b * n_tiles;
    const int32_t* blk = blocks + (size_t)b * kBlockInts;
    const int slot = blk[0], cnt = blk[1];
    const int pair = col < cnt ? blk[2 + col] : -1;
    const int rg = tile * 16, ru = I + tile * 16;
    const uint8_t* wg = w13 + ((size_t)slot * 2 * I + rg + col) * H + kg * 16;
    const uint8_t* wu = w13 + ((size_t)slot * 2 * I + ru + col) * H + kg * 16;
    const float* sg = w13_scale + ((size_t)slot * nrb + rg / kFp8Blk) * nkb;
    const float* su = w13_scale + ((size_t)slot * nrb + ru / kFp8Blk) * nkb;
    const uint16_t* xr = x + (size_t)(pair >= 0 ? pair / k : 0) * H + kg * 16;
    f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    for (int kb = kb0; kb < kb1; ++kb) {
      f32x4_t tg = {0.f, 0.f, 0.f, 0.f}, tu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k0 = kb * kFp8Blk + h * 64;
        const u32x4_t qg = ldg16_stream(wg + k0);
        const u32x4_t qu = ldg16_stream(wu + k0);
        u32x4_t b0 = {0u, 0u, 0u, 0u}, b1 = {0u, 0u, 0u, 0u};
        if (pair >= 0) {
          b0 = ldg16(xr + k0);
          b1 = ldg16(xr + k0 + 8);
        }
        u32x4_t g0, g1, u0, u1;
        fp8x16_to_bf16(qg, g0, g1);
        fp8x16_to_bf16(qu, u0, u1);
        tg = mfma16x16x32_bf16(g0, b0, tg);
        tg = mfma16x16x32_bf16(g1, b1, tg);
        tu = mfma16x16x32_bf16(u0, b0, tu);
        tu = mfma16x16x32_bf16(u1, b1, tu);
      }
      const float scg = sg[kb], scu = su[kb];
      ag += scg * tg;
      au += scu * tu;
    }
    red[wave][0][lane] = ag;
    red[wave][1][lane] = au;
    __syncthreads();
    if (wave == 0 && pair >= 0) {
      f32x4_t g = red[0][0][lane], u = red[0][1][lane];
#pragma unroll
      for (int w = 1; w < kKS; ++w) {
        g += red[w][0][lane];
        u += red[w][1][lane];
      }
      uint16_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gv = g[r];
        o[r] = f32_to_bf16_bits(gv / (1.0f + expf(-gv)) * u[r]);
      }
      u32x2_t packed = {(uint32_t)o[0] | ((uint32_t)o[1] << 16),
                        (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
      *reinterpret_cast<u32x2_t*>(act + (size_t)pair * I + tile * 16 + kg * 4) = packed;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(64 * kKS) void moe_gemm2_fp8_kernel(
    const uint16_t* __restrict__ act, const uint8_t* __restrict__ w2,
    const float* __restrict__ w2_scale, const int32_t* __restrict__ plan,
    const float* __restrict__ topk_w, int H, int I, float* __restrict__ partial) {
  __shared__ f32x4_t red[kKS][64];
  const int n_blocks = plan[0];
  const int n_tiles = H / 16;
  const int total = n_blocks * n_tiles;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kg = lane >> 4;
  const int nkb = I / kFp8Blk;
  const int nrb = H / kFp8Blk;
  const int kb0 = wave * nkb / kKS, kb1 = (wave + 1) * nkb / kKS;
  const int32_t* blocks = plan + kPlanHeader;

  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int b = item / n_tiles, tile = item - b * n_tiles;
    const int32_t* blk = blocks + (size_t)b * kBlockInts;
    const int slot = blk[0], cnt = blk[1];
    const int pair = col < cnt ? blk[2 + col] : -1;
    const uint8_t* wr = w2 + ((size_t)slot * H + (size_t)tile * 16 + col) * I + kg * 16;
    const float* sr = w2_scale + ((size_t)slot * nrb + (tile * 16) / kFp8Blk) * nkb;
    const uint16_t* ar = act + (size_t)(pair >= 0 ? pair : 0) * I + kg * 16;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int kb = kb0; kb < kb1; ++kb) {
      f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k0 = kb * kFp8Blk + h * 64;
        const u32x4_t q = ldg16_stream(wr + k0);
        u32x4_t b0 = {0u, 0u, 0u, 0u}, b1 = {0u, 0u, 0u, 0u};
        if (pair >= 0) {
          b0 = ldg16(ar + k0);
          b1 = ldg16(ar + k0 + 8);
        }
        u32x4_t a0, a1;
        fp8x16_to_bf16(q, a0, a1);
        t = mfma16x16x32_bf16(a0, b0, t);
        t = mfma16x16x32_bf16(a1, b1, t);
      }
      acc += sr[kb] * t;
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && pair >= 0) {
      f32x4_t s = red[0][lane];
#pragma unroll
      for (int w = 1; w < kKS; ++w) s += red[w][lane];
      const float wv = topk_w[pair];
      f32x4_t o = {wv * s[0], wv * s[1], wv * s[2], wv * s[3]};
      *reinterpret_cast<f32x4_t*>(partial + (size_t)pair * H + tile * 16 + kg * 4) = o;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Combine: out[t, h] = bf16(scale * sum_j valid ? partial[t*k+j, h] : 0
//                           + shared[t, h]); j ascending.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float* __restrict__ partial, const int32_t* __restrict__ valid, int k, int H,
    float scale, const uint16_t* __restrict__ shared, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (h >= H) return;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < k; ++j) {
    const int p = t * k + j;
    if (valid[p]) acc += *reinterpret_cast<const f32x4_t*>(partial + (size_t)p * H + h);
  }
  uint16_t o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = scale * acc[r];
    if (shared != nullptr) v += bf16_bits_to_f32(shared[(size_t)t * H + h + r]);
    o[r] = f32_to_bf16_bits(v);
  }
  u32x2_t packed = {(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
  *reinterpret_cast<u32x2_t*>(out + (size_t)t * H + h) = packed;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Workspace {
  int32_t* plan;
  uint16_t* act;
  float* partial;
};

size_t workspace_bytes(int T, int H, int I, int k, Workspace* ws, void* base) {
  const int P = T * k;
  size_t off = 0;
  const size_t plan_b = align_up(plan_ints(P) * sizeof(int32_t), 256);
  const size_t act_b = align_up((size_t)P * I * sizeof(uint16_t), 256);
  const size_t part_b = align_up((size_t)P * H * sizeof(float), 256);
  if (ws != nullptr) {
    char* b = (char*)base;
    ws->plan = (int32_t*)(b + off);
    ws->act = (uint16_t*)(b + off + plan_b);
    ws->partial = (float*)(b + off + plan_b + act_b);
  }
  return plan_b + act_b + part_b;
}

int grid_for(int P, int n_tiles) {
  const long items = (long)P * n_tiles;  // upper bound on (block, tile) items
  const long cap = 8192;
  return (int)(items < cap ? (items > 0 ? items : 1) : cap);
}

int check_common(int T, int H, int I, int k, int E, int S, const void* x, const void* w13,
                 const void* w2, const float* tw, const int32_t* ti, void* ws, size_t ws_bytes,
                 void* out) {
  if (T < 0 || H <= 0 || I <= 0 || k <= 0 || k > SLUICE_MAX_TOPK || E <= 0 || S <= 0 ||
      S > SLUICE_MAX_SLOTS)
    return SLUICE_E_INVAL;
  if ((long)T * k > SLUICE_MAX_PAIRS) return SLUICE_E_INVAL;
  if (H % 32 != 0 || H % (16 * kG2T) != 0 || I % 32 != 0) return SLUICE_E_INVAL;
  if (T == 0) return SLUICE_OK;
  if (!x || !w13 || !w2 || !tw || !ti || !ws || !out) return SLUICE_E_INVAL;
  if (ws_bytes < workspace_bytes(T, H, I, k, nullptr, nullptr)) return SLUICE_E_INVAL;
  if (((uintptr_t)x | (uintptr_t)w13 | (uintptr_t)w2 | (uintptr_t)ws | (uintptr_t)out) & 15)
    return SLUICE_E_INVAL;
  return SLUICE_OK;
}

}  // namespace

extern "C" size_t sluice_moe_plan_ints(int T, int k) { return plan_ints(T * k); }

extern "C" size_t sluice_fused_experts_workspace(int T, int H, int I, int k) {
  if (T <= 0 || k <= 0) return 256;
  return workspace_bytes(T, H, I, k, nullptr, nullptr);
}

extern "C" int sluice_moe_align(const int32_t* topk_ids, int T, int k, const int32_t* expert_map,
                                int E, int S, int32_t* plan, sluice_stream_t stream) {
  if (T < 0 || k <= 0 || E <= 0 || S <= 0 || S > SLUICE_MAX_SLOTS ||
      (long)T * k > SLUICE_MAX_PAIRS || plan == nullptr)
    return SLUICE_E_INVAL;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kAlignThreads), 0, (hipStream_t)stream,
                     topk_ids, T * k, expert_map, E, S, plan);
  return (int)hipGetLastError();
}

static int launch_combine(const Workspace& w, int T, int k, int H, float scale, const void* shared,
                          void* out, hipStream_t st) {
  const int P = T * k;
  const int32_t* valid = w.plan + kPlanHeader + (size_t)kBlockInts * P;
  dim3 grid((H / 4 + 255) / 256, T);
  hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, st, w.partial, valid, k, H, scale,
                     (const uint16_t*)shared, (uint16_t*)out);
  return (int)hipGetLastError();
}

extern "C" int sluice_fused_experts_bf16(const void* x, const void* w13, const void* w2,
                                         const float* topk_w, const int32_t* topk_ids,
                                         const int32_t* expert_map, int T, int H, int I, int k,
                                         int E, int S, float scale, const void* shared,
                                         void* workspace, size_t workspace_bytes_, void* out,
                                         sluice_stream_t stream) {
  int rc = check_common(T, H, I, k, E, S, x, w13, w2, topk_w, topk_ids, workspace,
                        workspace_bytes_, out);
  if (rc != SLUICE_OK || T == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  Workspace w;
  workspace_bytes(T, H, I, k, &w, workspace);
  const int P = T * k;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kAlignThreads), 0, st, topk_ids, P,
                     expert_map, E, S, w.plan);
  SLUICE_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(moe_gemm1_bf16_kernel, dim3(grid_for(P, I / 16)), dim3(64 * kG1KS), 0, st,
                     (const uint16_t*)x, (const uint16_t*)w13, w.plan, H, I, k, w.act);
  SLUICE_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(moe_gemm2_bf16_kernel, dim3(grid_for(P, H / (16 * kG2T))),
                     dim3(64 * kG2KS), 0, st, w.act, (const uint16_t*)w2, w.plan, topk_w, H, I,
                     w.partial);
  SLUICE_HIP_CHECK(hipGetLastError());
  return launch_combine(w, T, k, H, scale, shared, out, st);
}

extern "C" int sluice_moe_gemm1_bf16(const void* x, const void* w13, const int32_t* plan, int T,
                                     int H, int I, int k, void* act, sluice_stream_t stream) {
  if (T <= 0 || k <= 0 || H <= 0 || I <= 0 || H % 32 || I % 32 || (long)T * k > SLUICE_MAX_PAIRS ||
      !x || !w13 || !plan || !act)
    return SLUICE_E_INVAL;
  hipLaunchKernelGGL(moe_gemm1_bf16_kernel, dim3(grid_for(T * k, I / 16)), dim3(64 * kG1KS), 0,
                     (hipStream_t)stream, (const uint16_t*)x, (const uint16_t*)w13, plan, H, I, k,
                     (uint16_t*)act);
  return (int)hipGetLastError();
}

extern "C" int sluice_moe_gemm2_bf16(const void* act, const void* w2, const int32_t* plan,
                                     const float* topk_w, int T, int H, int I, int k,
                                     float* partial, sluice_stream_t stream) {
  if (T <= 0 || k <= 0 || H <= 0 || I <= 0 || H % (16 * kG2T) || I % 32 ||
      (long)T * k > SLUICE_MAX_PAIRS || !act || !w2 || !plan || !topk_w || !partial)
    return SLUICE_E_INVAL;
  hipLaunchKernelGGL(moe_gemm2_bf16_kernel, dim3(grid_for(T * k, H / (16 * kG2T))),
                     dim3(64 * kG2KS), 0, (hipStream_t)stream, (const uint16_t*)act,
                     (const uint16_t*)w2, plan, topk_w, H, I, partial);
  return (int)hipGetLastError();
}

extern "C" int sluice_moe_combine(const float* partial, const int32_t* plan, int T, int k, int H,
                                  float scale, const void* shared, void* out,
                                  sluice_stream_t stream) {
  if (T <= 0 || k <= 0 || H <= 0 || H % 4 || (long)T * k > SLUICE_MAX_PAIRS || !partial || !plan ||
      !out)
    return SLUICE_E_INVAL;
  Workspace w;
  w.plan = const_cast<int32_t*>(plan);
  w.partial = const_cast<float*>(partial);
  w.act = nullptr;
  return launch_combine(w, T, k, H, scale, shared, out, (hipStream_t)stream);
}

extern "C" int sluice_fused_experts_fp8(const void* x, const void* w13, const float* w13_scale,
                                        const void* w2, const float* w2_scale, int block_n,
                                        int block_k, const float* topk_w,
                                        const int32_t* topk_ids, const int32_t* expert_map, int T,
                                        int H, int I, int k, int E, int S, float scale,
                                        const void* shared, void* workspace,
                                        size_t workspace_bytes_, void* out,
                                        sluice_stream_t stream) {
  if (block_n != kFp8Blk || block_k != kFp8Blk) return SLUICE_E_INVAL;
  if (H % kFp8Blk != 0 || I % kFp8Blk != 0) return SLUICE_E_INVAL;
  int rc = check_common(T, H, I, k, E, S, x, w13, w2, topk_w, topk_ids, workspace,
                        workspace_bytes_, out);
  if (rc != SLUICE_OK || T == 0) return rc;
  if (w13_scale == nullptr || w2_scale == nullptr) return SLUICE_E_INVAL;
  hipStream_t st = (hipStream_t)stream;
  Workspace w;
  workspace_bytes(T, H, I, k, &w, workspace);
  const int P = T * k;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kAlignThreads), 0, st, topk_ids, P,
                     expert_map, E, S, w.plan);
  SLUICE_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(moe_gemm1_fp8_kernel, dim3(grid_for(P, I / 16)), dim3(64 * kKS), 0, st,
                     (const uint16_t*)x, (const uint8_t*)w13, w13_scale, w.plan, H, I, k, w.act);
  SLUICE_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(moe_gemm2_fp8_kernel, dim3(grid_for(P, H / 16)), dim3(64 * kKS), 0, st,
                     w.act, (const uint8_t*)w2, w2_scale, w.plan, topk_w, H, I, w.partial);
  SLUICE_HIP_CHECK(hipGetLastError());
  return launch_combine(w, T, k, H, scale, shared, out, st);
}
