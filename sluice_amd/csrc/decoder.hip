// Kernels of the synthetic decoders around the routed-MoE path (not part of
// the reference's interface; see include/sluice_decoder.h).  Each replaces a
// chain of small torch ops with one launch: a decode step of a 27-48 layer
// model otherwise spends most of its time launching 2-5 us kernels.
#include <math.h>

#include <type_traits>

#include "common.h"
#include "sluice_decoder.h"
#include "stream.h"

namespace {

constexpr int kT = 256;  // threads per workgroup (4 waves)

__device__ __forceinline__ float wave_sum(float v) { return wave_sum_f32(v); }

__device__ __forceinline__ float wave_max(float v) { return wave_max_f32(v); }

// Block-wide sum / max over kT threads (all threads get the result).
__device__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < kT / 64; ++i) s += red[i];
  return s;
}

__device__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = -INFINITY;
  for (int i = 0; i < kT / 64; ++i) s = fmaxf(s, red[i]);
  return s;
}

__device__ __forceinline__ float bf(uint16_t b) { return bf16_bits_to_f32(b); }

__device__ __forceinline__ void unpack8(u32x4_t v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}

// ---------------------------------------------------------------------------
// Residual add + RMSNorm.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kT) void add_rmsnorm_kernel(uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ delta,
                                                         const uint16_t* __restrict__ w,
                                                         uint16_t* __restrict__ out, int H,
                                                         float eps) {
  __shared__ float red[kT / 64];
  const int r = blockIdx.x;
  uint16_t* xr = x + (size_t)r * H;
  const uint16_t* dr = delta != nullptr ? delta + (size_t)r * H : nullptr;
  float ss = 0.f;
  for (int i = threadIdx.x * 8; i < H; i += kT * 8) {
    float v[8];
    unpack8(*reinterpret_cast<const u32x4_t*>(xr + i), v);
    if (dr != nullptr) {
      float d[8];
      unpack8(*reinterpret_cast<const u32x4_t*>(dr + i), d);
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = pack2(v[2 * j] + d[2 * j], v[2 * j + 1] + d[2 * j + 1]);
      *reinterpret_cast<u32x4_t*>(xr + i) = o;
      unpack8(o, v);  // the rounded sum, as the residual stream holds it
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
  }
  const float rstd = rsqrtf(block_sum(ss, red) / (float)H + eps);
  for (int i = threadIdx.x * 8; i < H; i += kT * 8) {
    float v[8], g[8];
    unpack8(*reinterpret_cast<const u32x4_t*>(xr + i), v);
    unpack8(*reinterpret_cast<const u32x4_t*>(w + i), g);
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack2(v[2 * j] * rstd * g[2 * j], v[2 * j + 1] * rstd * g[2 * j + 1]);
    *reinterpret_cast<u32x4_t*>(out + (size_t)r * H + i) = o;
  }
}

// The same for H <= NI * 2048: every load (x, delta, w) goes out at once
// and the rows stay in registers, so the kernel waits on memory once.
template <int NI>
__global__ __launch_bounds__(kT) void add_rmsnorm_reg_kernel(uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ delta,
                                                             const uint16_t* __restrict__ w,
                                                             uint16_t* __restrict__ out, int H,
                                                             float eps) {
  __shared__ float red[kT / 64];
  const int r = blockIdx.x;
  uint16_t* xr = x + (size_t)r * H;
  const uint16_t* dr = delta != nullptr ? delta + (size_t)r * H : nullptr;
  u32x4_t xv[NI], dv[NI], wv[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int i = threadIdx.x * 8 + j * kT * 8;
    if (i < H) {
      xv[j] = *reinterpret_cast<const u32x4_t*>(xr + i);
      wv[j] = *reinterpret_cast<const u32x4_t*>(w + i);
      if (dr != nullptr) dv[j] = *reinterpret_cast<const u32x4_t*>(dr + i);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int i = threadIdx.x * 8 + j * kT * 8;
    if (i < H) {
      if (dr != nullptr) {
        float v[8], d[8];
        unpack8(xv[j], v);
        unpack8(dv[j], d);
        u32x4_t o;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          o[q] = pack2(v[2 * q] + d[2 * q], v[2 * q + 1] + d[2 * q + 1]);
        *reinterpret_cast<u32x4_t*>(xr + i) = o;
        xv[j] = o;  // the rounded sum, as the residual stream holds it
      }
      float v[8];
      unpack8(xv[j], v);
#pragma unroll
      for (int q = 0; q < 8; ++q) ss += v[q] * v[q];
    }
  }
  const float rstd = rsqrtf(block_sum(ss, red) / (float)H + eps);
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int i = threadIdx.x * 8 + j * kT * 8;
    if (i < H) {
      float v[8], g[8];
      unpack8(xv[j], v);
      unpack8(wv[j], g);
      u32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack2(v[2 * q] * rstd * g[2 * q], v[2 * q + 1] * rstd * g[2 * q + 1]);
      *reinterpret_cast<u32x4_t*>(out + (size_t)r * H + i) = o;
    }
  }
}

// ---------------------------------------------------------------------------
// SwiGLU activation.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kT) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                      uint16_t* __restrict__ out, int I) {
  const int r = blockIdx.y;
  const int i = (blockIdx.x * kT + threadIdx.x) * 4;
  if (i >= I) return;
  const uint16_t* g = gu + (size_t)r * 2 * I + i;
  const uint16_t* u = g + I;
  const u32x2_t gv = *reinterpret_cast<const u32x2_t*>(g);
  const u32x2_t uv = *reinterpret_cast<const u32x2_t*>(u);
  float o[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float g0 = __uint_as_float(gv[j] << 16), g1 = __uint_as_float(gv[j] & 0xffff0000u);
    const float u0 = __uint_as_float(uv[j] << 16), u1 = __uint_as_float(uv[j] & 0xffff0000u);
    o[2 * j] = g0 / (1.0f + expf(-g0)) * u0;
    o[2 * j + 1] = g1 / (1.0f + expf(-g1)) * u1;
  }
  *reinterpret_cast<u32x2_t*>(out + (size_t)r * I + i) = u32x2_t{pack2(o[0], o[1]), pack2(o[2], o[3])};
}

// ---------------------------------------------------------------------------
// Router logits: one workgroup per expert, the 4 waves split H.
// ---------------------------------------------------------------------------
constexpr int kMaxRows = 16;

// Lane partial sums of one expert's logits for every token row over the H
// quarter q: lane covers 8 elements per 512-wide step.  MAXR >= rows rows are
// loaded unconditionally (rows past the last repeat it), so each step's
// loads are all in flight together (loads under per-row conditions were
// each waited for before the next was issued).
template <int MAXR>
__device__ __forceinline__ void gate_partial(const uint16_t* __restrict__ hn,
                                             const uint16_t* __restrict__ wr, int rows, int H,
                                             int q, float (&acc)[MAXR]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < MAXR; ++t) acc[t] = 0.f;
  const int h0 = q * (H / 4), h1 = h0 + H / 4;
  for (int i = h0 + lane * 8; i < h1; i += 64 * 8) {
    const u32x4_t wq = *reinterpret_cast<const u32x4_t*>(wr + i);
    u32x4_t xq[MAXR];
#pragma unroll
    for (int t = 0; t < MAXR; ++t) {
      const int tt = t < rows ? t : rows - 1;
      xq[t] = *reinterpret_cast<const u32x4_t*>(hn + (size_t)tt * H + i);
    }
    float wv[8];
    unpack8(wq, wv);
#pragma unroll
    for (int t = 0; t < MAXR; ++t) {
      float xv[8];
      unpack8(xq[t], xv);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[t] += wv[j] * xv[j];
    }
  }
}

// The logit from the four quarter sums (quarters in order) plus the
// step's synthetic routing bias.
__device__ __forceinline__ float gate_finish(float q0, float q1, float q2, float q3,
                                             const float* __restrict__ bias_table,
                                             const int64_t* __restrict__ step, int n_steps,
                                             int bias_rows, int t, int e, int E) {
  float v = q0 + q1 + q2 + q3;
  if (bias_table != nullptr) {
    long long st = *step;
    st = ((st % n_steps) + n_steps) % n_steps;
    v += bias_table[((size_t)st * bias_rows + t) * E + e];
  }
  return v;
}

template <int MAXR>
__global__ __launch_bounds__(kT) void gate_logits_kernel(
    const uint16_t* __restrict__ hn, const uint16_t* __restrict__ wg,
    const float* __restrict__ bias_table, const int64_t* __restrict__ step, int n_steps,
    int bias_rows, int rows, int H, int E, float* __restrict__ out) {
  __shared__ float red[kT / 64][MAXR];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int e = blockIdx.x;
  float acc[MAXR];
  gate_partial<MAXR>(hn, wg + (size_t)e * H, rows, H, wave, acc);
#pragma unroll
  for (int t = 0; t < MAXR; ++t) {
    if (t < rows) {
      const float v = wave_sum(acc[t]);
      if (lane == 0) red[wave][t] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < rows) {
    const int t = threadIdx.x;
    out[(size_t)t * E + e] = gate_finish(red[0][t], red[1][t], red[2][t], red[3][t], bias_table,
                                         step, n_steps, bias_rows, t, e, E);
  }
}


constexpr int kMaxDeltaParts = 4;  // K parts of a projection the fused norm sums

// Residual add + RMSNorm + router logits in one launch, for the MoE layers'
// second norm.  grid (rows, ceil(E / EPW)): workgroup (t, b) normalises row
// t (the same per-thread element order and reductions as
// add_rmsnorm_reg_kernel, so hn is bit-identical to it) and takes experts
// EPW*b .. EPW*b + EPW-1 of that row (the same element order as
// gate_logits_kernel when H == 2048).  Workgroup (t, 0) writes the row's new
// residual to x_out (x is read by every workgroup of the row) and hn.
// H <= NI * 2048.
template <int NI, int EPW>
__global__ __launch_bounds__(kT) void add_rmsnorm_gate_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ delta,
    const float* __restrict__ dparts, int nparts,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ x_out, uint16_t* __restrict__ hn_out,
    const uint16_t* __restrict__ wg, const float* __restrict__ bias_table,
    const int64_t* __restrict__ step, int n_steps, int bias_rows, int H, int E, float eps,
    float* __restrict__ logits) {
  __shared__ float red[kT / 64][EPW + 1];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int t = blockIdx.x, e0 = blockIdx.y * EPW;
  const uint16_t* xr = x + (size_t)t * H;
  const uint16_t* dr = delta != nullptr ? delta + (size_t)t * H : nullptr;
  u32x4_t xv[NI], dv[NI], wv[NI], gv[EPW][NI];
  f32x4_t pv[kMaxDeltaParts][NI][2];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int i = tid * 8 + j * kT * 8;
    const int ic = i < H ? i : 0;
    xv[j] = ldg16(xr + ic);
    wv[j] = ldg16(w + ic);
    if (dr != nullptr) dv[j] = ldg16(dr + ic);
    if (dparts != nullptr) {
      // a projection's K parts [nparts][rows][H] (fp32): delta = bf16(sum in part order)
#pragma unroll
      for (int q = 0; q < kMaxDeltaParts; ++q) {
        const float* src = dparts + ((size_t)(q < nparts ? q : 0) * gridDim.x + t) * H + ic;
        pv[q][j][0] = *reinterpret_cast<const f32x4_t*>(src);
        pv[q][j][1] = *reinterpret_cast<const f32x4_t*>(src + 4);
      }
    }
#pragma unroll
    for (int u = 0; u < EPW; ++u) {
      const int e = e0 + u < E ? e0 + u : E - 1;
      gv[u][j] = ldg16(wg + (size_t)e * H + ic);
    }
  }
  if (dparts != nullptr) {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
      for (int q = 0; q < kMaxDeltaParts; ++q) {
        if (q < nparts) {
          s0 += pv[q][j][0];
          s1 += pv[q][j][1];
        }
      }
      dv[j] = u32x4_t{pack2(s0[0], s0[1]), pack2(s0[2], s0[3]), pack2(s1[0], s1[1]),
                      pack2(s1[2], s1[3])};
    }
    dr = xr;  // (any non-null pointer: the delta is in dv)
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    if (tid * 8 + j * kT * 8 < H) {
      if (dr != nullptr) {
        float v[8], d[8];
        unpack8(xv[j], v);
        unpack8(dv[j], d);
#pragma unroll
        for (int q = 0; q < 4; ++q) xv[j][q] = pack2(v[2 * q] + d[2 * q], v[2 * q + 1] + d[2 * q + 1]);
      }
      float v[8];
      unpack8(xv[j], v);
#pragma unroll
      for (int q = 0; q < 8; ++q) ss += v[q] * v[q];
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave][EPW] = ss;
  __syncthreads();
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kT / 64; ++i) sum += red[i][EPW];
  const float rstd = rsqrtf(sum / (float)H + eps);
  float acc[EPW];
#pragma unroll
  for (int u = 0; u < EPW; ++u) acc[u] = 0.f;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int i = tid * 8 + j * kT * 8;
    if (i >= H) continue;
    float v[8], g[8];
    unpack8(xv[j], v);
    unpack8(wv[j], g);
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = pack2(v[2 * q] * rstd * g[2 * q], v[2 * q + 1] * rstd * g[2 * q + 1]);
    if (blockIdx.y == 0) {
      *reinterpret_cast<u32x4_t*>(x_out + (size_t)t * H + i) = xv[j];
      *reinterpret_cast<u32x4_t*>(hn_out + (size_t)t * H + i) = o;
    }
    float hv[8];
    unpack8(o, hv);
#pragma unroll
    for (int u = 0; u < EPW; ++u) {
      float gw[8];
      unpack8(gv[u][j], gw);
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[u] += gw[q] * hv[q];
    }
  }
#pragma unroll
  for (int u = 0; u < EPW; ++u) {
    const float v = wave_sum(acc[u]);
    if (lane == 0) red[wave][u] = v;
  }
  __syncthreads();
  if (tid < EPW) {
    const int e = e0 + tid;
    if (e < E)
      logits[(size_t)t * E + e] = gate_finish(red[0][tid], red[1][tid], red[2][tid], red[3][tid],
                                              bias_table, step, n_steps, bias_rows, t, e, E);
  }
}

// Row buckets of the gate kernel: rows <= MAXR loaded per step.
template <typename F>
void with_row_bucket(int rows, F f) {
  if (rows <= 1)
    f(std::integral_constant<int, 1>{});
  else if (rows <= 4)
    f(std::integral_constant<int, 4>{});
  else if (rows <= 8)
    f(std::integral_constant<int, 8>{});
  else
    f(std::integral_constant<int, 16>{});
}

// ---------------------------------------------------------------------------
// MLA (DeepSeek-V2 latent attention, decode, absorbed up-projections).
// ---------------------------------------------------------------------------
constexpr int kLora = 512;
constexpr int kRope = 64;
constexpr int kMaxL = 4096;

// ---------------------------------------------------------------------------
// MLA decode on the matrix cores, three launches:
//   mla_absorb_kernel   q_lat = q_nope . W_uk per head as one MFMA product over
//                       the batch (W_uk read once per head, not per token),
//                       q_pe RoPE, and the new latent / rope-key cache rows;
//   mla_partial_kernel  per (token, split of the rows, 16 heads): scores
//                       S = [q_lat ; q_pe] . [ckv ; kpe]^T and the latent sum
//                       O = P . ckv on v_mfma_f32_16x16x32_bf16 (the 16 heads
//                       are the M dimension), online softmax over 64-row
//                       steps, the split's (max, sum, O) to a workspace;
//   mla_merge_kernel    per (token, head): the splits merged, then the value
//                       up-projection.
// The P . ckv product contracts over cache rows, so its ckv operand needs 8
// consecutive rows of one latent column per lane: the cache keeps a second,
// transposed copy, ckvt [c][L/32][512][32], whose 32-row blocks hold the rows
// in the K order of that product (mla_kpos), so both products load their
// operands with plain 16-byte loads.  Scores and P are bf16 MFMA operands
// (q_lat rounded to bf16), sums fp32, softmax in base 2.
// ---------------------------------------------------------------------------
constexpr int kMlaSplit = 32;  // row splits per token
constexpr int kMlaStep = 32;   // rows per step of a split (one 16-row tile per wave)
constexpr int kMlaRec = kLora + 4;  // per (token, split, head): m, l, -, -, O[512]

// Slot of row r (0..31) of a 32-row block in the transposed cache: K index
// 8g + j (j < 4) holds row 4g + j, 8g + 4 + j holds row 16 + 4g + j -- the
// rows lane group g holds in the score tiles of rows 0..15 and 16..31.
__host__ __device__ inline int mla_kpos(int r) {
  const int hi = r >> 4, q = r & 15;
  return 8 * (q >> 2) + 4 * hi + (q & 3);
}

// Rows per split for n rows: a multiple of the step.
__host__ __device__ inline int mla_chunk(int n) {
  const int per = (n + kMlaSplit - 1) / kMlaSplit;
  return (per + kMlaStep - 1) / kMlaStep * kMlaStep;
}

// grid (nh * 8 + c), kT threads.  Block b < nh * 8: head b / 8, latent
// columns 64 * (b % 8) .. +64 of q_lat for every token (wave w: 16 columns,
// tokens on M, K = nope); block 8 * h also ropes head h's q_pe.  Block
// nh * 8 + t: token t's cache rows.
__global__ __launch_bounds__(kT) void mla_absorb_kernel(
    const uint16_t* __restrict__ q, int q_stride, const uint16_t* __restrict__ kva,
    int kva_stride, const uint16_t* __restrict__ kv_norm, const uint16_t* __restrict__ w_ukt,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int64_t* __restrict__ pos, int c, int nh, int nope, int L, float eps,
    uint16_t* __restrict__ q_lat, uint16_t* __restrict__ q_pe, uint16_t* __restrict__ ckv,
    uint16_t* __restrict__ ckvt, uint16_t* __restrict__ kpe) {
  __shared__ float red[kT / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kTiles = kLora / 64;
  const int b = blockIdx.x;
  if (b < nh * kTiles) {
    const int h = b / kTiles, jt = b % kTiles;
    const int R = lane & 15, g = lane >> 4;
    const int j = jt * 64 + wave * 16 + R;
    const int qh = h * (nope + kRope);
    const uint16_t* arow = q + (size_t)(R < c ? R : 0) * q_stride + qh + 8 * g;
    const uint16_t* brow = w_ukt + ((size_t)h * kLora + j) * nope + 8 * g;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < nope; k0 += 128) {
      // four K steps' loads in flight (steps past nope re-load step 0 and
      // are skipped)
      u32x4_t av[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int k = k0 + 32 * u < nope ? k0 + 32 * u : 0;
        av[u] = ldg16(arow + k);
        bv[u] = ldg16(brow + k);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k0 + 32 * u < nope) acc = mfma16x16x32_bf16(av[u], bv[u], acc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * g + r;  // D row = token, column = j
      if (t < c) q_lat[((size_t)t * nh + h) * kLora + j] = f32_to_bf16_bits(acc[r]);
    }
    if (jt == 0) {
      for (int i = tid; i < c * (kRope / 2); i += kT) {
        const int t = i / (kRope / 2), d = i % (kRope / 2);
        const long long p = pos[t];
        if (p < 0 || p >= L) continue;
        const uint16_t* qr = q + (size_t)t * q_stride + qh + nope;
        const float x1 = bf(qr[d]), x2 = bf(qr[d + kRope / 2]);
        const float cs = cos_t[p * (kRope / 2) + d], sn = sin_t[p * (kRope / 2) + d];
        uint16_t* o = q_pe + ((size_t)t * nh + h) * kRope;
        o[d] = f32_to_bf16_bits(x1 * cs - x2 * sn);
        o[d + kRope / 2] = f32_to_bf16_bits(x2 * cs + x1 * sn);
      }
    }
    return;
  }
  // token t's cache rows: rmsnorm(kva[:lora]) * kv_norm, rope(kva[lora:])
  const int t = b - nh * kTiles;
  const long long p = pos[t];
  if (p < 0 || p >= L) return;
  const uint16_t* kr = kva + (size_t)t * kva_stride;
  const uint32_t v2 = reinterpret_cast<const uint32_t*>(kr)[tid];
  const float x0 = __uint_as_float(v2 << 16), x1 = __uint_as_float(v2 & 0xffff0000u);
  const float rstd = rsqrtf(block_sum(x0 * x0 + x1 * x1, red) / (float)kLora + eps);
  const uint32_t g2 = reinterpret_cast<const uint32_t*>(kv_norm)[tid];
  const uint32_t packed = pack2(x0 * rstd * __uint_as_float(g2 << 16),
                                x1 * rstd * __uint_as_float(g2 & 0xffff0000u));
  reinterpret_cast<uint32_t*>(ckv + ((size_t)t * L + p) * kLora)[tid] = packed;
  uint16_t* tcol = ckvt + (((size_t)t * (L / 32) + (p >> 5)) * kLora + 2 * tid) * 32 +
                   mla_kpos((int)(p & 31));
  tcol[0] = (uint16_t)packed;
  tcol[32] = (uint16_t)(packed >> 16);
  if (tid < kRope / 2) {
    const float cr = cos_t[p * (kRope / 2) + tid], sr = sin_t[p * (kRope / 2) + tid];
    const float a = bf(kr[kLora + tid]), bb = bf(kr[kLora + tid + kRope / 2]);
    uint16_t* krow = kpe + ((size_t)t * L + p) * kRope;
    krow[tid] = f32_to_bf16_bits(a * cr - bb * sr);
    krow[tid + kRope / 2] = f32_to_bf16_bits(bb * cr + a * sr);
  }
}

// grid (c, kMlaSplit, nh / 16), 2 waves.  Split s of token t covers rows
// [s * chunk, min(n, (s + 1) * chunk)) in steps of 32 rows: wave w scores
// rows +16w .. +16w+15 for the 16 heads (A = cache rows, B = q from LDS),
// the scores meet in LDS, both waves derive the same softmax state, and
// wave w accumulates latent columns 256w .. 256w+255 of O (A = P, B = ckvt).
constexpr int kMlaWaves = 2;
constexpr int kMlaQRow = kLora + kRope + 8;  // LDS row of one head's q (padded)

__global__ __launch_bounds__(kMlaWaves * 64) void mla_partial_kernel(
    const uint16_t* __restrict__ q_lat, const uint16_t* __restrict__ q_pe,
    const uint16_t* __restrict__ ckv, const uint16_t* __restrict__ ckvt,
    const uint16_t* __restrict__ kpe, const int64_t* __restrict__ pos, int nh, int L, float sl2,
    float* __restrict__ part) {
  __shared__ __align__(16) uint16_t qs[16 * kMlaQRow];
  __shared__ float sc[kMlaStep][17];  // scores [row][head], log2 units
  const int t = blockIdx.x, s = blockIdx.y, hg = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int R = lane & 15, g = lane >> 4;
  // The 16 heads' [q_lat ; q_pe] (72 16-byte pieces per head) go out before
  // the position is known; the first step's operands follow it, and q then
  // goes to LDS.
  constexpr int kPieces = 16 * 72 / (kMlaWaves * 64);
  static_assert(kPieces * kMlaWaves * 64 == 16 * 72, "q pieces per thread");
  u32x4_t qv[kPieces];
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const int i = tid + u * kMlaWaves * 64, hh = i / 72, k = i % 72;
    const size_t row = (size_t)t * nh + hg * 16 + hh;
    qv[u] = k < 64 ? ldg16(q_lat + row * kLora + 8 * k) : ldg16(q_pe + row * kRope + 8 * (k - 64));
  }
  const long long p = pos[t];
  if (p < 0 || p >= L) return;
  const int n = (int)p + 1;
  const int chunk = mla_chunk(n);
  const int r0 = s * chunk;
  if (r0 >= n) return;
  const int r1 = min(n, r0 + chunk);
  const uint16_t* cb = ckv + (size_t)t * L * kLora;
  const uint16_t* kb = kpe + (size_t)t * L * kRope;
  const uint16_t* tb = ckvt + (size_t)t * L * kLora;
  // A step's operands: a = the cache rows of this wave's score tile, vt =
  // the step's ckvt block, column tiles 16w + i.
  u32x4_t a[kLora / 32 + kRope / 32], vt[16];
  auto load_step = [&](int b0) {
    const int row = min(b0 + 16 * w + R, r1 - 1);
    const uint16_t* ar = cb + (size_t)row * kLora + 8 * g;
    const uint16_t* pr = kb + (size_t)row * kRope + 8 * g;
#pragma unroll
    for (int kk = 0; kk < kLora / 32; ++kk) a[kk] = ldg16(ar + 32 * kk);
    a[kLora / 32] = ldg16(pr);
    a[kLora / 32 + 1] = ldg16(pr + 32);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      vt[i] = ldg16(tb + ((size_t)(b0 >> 5) * kLora + 16 * (16 * w + i) + R) * 32 + 8 * g);
  };
  load_step(r0);
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const int i = tid + u * kMlaWaves * 64, hh = i / 72, k = i % 72;
    *reinterpret_cast<u32x4_t*>(&qs[hh * kMlaQRow + 8 * k]) = qv[u];
  }
  f32x4_t o[16];  // o[i][r] = O[head 4g + r][column 16 * (16w + i) + R]
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;  // head R's running max and sum
  const uint16_t* qrow = &qs[R * kMlaQRow + 8 * g];
  for (int b0 = r0; b0 < r1; b0 += kMlaStep) {
    if (b0 + kMlaStep > r1) {
      // rows past the last one hold whatever the cache held: zero them, so
      // that a non-finite stale value cannot meet its zero weight
      uint32_t keep[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int e = 2 * e2;
        const int lo = b0 + (e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4));
        keep[e2] = (lo < r1 ? 0x0000ffffu : 0u) | (lo + 1 < r1 ? 0xffff0000u : 0u);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) vt[i][e2] &= keep[e2];
    }
    __syncthreads();  // q is in LDS; the previous step's readers of sc are done
    // two accumulation chains (even and odd K steps) halve the dependent
    // product latency
    f32x4_t sa0 = {0.f, 0.f, 0.f, 0.f}, sa1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < kLora / 32 + kRope / 32; kk += 2) {
      sa0 = mfma16x16x32_bf16(a[kk], *reinterpret_cast<const u32x4_t*>(qrow + 32 * kk), sa0);
      sa1 = mfma16x16x32_bf16(a[kk + 1], *reinterpret_cast<const u32x4_t*>(qrow + 32 * kk + 32),
                              sa1);
    }
    const f32x4_t sacc = sa0 + sa1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rr = 16 * w + 4 * g + r;  // S^T[row 4g + r][head R] of the wave's tile
      sc[rr][R] = b0 + rr < r1 ? sacc[r] * sl2 : -INFINITY;
    }
    __syncthreads();
    // head R's step max over the 32 rows (lane group g reads rows 8g..8g+7)
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, sc[8 * g + i][R]);
    mx = rows4_max(mx);
    const float mn = fmaxf(m, mx);  // finite: row b0 is in every step
    const float f = __builtin_amdgcn_exp2f(m - mn);
    // P in the K order of ckvt (A operand: head R, K group g) and its sum
    u32x4_t pa;
    float ps = 0.f;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      float pv[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int e = 2 * e2 + u;
        pv[u] = __builtin_amdgcn_exp2f(sc[e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4)][R] - mn);
        ps += pv[u];
      }
      pa[e2] = pack2(pv[0], pv[1]);
    }
    ps = rows4_sum(ps);
    l = l * f + ps;
    m = mn;
    if (b0 > r0) {
      // o[i][r] is head 4g + r's: its factor comes from lane 4g + r (on the
      // first step o is still zero)
      float fr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) fr[r] = __shfl(f, 4 * g + r);
#pragma unroll
      for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[i][r] *= fr[r];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = mfma16x16x32_bf16(pa, vt[i], o[i]);
    if (b0 + kMlaStep < r1) load_step(b0 + kMlaStep);
  }
  float* rec = part + (((size_t)t * kMlaSplit + s) * nh + hg * 16) * kMlaRec;
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      rec[(size_t)(4 * g + r) * kMlaRec + 4 + 16 * (16 * w + i) + R] = o[i][r];
  if (w == 0 && g == 0) {
    rec[(size_t)R * kMlaRec] = m;
    rec[(size_t)R * kMlaRec + 1] = l;
  }
}

// grid (c, nh, ceil(vh / 64)), kT threads: the splits of (token, head)
// merged into the normalised latent output, then value columns 64z .. 64z+63
// of out = o_lat . w_uv[h]: a thread owns 8 columns and 16 latent rows (lane
// group and wave pick the rows), the 32 row groups meet in LDS.  Everything
// whose address does not depend on the position goes out first: the w_uv
// rows, every split's (max, sum) and the first 8 splits' partial sums (splits
// past the position are never used, so whatever they hold is harmless:
// they are selected away, not multiplied by 0).
__global__ __launch_bounds__(kT) void mla_merge_kernel(const float* __restrict__ part,
                                                       const uint16_t* __restrict__ w_uv,
                                                       const int64_t* __restrict__ pos, int nh,
                                                       int vh, int L, uint16_t* __restrict__ out) {
  __shared__ float ol[kLora];
  __shared__ float ws[kMlaSplit];
  __shared__ float pq[32][64];
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int c8 = lane & 7, jg = (lane >> 3) + 8 * wave;  // 32 row groups
  const int v = 64 * blockIdx.z + 8 * c8;
  const uint16_t* wv = w_uv + (size_t)h * kLora * vh + (v < vh ? v : 0);
  u32x4_t wr[kLora / 32];
#pragma unroll
  for (int u = 0; u < kLora / 32; ++u) wr[u] = ldg16(wv + (size_t)(jg + 32 * u) * vh);
  const float* rec = part + ((size_t)t * kMlaSplit * nh + h) * kMlaRec;
  const size_t sstride = (size_t)nh * kMlaRec;
  static_assert(2 * kT == kLora, "two latent columns per thread");
  f32x2_t pv[8];  // splits 0..7, columns 2 * tid, 2 * tid + 1
#pragma unroll
  for (int u = 0; u < 8; ++u)
    pv[u] = *reinterpret_cast<const f32x2_t*>(rec + u * sstride + 4 + 2 * tid);
  float ms = -INFINITY, ls = 0.f;
  if (tid < kMlaSplit) {
    ms = rec[tid * sstride];
    ls = rec[tid * sstride + 1];
  }
  const long long p = pos[t];
  if (p < 0 || p >= L) return;
  const int n = (int)p + 1;
  const int chunk = mla_chunk(n);
  const int na = (n + chunk - 1) / chunk;
  if (tid < 64) {
    const bool ok = tid < na;
    const float M = wave_max(ok ? ms : -INFINITY);
    const float e = ok ? __builtin_amdgcn_exp2f(ms - M) : 0.f;
    const float den = wave_sum(ok ? e * ls : 0.f);
    if (tid < kMlaSplit) ws[tid] = e / den;
  }
  __syncthreads();
  {
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (u < na) {
        v0 += ws[u] * pv[u][0];
        v1 += ws[u] * pv[u][1];
      }
    }
    for (int s0 = 8; s0 < na; s0 += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sp = s0 + u < na ? s0 + u : 0;
        pv[u] = *reinterpret_cast<const f32x2_t*>(rec + sp * sstride + 4 + 2 * tid);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (s0 + u < na) {
          v0 += ws[s0 + u] * pv[u][0];
          v1 += ws[s0 + u] * pv[u][1];
        }
      }
    }
    ol[2 * tid] = v0;
    ol[2 * tid + 1] = v1;
  }
  __syncthreads();
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.f;
#pragma unroll
  for (int u = 0; u < kLora / 32; ++u) {
    const float oj = ol[jg + 32 * u];
    float wf[8];
    unpack8(wr[u], wf);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] += oj * wf[k];
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) pq[jg][8 * c8 + k] = acc[k];
  __syncthreads();
  if (tid < 64 && 64 * (int)blockIdx.z + tid < vh) {
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) sum += pq[i][tid];
    out[((size_t)t * nh + h) * vh + 64 * blockIdx.z + tid] = f32_to_bf16_bits(sum);
  }
}

// ---------------------------------------------------------------------------
// GQA with per-head q/k RMSNorm (Qwen3-MoE), head_dim 128, in one launch:
// the head's q/k RMSNorm and RoPE, the new cache row, and attention over
// rows 0..pos[t].
//
// grid (c, nh), WAVES waves.  A wave is four 16-lane groups; lane `sub` of a
// group owns head columns 8*sub .. 8*sub + 7 of q, k and v (lanes sub and
// sub + 8 hold the rotate-half partners).  Group i takes cache rows i,
// i + NG, ... of each chunk of NG*RG rows (a wave's load reads 4
// consecutive rows), keeping a running max / sum / value accumulator of its
// own (online softmax); the groups' states are merged in LDS at the end.
// q . k runs on v_dot2_f32_bf16 with q rounded to bf16 (the cache's
// precision), fp32 sums; the softmax runs in base 2 (v_exp_f32) on scores
// scaled by log2(e).  The new row (position pos[t]) is computed in registers from qkv and
// enters group 0's state first; the first query head of each kv head writes
// it to the caches.  Every other cache row is only read, so no workgroup
// reads a row another one writes.
// ---------------------------------------------------------------------------

constexpr int kHd = 128;

// Sum over each 16-lane row of the wave, left in every lane of the row
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror).
__device__ __forceinline__ float row16_allsum(float v) {
  uint32_t u = __float_as_uint(v);
  u = __float_as_uint(__uint_as_float(u) + __uint_as_float(dpp_mov<0xb1, 0xf>(0u, u)));
  u = __float_as_uint(__uint_as_float(u) + __uint_as_float(dpp_mov<0x4e, 0xf>(0u, u)));
  u = __float_as_uint(__uint_as_float(u) + __uint_as_float(dpp_mov<0x141, 0xf>(0u, u)));
  u = __float_as_uint(__uint_as_float(u) + __uint_as_float(dpp_mov<0x140, 0xf>(0u, u)));
  return __uint_as_float(u);
}

// The value of lane sub ^ 8 of the same 16-lane row (row_ror:8).
__device__ __forceinline__ float row16_partner(float v) {
  return __uint_as_float(dpp_mov<0x128, 0xf>(0u, __float_as_uint(v)));
}

// rope(rmsnorm(x) * w) of one head for this lane's 8 columns.
__device__ __forceinline__ void head_norm_rope(u32x4_t x, u32x4_t w, const float* cs,
                                               const float* sn, float eps, bool first_half,
                                               float* r) {
  float f[8], wf[8], n[8];
  unpack8(x, f);
  unpack8(w, wf);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
  const float rstd = rsqrtf(row16_allsum(ss) / (float)kHd + eps);
#pragma unroll
  for (int j = 0; j < 8; ++j) n[j] = f[j] * rstd * wf[j];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float o = row16_partner(n[j]);
    r[j] = first_half ? n[j] * cs[j] - o * sn[j] : n[j] * cs[j] + o * sn[j];
  }
}

// Cache rows c0 + gi + NG*r (r < RG) of this lane's columns; rows at or past
// nc load row 0 (in bounds) and are masked by gqa_chunk.
template <int RG, int NG>
__device__ __forceinline__ void gqa_load_chunk(const uint16_t* __restrict__ k_cache,
                                               const uint16_t* __restrict__ v_cache, size_t cbase,
                                               int c0, int gi, int nc, u32x4_t* kr, u32x4_t* vr) {
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int l = c0 + gi + NG * r;
    const size_t off = (size_t)(l < nc ? l : 0) * kHd;
    kr[r] = ldg16(k_cache + cbase + off);
    vr[r] = ldg16(v_cache + cbase + off);
  }
}

// q . k over this lane's 8 columns (bf16 pairs, fp32 accumulation).
__device__ __forceinline__ float dot8_bf16(u32x4_t a, u32x4_t b) {
  float d = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // (the elements go through scalars: hipcc 7.2 bit-casts a vector element
    // expression as if it were element 0)
    const uint32_t aj = a[j], bj = b[j];
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, aj),
                                        __builtin_bit_cast(bf16x2_t, bj), d, false);
  }
  return d;
}

// One chunk into a group's online-softmax state: running max m and sum
// lsum of 2^score (scores carry the log2(e) factor), value accumulator acc
// of this lane's 8 columns.
template <int RG, int NG>
__device__ __forceinline__ void gqa_chunk(const u32x4_t* kr, const u32x4_t* vr, int c0, int gi,
                                          int nc, u32x4_t qb, float sl2, float& m, float& lsum,
                                          float* acc) {
  float s[RG];
  float mc = -INFINITY;
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const float d = row16_allsum(dot8_bf16(qb, kr[r])) * sl2;
    s[r] = c0 + gi + NG * r < nc ? d : -INFINITY;
    mc = fmaxf(mc, s[r]);
  }
  const float mn = fmaxf(m, mc);
  if (mn == -INFINITY) return;
  const float f = __builtin_amdgcn_exp2f(m - mn);
  lsum *= f;
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] *= f;
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const float pw = __builtin_amdgcn_exp2f(s[r] - mn);
    float vf[8];
    unpack8(vr[r], vf);
    lsum += pw;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += pw * vf[j];
  }
  m = mn;
}

// 8 waves, 2 rows per group per chunk (256 rows per chunk): measured in
// replayed graphs against 4 waves x 4 or 8 rows and 8 waves x 4 rows at
// positions 0..1000.
constexpr int kGqaWaves = 8;
constexpr int kGqaRows = 2;

template <int WAVES, int RG>
__global__ __launch_bounds__(WAVES * 64) void gqa_decode_kernel(
    const uint16_t* __restrict__ qkv, const float* __restrict__ qkv_parts, int nparts,
    const uint16_t* __restrict__ q_norm,
    const uint16_t* __restrict__ k_norm, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const int64_t* __restrict__ pos, int nh, int kvh, int L,
    float eps, float scale, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    uint16_t* __restrict__ out) {
  constexpr int NG = WAVES * 4;
  constexpr int CH = NG * RG;
  __shared__ float gacc[NG][kHd];
  __shared__ float gm[NG], gl[NG];
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int grp = nh / kvh, g = h / grp;
  const int sub = tid & 15, gi = tid >> 4;
  const int col = sub * 8;
  const uint16_t* xr = qkv + (size_t)t * (nh + 2 * kvh) * kHd;
  const size_t cbase = ((size_t)t * kvh + g) * L * kHd + col;

  // Everything that does not depend on the position goes out with its
  // load: the head's q, the new k and v, the norm weights and the first
  // chunk of cache rows (rows past the position are loaded, in bounds, and
  // masked below).
  u32x4_t xq, xk, xv;
  if (qkv_parts != nullptr) {
    // the projection's K parts [nparts][c][width] fp32: bf16(sum in part order)
    const size_t width = (size_t)(nh + 2 * kvh) * kHd;
    const int offs[3] = {h * kHd + col, (nh + g) * kHd + col, (nh + kvh + g) * kHd + col};
    f32x4_t pv[3][kMaxDeltaParts][2];
#pragma unroll
    for (int v = 0; v < 3; ++v)
#pragma unroll
      for (int q = 0; q < kMaxDeltaParts; ++q) {
        const float* src = qkv_parts + ((size_t)(q < nparts ? q : 0) * gridDim.x + t) * width + offs[v];
        pv[v][q][0] = *reinterpret_cast<const f32x4_t*>(src);
        pv[v][q][1] = *reinterpret_cast<const f32x4_t*>(src + 4);
      }
    u32x4_t xs[3];
#pragma unroll
    for (int v = 0; v < 3; ++v) {
      f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
      for (int q = 0; q < kMaxDeltaParts; ++q)
        if (q < nparts) {
          s0 += pv[v][q][0];
          s1 += pv[v][q][1];
        }
      xs[v] = u32x4_t{pack2(s0[0], s0[1]), pack2(s0[2], s0[3]), pack2(s1[0], s1[1]),
                      pack2(s1[2], s1[3])};
    }
    xq = xs[0];
    xk = xs[1];
    xv = xs[2];
  } else {
    xq = ldg16(xr + h * kHd + col);
    xk = ldg16(xr + (nh + g) * kHd + col);
    xv = ldg16(xr + (nh + kvh + g) * kHd + col);
  }
  const u32x4_t wq = ldg16(q_norm + col), wk = ldg16(k_norm + col);
  u32x4_t kr[RG], vr[RG];
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int l = gi + NG * r;
    const size_t off = (size_t)(l < L ? l : L - 1) * kHd;
    kr[r] = ldg16(k_cache + cbase + off);
    vr[r] = ldg16(v_cache + cbase + off);
  }
  const long long p = pos[t];
  if (p < 0 || p >= L) return;
  const int nc = (int)p;  // cache rows before the new one
  const int ci = (int)p * 64 + (sub & 7) * 8;
  float cs[8], sn[8];
  *reinterpret_cast<f32x4_t*>(cs) = *reinterpret_cast<const f32x4_t*>(cos_t + ci);
  *reinterpret_cast<f32x4_t*>(cs + 4) = *reinterpret_cast<const f32x4_t*>(cos_t + ci + 4);
  *reinterpret_cast<f32x4_t*>(sn) = *reinterpret_cast<const f32x4_t*>(sin_t + ci);
  *reinterpret_cast<f32x4_t*>(sn + 4) = *reinterpret_cast<const f32x4_t*>(sin_t + ci + 4);

  const bool first_half = sub < 8;
  float qf[8], kf[8];
  head_norm_rope(xq, wq, cs, sn, eps, first_half, qf);
  head_norm_rope(xk, wk, cs, sn, eps, first_half, kf);
  // q and the new k row in bf16 (the k row as the cache holds it)
  u32x4_t qb, kb;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    qb[j] = pack2(qf[2 * j], qf[2 * j + 1]);
    kb[j] = pack2(kf[2 * j], kf[2 * j + 1]);
  }
  if (h % grp == 0 && gi == 0) {
    *reinterpret_cast<u32x4_t*>(k_cache + cbase + (size_t)p * kHd) = kb;
    *reinterpret_cast<u32x4_t*>(v_cache + cbase + (size_t)p * kHd) = xv;
  }
  const float sl2 = scale * 1.4426950408889634f;  // scores in log2 units
  float m = -INFINITY, lsum = 0.f, acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  if (gi == 0) {
    m = row16_allsum(dot8_bf16(qb, kb)) * sl2;
    lsum = 1.f;
    unpack8(xv, acc);
  }

  // Chunks alternate between two register buffers: the next chunk's loads
  // are in flight while this one is scored and accumulated.
  u32x4_t kr2[RG], vr2[RG];
  for (int c0 = 0; c0 < nc; c0 += 2 * CH) {
    if (c0 + CH < nc) gqa_load_chunk<RG, NG>(k_cache, v_cache, cbase, c0 + CH, gi, nc, kr2, vr2);
    gqa_chunk<RG, NG>(kr, vr, c0, gi, nc, qb, sl2, m, lsum, acc);
    if (c0 + CH >= nc) break;
    if (c0 + 2 * CH < nc) gqa_load_chunk<RG, NG>(k_cache, v_cache, cbase, c0 + 2 * CH, gi, nc, kr, vr);
    gqa_chunk<RG, NG>(kr2, vr2, c0 + CH, gi, nc, qb, sl2, m, lsum, acc);
  }

  if (sub == 0) {
    gm[gi] = m;
    gl[gi] = lsum;
  }
  *reinterpret_cast<f32x4_t*>(&gacc[gi][col]) = *reinterpret_cast<const f32x4_t*>(acc);
  *reinterpret_cast<f32x4_t*>(&gacc[gi][col + 4]) = *reinterpret_cast<const f32x4_t*>(acc + 4);
  __syncthreads();
  if (tid < kHd / 2) {
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < NG; ++i) M = fmaxf(M, gm[i]);
    float den = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const float f = __builtin_amdgcn_exp2f(gm[i] - M);  // empty groups: 2^-inf = 0
      den += f * gl[i];
      a0 += f * gacc[i][2 * tid];
      a1 += f * gacc[i][2 * tid + 1];
    }
    const float inv = 1.0f / den;
    *reinterpret_cast<uint32_t*>(out + ((size_t)t * nh + h) * kHd + 2 * tid) =
        pack2(a0 * inv, a1 * inv);
  }
}

// ---------------------------------------------------------------------------
// Skinny GEMMs for decode, T <= 16 tokens, weights streamed by stream_bf16:
//   plain: y [T, N] = x [T, K] . W [N, K]^T;
//   GLU:   y [T, Ni] = silu(g) * u with g|u = x . W^T and W [2*Ni, K] holding
//          the gate rows then the up rows (the activation is applied to the
//          fp32 sums, so the [T, 2*Ni] product never exists).
// A work item is a pair of 16-row tiles (32 consecutive rows; for GLU the
// gate and up rows of the same 16 channels) and a part of K; the host
// splits K into `ks` parts so that the items spread over the CUs (one CU
// streams only ~27 GB/s, so a small matrix in few items leaves most of HBM
// idle).  The item's 4 waves split its chunks and reduce in LDS.  With
// ks > 1 an item writes its fp32 partial tiles to the workspace with
// device-coherent stores and counts itself on the item's counter; the
// item's last part sums the parts in part order (the result does not
// depend on which part finishes last), finishes y and re-arms the counter.
// ---------------------------------------------------------------------------
constexpr int kLinWaves = 4;
constexpr int kLinD = 2;
constexpr int kLinMaxCus = 1024;        // workspace bound: ks * items <= 2 * CUs
constexpr size_t kLinPartBytes = (size_t)2 * kLinMaxCus * 32 * 16 * sizeof(float);

struct LinLds {
  f32x4_t red[kLinWaves][2][64];
  u32x4_t stage[kLinWaves][kStageVecs];
  int last;
};

// Finish 4 rows of token col: plain -> two bf16 row groups (t = 0, 1);
// GLU -> one bf16 group of silu(g) * u.
template <bool GLU>
__device__ __forceinline__ void lin_store(uint16_t* __restrict__ y, int ny, int col, int r0,
                                          int kg, bool two, f32x4_t v0, f32x4_t v1) {
  if (GLU) {
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = v0[r] / (1.0f + expf(-v0[r])) * v1[r];
    *reinterpret_cast<u32x2_t*>(y + (size_t)col * ny + r0 + kg * 4) =
        u32x2_t{pack2(o[0], o[1]), pack2(o[2], o[3])};
  } else {
    *reinterpret_cast<u32x2_t*>(y + (size_t)col * ny + r0 + kg * 4) =
        u32x2_t{pack2(v0[0], v0[1]), pack2(v0[2], v0[3])};
    if (two)
      *reinterpret_cast<u32x2_t*>(y + (size_t)col * ny + r0 + 16 + kg * 4) =
          u32x2_t{pack2(v1[0], v1[1]), pack2(v1[2], v1[3])};
  }
}

// GLU: item i covers channels 16*i .. +16 (ny = Ni = N / 2); plain: rows
// 32*i .. +32 (ny = N).
template <bool GLU>
__global__ __launch_bounds__(64 * kLinWaves) void linear_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int T, int N, int K, int ks,
    uint16_t* __restrict__ y, float* __restrict__ parts, int* __restrict__ counters,
    float* __restrict__ split) {
  __shared__ LinLds l;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kg = lane >> 4;
  const int item = blockIdx.x / ks, part = blockIdx.x - item * ks;
  const int nc = K / 64;
  const int p0 = part * nc / ks, p1 = (part + 1) * nc / ks;
  const int c0 = p0 + wave * (p1 - p0) / kLinWaves, c1 = p0 + (wave + 1) * (p1 - p0) / kLinWaves;
  const int ny = GLU ? N / 2 : N;
  const int r0 = GLU ? item * 16 : item * 32;
  const bool two = GLU || r0 + 16 < N;  // plain, N % 32 == 16: the last item holds 16 rows
  const uint16_t* a0 = w + (size_t)r0 * K;
  const uint16_t* a1 = GLU ? w + (size_t)(ny + r0) * K : (two ? a0 + (size_t)16 * K : a0);
  const uint16_t* xr = x + (size_t)(col < T ? col : T - 1) * K;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  stream_bf16<kTokPlain, kLinD>(a0, a1, K, xr, c0, c1 - c0, l.stage[wave], acc0, acc1);
  l.red[wave][0][lane] = acc0;
  l.red[wave][1][lane] = acc1;
  __syncthreads();
  // lane (col, kg) of wave 0 owns rows kg*4 .. +4 of both tiles for token col
  if (wave == 0 && col < T) {
    f32x4_t v0 = l.red[0][0][lane], v1 = l.red[0][1][lane];
#pragma unroll
    for (int u = 1; u < kLinWaves; ++u) {
      v0 += l.red[u][0][lane];
      v1 += l.red[u][1][lane];
    }
    if (!GLU && split != nullptr) {
      // the parts themselves, row-major [ks][T][N], for the next kernel to sum
      float* dst = split + ((size_t)part * T + col) * N + r0 + kg * 4;
      *reinterpret_cast<f32x4_t*>(dst) = v0;
      if (two) *reinterpret_cast<f32x4_t*>(dst + 16) = v1;
      return;
    }
    if (ks == 1) {
      lin_store<GLU>(y, ny, col, r0, kg, two, v0, v1);
    } else {
      // parts [ks][T][2 tiles][items * 16], tile-major so both tiles of an item sit together
      float* dst = parts + (((size_t)part * T + col) * 2) * (size_t)(gridDim.x / ks) * 16 +
                   (size_t)item * 16 + kg * 4;
      const size_t tstride = (size_t)(gridDim.x / ks) * 16;
      st8_coh(dst, __float_as_uint(v0[0]), __float_as_uint(v0[1]));
      st8_coh(dst + 2, __float_as_uint(v0[2]), __float_as_uint(v0[3]));
      st8_coh(dst + tstride, __float_as_uint(v1[0]), __float_as_uint(v1[1]));
      st8_coh(dst + tstride + 2, __float_as_uint(v1[2]), __float_as_uint(v1[3]));
    }
    if (ks > 1) __builtin_amdgcn_s_waitcnt(0);  // written through before the part is counted
  }
  if (ks == 1 || split != nullptr) return;
  __syncthreads();
  if (threadIdx.x == 0) {
    l.last = atomicAdd(&counters[item], 1) == ks - 1;
    if (l.last) atomicExch(&counters[item], 0);
  }
  __syncthreads();
  if (!l.last || wave != 0 || col >= T) return;
  const size_t tstride = (size_t)(gridDim.x / ks) * 16;
  f32x4_t v0 = {0.f, 0.f, 0.f, 0.f}, v1 = v0;
  for (int p = 0; p < ks; ++p) {
    const float* src = parts + (((size_t)p * T + col) * 2) * tstride + (size_t)item * 16 + kg * 4;
    v0 += __builtin_bit_cast(f32x4_t, ld16_coh(src));
    v1 += __builtin_bit_cast(f32x4_t, ld16_coh(src + tstride));
  }
  lin_store<GLU>(y, ny, col, r0, kg, two, v0, v1);
}

int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n < kLinMaxCus ? n : kLinMaxCus;
  }
  return cus[dev];
}

// Parts of K per item, from per-kernel costs measured in replayed graphs on
// MI355X (decode shapes, T = 1 and 8, N 2048-21888, K 2048-10944): the
// hand-off of a split costs about as much as streaming a 3072-long row slice
// on one CU, so K up to 3072 stays whole; longer K splits in 3 (up to 4096)
// or 4.  ks * items <= 2 * CUs keeps the partials within the workspace bound.
int linear_parts(int items, int K, int T, int cus) {
  (void)T;
  const int nc = K / 64;
  int ks = nc <= 48 ? 1 : nc <= 64 ? 3 : 4;
  if (ks > nc) ks = nc;
  while (ks > 1 && (long)items * ks > 2L * cus) --ks;
  return ks;
}

template <bool GLU>
int launch_linear(const void* x, const void* w, int T, int N, int K, void* y, void* ws,
                  hipStream_t st) {
  const int items = GLU ? N / 32 : (N + 31) / 32;
  const int ks = ws != nullptr ? linear_parts(items, K, T, device_cus()) : 1;
  float* parts = (float*)ws;
  int* counters = ws != nullptr ? (int*)((char*)ws + kLinPartBytes) : nullptr;
  hipLaunchKernelGGL((linear_kernel<GLU>), dim3(items * ks), dim3(64 * kLinWaves), 0, st,
                     (const uint16_t*)x, (const uint16_t*)w, T, N, K, ks, (uint16_t*)y, parts,
                     counters, (float*)nullptr);
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Greedy next token: out[t] = argmax_n x[t, n] (first index on ties), one
// workgroup per row.  A graph-safe replacement for a library reduction that
// would record a memset of its cross-block semaphores.
// ---------------------------------------------------------------------------
constexpr int kArg = 1024;

__global__ __launch_bounds__(kArg) void argmax_kernel(const uint16_t* __restrict__ x, int N,
                                                      int64_t* __restrict__ out) {
  __shared__ float bv[kArg / 64];
  __shared__ int bi[kArg / 64];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* row = x + (size_t)t * N;
  float best = -INFINITY;
  int besti = N;  // sentinel above every index
  if ((N & 7) == 0 && ((uintptr_t)row & 15) == 0) {
    // 8 values per 16-byte load, 4 loads in flight per thread; a thread's
    // indices only grow, so a strict '>' keeps the first of equal values
    const int nv = N / 8;
    const u32x4_t* rv = reinterpret_cast<const u32x4_t*>(row);
    for (int v0 = tid; v0 < nv; v0 += 4 * kArg) {
      u32x4_t q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int v = v0 + u * kArg;
        q[u] = rv[v < nv ? v : v0];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int v = v0 + u * kArg;
        if (v < nv) {
          float f[8];
          unpack8(q[u], f);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (f[e] > best || (besti == N && f[e] == best)) {
              best = f[e];
              besti = v * 8 + e;
            }
        }
      }
    }
  } else {
    for (int i = tid; i < N; i += kArg) {
      const float v = bf(row[i]);
      if (v > best || (besti == N && v == best)) {
        best = v;
        besti = i;
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off, SLUICE_WAVE);
    const int oi = __shfl_xor(besti, off, SLUICE_WAVE);
    if (ov > best || (ov == best && oi < besti)) {
      best = ov;
      besti = oi;
    }
  }
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = besti;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArg / 64; ++w)
      if (bv[w] > best || (bv[w] == best && bi[w] < besti)) {
        best = bv[w];
        besti = bi[w];
      }
    out[t] = besti < N ? besti : 0;
  }
}

}  // namespace

extern "C" int sluice_dec_argmax(const void* x, int T, int N, int64_t* out,
                                 sluice_stream_t stream) {
  if (T < 0 || N <= 0 || x == nullptr || out == nullptr) return SLUICE_E_INVAL;
  if (T == 0) return SLUICE_OK;
  hipLaunchKernelGGL(argmax_kernel, dim3(T), dim3(kArg), 0, (hipStream_t)stream,
                     (const uint16_t*)x, N, out);
  return (int)hipGetLastError();
}

extern "C" size_t sluice_dec_linear_workspace(void) {
  return kLinPartBytes + (size_t)kLinMaxCus * sizeof(int);
}

extern "C" int sluice_dec_linear(const void* x, const void* w, int T, int N, int K, void* y,
                                 void* workspace, sluice_stream_t stream) {
  if (T < 0 || T > 16 || N <= 0 || N % 16 != 0 || K <= 0 || K % 64 != 0 || x == nullptr ||
      w == nullptr || y == nullptr)
    return SLUICE_E_INVAL;
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)workspace) & 15 || (uintptr_t)y & 7)
    return SLUICE_E_INVAL;
  if (T == 0) return SLUICE_OK;
  return launch_linear<false>(x, w, T, N, K, y, workspace, (hipStream_t)stream);
}

// K parts of a projection whose parts the next kernel sums (no hand-off).
// Measured in replayed graphs with distinct weights per launch (T = 1 and 8):
// 4 parts for K <= 2048 (N = 2048: 3.8 vs 5.6 us whole; N = 5120: 5.9 vs
// 6.1), 3 for K <= 4096 (N = 2048: 5.3 vs 8.7 us whole, 5.8 with 4), 4 beyond.
int split_parts(int items, int K, int T) {
  (void)items;
  (void)T;
  const int nc = K / 64;
  int ks = nc <= 32 ? 4 : nc <= 64 ? 3 : 4;
  while (ks > 1 && nc < 8 * ks) --ks;  // at least 8 chunks per part
  return ks;
}

extern "C" int sluice_dec_linear_split_parts(int T, int N, int K) {
  if (T <= 0 || T > 16 || N <= 0 || N % 16 != 0 || K <= 0 || K % 64 != 0) return 0;
  return split_parts((N + 31) / 32, K, T);
}

extern "C" int sluice_dec_linear_split(const void* x, const void* w, int T, int N, int K,
                                       float* parts, sluice_stream_t stream) {
  if (T < 0 || T > 16 || N <= 0 || N % 16 != 0 || K <= 0 || K % 64 != 0 || x == nullptr ||
      w == nullptr || parts == nullptr)
    return SLUICE_E_INVAL;
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)parts) & 15) return SLUICE_E_INVAL;
  if (T == 0) return SLUICE_OK;
  const int items = (N + 31) / 32;
  const int ks = split_parts(items, K, T);
  hipLaunchKernelGGL((linear_kernel<false>), dim3(items * ks), dim3(64 * kLinWaves), 0,
                     (hipStream_t)stream, (const uint16_t*)x, (const uint16_t*)w, T, N, K, ks,
                     (uint16_t*)nullptr, (float*)nullptr, (int*)nullptr, parts);
  return (int)hipGetLastError();
}

extern "C" int sluice_dec_linear_glu(const void* x, const void* w, int T, int N, int K, void* y,
                                     void* workspace, sluice_stream_t stream) {
  if (T < 0 || T > 16 || N <= 0 || N % 32 != 0 || K <= 0 || K % 64 != 0 || x == nullptr ||
      w == nullptr || y == nullptr)
    return SLUICE_E_INVAL;
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)workspace) & 15 || (uintptr_t)y & 7)
    return SLUICE_E_INVAL;
  if (T == 0) return SLUICE_OK;
  return launch_linear<true>(x, w, T, N, K, y, workspace, (hipStream_t)stream);
}

extern "C" int sluice_dec_add_rmsnorm(void* x, const void* delta, const void* w, void* out,
                                      int rows, int H, float eps, sluice_stream_t stream) {
  if (rows < 0 || H <= 0 || H % 8 != 0 || x == nullptr || w == nullptr || out == nullptr)
    return SLUICE_E_INVAL;
  if (((uintptr_t)x | (uintptr_t)delta | (uintptr_t)w | (uintptr_t)out) & 15) return SLUICE_E_INVAL;
  if (rows == 0) return SLUICE_OK;
  const int ni = (H + kT * 8 - 1) / (kT * 8);
  auto* xp = (uint16_t*)x;
  auto* dp = (const uint16_t*)delta;
  auto* wp = (const uint16_t*)w;
  auto* op = (uint16_t*)out;
  hipStream_t st = (hipStream_t)stream;
  if (ni <= 1)
    hipLaunchKernelGGL(add_rmsnorm_reg_kernel<1>, dim3(rows), dim3(kT), 0, st, xp, dp, wp, op, H,
                       eps);
  else if (ni <= 2)
    hipLaunchKernelGGL(add_rmsnorm_reg_kernel<2>, dim3(rows), dim3(kT), 0, st, xp, dp, wp, op, H,
                       eps);
  else if (ni <= 4)
    hipLaunchKernelGGL(add_rmsnorm_reg_kernel<4>, dim3(rows), dim3(kT), 0, st, xp, dp, wp, op, H,
                       eps);
  else
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(rows), dim3(kT), 0, st, xp, dp, wp, op, H, eps);
  return (int)hipGetLastError();
}

extern "C" int sluice_dec_silu_mul(const void* gu, void* out, int rows, int I,
                                   sluice_stream_t stream) {
  if (rows < 0 || I <= 0 || I % 4 != 0 || gu == nullptr || out == nullptr) return SLUICE_E_INVAL;
  if (((uintptr_t)gu | (uintptr_t)out) & 7) return SLUICE_E_INVAL;
  if (rows == 0) return SLUICE_OK;
  dim3 grid((I / 4 + kT - 1) / kT, rows);
  hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(kT), 0, (hipStream_t)stream,
                     (const uint16_t*)gu, (uint16_t*)out, I);
  return (int)hipGetLastError();
}

extern "C" int sluice_dec_gate_logits(const void* hn, const void* wg, const float* bias_table,
                                      const int64_t* step, int n_steps, int bias_rows, int rows,
                                      int H, int E, float* out, sluice_stream_t stream) {
  if (rows < 0 || rows > kMaxRows || H <= 0 || H % 32 != 0 || E <= 0 || hn == nullptr ||
      wg == nullptr || out == nullptr)
    return SLUICE_E_INVAL;
  if (bias_table != nullptr && (step == nullptr || n_steps <= 0 || bias_rows < rows))
    return SLUICE_E_INVAL;
  if (((uintptr_t)hn | (uintptr_t)wg) & 15) return SLUICE_E_INVAL;
  if (rows == 0) return SLUICE_OK;
  with_row_bucket(rows, [&](auto mr) {
    constexpr int R = decltype(mr)::value;
    hipLaunchKernelGGL((gate_logits_kernel<R>), dim3(E), dim3(kT), 0, (hipStream_t)stream,
                       (const uint16_t*)hn, (const uint16_t*)wg, bias_table, step, n_steps,
                       bias_rows, rows, H, E, out);
  });
  return (int)hipGetLastError();
}

// Experts per workgroup of the fused norm + router kernel: 4 measured
// faster than 8 or 16 in replayed graphs (more workgroups, each shorter).
constexpr int kNormGateEpw = 4;

extern "C" int sluice_dec_add_rmsnorm_gate_ok(int rows, int H) {
  return rows >= 0 && rows <= kMaxRows && H > 0 && H % 8 == 0 && H <= 4 * kT * 8;
}

extern "C" int sluice_dec_add_rmsnorm_gate(const void* x, const void* delta,
                                          const float* delta_parts, int n_parts, const void* w,
                                          void* x_out, void* hn_out, const void* wg,
                                          const float* bias_table, const int64_t* step,
                                          int n_steps, int bias_rows, int rows, int H, int E,
                                          float eps, float* logits, sluice_stream_t stream) {
  if (!sluice_dec_add_rmsnorm_gate_ok(rows, H) || E <= 0 || !x || !w || !x_out || !hn_out || !wg ||
      !logits)
    return SLUICE_E_INVAL;
  if (delta_parts != nullptr &&
      (delta != nullptr || n_parts < 1 || n_parts > kMaxDeltaParts || ((uintptr_t)delta_parts & 15)))
    return SLUICE_E_INVAL;
  if (bias_table != nullptr && (step == nullptr || n_steps <= 0 || bias_rows < rows))
    return SLUICE_E_INVAL;
  if (((uintptr_t)x | (uintptr_t)delta | (uintptr_t)w | (uintptr_t)x_out | (uintptr_t)hn_out |
       (uintptr_t)wg) & 15)
    return SLUICE_E_INVAL;
  if (rows == 0) return SLUICE_OK;
  constexpr int EPW = kNormGateEpw;
  const dim3 grid(rows, (E + EPW - 1) / EPW);
  hipStream_t st = (hipStream_t)stream;
  auto go = [&](auto ni) {
    constexpr int NI = decltype(ni)::value;
    hipLaunchKernelGGL((add_rmsnorm_gate_kernel<NI, EPW>), grid, dim3(kT), 0, st,
                       (const uint16_t*)x, (const uint16_t*)delta, delta_parts, n_parts,
                       (const uint16_t*)w,
                       (uint16_t*)x_out, (uint16_t*)hn_out, (const uint16_t*)wg, bias_table, step,
                       n_steps, bias_rows, H, E, eps, logits);
  };
  const int ni = (H + kT * 8 - 1) / (kT * 8);
  if (ni <= 1)
    go(std::integral_constant<int, 1>{});
  else if (ni <= 2)
    go(std::integral_constant<int, 2>{});
  else
    go(std::integral_constant<int, 4>{});
  return (int)hipGetLastError();
}

extern "C" size_t sluice_dec_mla_workspace(int c, int nh) {
  if (c <= 0 || nh <= 0) return 0;
  const size_t ql = (size_t)c * nh * (kLora + kRope) * sizeof(uint16_t);
  return (ql + 255) / 256 * 256 + (size_t)c * kMlaSplit * nh * kMlaRec * sizeof(float);
}

extern "C" int sluice_dec_mla_decode(const void* q, int q_stride, const void* kva,
                                     int kva_stride, const void* kv_norm, const void* w_ukt,
                                     const void* w_uv, const float* cos_t, const float* sin_t,
                                     const int64_t* pos, int c, int nh, int nope, int rope,
                                     int lora, int vh, int L, float eps, float scale,
                                     void* ckv_cache, void* ckvt_cache, void* kpe_cache,
                                     void* work, void* out, sluice_stream_t stream) {
  if (c < 0 || c > 16 || nh <= 0 || nh % 16 != 0 || nope <= 0 || nope % 32 != 0 ||
      rope != kRope || lora != kLora || vh <= 0 || vh > 256 || vh % 8 != 0 || L <= 0 ||
      L > kMaxL || L % 32 != 0 || q_stride < nh * (nope + rope) || q_stride % 8 != 0 ||
      kva_stride < lora + rope || kva_stride % 2 != 0)
    return SLUICE_E_INVAL;
  if (!q || !kva || !kv_norm || !w_ukt || !w_uv || !cos_t || !sin_t || !pos || !ckv_cache ||
      !ckvt_cache || !kpe_cache || !work || !out)
    return SLUICE_E_INVAL;
  if ((((uintptr_t)q | (uintptr_t)w_ukt | (uintptr_t)w_uv | (uintptr_t)ckv_cache |
        (uintptr_t)ckvt_cache | (uintptr_t)kpe_cache | (uintptr_t)work) & 15) != 0 ||
      (((uintptr_t)kva | (uintptr_t)kv_norm) & 3) != 0)
    return SLUICE_E_INVAL;
  if (c == 0) return SLUICE_OK;
  hipStream_t st = (hipStream_t)stream;
  uint16_t* q_lat = (uint16_t*)work;
  uint16_t* q_pe = q_lat + (size_t)c * nh * kLora;
  const size_t ql = (size_t)c * nh * (kLora + kRope) * sizeof(uint16_t);
  float* part = (float*)((char*)work + (ql + 255) / 256 * 256);
  hipLaunchKernelGGL(mla_absorb_kernel, dim3(nh * (kLora / 64) + c), dim3(kT), 0, st,
                     (const uint16_t*)q, q_stride, (const uint16_t*)kva, kva_stride,
                     (const uint16_t*)kv_norm, (const uint16_t*)w_ukt, cos_t, sin_t, pos, c, nh,
                     nope, L, eps, q_lat, q_pe, (uint16_t*)ckv_cache, (uint16_t*)ckvt_cache,
                     (uint16_t*)kpe_cache);
  hipLaunchKernelGGL(mla_partial_kernel, dim3(c, kMlaSplit, nh / 16), dim3(kMlaWaves * 64), 0,
                     st, q_lat,
                     q_pe, (const uint16_t*)ckv_cache, (const uint16_t*)ckvt_cache,
                     (const uint16_t*)kpe_cache, pos, nh, L, scale * 1.4426950408889634f, part);
  hipLaunchKernelGGL(mla_merge_kernel, dim3(c, nh, (vh + 63) / 64), dim3(kT), 0, st, part,
                     (const uint16_t*)w_uv, pos, nh, vh, L, (uint16_t*)out);
  return (int)hipGetLastError();
}

extern "C" int sluice_dec_gqa_decode(const void* qkv, const float* qkv_parts, int n_parts,
                                     const void* q_norm, const void* k_norm,
                                     const float* cos_t, const float* sin_t, const int64_t* pos,
                                     int c, int nh, int kvh, int hd, int L, float eps, float scale,
                                     void* k_cache, void* v_cache, void* out,
                                     sluice_stream_t stream) {
  if (c < 0 || nh <= 0 || kvh <= 0 || nh % kvh != 0 || hd != kHd || L <= 0 || L > kMaxL)
    return SLUICE_E_INVAL;
  if ((qkv == nullptr) == (qkv_parts == nullptr)) return SLUICE_E_INVAL;  // exactly one
  if (qkv_parts != nullptr && (n_parts < 1 || n_parts > kMaxDeltaParts)) return SLUICE_E_INVAL;
  if (!q_norm || !k_norm || !cos_t || !sin_t || !pos || !k_cache || !v_cache || !out)
    return SLUICE_E_INVAL;
  if ((((uintptr_t)qkv | (uintptr_t)qkv_parts | (uintptr_t)q_norm | (uintptr_t)k_norm | (uintptr_t)cos_t |
        (uintptr_t)sin_t | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15) != 0 ||
      ((uintptr_t)out & 3) != 0)
    return SLUICE_E_INVAL;
  if (c == 0) return SLUICE_OK;
  hipLaunchKernelGGL((gqa_decode_kernel<kGqaWaves, kGqaRows>), dim3(c, nh),
                     dim3(kGqaWaves * 64), 0, (hipStream_t)stream, (const uint16_t*)qkv,
                     qkv_parts, n_parts, (const uint16_t*)q_norm, (const uint16_t*)k_norm, cos_t, sin_t, pos, nh, kvh,
                     L, eps, scale, (uint16_t*)k_cache, (uint16_t*)v_cache, (uint16_t*)out);
  return (int)hipGetLastError();
}

