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

// grid (c, nh + 1): y < nh -> query head y; y == nh -> the token's kv row.
__global__ __launch_bounds__(kT) void mla_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kva,
    const uint16_t* __restrict__ kv_norm, const uint16_t* __restrict__ w_uk,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int64_t* __restrict__ pos, int nh, int nope, int q_stride, int kva_stride, int L,
    float eps, float* __restrict__ q_lat, float* __restrict__ q_pe,
    uint16_t* __restrict__ ckv_cache, uint16_t* __restrict__ kpe_cache) {
  __shared__ float qn[256];
  __shared__ float red[kT / 64];
  __shared__ float ql_part[kT / 64][kLora];
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const long long p = pos[t];
  if (p < 0 || p >= L) return;
  const float* cr = cos_t + p * (kRope / 2);
  const float* sr = sin_t + p * (kRope / 2);
  if (h < nh) {
    const uint16_t* qh = q + (size_t)t * q_stride + (size_t)h * (nope + kRope);
    for (int d = tid; d < nope; d += kT) qn[d] = bf(qh[d]);
    if (tid < kRope / 2) {
      const float x1 = bf(qh[nope + tid]), x2 = bf(qh[nope + tid + kRope / 2]);
      float* o = q_pe + ((size_t)t * nh + h) * kRope;
      o[tid] = x1 * cr[tid] - x2 * sr[tid];
      o[tid + kRope / 2] = x2 * cr[tid] + x1 * sr[tid];
    }
    __syncthreads();
    // q_lat[j] = sum_d q_nope[d] w_uk[h][d][j]: wave w takes rows d = w, w+4,
    // ..., a lane owns columns 8*lane..+8 (16-byte loads, 4 rows in flight);
    // the waves' sums meet in LDS.
    const int wave = tid >> 6, lane = tid & 63;
    const uint16_t* wk = w_uk + (size_t)h * nope * kLora + lane * 8;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int d0 = wave; d0 < nope; d0 += 16) {
      u32x4_t wv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int d = d0 + 4 * u;
        wv[u] = *reinterpret_cast<const u32x4_t*>(wk + (size_t)(d < nope ? d : 0) * kLora);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int d = d0 + 4 * u;
        const float qd = d < nope ? qn[d] : 0.f;
        float c[8];
        unpack8(wv[u], c);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += qd * c[j];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ql_part[wave][lane * 8 + j] = acc[j];
    __syncthreads();
    float* o = q_lat + ((size_t)t * nh + h) * kLora;
    for (int j = tid; j < kLora; j += kT)
      o[j] = ql_part[0][j] + ql_part[1][j] + ql_part[2][j] + ql_part[3][j];
    return;
  }
  // kv row: rmsnorm(kva[:lora]) * kv_norm, rope(kva[lora:])
  const uint16_t* kr = kva + (size_t)t * kva_stride;
  const uint32_t v2 = reinterpret_cast<const uint32_t*>(kr)[tid];
  const float x0 = __uint_as_float(v2 << 16), x1 = __uint_as_float(v2 & 0xffff0000u);
  const float rstd = rsqrtf(block_sum(x0 * x0 + x1 * x1, red) / (float)kLora + eps);
  const uint32_t g2 = reinterpret_cast<const uint32_t*>(kv_norm)[tid];
  uint32_t* crow = reinterpret_cast<uint32_t*>(ckv_cache + ((size_t)t * L + p) * kLora);
  crow[tid] = pack2(x0 * rstd * __uint_as_float(g2 << 16),
                    x1 * rstd * __uint_as_float(g2 & 0xffff0000u));
  if (tid < kRope / 2) {
    const float a = bf(kr[kLora + tid]), b = bf(kr[kLora + tid + kRope / 2]);
    uint16_t* krow = kpe_cache + ((size_t)t * L + p) * kRope;
    krow[tid] = f32_to_bf16_bits(a * cr[tid] - b * sr[tid]);
    krow[tid + kRope / 2] = f32_to_bf16_bits(b * cr[tid] + a * sr[tid]);
  }
}

// grid (c, nh), kA threads.  Scores: each wave takes rows l = wave,
// wave + W, ... four at a time (four independent 1 KB loads and reductions
// in flight); the latent sum: each wave accumulates its rows (a lane owns 8
// latent columns, 16-byte loads, four rows in flight) and the waves are
// summed in LDS; the value projection: a thread owns 2 value columns and a
// slice of the latent rows, eight rows of w_uv in flight.
constexpr int kA = 1024;
constexpr int kAW = kA / 64;

__global__ __launch_bounds__(kA) void mla_attend_kernel(
    const float* __restrict__ q_lat, const float* __restrict__ q_pe,
    const uint16_t* __restrict__ ckv_cache, const uint16_t* __restrict__ kpe_cache,
    const uint16_t* __restrict__ w_uv, const int64_t* __restrict__ pos, int nh, int vh, int L,
    float scale, uint16_t* __restrict__ out) {
  __shared__ float s[kMaxL];
  __shared__ float part[kAW][kLora];
  __shared__ float ol[kLora];
  __shared__ float red[kAW];
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const long long p = pos[t];
  if (p < 0 || p >= L) return;
  const int n = (int)p + 1;
  const uint16_t* cb = ckv_cache + (size_t)t * L * kLora;
  const uint16_t* kb = kpe_cache + (size_t)t * L * kRope;
  float ql[8];
  {
    const float* qrow = q_lat + ((size_t)t * nh + h) * kLora + lane * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) ql[j] = qrow[j];
  }
  const float qp = q_pe[((size_t)t * nh + h) * kRope + lane];
  constexpr int U = 8;  // cache rows in flight per wave
  float lmax = -INFINITY;
  for (int l0 = wave; l0 < n; l0 += U * kAW) {
    float dsum[U];
    u32x4_t cv[U];
    uint16_t kv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int l = l0 + u * kAW;
      const int lc = l < n ? l : 0;
      cv[u] = *reinterpret_cast<const u32x4_t*>(cb + (size_t)lc * kLora + lane * 8);
      kv[u] = kb[(size_t)lc * kRope + lane];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float c[8];
      unpack8(cv[u], c);
      float d = qp * bf(kv[u]);
#pragma unroll
      for (int j = 0; j < 8; ++j) d += ql[j] * c[j];
      dsum[u] = d;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) dsum[u] = wave_sum(dsum[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int l = l0 + u * kAW;
      if (l < n) {
        const float d = dsum[u] * scale;
        if (lane == 0) s[l] = d;
        lmax = fmaxf(lmax, d);
      }
    }
  }
  // block max
  lmax = wave_max(lmax);
  if (lane == 0) red[wave] = lmax;
  __syncthreads();
  float m = -INFINITY;
  for (int i = 0; i < kAW; ++i) m = fmaxf(m, red[i]);
  __syncthreads();
  float psum = 0.f;
  for (int l = tid; l < n; l += kA) {
    const float e = expf(s[l] - m);
    s[l] = e;
    psum += e;
  }
  psum = wave_sum(psum);
  if (lane == 0) red[wave] = psum;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < kAW; ++i) tot += red[i];
  const float inv = 1.0f / tot;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  for (int l0 = wave; l0 < n; l0 += U * kAW) {
    u32x4_t cv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int l = l0 + u * kAW;
      cv[u] = *reinterpret_cast<const u32x4_t*>(cb + (size_t)(l < n ? l : 0) * kLora + lane * 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int l = l0 + u * kAW;
      const float pl = l < n ? s[l] : 0.f;
      float c[8];
      unpack8(cv[u], c);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += pl * c[j];
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) part[wave][lane * 8 + j] = acc[j];
  __syncthreads();
  for (int j = tid; j < kLora; j += kA) {
    float v = 0.f;
    for (int w = 0; w < kAW; ++w) v += part[w][j];
    ol[j] = v * inv;
  }
  __syncthreads();
  // out[v] = o_lat . w_uv[h][:, v]: thread = (column pair, slice of kAW rows' worth)
  const uint16_t* wv = w_uv + (size_t)h * kLora * vh;
  float* pq = &part[0][0];  // reused: [kAW][128] partial sums
  constexpr int kRows = kLora / kAW;
  for (int v0 = 0; v0 < vh; v0 += 128) {
    const int vp = v0 + 2 * lane;
    float a0 = 0.f, a1 = 0.f;
    if (vp < vh) {
      const uint16_t* col = wv + vp;
      const int j0 = wave * kRows;
      for (int j = j0; j < j0 + kRows; j += 8) {
        uint32_t w8[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w8[u] = *reinterpret_cast<const uint32_t*>(col + (size_t)(j + u) * vh);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          a0 += ol[j + u] * __uint_as_float(w8[u] << 16);
          a1 += ol[j + u] * __uint_as_float(w8[u] & 0xffff0000u);
        }
      }
    }
    pq[wave * 128 + 2 * lane] = a0;
    pq[wave * 128 + 2 * lane + 1] = a1;
    __syncthreads();
    if (tid < 128 && v0 + tid < vh) {
      float v = 0.f;
      for (int w = 0; w < kAW; ++w) v += pq[w * 128 + tid];
      out[((size_t)t * nh + h) * vh + v0 + tid] = f32_to_bf16_bits(v);
    }
    __syncthreads();
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
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_norm,
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
  const u32x4_t xq = ldg16(xr + h * kHd + col);
  const u32x4_t xk = ldg16(xr + (nh + g) * kHd + col);
  const u32x4_t xv = ldg16(xr + (nh + kvh + g) * kHd + col);
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
    uint16_t* __restrict__ y, float* __restrict__ parts, int* __restrict__ counters) {
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
  if (ks == 1) return;
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
                     counters);
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

extern "C" int sluice_dec_mla_prep(const void* q, int q_stride, const void* kva, int kva_stride,
                                   const void* kv_norm, const void* w_uk, const float* cos_t,
                                   const float* sin_t, const int64_t* pos, int c, int nh, int nope,
                                   int rope, int lora, int L, float eps, float* q_lat, float* q_pe,
                                   void* ckv_cache, void* kpe_cache, sluice_stream_t stream) {
  if (c < 0 || nh <= 0 || nope <= 0 || nope > 256 || nope % 2 != 0 || rope != kRope ||
      lora != kLora || L <= 0 || L > kMaxL || q_stride < nh * (nope + rope) ||
      kva_stride < lora + rope || kva_stride % 2 != 0)
    return SLUICE_E_INVAL;
  if (((uintptr_t)kva | (uintptr_t)kv_norm | (uintptr_t)w_uk | (uintptr_t)ckv_cache) & 3)
    return SLUICE_E_INVAL;
  if (!q || !kva || !kv_norm || !w_uk || !cos_t || !sin_t || !pos || !q_lat || !q_pe ||
      !ckv_cache || !kpe_cache)
    return SLUICE_E_INVAL;
  if (c == 0) return SLUICE_OK;
  hipLaunchKernelGGL(mla_prep_kernel, dim3(c, nh + 1), dim3(kT), 0, (hipStream_t)stream,
                     (const uint16_t*)q, (const uint16_t*)kva, (const uint16_t*)kv_norm,
                     (const uint16_t*)w_uk, cos_t, sin_t, pos, nh, nope, q_stride, kva_stride, L,
                     eps, q_lat, q_pe, (uint16_t*)ckv_cache, (uint16_t*)kpe_cache);
  return (int)hipGetLastError();
}

extern "C" int sluice_dec_mla_attend(const float* q_lat, const float* q_pe, const void* ckv_cache,
                                     const void* kpe_cache, const void* w_uv, const int64_t* pos,
                                     int c, int nh, int rope, int lora, int vh, int L, float scale,
                                     void* out, sluice_stream_t stream) {
  if (c < 0 || nh <= 0 || rope != kRope || lora != kLora || vh <= 0 || vh > 256 || vh % 2 ||
      L <= 0 || L > kMaxL)
    return SLUICE_E_INVAL;
  if (!q_lat || !q_pe || !ckv_cache || !kpe_cache || !w_uv || !pos || !out) return SLUICE_E_INVAL;
  if ((uintptr_t)ckv_cache & 15) return SLUICE_E_INVAL;
  if (c == 0) return SLUICE_OK;
  hipLaunchKernelGGL(mla_attend_kernel, dim3(c, nh), dim3(kA), 0, (hipStream_t)stream, q_lat,
                     q_pe, (const uint16_t*)ckv_cache, (const uint16_t*)kpe_cache,
                     (const uint16_t*)w_uv, pos, nh, vh, L, scale, (uint16_t*)out);
  return (int)hipGetLastError();
}

extern "C" int sluice_dec_gqa_decode(const void* qkv, const void* q_norm, const void* k_norm,
                                     const float* cos_t, const float* sin_t, const int64_t* pos,
                                     int c, int nh, int kvh, int hd, int L, float eps, float scale,
                                     void* k_cache, void* v_cache, void* out,
                                     sluice_stream_t stream) {
  if (c < 0 || nh <= 0 || kvh <= 0 || nh % kvh != 0 || hd != kHd || L <= 0 || L > kMaxL)
    return SLUICE_E_INVAL;
  if (!qkv || !q_norm || !k_norm || !cos_t || !sin_t || !pos || !k_cache || !v_cache || !out)
    return SLUICE_E_INVAL;
  if ((((uintptr_t)qkv | (uintptr_t)q_norm | (uintptr_t)k_norm | (uintptr_t)cos_t |
        (uintptr_t)sin_t | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15) != 0 ||
      ((uintptr_t)out & 3) != 0)
    return SLUICE_E_INVAL;
  if (c == 0) return SLUICE_OK;
  hipLaunchKernelGGL((gqa_decode_kernel<kGqaWaves, kGqaRows>), dim3(c, nh),
                     dim3(kGqaWaves * 64), 0, (hipStream_t)stream, (const uint16_t*)qkv,
                     (const uint16_t*)q_norm, (const uint16_t*)k_norm, cos_t, sin_t, pos, nh, kvh,
                     L, eps, scale, (uint16_t*)k_cache, (uint16_t*)v_cache, (uint16_t*)out);
  return (int)hipGetLastError();
}

