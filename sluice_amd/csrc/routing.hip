// a1: top-k routing over 64..1024 expert logits, one wave64 per token.
//
// Replaces vLLM's select_experts as called from the router-split entry
// (src/sluice/offloader.py:2583-2585).  The closed forms it computes are the
// textbook ones the supported models use:
//   softmax greedy (DeepSeek-V2-Lite, no renorm) and softmax + renorm (Qwen3
//   MoE); sigmoid + score-correction bias, group-limited by the sum of each
//   group's two best biased scores, weights from the unbiased sigmoid,
//   renormalised and scaled (DeepSeek-V3).
//
// Selection: k rounds of a wave-wide argmax over (key, expert id) in the
// order "greater key, or equal key and lower id", each round reducing with
// xor-shuffles and retiring the winner in its owning lane.  Round r picks the
// candidate that exactly r eligible candidates beat, so outputs come out
// best-first with ties going to the lower id, with no sort and no pass over
// all E keys per lane (an exact-rank pass of that kind cost ~45 us at
// E = 256).  Softmax is monotone, so selection runs on the logits themselves;
// sigmoid scores are evaluated in fp64 and rounded to fp32 once, so that
// selection on fp32(s + bias) is reproducible bit for bit on the host.
//
// The kernel is instantiated per scoring mode and per experts-per-lane (NV =
// 1, 2, 4, 16) so each launch runs compact straight-line code: a decode step
// launches it once per MoE layer, where cold instruction fetch, not
// arithmetic, is what a bloated variant pays for.
#include <math.h>

#include "common.h"

namespace {

__device__ __forceinline__ float load_logit(const void* p, int dtype, size_t i) {
  if (dtype == 1) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, SLUICE_WAVE));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, SLUICE_WAVE);
  return v;
}

template <int NV, int SCORING>
__global__ __launch_bounds__(SLUICE_WAVE) void route_topk_kernel(
    const void* __restrict__ logits, int dtype, int E, int k, int renorm, float scale,
    const float* __restrict__ bias, int n_group, int topk_group, int32_t* __restrict__ ids_out,
    float* __restrict__ w_out) {
  __shared__ float s_key[SLUICE_MAX_EXPERTS];  // selection keys (group scores read them)
  __shared__ float s_gscore[SLUICE_WAVE];
  __shared__ int s_gok[SLUICE_WAVE];
  __shared__ int s_sel[SLUICE_MAX_TOPK];
  __shared__ float s_w[SLUICE_MAX_TOPK];

  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const size_t row = (size_t)t * E;

  float key[NV], raw[NV];
  bool ok[NV];
  float lmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = lane + j * SLUICE_WAVE;
    ok[j] = e < E;
    key[j] = -INFINITY;
    raw[j] = 0.0f;
    if (ok[j]) {
      const float l = load_logit(logits, dtype, row + e);
      if (SCORING == 0) {
        raw[j] = l;
        key[j] = l;
        lmax = fmaxf(lmax, l);
      } else {
        raw[j] = (float)(1.0 / (1.0 + exp(-(double)l)));
        key[j] = raw[j] + (bias != nullptr ? bias[e] : 0.0f);
      }
      s_key[e] = key[j];
    }
  }

  if (n_group > 1) {
    const int gsize = E / n_group;
    if (gsize <= SLUICE_WAVE && (gsize & (gsize - 1)) == 0) {
      // A group is gsize consecutive lanes of one register: reduce its two
      // best keys with xor-shuffles inside the group.
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        float b1 = key[j], b2 = -INFINITY;
        for (int off = 1; off < gsize; off <<= 1) {
          const float o1 = __shfl_xor(b1, off, SLUICE_WAVE);
          const float o2 = __shfl_xor(b2, off, SLUICE_WAVE);
          const float hi = fmaxf(b1, o1), lo = fminf(b1, o1);
          b2 = fmaxf(lo, fmaxf(b2, o2));
          b1 = hi;
        }
        const int e = lane + j * SLUICE_WAVE;
        // softmax: group max; sigmoid: sum of the two best biased scores
        if (e < E && (e & (gsize - 1)) == 0)
          s_gscore[e / gsize] = (SCORING == 0 || gsize < 2) ? b1 : b1 + b2;
      }
    } else {
      __syncthreads();
      if (lane < n_group) {
        const int g0 = lane * gsize;
        float b1 = -INFINITY, b2 = -INFINITY;
        for (int e = g0; e < g0 + gsize; ++e) {
          const float v = s_key[e];
          if (v > b1) {
            b2 = b1;
            b1 = v;
          } else if (v > b2) {
            b2 = v;
          }
        }
        s_gscore[lane] = (SCORING == 0 || gsize < 2) ? b1 : b1 + b2;
      }
    }
    __syncthreads();
    if (lane < n_group) {
      const float mine = s_gscore[lane];
      int rank = 0;
      for (int h = 0; h < n_group; ++h) {
        const float o = s_gscore[h];
        rank += (o > mine || (o == mine && h < lane)) ? 1 : 0;
      }
      s_gok[lane] = rank < topk_group ? 1 : 0;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = lane + j * SLUICE_WAVE;
      if (ok[j]) ok[j] = s_gok[e / gsize] != 0;
    }
  }
  // k rounds of a wave argmax; the winner's owner records it and retires it.
  bool live[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) live[j] = ok[j];
  for (int r = 0; r < k; ++r) {
    float bk = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = lane + j * SLUICE_WAVE;
      if (live[j] && (key[j] > bk || (key[j] == bk && e < bi))) {
        bk = key[j];
        bi = e;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ok2 = __shfl_xor(bk, off, SLUICE_WAVE);
      const int oi = __shfl_xor(bi, off, SLUICE_WAVE);
      if (ok2 > bk || (ok2 == bk && oi < bi)) {
        bk = ok2;
        bi = oi;
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (bi == lane + j * SLUICE_WAVE) {
        live[j] = false;
        s_sel[r] = bi;
        s_w[r] = raw[j];  // softmax: the logit, weighted below
      }
    }
    if (bi == 0x7fffffff && lane == 0) {  // only NaN keys left: no expert, no weight
      s_sel[r] = -1;
      s_w[r] = SCORING == 0 ? -INFINITY : 0.0f;
    }
  }

  // Weights of the winners, in selection order.
  float m = 0.0f, z = 1.0f;
  if (SCORING == 0) {
    m = wave_max(lmax);
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (lane + j * SLUICE_WAVE < E) part += expf(raw[j] - m);
    z = wave_sum(part);
  }
  __syncthreads();
  if (SCORING == 0 && lane < k) s_w[lane] = expf(s_w[lane] - m) / z;
  __syncthreads();
  if (lane < k) {
    float w = s_w[lane];
    if (renorm) {
      float sum = 0.0f;
      for (int r = 0; r < k; ++r) sum += s_w[r];
      w = SCORING == 0 ? w / sum : w / (sum + 1e-20f);
    }
    ids_out[(size_t)t * k + lane] = s_sel[lane];
    w_out[(size_t)t * k + lane] = w * scale;
  }
}

template <int NV>
void launch(int scoring, dim3 grid, hipStream_t st, const void* logits, int dtype, int E, int k,
            int renorm, float scale, const float* bias, int ng, int tg, int32_t* ids, float* w) {
  if (scoring == 0)
    hipLaunchKernelGGL((route_topk_kernel<NV, 0>), grid, dim3(SLUICE_WAVE), 0, st, logits, dtype,
                       E, k, renorm, scale, bias, ng, tg, ids, w);
  else
    hipLaunchKernelGGL((route_topk_kernel<NV, 1>), grid, dim3(SLUICE_WAVE), 0, st, logits, dtype,
                       E, k, renorm, scale, bias, ng, tg, ids, w);
}

}  // namespace

extern "C" int sluice_route_topk(const void* logits, int logits_dtype, int T, int E, int k,
                                 int scoring, int renorm, float scale, const float* bias,
                                 int n_group, int topk_group, int32_t* ids_out, float* w_out,
                                 sluice_stream_t stream) {
  if (T < 0 || E <= 0 || E > SLUICE_MAX_EXPERTS || k <= 0 || k > SLUICE_MAX_TOPK || k > E)
    return SLUICE_E_INVAL;
  if (logits_dtype != 0 && logits_dtype != 1) return SLUICE_E_INVAL;
  if (scoring != 0 && scoring != 1) return SLUICE_E_INVAL;
  if (n_group < 1) n_group = 1;
  if (n_group > 1) {
    if (n_group > SLUICE_WAVE || E % n_group != 0) return SLUICE_E_INVAL;
    if (topk_group < 1 || topk_group > n_group) return SLUICE_E_INVAL;
    if (topk_group * (E / n_group) < k) return SLUICE_E_INVAL;
  }
  if (T == 0) return SLUICE_OK;
  if (logits == nullptr || ids_out == nullptr || w_out == nullptr) return SLUICE_E_INVAL;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(T);
  const int nv = (E + SLUICE_WAVE - 1) / SLUICE_WAVE;
  if (nv <= 1)
    launch<1>(scoring, grid, st, logits, logits_dtype, E, k, renorm, scale, bias, n_group,
              topk_group, ids_out, w_out);
  else if (nv <= 2)
    launch<2>(scoring, grid, st, logits, logits_dtype, E, k, renorm, scale, bias, n_group,
              topk_group, ids_out, w_out);
  else if (nv <= 4)
    launch<4>(scoring, grid, st, logits, logits_dtype, E, k, renorm, scale, bias, n_group,
              topk_group, ids_out, w_out);
  else
    launch<16>(scoring, grid, st, logits, logits_dtype, E, k, renorm, scale, bias, n_group,
               topk_group, ids_out, w_out);
  return (int)hipGetLastError();
}
