// a1: top-k routing over 64..1024 expert logits, one wave64 per token.
//
// Replaces vLLM's select_experts as called from the router-split entry
// (src/sluice/offloader.py:2583-2585).  The closed forms it computes are the
// textbook ones the supported models use:
//   softmax greedy (DeepSeek-V2-Lite, no renorm) and softmax + renorm (Qwen3
//   MoE); sigmoid + score-correction bias, group-limited by the sum of each
//   group's two best biased scores, weights from the unbiased sigmoid,
//   renormalised and scaled (DeepSeek-V3).
// Selection is an exact k-round wave argmax (no sort): every round each lane
// offers its best not-yet-taken candidate and a 6-step xor-shuffle reduction
// picks the wave winner, ties going to the lower expert id.  Softmax is
// monotone, so selection runs on the logits themselves; sigmoid scores are
// evaluated in fp64 and rounded to fp32 once so that selection on
// fp32(s + bias) is reproducible bit for bit on the host.
#include <math.h>

#include "common.h"

namespace {

constexpr int kMaxPerLane = SLUICE_MAX_EXPERTS / SLUICE_WAVE;  // 16

__device__ __forceinline__ bool better(float v1, int i1, float v2, int i2) {
  return v1 > v2 || (v1 == v2 && i1 < i2);
}

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

__global__ __launch_bounds__(SLUICE_WAVE) void route_topk_kernel(
    const void* __restrict__ logits, int dtype, int E, int k, int scoring,
    int renorm, float scale, const float* __restrict__ bias, int n_group,
    int topk_group, int32_t* __restrict__ ids_out, float* __restrict__ w_out) {
  __shared__ float s_raw[SLUICE_MAX_EXPERTS];  // logit (softmax) or sigmoid s
  __shared__ float s_key[SLUICE_MAX_EXPERTS];  // selection key
  __shared__ float s_gscore[SLUICE_WAVE];
  __shared__ int s_gok[SLUICE_WAVE];
  __shared__ int s_sel[SLUICE_MAX_TOPK];

  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const size_t row = (size_t)t * E;
  const int nv = (E + SLUICE_WAVE - 1) / SLUICE_WAVE;

  float key[kMaxPerLane];
  bool eligible[kMaxPerLane];
  float lmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    const int e = lane + j * SLUICE_WAVE;
    key[j] = -INFINITY;
    eligible[j] = false;
    if (j < nv && e < E) {
      const float l = load_logit(logits, dtype, row + e);
      float raw, kv;
      if (scoring == 0) {
        raw = l;
        kv = l;
      } else {
        raw = (float)(1.0 / (1.0 + exp(-(double)l)));
        kv = raw + (bias != nullptr ? bias[e] : 0.0f);
      }
      s_raw[e] = raw;
      s_key[e] = kv;
      key[j] = kv;
      eligible[j] = true;
      lmax = fmaxf(lmax, l);
    }
  }

  if (n_group > 1) {
    __syncthreads();
    const int gsize = E / n_group;
    if (lane < n_group) {
      const int g0 = lane * gsize;
      float score;
      if (scoring == 0) {
        score = -INFINITY;
        for (int e = g0; e < g0 + gsize; ++e) score = fmaxf(score, s_key[e]);
      } else {
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
        score = gsize >= 2 ? b1 + b2 : b1;
      }
      s_gscore[lane] = score;
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
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + j * SLUICE_WAVE;
      if (eligible[j]) eligible[j] = s_gok[e / gsize] != 0;
    }
  }

  // k rounds of exact wave argmax.
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + j * SLUICE_WAVE;
      if (eligible[j] && better(key[j], e, bv, bi)) {
        bv = key[j];
        bi = e;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, SLUICE_WAVE);
      const int oi = __shfl_xor(bi, off, SLUICE_WAVE);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    // bi is uniform across the wave; its owner retires it.
    if (bi != 0x7fffffff && (bi & (SLUICE_WAVE - 1)) == lane) {
#pragma unroll
      for (int j = 0; j < kMaxPerLane; ++j)
        if (lane + j * SLUICE_WAVE == bi) eligible[j] = false;
    }
    if (lane == 0) s_sel[r] = bi;
  }
  __syncthreads();

  // Weights.
  float denom_all = 1.0f;
  if (scoring == 0) {
    const float m = wave_max(lmax);
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + j * SLUICE_WAVE;
      if (j < nv && e < E) part += expf(s_raw[e] - m);
    }
    denom_all = wave_sum(part);
    if (lane == 0) {
      float w[SLUICE_MAX_TOPK];
      float wsum = 0.0f;
      for (int r = 0; r < k; ++r) {
        const int e = s_sel[r];
        w[r] = (e < E) ? expf(s_raw[e] - m) / denom_all : 0.0f;
        wsum += w[r];
      }
      for (int r = 0; r < k; ++r) {
        float v = renorm ? w[r] / wsum : w[r];
        ids_out[(size_t)t * k + r] = s_sel[r] < E ? s_sel[r] : -1;
        w_out[(size_t)t * k + r] = v * scale;
      }
    }
  } else {
    if (lane == 0) {
      float w[SLUICE_MAX_TOPK];
      float wsum = 0.0f;
      for (int r = 0; r < k; ++r) {
        const int e = s_sel[r];
        w[r] = (e < E) ? s_raw[e] : 0.0f;
        wsum += w[r];
      }
      for (int r = 0; r < k; ++r) {
        float v = renorm ? w[r] / (wsum + 1e-20f) : w[r];
        ids_out[(size_t)t * k + r] = s_sel[r] < E ? s_sel[r] : -1;
        w_out[(size_t)t * k + r] = v * scale;
      }
    }
  }
}

}  // namespace

extern "C" int sluice_route_topk(const void* logits, int logits_dtype, int T,
                                 int E, int k, int scoring, int renorm,
                                 float scale, const float* bias, int n_group,
                                 int topk_group, int32_t* ids_out, float* w_out,
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
  hipLaunchKernelGGL(route_topk_kernel, dim3(T), dim3(SLUICE_WAVE), 0,
                     (hipStream_t)stream, logits, logits_dtype, E, k, scoring,
                     renorm, scale, bias, n_group, topk_group, ids_out, w_out);
  return (int)hipGetLastError();
}
