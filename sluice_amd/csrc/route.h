// Top-k routing of one token by one wave64 (gfx950).
//
// route_topk_kernel runs it with one wave per token; any kernel that routes
// with it gets the same ids and weight bits from the same logits.
//
// The closed forms are those of vLLM's select_experts as the router-split
// entry calls it (src/sluice/offloader.py:2583-2585):
//   softmax greedy (DeepSeek-V2-Lite, no renorm) and softmax + renorm (Qwen3
//   MoE); sigmoid + score-correction bias, group-limited by the sum of each
//   group's two best biased scores, weights from the unbiased sigmoid,
//   renormalised and scaled (DeepSeek-V3).
//
// Selection: k rounds of a wave-wide argmax over (key, expert id) in the
// order "greater key, or equal key and lower id", each round a DPP max over
// order-preserving key codes plus one ballot per register for the lowest id
// holding the winning code, the winner retired in its owning lane.  Round r picks the
// candidate that exactly r eligible candidates beat, so outputs come out
// best-first with ties going to the lower id.  Softmax is monotone, so
// selection runs on the logits themselves; sigmoid scores are evaluated in
// fp64 and rounded to fp32 once, so that selection on fp32(s + bias) is
// reproducible bit for bit on the host.
#pragma once

#include <math.h>

#include "common.h"

// The lanes of one wave exchange values through LDS between these points.
// LDS operations of one wave execute in program order, so only the compiler
// has to be kept from moving accesses across them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Order-preserving map of a float key to uint32 (greater key, greater code;
// -0 and +0 share a code, as they compare equal; -inf is 0x007fffff); 0
// marks "no candidate" and NaN keys never compete.
__device__ __forceinline__ uint32_t route_key_code(float x) {
  const uint32_t u = x == 0.0f ? 0u : __float_as_uint(x);
  if (x != x) return 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One wave's LDS for routing a token over up to MAXE experts.
template <int MAXE>
struct RouteLds {
  float key[MAXE];  // selection keys (group scores of irregular groups read them)
  float gscore[SLUICE_WAVE];
  int gok[SLUICE_WAVE];
};

// Routes one token: logit(e) returns the token's fp32 logit of expert e.
// Writes ids[0..k) and w[0..k) (best first).  Every lane of the wave calls
// it; NV * 64 >= E, E <= MAXE.
template <int NV, int SCORING, int MAXE, typename LogitFn>
__device__ __forceinline__ void route_token(LogitFn logit, int E, int k, int renorm, float scale,
                                            const float* __restrict__ bias, int n_group,
                                            int topk_group, RouteLds<MAXE>& l,
                                            int32_t* __restrict__ ids, float* __restrict__ w_out) {
  const int lane = threadIdx.x & (SLUICE_WAVE - 1);
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
      const float x = logit(e);
      if (SCORING == 0) {
        raw[j] = x;
        key[j] = x;
        lmax = fmaxf(lmax, x);
      } else {
        raw[j] = (float)(1.0 / (1.0 + exp(-(double)x)));
        key[j] = raw[j] + (bias != nullptr ? bias[e] : 0.0f);
      }
      l.key[e] = key[j];
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
          l.gscore[e / gsize] = (SCORING == 0 || gsize < 2) ? b1 : b1 + b2;
      }
    } else {
      wave_lds_sync();
      if (lane < n_group) {
        const int g0 = lane * gsize;
        float b1 = -INFINITY, b2 = -INFINITY;
        for (int e = g0; e < g0 + gsize; ++e) {
          const float v = l.key[e];
          if (v > b1) {
            b2 = b1;
            b1 = v;
          } else if (v > b2) {
            b2 = v;
          }
        }
        l.gscore[lane] = (SCORING == 0 || gsize < 2) ? b1 : b1 + b2;
      }
    }
    wave_lds_sync();
    if (lane < n_group) {
      const float mine = l.gscore[lane];
      int rank = 0;
      for (int h = 0; h < n_group; ++h) {
        const float o = l.gscore[h];
        rank += (o > mine || (o == mine && h < lane)) ? 1 : 0;
      }
      l.gok[lane] = rank < topk_group ? 1 : 0;
    }
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = lane + j * SLUICE_WAVE;
      if (ok[j]) ok[j] = l.gok[e / gsize] != 0;
    }
  }
  // k rounds of a wave argmax over (key code, expert id): the largest code
  // wins, equal codes go to the lower id (the lowest lane of the first
  // register holding the code).  Winners are uniform across the wave; lane r
  // keeps round r's id and raw value.
  uint32_t code[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) code[j] = ok[j] ? route_key_code(key[j]) : 0u;
  int my_id = -1;
  float my_w = SCORING == 0 ? -INFINITY : 0.0f;  // round without a candidate
  for (int r = 0; r < k; ++r) {
    uint32_t best = 0u;
#pragma unroll
    for (int j = 0; j < NV; ++j) best = code[j] > best ? code[j] : best;
    const uint32_t top = wave_max_u32(best);
    if (top == 0u) break;  // only NaN keys (or none) left: no expert, no weight
    int jw = 0;
    uint64_t m = 0;
#pragma unroll
    for (int j = NV - 1; j >= 0; --j) {
      const uint64_t b = __ballot(code[j] == top);
      if (b != 0) {
        jw = j;
        m = b;
      }
    }
    const int lw = __builtin_ctzll(m);
    float rv = raw[0];
#pragma unroll
    for (int j = 1; j < NV; ++j) rv = jw == j ? raw[j] : rv;
    rv = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(rv), lw));
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (j == jw && lane == lw) code[j] = 0u;  // retired
    if (lane == r) {
      my_id = jw * SLUICE_WAVE + lw;
      my_w = rv;  // softmax: the logit, weighted below
    }
  }

  // Weights of the winners, in selection order.
  if (SCORING == 0) {
    const float mx = wave_max_f32(lmax);
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (lane + j * SLUICE_WAVE < E) part += expf(raw[j] - mx);
    const float z = wave_sum_f32(part);
    my_w = expf(my_w - mx) / z;
  }
  if (renorm) {
    const float sum = wave_sum_f32(lane < k ? my_w : 0.0f);
    my_w = SCORING == 0 ? my_w / sum : my_w / (sum + 1e-20f);
  }
  if (lane < k) {
    ids[lane] = my_id;
    w_out[lane] = my_w * scale;
  }
  wave_lds_sync();  // the wave may route its next token with the same LDS
}
