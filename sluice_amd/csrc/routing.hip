// a1: top-k routing over 64..1024 expert logits, one wave64 per token.
//
// Replaces vLLM's select_experts as called from the router-split entry
// (src/sluice/offloader.py:2583-2585); the per-token selection and weights
// are route_token (route.h), shared with the decoder's fused gate + routing
// kernel.  An exact-rank pass over all E keys per lane cost ~45 us at
// E = 256; the k rounds of a wave argmax that route_token runs do not.
//
// The kernel is instantiated per scoring mode and per experts-per-lane (NV =
// 1, 2, 4, 16) so each launch runs compact straight-line code: a decode step
// launches it once per MoE layer, where cold instruction fetch, not
// arithmetic, is what a bloated variant pays for.
#include "common.h"
#include "route.h"

namespace {

__device__ __forceinline__ float load_logit(const void* p, int dtype, size_t i) {
  if (dtype == 1) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

template <int NV, int SCORING>
__global__ __launch_bounds__(SLUICE_WAVE) void route_topk_kernel(
    const void* __restrict__ logits, int dtype, int E, int k, int renorm, float scale,
    const float* __restrict__ bias, int n_group, int topk_group, int32_t* __restrict__ ids_out,
    float* __restrict__ w_out) {
  __shared__ RouteLds<NV * SLUICE_WAVE> l;
  const int t = blockIdx.x;
  const size_t row = (size_t)t * E;
  route_token<NV, SCORING>([&](int e) { return load_logit(logits, dtype, row + e); }, E, k,
                           renorm, scale, bias, n_group, topk_group, l, ids_out + (size_t)t * k,
                           w_out + (size_t)t * k);
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
