// Measurement probe: a plain streaming read of a device buffer, timed beside
// the expert kernels at the same bytes per launch, so their HBM fraction can
// be set against what a kernel that only reads reaches at that launch size
// (ramp-up and tail included).  Not on the hot path.
#include "common.h"
#include "sluice_probe.h"

namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeU = 4;       // 16-byte loads in flight per thread
constexpr int kProbeGrid = 4096;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const u32x4_t* __restrict__ p,
                                                                   size_t n,
                                                                   uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * kProbeThreads * kProbeU;
  for (size_t i = (size_t)blockIdx.x * kProbeThreads * kProbeU + threadIdx.x; i < n; i += stride) {
    u32x4_t v[kProbeU];
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) {
      const size_t j = i + (size_t)u * kProbeThreads;
      v[u] = j < n ? ldg16_stream(p + j) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  // never true for the probe's inputs in practice; keeps every load live
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace

extern "C" int sluice_read_probe(const void* src, size_t bytes, uint32_t* sink,
                                 sluice_stream_t stream) {
  if (src == nullptr || sink == nullptr || (bytes & 15) != 0 || ((uintptr_t)src & 15) != 0)
    return SLUICE_E_INVAL;
  const size_t n = bytes / 16;
  if (n == 0) return SLUICE_OK;
  const size_t per_block = (size_t)kProbeThreads * kProbeU;
  const size_t blocks = (n + per_block - 1) / per_block;
  const int grid = (int)(blocks < (size_t)kProbeGrid ? blocks : (size_t)kProbeGrid);
  hipLaunchKernelGGL(read_probe_kernel, dim3(grid), dim3(kProbeThreads), 0, (hipStream_t)stream,
                     (const u32x4_t*)src, n, sink);
  return (int)hipGetLastError();
}
