// Gap timeline tracing (internal to libsluice_hip; opt-in build).
//
// Built with -DSLUICE_TRACE (sluice_amd/build.py --trace ->
// libsluice_hip_trace.so), the gap kernel, the expert product's split launch
// and the combine stamp events with the device wall clock (s_memrealtime,
// the constant-rate clock every wait here is bounded on), and the host gap
// service stamps its steps with CLOCK_MONOTONIC; sluice_trace_calibrate
// relates the two clocks.  sluice_amd/timeline.py reads both rings and splits
// a decode step's link-idle time into its parts.  In the default build every
// hook compiles to nothing and the entry points return SLUICE_E_STATE.
//
// Device record: word 0 = tag << 56 | value (56 bits), word 1 = wall clock.
// Host record: tag, layer id, stamp, value, seconds.
//   device, gap kernel (value = layer id << 24 | stamp):
//     1 stamp taken   2 record posted   3 answer read   4 kernel end
//   device, expert product:
//     10 a pending slot's ready mark seen by its poller (slot << 24 | stamp)
//     11 split launch started (grid)        13 combine started (T)
//     14 a pending gemm1 item's slot wait ended (ticket)
//     15 a pending gemm1 item done (ticket)
//     17 a pending gemm2 item's gemm1 count reached (ticket)
//     16 a pending gemm2 item done (ticket)
//   host, gap service (layer id = the device map address >> 8):
//     21 record copied out (v = misses the device counted)
//     22 bookkeeping done (v = stream-ins)
//     23 first row copy over the link issued (v = experts before it in copy
//        order: those served from staged rows)
//     24 device answered (v = row copies per expert)
//     25 every row copy issued (v = signals)
//     26 expert j (copy order) landed (v = j)
//     27 expert j's slot marked ready (v = j)
//     28 staging chunk issued, 29 staging chunk seen landed (stamp 0,
//        v = KiB << 1 | staging lane)
#pragma once

#include "common.h"

#ifdef SLUICE_TRACE

constexpr unsigned kTraceDevRing = 1u << 20;  // device records per translation unit

// Each translation unit that traces keeps its own ring.
static __device__ unsigned long long g_trace_dev[kTraceDevRing][2];
static __device__ unsigned int g_trace_dev_n;

__device__ __forceinline__ void trace_dev(unsigned tag, unsigned long long value) {
  const unsigned i = atomicAdd(&g_trace_dev_n, 1u) & (kTraceDevRing - 1);
  g_trace_dev[i][0] = ((unsigned long long)tag << 56) | (value & ((1ull << 56) - 1));
  g_trace_dev[i][1] = wall_clock64();
}

__device__ __forceinline__ unsigned long long trace_id(const void* p) {
  return ((unsigned long long)(uintptr_t)p >> 8) & 0xffffffffull;
}

#define SLUICE_DTRACE(tag, value) trace_dev((tag), (value))
#define SLUICE_TRACE_GAP(tag, map, stamp) \
  trace_dev((tag), (trace_id(map) << 24) | ((unsigned long long)(stamp) & 0xffffff))

// Copies this translation unit's ring and count out (host).
inline int trace_dev_read(unsigned long long* out, unsigned* n) {
  SLUICE_HIP_CHECK(hipMemcpyFromSymbol(n, HIP_SYMBOL(g_trace_dev_n), sizeof(unsigned)));
  if (out != nullptr)
    SLUICE_HIP_CHECK(hipMemcpyFromSymbol(out, HIP_SYMBOL(g_trace_dev), sizeof(g_trace_dev)));
  return SLUICE_OK;
}
inline int trace_dev_reset() {
  const unsigned z = 0;
  SLUICE_HIP_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_dev_n), &z, sizeof(z)));
  return SLUICE_OK;
}

#else

#define SLUICE_DTRACE(tag, value) ((void)0)
#define SLUICE_TRACE_GAP(tag, map, stamp) ((void)0)

#endif
