/* Measurement probe of libsluice_hip (no counterpart in the reference: it
 * calibrates the expert kernels' HBM fraction, it is not on the path). */
#ifndef SLUICE_PROBE_H
#define SLUICE_PROBE_H

#include "sluice.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A plain streaming read of `bytes` (multiple of 16, 16-byte aligned) at
 * src, on `stream`: 16-byte non-temporal loads, 4 per thread in flight,
 * at most 4096 workgroups of 256 threads.  sink (device, 4 bytes) is only
 * written when the xor of everything read equals one fixed constant, which
 * keeps the loads live.  Timing it at an expert kernel's bytes per launch
 * gives what a kernel that only reads reaches at that launch size. */
int sluice_read_probe(const void* src, size_t bytes, uint32_t* sink, sluice_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif
