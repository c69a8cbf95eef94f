// The decode kernel of coded host stores (codec.h), built on its own into
// sluice_amd/codec_decode.hsaco (a code object with no host part) and
// dispatched by codec.hip on an HSA queue of the library's own: the expert
// product that waits for a decoded slot may hold an in-order hardware queue
// that HIP streams share, and a decode queued behind it would never run.
//
// The decode is byte work bound by HBM: per chunk of 2048 values each lane
// reads 8 sign/mantissa bytes and 4 nibble bytes (coalesced across the
// wave) and writes 16 bytes of bf16; the chunk's base exponent and escape
// offsets are one scalar load each.  The kernel
// allocates few registers and no LDS, so that it fits beside the expert
// product's waiting workgroups (sluice_amd/build.py checks its registers),
// and reads no implicit kernel arguments (the grid size is in the job), so
// its kernarg segment is the job alone.
#include "codec.h"
#include "common.h"

namespace {

constexpr int kCodecUnroll = 4;  // chunks a workgroup decodes per round
static_assert(kCodecChunk == 8 * kCodecThreads, "a lane decodes 8 values of a chunk");

// Device-coherent stores (written through the L2 of this XCD to memory):
// the decoded rows are read by workgroups on every XCD, and with coherent
// stores no wave has to write back a whole L2 before the slot is marked.
__device__ __forceinline__ void st16_coh(void* p, const u32x4_t& v) {
  uint64_t* q = static_cast<uint64_t*>(p);
  __hip_atomic_store(q, (uint64_t)v[0] | (uint64_t)v[1] << 32, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, (uint64_t)v[2] | (uint64_t)v[3] << 32, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

extern "C" __global__ __launch_bounds__(kCodecThreads) void sluice_codec_decode_kernel(CodecJob job) {
  // A workgroup decodes kCodecUnroll chunks of 2048 values per round, each
  // lane 8 values of each; the chunk, its part and its base exponent are the
  // same for the whole workgroup (scalar loads).  After the round's stores,
  // the escapes of its chunks are patched in parallel, one lane per entry.
  uint32_t total = 0;
#pragma unroll
  for (int q = 0; q < kCodecMaxParts; ++q) total += q < job.n_part ? job.part[q].n_chunk : 0u;
  const uint32_t tid = __builtin_amdgcn_workitem_id_x();
  const uint32_t wg = __builtin_amdgcn_workgroup_id_x();
  for (uint32_t c0 = wg * kCodecUnroll; c0 < total; c0 += job.n_wg * kCodecUnroll) {
    const uint8_t* src[kCodecUnroll];
    uint16_t* dst[kCodecUnroll];
    uint32_t loc[kCodecUnroll], nchk[kCodecUnroll], n_esc[kCodecUnroll];
    u32x2_t sm[kCodecUnroll];
    uint32_t nb[kCodecUnroll], base[kCodecUnroll];
#pragma unroll
    for (int u = 0; u < kCodecUnroll; ++u) {
      // the part holding chunk c (static indices: the job stays in registers)
      const uint32_t c = min(c0 + u, total - 1);
      uint32_t first = 0;
      CodecPart pt = job.part[0];
#pragma unroll
      for (int q = 1; q < kCodecMaxParts; ++q)
        if (q < job.n_part && c - first >= pt.n_chunk) {
          first += pt.n_chunk;
          pt = job.part[q];
        }
      loc[u] = c - first;
      nchk[u] = pt.n_chunk;
      n_esc[u] = pt.n_esc;
      src[u] = pt.src;
      dst[u] = pt.dst + (size_t)loc[u] * kCodecChunk + 8 * tid;
      const size_t n = (size_t)pt.n_chunk * kCodecChunk;
      sm[u] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x2_t*>(pt.src + (size_t)loc[u] * kCodecChunk + 8 * tid));
      nb[u] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(
          pt.src + n + (size_t)loc[u] * (kCodecChunk / 2) + 4 * tid));
      base[u] = pt.src[codec_base_off(n) + loc[u]];
    }
#pragma unroll
    for (int u = 0; u < kCodecUnroll; ++u) {
      if (c0 + u >= total) break;
      // Two values per 32-bit word, lane-parallel within the word: value 2p
      // in the low half, 2p + 1 in the high half.  The sign/mantissa bytes
      // and the byte of nibbles of pair p are placed at bytes 0 and 2 by
      // byte permutes (selector 0x0c gives a zero byte).
      const uint32_t base2 = base[u] | base[u] << 16;
      uint32_t out[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t b0 = (uint32_t)(2 * k) & 3u;
        const uint32_t t = __builtin_amdgcn_perm(0u, sm[u][k >> 1],
                                                 b0 | 0x0c00u | (b0 + 1) << 16 | 0x0c000000u);
        const uint32_t x = __builtin_amdgcn_perm(0u, nb[u],
                                                 (uint32_t)k | 0x0c00u | (uint32_t)k << 16 |
                                                     0x0c000000u);
        const uint32_t code = ((x & 0x00f00000u) >> 4) | (x & 0xfu);
        // a half whose code is kCodecZero takes exponent 0
        const uint32_t y = code ^ (kCodecZero | kCodecZero << 16);
        const uint32_t zero = ((y | (y >> 1) | (y >> 2) | (y >> 3)) & 0x00010001u) ^ 0x00010001u;
        const uint32_t ex = ((code + base2) & 0x00ff00ffu) & ~(zero * 0xffu);
        out[k] = ((t & 0x00800080u) << 8) | (t & 0x007f007fu) | (ex << 7);
      }
      st16_coh(dst[u], u32x4_t{out[0], out[1], out[2], out[3]});
    }
    // Escapes (about 1 value in 6000 of a N(0, 0.02) row, a few per round):
    // stored again over the values above once every lane's stores completed.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kCodecUnroll; ++u) {
      if (c0 + u >= total) break;
      const size_t n = (size_t)nchk[u] * kCodecChunk;
      const uint32_t* off = reinterpret_cast<const uint32_t*>(src[u] + codec_esc_off_off(n));
      const uint32_t* esc = reinterpret_cast<const uint32_t*>(src[u] + codec_esc_off(n));
      const uint32_t e0 = min(off[loc[u]], n_esc[u]), e1 = min(off[loc[u] + 1], n_esc[u]);
      for (uint32_t e = e0 + tid; e < e1; e += kCodecThreads) {
        const uint32_t ent = esc[e], pos = (ent >> 8) & (uint32_t)(kCodecChunk - 1);
        const uint32_t sb = src[u][(size_t)loc[u] * kCodecChunk + pos];
        uint16_t* d = dst[u] - 8 * tid + pos;
        __hip_atomic_store(d, (uint16_t)(((sb & 0x80u) << 8) | ((ent & 0xffu) << 7) | (sb & 0x7fu)),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // Every lane's coherent stores have completed (reached memory) before its
  // workgroup counts itself; the last workgroup to count publishes the job.
  // The readers take a system-scope acquire (an L2 invalidate) after they
  // see the mark, so no write-back is needed here.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(job.wg_count, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    if (prev == job.n_wg - 1) {
      __hip_atomic_store(job.wg_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (job.ready != nullptr)
        __hip_atomic_store(job.ready, job.stamp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      if (job.done != nullptr)
        __hip_atomic_store(job.done, job.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}
