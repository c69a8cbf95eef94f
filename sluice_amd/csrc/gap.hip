// a3-a8: the streaming gap on MI355X.
//
// The reference's gap (src/sluice/offloader.py:2362-2467) is an eager host
// region between captured graph pieces: topk_ids.to("cpu") synchronises the
// stream (2406), the host runs the SLRU bookkeeping, streams misses on a copy
// stream (2443-2464, 2709-2723) and rewrites the standing expert map
// (2083-2123).  Here the gap is split at the one point where the host is
// really needed:
//
//   gap_kernel (device, capturable, one workgroup)
//     - builds the step's sorted unique selected ids in LDS (ballot
//       compaction) and counts the owned ids the standing map does not hold;
//     - posts them to the layer's mailbox in host-mapped pinned memory as
//       8-byte words that each carry the record's stamp, so the words need
//       no ordering and the kernel never waits for its bus writes to land;
//     - writes the gap op's fresh copy of hidden_states;
//     - waits for the host ONLY when residency has to change (a miss, or no
//       standing map yet), then installs the map the host sent.  A step
//       without misses leaves slots and map untouched whatever the SLRU
//       does, so the device runs on without a host round trip.
//
//   serve (host): consumes each posted record in stamp order and runs the
//     reference's bookkeeping exactly (slru::Cache::gap: fast-hit, touches,
//     claimed set, victims, overflow).  For a waiting device it answers with
//     the standing slot table and the slots being filled, issues the misses'
//     row copies as SDMA copies through the HSA runtime (two engines), and
//     marks each filled slot ready once its rows landed (the expert product
//     waits per slot).  It runs inline
//     (sluice_layer_gap: launch + serve, the reference's eager op) or on a
//     native server thread (sluice_gap_server_*), which makes the gap op
//     capturable, so a whole decode step replays as one hipGraph.
//
//   staging rows (sluice_layer_set_staging): copies in HBM of the experts a
//     layer selects most often but does not hold, which the server thread
//     fills while the host link idles; a miss on one is copied into its slot
//     from HBM before the device is answered.
//
//   coded host stores (sluice_layer_set_codec): a miss copies its expert's
//     losslessly coded rows (12 bits per bf16 value) over the link into a
//     ring in HBM, and a decode job on the library's own HSA queue writes
//     the rows into the slot and marks it ready; staging rows then hold
//     coded rows, decoded from where they lie.
//
// Ordering: a gap kernel runs only after all earlier work on its stream has
// completed, so when the host sees its record no kernel of that stream can
// still read a slot about to be overwritten (what the reference fences with
// an event from the compute stream, 2443-2447); where the reference makes
// the compute stream wait for the copies (2464), the expert product waits
// for each filled slot's ready mark.
//
// Every device wait is bounded (SLUICE_GAP_TIMEOUT_S, default 20 s, measured
// on the constant-rate wall clock) and also ends when the host raises the
// process-wide abort flag; the kernel then leaves the map unchanged and
// reports the outcome in the mailbox.
#include <immintrin.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <deque>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include "codec.h"
#include "common.h"
#include "plan.h"
#include "slotwait.h"
#include "slru.h"
#include "stamp.h"
#include "trace.h"

namespace {

constexpr int kLookupThreads = 256;
constexpr int kWaves = kLookupThreads / SLUICE_WAVE;
constexpr int kCopyU = 8;  // hidden-state vectors per thread in flight in the gap kernel

// ---------------------------------------------------------------------------
// Stand-alone lookup (sluice_slot_lookup): sorted unique ids + miss count.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kLookupThreads) void slot_lookup_kernel(
    const int32_t* __restrict__ ids, int n, const int32_t* __restrict__ map,
    const int32_t* __restrict__ local_of, int E, sluice_gap_record* rec, int32_t stamp) {
  __shared__ int present[SLUICE_MAX_EXPERTS];
  __shared__ int wcount[kWaves];
  __shared__ int wmiss[kWaves];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  for (int e = tid; e < E; e += kLookupThreads) present[e] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += kLookupThreads) {
    const int g = ids[i];
    if ((unsigned)g < (unsigned)E) present[g] = 1;
  }
  __syncthreads();

  int base = 0, miss = 0;
  for (int c = 0; c < E; c += kLookupThreads) {
    const int e = c + tid;
    const bool f = e < E && present[e] != 0;
    const bool m = f && map != nullptr && (local_of == nullptr || local_of[e] >= 0) && map[e] < 0;
    const uint64_t fb = __ballot(f);
    const uint64_t mb = __ballot(m);
    if (lane == 0) {
      wcount[wave] = __popcll(fb);
      wmiss[wave] = __popcll(mb);
    }
    __syncthreads();
    int off = base;
    for (int w = 0; w < wave; ++w) off += wcount[w];
    if (f) rec->uniq[off + mask_rank(fb)] = e;
    for (int w = 0; w < kWaves; ++w) {
      base += wcount[w];
      miss += wmiss[w];
    }
    __syncthreads();
  }
  __threadfence_system();
  __syncthreads();
  if (tid == 0) {
    rec->n_uniq = base;
    rec->n_miss = miss;
    __threadfence_system();
    __hip_atomic_store(const_cast<int32_t*>(&rec->stamp), stamp, __ATOMIC_RELEASE,
                       __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

struct SlotTable {
  int32_t n;
  int32_t g[SLUICE_MAX_SLOTS];
};

// map[g] = s for every slot s holding global id g, -1 elsewhere.  A classic
// wave also clears the device's "standing map seen" flag (standing_flag),
// so the layer's next gap waits for the host to reinstall the standing map.
__global__ __launch_bounds__(256) void map_refresh_kernel(int32_t* __restrict__ map, int E,
                                                          SlotTable tab,
                                                          int32_t* __restrict__ standing_flag) {
  __shared__ int m[SLUICE_MAX_EXPERTS];
  if (standing_flag != nullptr && threadIdx.x == 0) *standing_flag = 0;
  for (int e = threadIdx.x; e < E; e += 256) m[e] = -1;
  __syncthreads();
  for (int s = threadIdx.x; s < tab.n; s += 256) {
    const int g = tab.g[s];
    if ((unsigned)g < (unsigned)E) m[g] = s;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) map[e] = m[e];
}

// ---------------------------------------------------------------------------
// Mailbox of one layer (host pinned, coherent, mapped into the device).
// ---------------------------------------------------------------------------
// A record.  Every word carries the record's stamp in its low half, so the
// host takes a word once its stamp matches and the device needs no ordering
// (and no wait) between the words.
struct GapRecord {
  uint64_t hdr;  // stamp | n_uniq << 32 | n_miss << 43 | waits << 54
  uint64_t pad[7];
  uint64_t ent[SLUICE_MAX_EXPERTS];  // stamp | id << 32: sorted unique selected ids
};

// Records of a layer rotate through kRing slots (record s in slot s % kRing,
// stamps wrapping at a multiple of kRing: stamp.h), so the device need not
// know whether the host has copied out the previous record: only the one
// kRing records back, which it checks against the last ack it read and
// re-reads over the bus only when that is too old (once every kRing - 1 gaps
// at most, when the host keeps up).
using sluice_stamp::kRing;

struct GapMailbox {
  // written by the device
  GapRecord rec[kRing];
  int32_t dev_status;  // first failed device wait (sticky; 0 = none)
  int32_t dev_pad[15];
  // written by the host
  int32_t ack_stamp;   // last record the host has copied out
  int32_t resp_stamp;  // stamp the response below answers (written last)
  int32_t resp_code;   // 0: install slot_global as the map; else leave it
  int32_t standing;    // the device map is the standing map
  int32_t n_slots;
  int32_t n_fill;      // slots the answered gap filled (their rows may still stream)
  int32_t host_pad[10];
  int32_t slot_global[SLUICE_MAX_SLOTS];  // slot -> global id, -1 = empty
  int32_t fill[SLUICE_MAX_SLOTS];         // the filled slots
  int32_t fill_src[SLUICE_MAX_SLOTS];     // the host row (local expert) each fill takes
  int32_t slot_ready[SLUICE_MAX_SLOTS];   // stamp of the last gap whose rows into the slot landed
};

constexpr int kRecCountBits = 11;  // n_uniq, n_miss <= SLUICE_MAX_EXPERTS
static_assert(SLUICE_MAX_EXPERTS < (1 << kRecCountBits), "record count field");

__host__ __device__ inline uint64_t rec_word(int32_t stamp, uint32_t hi) {
  return (uint64_t)(uint32_t)stamp | ((uint64_t)hi << 32);
}
__host__ __device__ inline uint32_t rec_hdr_hi(int n_uniq, int n_miss, int waits) {
  return (uint32_t)n_uniq | ((uint32_t)n_miss << kRecCountBits) |
         ((uint32_t)waits << (2 * kRecCountBits));
}
inline int32_t rec_stamp(uint64_t w) { return (int32_t)(uint32_t)w; }

// The mailbox is coherent host memory, which the device reaches uncached
// over the bus.  A system-scope store is written through; an aligned 8-byte
// store is one bus write, so a record word is seen whole or not at all.
__device__ __forceinline__ void st_host(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_host64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ int32_t ld_host(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ int32_t ld_sys(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Records from stamp b forward to stamp a (stamp.h).
__host__ __device__ inline int32_t stamp_dist(int32_t a, int32_t b) {
  return sluice_stamp::dist(a, b);
}

// Spin until the host's ack *p is at most kRing stamps behind stamp s, so
// that record s's slot is free; the last value read goes to *seen.  0, or
// SLUICE_E_ABORTED / SLUICE_E_TIMEOUT.
__device__ int wait_slot(const int32_t* p, int32_t s, const int32_t* abort_flag,
                         const long long* bound, int32_t* seen) {
  const long long t0 = wall_clock64();
  const long long timeout_ticks = *bound;
  for (;;) {
    const int32_t v = ld_host(p);
    *seen = v;
    if (stamp_dist(s, v) <= kRing) return 0;
    if (ld_host(abort_flag) != 0) return SLUICE_E_ABORTED;
    if (wall_clock64() - t0 > timeout_ticks) return SLUICE_E_TIMEOUT;
    __builtin_amdgcn_s_sleep(4);
  }
}

// Spin until *p == want (acquire on success when ACQ: the caller then reads
// what the host wrote before *p).  0, or SLUICE_E_ABORTED / SLUICE_E_TIMEOUT.
template <bool ACQ>
__device__ int wait_eq(const int32_t* p, int32_t want, const int32_t* abort_flag,
                       const long long* bound) {
  const long long t0 = wall_clock64();
  const long long timeout_ticks = *bound;
  for (;;) {
    if (ld_host(p) == want) {
      if (ACQ) (void)ld_sys(p);
      return 0;
    }
    if (ld_host(abort_flag) != 0) return SLUICE_E_ABORTED;
    if (wall_clock64() - t0 > timeout_ticks) return SLUICE_E_TIMEOUT;
    __builtin_amdgcn_s_sleep(4);
  }
}

// dev_state: [0] last stamp issued, [1] 1 once the host has installed a
// standing map (device-side copy of mb->standing, which never goes back to
// 0, so later gaps skip that bus read), [2] the last host ack read.
constexpr int kGapMaxPerThread = SLUICE_MAX_EXPERTS / kLookupThreads;

// Per-expert params whose rows are small (fp8 block-scale rows, a few KB):
// the layer keeps a copy of all their rows in HBM, and a gap that answers
// before its rows land copies them into the filled slots itself, right
// after it installs the map.  On a copy engine such a row would queue
// behind the big rows of its lane and cost a completion of its own; as a
// HIP-stream copy it ran as a runtime copy kernel on the CUs, which the
// expert product's pending workgroups, waiting for these slots, could hold;
// and a read of host memory issued while the copy engine fills the link
// waits tens of microseconds behind it.  (The big rows stay on the copy
// engines, which need no CU.)
constexpr int kMaxPull = 4;
constexpr size_t kPullMaxRowBytes = 32 << 10;
struct PullRows {
  int n;                         // params copied by the gap kernel
  int rows;                      // host rows of each (the layer's local experts)
  int vecs[kMaxPull];            // 16-byte vectors per row
  const u32x4_t* src[kMaxPull];  // all rows of the param, in HBM
  u32x4_t* dst[kMaxPull];        // slot rows
};
constexpr int kPullU = 8;  // vectors per thread in flight

// Copy the pulled params' rows of the nf fills (slot fslot[f] takes row
// fsrc[f]) from their HBM copy into the slots: every (param, fill, vector)
// index in one flat range, kPullU loads in flight per thread.
__device__ void pull_rows(const PullRows& pull, const int* fslot, const int* fsrc, int nf, int S,
                          int tid) {
  int per_fill = 0;
  for (int p = 0; p < pull.n; ++p) per_fill += pull.vecs[p];
  const int total = nf * per_fill;
  for (int j0 = 0; j0 < total; j0 += kPullU * kLookupThreads) {
    u32x4_t v[kPullU];
    u32x4_t* dst[kPullU];
#pragma unroll
    for (int u = 0; u < kPullU; ++u) {
      const int j = j0 + u * kLookupThreads + tid;
      dst[u] = nullptr;
      if (j >= total) continue;
      const int f = j / per_fill;
      int w = j - f * per_fill, p = 0;
      while (p + 1 < pull.n && w >= pull.vecs[p]) w -= pull.vecs[p++];
      const int sl = fslot[f], src = fsrc[f];
      if ((unsigned)sl >= (unsigned)S || (unsigned)src >= (unsigned)pull.rows) continue;
      v[u] = pull.src[p][(size_t)src * pull.vecs[p] + w];
      dst[u] = pull.dst[p] + (size_t)sl * pull.vecs[p] + w;
    }
#pragma unroll
    for (int u = 0; u < kPullU; ++u)
      if (dst[u] != nullptr) *dst[u] = v[u];
  }
}

// pending [S]: the stamp of the gap that filled each slot, while its rows may
// still stream (0 = none); prev: [0] = count, [1..] = the slots the last
// waiting gap filled, cleared by the next gap (the expert product of that
// gap's step waited for each of them).
__global__ __launch_bounds__(kLookupThreads) void gap_kernel(
    const int32_t* __restrict__ ids, int n, int32_t* __restrict__ map,
    const int32_t* __restrict__ local_of, int E, GapMailbox* mb, int32_t* dev_state,
    int32_t* __restrict__ pending, int32_t* __restrict__ prev, int S, const int32_t* abort_flag,
    const long long* bound, const u32x4_t* __restrict__ copy_src, u32x4_t* __restrict__ copy_dst,
    int copy_vecs, int32_t* __restrict__ plan, PullRows pull) {
  __shared__ int present[SLUICE_MAX_EXPERTS];
  __shared__ int s_fslot[SLUICE_MAX_SLOTS], s_fsrc[SLUICE_MAX_SLOTS];
  __shared__ sluice_plan::Scratch psc;
  __shared__ int s_uniq[SLUICE_MAX_EXPERTS];
  __shared__ int wcount[kWaves];
  __shared__ int wmiss[kWaves];
  __shared__ int s_stamp, s_status, s_waits, s_standing;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  // Loads that do not depend on each other go out together: the op's fresh
  // copy of hidden_states (its first kCopyU vectors per thread, stored after
  // the record is written), and the map / ownership of this thread's
  // experts.  (every copy load is issued, clamped into the buffer)
  u32x4_t cv[kCopyU];
  if (copy_vecs > 0) {
#pragma unroll
    for (int u = 0; u < kCopyU; ++u) {
      const int i = u * kLookupThreads + tid;
      cv[u] = copy_src[i < copy_vecs ? i : copy_vecs - 1];
    }
  }
  // (with a plan to build, the map is staged for it as it is read, and no
  // slot is pending until this gap installs its fills: the previous gap's
  // pending slots are cleared below, and only a gap's install marks any)
  bool unmapped[kGapMaxPerThread];
#pragma unroll
  for (int c = 0; c < kGapMaxPerThread; ++c) {
    const int e = c * kLookupThreads + tid;
    const int mv = e < E ? map[e] : -1;
    unmapped[c] = e < E && local_of[e] >= 0 && mv < 0;
    if (plan != nullptr && e < E) psc.slot_of[e] = mv;
  }
  if (plan != nullptr)
    for (int i = tid; i < S; i += kLookupThreads) psc.pend[i] = 0;
  int32_t s = 0, seen = 0;
  bool fresh = false;
  if (tid == 0) {
    s = sluice_stamp::next(dev_state[0]);
    SLUICE_TRACE_GAP(1, map, s);
    s_standing = dev_state[1];
    seen = dev_state[2];
  }
  for (int e = tid; e < E; e += kLookupThreads) present[e] = 0;
  {
    const int np = prev[0];
    for (int i = tid; i < np; i += kLookupThreads) pending[prev[1 + i]] = 0;
  }
  __syncthreads();
  if (tid == 0) prev[0] = 0;
  // Record s reuses the slot of record s - kRing, which the host must have
  // copied out (it normally has, long ago).  When the last ack read does not
  // show it, a fresh read goes out now and is checked after the compaction.
  if (tid == 0 && stamp_dist(s, seen) > kRing) {
    seen = ld_host(&mb->ack_stamp);
    fresh = true;
  }
  int id0 = -1;  // ids[tid], kept for the plan
  for (int i = tid; i < n; i += kLookupThreads) {
    const int g = ids[i];
    if (i == tid) id0 = g;
    if ((unsigned)g < (unsigned)E) present[g] = 1;
  }
  __syncthreads();
  // Sorted unique selected ids into LDS (ballot compaction); misses = owned
  // selected ids the device map does not hold.
  int base = 0, miss = 0;
#pragma unroll
  for (int c = 0; c < kGapMaxPerThread; ++c) {
    if (c * kLookupThreads >= E) break;
    const int e = c * kLookupThreads + tid;
    const bool f = e < E && present[e] != 0;
    const bool m = f && unmapped[c];
    const uint64_t fb = __ballot(f);
    const uint64_t mbits = __ballot(m);
    if (lane == 0) {
      wcount[wave] = __popcll(fb);
      wmiss[wave] = __popcll(mbits);
    }
    __syncthreads();
    int off = base;
    for (int w = 0; w < wave; ++w) off += wcount[w];
    if (f) s_uniq[off + mask_rank(fb)] = e;
    for (int w = 0; w < kWaves; ++w) {
      base += wcount[w];
      miss += wmiss[w];
    }
    __syncthreads();
  }
  if (tid == 0) {
    s_stamp = s;
    s_status = 0;
    if (stamp_dist(s, seen) > kRing)
      s_status = wait_slot(&mb->ack_stamp, s, abort_flag, bound, &seen);
    if (fresh) dev_state[2] = seen;
    s_waits = 0;
    if (s_status == 0) {
      if (!s_standing && ld_host(&mb->standing) != 0) {
        s_standing = 1;
        dev_state[1] = 1;
      }
      s_waits = (miss > 0 || !s_standing) ? 1 : 0;
      dev_state[0] = s;
    } else {
      st_host(&mb->dev_status, s_status);
    }
  }
  __syncthreads();
  if (s_status == 0) {
    // the record: entries and header in any order (each word is stamped)
    const int32_t s = s_stamp;
    GapRecord* r = &mb->rec[sluice_stamp::slot(s)];
    for (int i = tid; i < base; i += kLookupThreads)
      st_host64(&r->ent[i], rec_word(s, (uint32_t)s_uniq[i]));
    if (tid == 0) st_host64(&r->hdr, rec_word(s, rec_hdr_hi(base, miss, s_waits)));
    if (tid == 0) SLUICE_TRACE_GAP(2, map, s);
  }
#pragma unroll
  for (int u = 0; u < kCopyU; ++u) {
    const int i = u * kLookupThreads + tid;
    if (i < copy_vecs) copy_dst[i] = cv[u];
  }
  for (int i0 = kCopyU * kLookupThreads; i0 < copy_vecs; i0 += kCopyU * kLookupThreads) {
#pragma unroll
    for (int u = 0; u < kCopyU; ++u) {
      const int i = i0 + u * kLookupThreads + tid;
      cv[u] = copy_src[i < copy_vecs ? i : copy_vecs - 1];
    }
#pragma unroll
    for (int u = 0; u < kCopyU; ++u) {
      const int i = i0 + u * kLookupThreads + tid;
      if (i < copy_vecs) copy_dst[i] = cv[u];
    }
  }
  if (s_waits) {
    if (tid == 0) {
      const int st = wait_eq<true>(&mb->resp_stamp, s_stamp, abort_flag, bound);
      s_status = st != 0 ? st : ld_sys(&mb->resp_code);
      SLUICE_TRACE_GAP(3, map, s_stamp);
      if (st != 0) st_host(&mb->dev_status, st);
    }
    __syncthreads();
    if (s_status == 0) {
      // Install the standing map the host sent.  The answer was acquired
      // above, so its words are read relaxed, all in one bus round trip:
      // the slot table and the fill list (both at most S entries) with
      // their counts.
      constexpr int kPer = SLUICE_MAX_SLOTS / kLookupThreads;
      static_assert(SLUICE_MAX_SLOTS % kLookupThreads == 0, "answer words per thread");
      int sg[kPer], fl[kPer], fs[kPer];
      const int ns_word = ld_host(&mb->n_slots), nf_word = ld_host(&mb->n_fill);
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int i = u * kLookupThreads + tid;
        sg[u] = i < S ? ld_host(&mb->slot_global[i]) : -1;
        fl[u] = i < S ? ld_host(&mb->fill[i]) : -1;
        fs[u] = i < S && pull.n > 0 ? ld_host(&mb->fill_src[i]) : -1;
      }
      const int nS = min(ns_word, S);
      for (int e = tid; e < E; e += kLookupThreads) present[e] = -1;
      __syncthreads();
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int sl = u * kLookupThreads + tid;
        if (sl < nS && (unsigned)sg[u] < (unsigned)E) present[sg[u]] = sl;
      }
      __syncthreads();
      for (int e = tid; e < E; e += kLookupThreads) {
        map[e] = present[e];
        if (plan != nullptr) psc.slot_of[e] = present[e];
      }
      // The slots the host is still filling: the expert product waits for
      // them.  Their poll claims and seen marks (after the fill list) start
      // over.
      int32_t* claim = prev + 1 + S;
      const int nf = min(nf_word, S);
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int i = u * kLookupThreads + tid;
        if (i >= nf) continue;
        const int sl = fl[u];
        const int ok = (unsigned)sl < (unsigned)S;
        if (ok) {
          pending[sl] = s_stamp;
          claim[sl] = 0;
          claim[S + sl] = 0;
          if (plan != nullptr) psc.pend[sl] = 1;
        }
        prev[1 + i] = ok ? sl : 0;
        s_fslot[i] = ok ? sl : -1;
        s_fsrc[i] = fs[u];
      }
      if (tid == 0) prev[0] = nf;
      if (pull.n > 0 && nf > 0) {
        __syncthreads();
        pull_rows(pull, s_fslot, s_fsrc, nf, S, tid);
      }
    }
  }
  // The expert product's plan of these ids over the map (and pending marks)
  // this gap leaves behind, staged above, so the product needs no align
  // launch of its own.
  if (plan != nullptr) (void)sluice_plan::plan_build_staged(id0, ids, n, E, S, psc, plan);
#ifdef SLUICE_TRACE
  __syncthreads();
  if (tid == 0) SLUICE_TRACE_GAP(4, map, s_stamp);
#endif
}

// Resynchronisation after a failed gap: the pulled params' rows of every
// slot the host's cache holds (mb->fill / fill_src, nf entries), so that a
// gap the host answered but the device never installed (its wait ended
// first) leaves no slot without its small rows.
__global__ __launch_bounds__(kLookupThreads) void pull_slots_kernel(const GapMailbox* mb, int nf,
                                                                    int S, PullRows pull) {
  __shared__ int s_fslot[SLUICE_MAX_SLOTS], s_fsrc[SLUICE_MAX_SLOTS];
  for (int i = threadIdx.x; i < nf; i += kLookupThreads) {
    s_fslot[i] = ld_host(&mb->fill[i]);
    s_fsrc[i] = ld_host(&mb->fill_src[i]);
  }
  __syncthreads();
  pull_rows(pull, s_fslot, s_fsrc, nf, S, threadIdx.x);
}

// ---------------------------------------------------------------------------
// Per-device resources: the copy lanes (default priority, non-blocking
// streams) and the wall-clock rate; one process-wide abort flag in pinned
// memory.
//
// Expert rows go over kLanes copy streams, each per-expert param on the lane
// its layer assigned it (the lanes' row bytes balanced).  Every
// hipMemcpyAsync leaves the copy engine idle for ~9 us between copies on one
// stream (measured on MI355X, also through HSA's own async copy), and a bf16
// expert is two copies (w13 and w2 rows), an fp8 expert four: on one stream
// 326.9 us per 17.3 MB expert (52.9 GB/s), 1306 us for four; with w13 and w2
// on two streams the engines' gaps overlap the other lane's transfer, 318.4
// and 1237 us (55.95 GB/s, against 56.3 GB/s for 64 MiB copies).
// ---------------------------------------------------------------------------
constexpr int kLanes = 2;

// Staging (sluice_layer_set_staging): rows in HBM outside the slots, each a
// copy of one expert the layer selects often but does not hold, filled from
// the host store while the link idles, in chunks on kStageLanes SDMA engines
// of their own (at most kStageLanes chunks in flight per gap server, so a
// gap whose copies start meanwhile shares the link with at most that).  A
// miss whose expert is staged is copied into its slot from there by the
// runtime's device-to-device copy (a copy kernel: 17.3 MB in ~29 us on
// MI355X, against ~310 us over the link).
constexpr int kStageLanes = 2;
constexpr size_t kStageChunk = 2 << 20;
constexpr int kMaxStageRows = 8;
constexpr int kStageHalfLife = 4096;  // gaps between halvings of the selection counts

double now_s();

#ifdef SLUICE_TRACE
// Host ring of the gap service's steps (see trace.h).
struct TraceHostRec {
  uint32_t tag, layer;
  int32_t stamp, value;
  double t;
};
constexpr unsigned kTraceHostRing = 1u << 18;
TraceHostRec g_trace_host[kTraceHostRing];
std::atomic<unsigned> g_trace_host_n{0};
void trace_host(uint32_t tag, const void* map, int32_t stamp, int32_t value) {
  const unsigned i = g_trace_host_n.fetch_add(1, std::memory_order_relaxed) & (kTraceHostRing - 1);
  g_trace_host[i] = {tag, (uint32_t)(((uintptr_t)map >> 8) & 0xffffffffu), stamp, value, now_s()};
}
#define SLUICE_HTRACE(tag, L, stamp, value) trace_host((tag), (L)->map_dev, (stamp), (value))
#else
#define SLUICE_HTRACE(tag, L, stamp, value) ((void)0)
#endif

double gap_timeout_s();
long long bound_ticks(long long clock_khz) {
  return (long long)(gap_timeout_s() * 1000.0 * (double)clock_khz);
}

struct DeviceRes {
  hipStream_t copy[kLanes] = {};
  // The streamed gap's row copies go to the SDMA engines through the HSA
  // runtime (the one HIP itself runs on), not through HIP streams: a HIP
  // stream shares an in-order hardware queue with other streams once a
  // process has more streams than hardware queues (GPU_MAX_HW_QUEUES), and
  // a copy, or the marker of its completion event, queued behind the expert
  // product that waits for it would never run.  An SDMA copy's completion
  // signal needs no compute queue.  Lane l's rows go to engine[l] (0: the
  // runtime's choice).
  bool hsa = false;
  hsa_agent_t gpu_agent{}, cpu_agent{};
  uint32_t engine[kLanes] = {};
  // staging: the engines that fill staging rows from the host (0: none
  // free, no staging)
  uint32_t stage_engine[kStageLanes] = {};
  long long clock_khz = 0;
  // device word: the bound of every device wait, in wall-clock ticks; the
  // kernels read it when they start to wait (sluice_gap_set_timeout
  // rewrites it, so graphs captured earlier follow the new bound)
  long long* bound_dev = nullptr;
};
constexpr int kMaxDevices = 64;
DeviceRes g_dev[kMaxDevices];
std::mutex g_dev_mu;
int32_t* g_abort_host = nullptr;
int32_t* g_abort_dev = nullptr;

hsa_status_t first_cpu_agent(hsa_agent_t agent, void* data) {
  hsa_device_type_t t;
  if (hsa_agent_get_info(agent, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS)
    return HSA_STATUS_SUCCESS;
  if (t != HSA_DEVICE_TYPE_CPU) return HSA_STATUS_SUCCESS;
  *static_cast<hsa_agent_t*>(data) = agent;
  return HSA_STATUS_INFO_BREAK;
}

// The HSA agents of this device (the owner of its device memory) and of the
// host, and one SDMA engine per copy lane among those the runtime reports
// available for host-to-device copies.
int hsa_setup(DeviceRes& r) {
  if (hsa_init() != HSA_STATUS_SUCCESS) return SLUICE_E_COPY;  // counted: HIP holds one too
  hsa_amd_pointer_info_t info;
  memset(&info, 0, sizeof(info));
  info.size = sizeof(info);
  if (hsa_amd_pointer_info(r.bound_dev, &info, nullptr, nullptr, nullptr) != HSA_STATUS_SUCCESS ||
      info.type == HSA_EXT_POINTER_TYPE_UNKNOWN)
    return SLUICE_E_COPY;
  r.gpu_agent = info.agentOwner;
  hsa_agent_t cpu{};
  const hsa_status_t st = hsa_iterate_agents(first_cpu_agent, &cpu);
  if ((st != HSA_STATUS_SUCCESS && st != HSA_STATUS_INFO_BREAK) || cpu.handle == 0)
    return SLUICE_E_COPY;
  r.cpu_agent = cpu;
  uint32_t mask = 0;
  if (hsa_amd_memory_copy_engine_status(r.gpu_agent, r.cpu_agent, &mask) != HSA_STATUS_SUCCESS)
    mask = 0;
  int l = 0;
  uint32_t used = 0;
  for (uint32_t bit = 1; bit != 0 && l < kLanes; bit <<= 1)
    if (mask & bit) {
      r.engine[l++] = bit;
      used |= bit;
    }
  for (; l < kLanes; ++l) r.engine[l] = l > 0 ? r.engine[l - 1] : 0;
  // staging engines: reported host-to-device engines neither lane uses
  // (only engines the runtime reports for a direction are used for it)
  int ls = 0;
  for (uint32_t bit = 1; bit != 0 && ls < kStageLanes; bit <<= 1)
    if ((mask & bit) && !(used & bit)) {
      r.stage_engine[ls++] = bit;
      used |= bit;
    }
  if (ls < kStageLanes)
    for (uint32_t& e : r.stage_engine) e = 0;
  r.hsa = true;
  return SLUICE_OK;
}

int device_res(int dev, DeviceRes** out) {
  if (dev < 0 || dev >= kMaxDevices) return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> lk(g_dev_mu);
  DeviceRes& r = g_dev[dev];
  if (r.copy[kLanes - 1] == nullptr) {
    int khz = 0;
    SLUICE_HIP_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
    for (hipStream_t& s : r.copy)
      if (s == nullptr) SLUICE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    r.clock_khz = khz > 0 ? khz : 100000;
  }
  if (r.bound_dev == nullptr) {
    long long* b = nullptr;
    SLUICE_HIP_CHECK(hipMalloc((void**)&b, 256));
    const long long ticks = bound_ticks(r.clock_khz);
    SLUICE_HIP_CHECK(hipMemcpy(b, &ticks, sizeof(ticks), hipMemcpyHostToDevice));
    r.bound_dev = b;
  }
  if (!r.hsa) {
    const int rc = hsa_setup(r);
    if (rc != SLUICE_OK) return rc;
  }
  if (g_abort_host == nullptr) {
    void* p = nullptr;
    SLUICE_HIP_CHECK(hipHostMalloc(&p, 256, hipHostMallocCoherent | hipHostMallocMapped |
                                                hipHostMallocPortable));
    static_cast<int32_t*>(p)[0] = 0;
    void* dp = nullptr;
    SLUICE_HIP_CHECK(hipHostGetDevicePointer(&dp, p, 0));
    g_abort_host = static_cast<int32_t*>(p);
    g_abort_dev = static_cast<int32_t*>(dp);
  }
  *out = &r;
  return SLUICE_OK;
}

double now_s() {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

// The bound of every gap wait (device and host), in seconds: set by
// sluice_gap_set_timeout, else SLUICE_GAP_TIMEOUT_S, else 20.
std::atomic<double> g_timeout_set{0.0};

// Failure injection (sluice_gap_inject_copy_failure): row copies a served
// gap may still issue before one fails; < 0 = disarmed.
std::atomic<int> g_fail_after{-1};

// Whether a missing gap is answered before its rows land (the expert
// product then waits per filled slot) or, as the reference orders it, only
// after every row landed (sluice_gap_set_pipelined).
std::atomic<int> g_pipelined{1};

double gap_timeout_s() {
  const double set = g_timeout_set.load(std::memory_order_relaxed);
  if (set > 0) return set;
  static double v = [] {
    const char* s = getenv("SLUICE_GAP_TIMEOUT_S");
    double t = s ? atof(s) : 20.0;
    return t > 0 ? t : 20.0;
  }();
  return v;
}

int32_t next_stamp(int32_t s) { return sluice_stamp::next(s); }

}  // namespace

struct ParamRows {
  char* slot_base;
  const char* host_base;
  size_t row_bytes;
  int lane;                 // copy lane of this param's rows
  char* rows_dev = nullptr;  // HBM copy of all host rows when the gap kernel pulls them
  hsa_agent_t host_agent{};  // the agent owning the host rows (0: the first CPU agent)
  // Coded host store (sluice_layer_set_codec; nullptr: the rows stream as
  // they are): expert `local`'s coded row at coded_base + local *
  // coded_stride, coded_len[local] bytes.
  char* coded_base = nullptr;
  size_t coded_stride = 0;
  std::vector<uint32_t> coded_len;
  hsa_agent_t coded_agent{};
};

// Decode resources of a gap server whose layers hold coded host stores: the
// device's decode queue, the word the jobs' last workgroups release their
// sequence numbers into (jobs on the queue complete in order), and the ring
// in HBM that coded rows land in before they are decoded into slots.
struct CodecRes {
  int device = 0;
  CodecQueue* queue = nullptr;
  uint32_t* wg_count = nullptr;             // device word, 0 between jobs
  unsigned long long* done_host = nullptr;  // host-mapped: the last job completed
  unsigned long long* done_dev = nullptr;
  char* ring = nullptr;
  size_t ring_bytes = 0, head = 0;
  // ring regions in allocation order; a region is free again once the job
  // that decodes it completed (or its copies failed)
  struct Use {
    int64_t id;
    size_t off, len;
    unsigned long long seq;
    int state;
  };
  std::deque<Use> uses;
  int64_t next_use = 0;
  unsigned long long seq = 0;  // the last job launched (server thread)
  std::atomic<unsigned long long> launched{0};  // the same, for other threads
};

struct sluice_gap_server;

struct sluice_layer {
  slru::Cache c;
  std::mutex mu;  // guards c, params, bytes against the server thread
  int32_t* map_dev = nullptr;
  std::vector<ParamRows> params;
  int device = -1;
  GapMailbox* mb = nullptr;      // host pointer
  GapMailbox* mb_dev = nullptr;  // device view of the same memory
  int32_t* dev_block = nullptr;  // [E] local_of, then last stamp, standing seen, last ack read
  int32_t host_stamp = 0;        // last record copied out
  std::atomic<int32_t> done_stamp{0};  // last record fully served
  int64_t bytes = 0;
  sluice_gap_server* server = nullptr;
  std::vector<int> streams;
  std::vector<int32_t> uniq;
  // classic (wave) step: the plan, how far it has run, and its events
  slru::Plan plan;
  int plan_next = 0;          // next wave to run
  bool plan_in_wave = false;  // between classic_wave and classic_wave_done
  int plan_copied = 0;        // waves whose row copies have been issued
  std::vector<hipEvent_t> wave_ev, copy_ev;
  hipEvent_t pre_ev = nullptr;
  int32_t* ids_host = nullptr;  // pinned staging of the step's ids
  size_t ids_cap = 0;
  int64_t classic_steps = 0, classic_waves = 0;
  // one HSA completion signal per row copy of a gap (armed at 1; the copy
  // completes it); the first armed_copies of them may still be in flight
  // after a failed stream-in
  std::vector<hsa_signal_t> fill_sig;
  int armed_copies = 0;
  unsigned lane_mask = 0;  // lanes that carry some param's rows
  std::vector<int> order, sig_end;  // a gap's streams in copy order; each one's last signal + 1
  // Staging rows (sluice_layer_set_staging).  Row r holds (or is being
  // filled with) expert `local`; its bytes are the non-pulled params' rows
  // one after the other (stage_dev[p] + r * row_bytes for param p).
  struct StageRow {
    int local = -1;
    int state = 0;      // kStageEmpty / kStageCopying / kStageReady
    size_t issued = 0;  // bytes whose copies were issued
    int in_flight = 0;  // of its chunks
    unsigned long long busy_seq = 0;  // decode job that reads the row (coded stores)
  };
  std::vector<StageRow> stage;
  std::vector<char*> stage_dev;  // per param (nullptr: pulled, or no staging)
  size_t stage_bytes = 0;        // one staged expert
  hsa_signal_t stage_sig[kStageLanes] = {};
  int stage_sig_row[kStageLanes] = {-1, -1};  // row of the chunk a signal tracks
  size_t stage_sig_bytes[kStageLanes] = {};
  std::vector<uint32_t> sel_count;  // [local_n] how often each expert was selected
  int stage_gaps = 0;
  bool stage_dirty = false;   // a gap was served since the rows were chosen
  bool stage_broken = false;  // a staging copy failed: none until resync
  int64_t stage_filled = 0, stage_h2d = 0, stage_hits = 0, stage_hit_bytes = 0;
  std::vector<size_t> stage_row_bytes;  // per param: bytes of one row in its staging buffer
  // coded host stores (sluice_layer_set_codec): the params coded, and the
  // decode resources of the gap server serving the layer (nullptr: none)
  uint32_t codec_mask = 0;
  struct CodecRes* codec = nullptr;
  std::vector<size_t> ring_off;  // a gap's streams: offset of each one's coded rows in the ring
  std::vector<int64_t> use_id;   // and the ring use holding them (0: none)
  std::vector<int> srow_of;      // and the staging row each one is served from (-1: none)
  int64_t link_bytes = 0;        // bytes of served gaps' row copies over the link
  int64_t decodes = 0, decodes_staged = 0;
};

namespace {

int layer_device_init(sluice_layer* L) {
  if (L->mb != nullptr) return SLUICE_OK;
  SLUICE_HIP_CHECK(hipGetDevice(&L->device));
  DeviceRes* R = nullptr;
  int rc = device_res(L->device, &R);
  if (rc) return rc;
  void* p = nullptr;
  SLUICE_HIP_CHECK(hipHostMalloc(&p, sizeof(GapMailbox), hipHostMallocCoherent |
                                                             hipHostMallocMapped));
  memset(p, 0, sizeof(GapMailbox));
  L->mb = static_cast<GapMailbox*>(p);
  void* dp = nullptr;
  SLUICE_HIP_CHECK(hipHostGetDevicePointer(&dp, p, 0));
  L->mb_dev = static_cast<GapMailbox*>(dp);
  const int E = L->c.E, S = L->c.S;
  // [E] local_of | last stamp, standing map seen, last ack read | [S] pending
  // | prev count, [S] prev fills | [S] claim | [S] seen
  const size_t n = (size_t)E + 3 + S + 1 + S + S + S;
  SLUICE_HIP_CHECK(hipMalloc((void**)&L->dev_block, sizeof(int32_t) * n));
  std::vector<int32_t> blk(L->c.local_of.begin(), L->c.local_of.end());
  blk.resize(n, 0);
  SLUICE_HIP_CHECK(hipMemcpy(L->dev_block, blk.data(), sizeof(int32_t) * n,
                             hipMemcpyHostToDevice));
  if (L->map_dev != nullptr) {
    SlotWait w;
    w.pending = L->dev_block + E + 3;
    w.ready = L->mb_dev->slot_ready;
    w.claim = L->dev_block + E + 3 + S + 1 + S;
    w.seen = w.claim + S;
    w.abort_flag = g_abort_dev;
    w.status = &L->mb_dev->dev_status;
    w.bound = R->bound_dev;
    slotwait_register(L->map_dev, w);
  }
  return SLUICE_OK;
}

constexpr int kNothing = 1;  // serve_one: no record posted yet (non-blocking)

// Answer the device's gap `stamp`: on success the standing slot table and
// the slots being filled (the product waits for each one's ready mark).
void respond(sluice_layer* L, int32_t stamp, int code, int n_fill) {
  GapMailbox* mb = L->mb;
  if (code == SLUICE_OK) {
    L->c.slot_globals(mb->slot_global);
    mb->n_slots = L->c.S;
    mb->standing = 1;
    for (int i = 0; i < n_fill; ++i) {
      mb->fill[i] = L->streams[2 * i + 1];
      mb->fill_src[i] = L->streams[2 * i];
    }
    mb->n_fill = n_fill;
  } else {
    mb->n_fill = 0;
  }
  mb->resp_code = code;
  __atomic_store_n(&mb->resp_stamp, stamp, __ATOMIC_RELEASE);
}

// Every row copy of a gap has a completion signal of its own, armed at 1,
// and an expert's slot is marked ready once all of its copies completed:
// the product of each expert starts as soon as its own rows landed (a
// completion costs the copy engine nothing, unlike a HIP event recorded
// between copies, which idled it ~6 us).  The runtime completes a signal by
// decrementing it, a tool that wraps the copy may store zero instead: one
// signal per copy is right under either.
//
// Spin until signal `sig` reached zero (bounded).  0, or SLUICE_E_COPY (a
// copy reported an error: the runtime sets the signal negative) or
// SLUICE_E_TIMEOUT.
int wait_signal(hsa_signal_t sig) {
  const double t0 = now_s();
  unsigned spins = 0;
  for (;;) {
    const hsa_signal_value_t v = hsa_signal_load_scacquire(sig);
    if (v == 0) return SLUICE_OK;
    if (v < 0) return SLUICE_E_COPY;
    _mm_pause();
    if ((++spins & 1023u) == 0 && now_s() - t0 > gap_timeout_s()) return SLUICE_E_TIMEOUT;
  }
}

// Wait (bounded) until no copy of the layer's last stream-in is in flight
// (a copy that failed is not in flight either).  0 or SLUICE_E_TIMEOUT.
int drain_copies(sluice_layer* L) {
  for (int c = 0; c < L->armed_copies && c < (int)L->fill_sig.size(); ++c)
    if (wait_signal(L->fill_sig[c]) == SLUICE_E_TIMEOUT) return SLUICE_E_TIMEOUT;
  return SLUICE_OK;
}

// ---------------------------------------------------------------------------
// Decode of coded experts (sluice_layer_set_codec), under a gap server.
// ---------------------------------------------------------------------------
constexpr int kUsePending = 0, kUseLaunched = 1, kUseDead = 2;
constexpr size_t kRingAlign = 256;
size_t ring_round(size_t v) { return (v + kRingAlign - 1) & ~(kRingAlign - 1); }

bool coded(const ParamRows& p) { return p.coded_base != nullptr; }

bool has_coded(const sluice_layer* L) {
  for (const ParamRows& p : L->params)
    if (coded(p)) return true;
  return false;
}

unsigned long long codec_done(const CodecRes* C) {
  return __atomic_load_n(C->done_host, __ATOMIC_ACQUIRE);
}

// Wait (bounded) until job `seq` has completed.
int codec_wait(const CodecRes* C, unsigned long long seq) {
  const double t0 = now_s();
  unsigned spins = 0;
  while (codec_done(C) < seq) {
    _mm_pause();
    if ((++spins & 1023u) == 0 && now_s() - t0 > gap_timeout_s()) return SLUICE_E_TIMEOUT;
  }
  return SLUICE_OK;
}

void ring_reap(CodecRes* C) {
  const unsigned long long done = codec_done(C);
  while (!C->uses.empty()) {
    const CodecRes::Use& u = C->uses.front();
    if (u.state == kUseDead || (u.state == kUseLaunched && u.seq <= done)) C->uses.pop_front();
    else break;
  }
  if (C->uses.empty()) C->head = 0;
}

// A ring region of len bytes after the live ones (their order is the
// allocation order): its use id, or 0 while the live regions leave no room.
int64_t ring_take(CodecRes* C, size_t len, size_t* off) {
  ring_reap(C);
  size_t at = 0;
  if (C->uses.empty()) {
    if (len > C->ring_bytes) return 0;
  } else {
    const size_t tail = C->uses.front().off;
    if (C->head > tail) {  // live: [tail, head)
      if (C->head + len <= C->ring_bytes) at = C->head;
      else if (len <= tail) at = 0;
      else return 0;
    } else {  // live: [tail, end) and [0, head)
      if (C->head + len <= tail) at = C->head;
      else return 0;
    }
  }
  C->uses.push_back({++C->next_use, at, len, 0, kUsePending});
  C->head = at + len;
  *off = at;
  return C->next_use;
}

void ring_set(CodecRes* C, int64_t id, int state, unsigned long long seq) {
  for (auto it = C->uses.rbegin(); it != C->uses.rend(); ++it)
    if (it->id == id) {
      it->state = state;
      it->seq = seq;
      return;
    }
}

// Launch the decode of expert `local`'s coded rows into `slot`: from the
// ring at `ring_at`, or from staging row `srow` (>= 0).  The job's last
// workgroup marks the slot ready for gap `stamp`.  *seq: the job's number.
int launch_decode(sluice_layer* L, CodecRes* C, int local, int slot, int srow, size_t ring_at,
                  int32_t stamp, unsigned long long* seq) {
  CodecJob job{};
  size_t at = ring_at;
  for (size_t pi = 0; pi < L->params.size(); ++pi) {
    const ParamRows& p = L->params[pi];
    if (!coded(p)) continue;
    if (job.n_part == kCodecMaxParts) return SLUICE_E_STATE;
    const size_t n = p.row_bytes / 2;
    const char* src = srow >= 0 ? L->stage_dev[pi] + (size_t)srow * L->stage_row_bytes[pi]
                                : C->ring + at;
    job.part[job.n_part++] = {(const uint8_t*)src,
                              (uint16_t*)(p.slot_base + (size_t)slot * p.row_bytes),
                              (uint32_t)(n / kCodecChunk), codec_escapes(n, p.coded_len[local])};
    at += ring_round(p.coded_len[local]);
  }
  job.wg_count = C->wg_count;
  job.ready = &L->mb_dev->slot_ready[slot];
  job.stamp = stamp;
  job.done = C->done_dev;
  job.seq = C->seq + 1;
  const int rc = codec_dispatch(C->queue, job);
  if (rc != SLUICE_OK) return rc == SLUICE_E_INVAL ? SLUICE_E_STATE : rc;
  *seq = ++C->seq;
  C->launched.store(C->seq, std::memory_order_release);
  ++L->decodes;
  if (srow >= 0) ++L->decodes_staged;
  return SLUICE_OK;
}

// The bytes of expert `local`'s rows that cross the link: its coded rows
// where the store is coded (under a server's decode), else the rows.
size_t link_bytes_of(const sluice_layer* L, int local, bool use_codec) {
  size_t b = 0;
  for (const ParamRows& p : L->params)
    if (p.rows_dev == nullptr)
      b += use_codec && coded(p) ? (size_t)p.coded_len[local] : p.row_bytes;
  return b;
}

// ---------------------------------------------------------------------------
// Staging rows (L->mu held by the callers that other threads may race; the
// gap server's own thread is the only one that issues staging copies).
// ---------------------------------------------------------------------------
constexpr int kStageEmpty = 0, kStageCopying = 1, kStageReady = 2;

// The row holding expert `local` whole, or -1.
int stage_ready_row(const sluice_layer* L, int local) {
  for (size_t r = 0; r < L->stage.size(); ++r)
    if (L->stage[r].state == kStageReady && L->stage[r].local == local) return (int)r;
  return -1;
}

// Bytes of expert `local` a staging row holds: its coded rows where the
// store is coded, else its rows (the params the gap kernel pulls aside).
size_t stage_total(const sluice_layer* L, int local) {
  size_t b = 0;
  for (size_t pi = 0; pi < L->params.size(); ++pi) {
    if (L->stage_dev[pi] == nullptr) continue;
    const ParamRows& p = L->params[pi];
    b += coded(p) ? (size_t)p.coded_len[local] : p.row_bytes;
  }
  return b;
}

// A row still has bytes to copy.
bool stage_has_copy(const sluice_layer* L) {
  for (const sluice_layer::StageRow& row : L->stage)
    if (row.state == kStageCopying && row.issued < stage_total(L, row.local)) return true;
  return false;
}

// A decode job still reads the row.
bool stage_busy(const sluice_layer* L, const sluice_layer::StageRow& row) {
  return L->codec != nullptr && row.busy_seq > codec_done(L->codec);
}

// Count the gap's selections: the staging candidates are the experts the
// layer selects most often among those it does not hold (counts halved
// every kStageHalfLife gaps, so they follow a drifting routing).
void stage_count(sluice_layer* L) {
  if (L->stage.empty()) return;
  for (int32_t g : L->uniq) {
    const int loc = (g >= 0 && g < L->c.E) ? L->c.local_of[g] : -1;
    if (loc >= 0 && loc < L->c.local_n) ++L->sel_count[loc];
  }
  if (++L->stage_gaps >= kStageHalfLife) {
    L->stage_gaps = 0;
    for (uint32_t& v : L->sel_count) v >>= 1;
  }
  L->stage_dirty = true;
}

// Completed staging chunks; a row whose chunks all landed becomes ready.
// A failed chunk empties its row and stops the layer's staging until
// sluice_layer_gap_resync.
void stage_poll(sluice_layer* L) {
  for (int l = 0; l < kStageLanes; ++l) {
    const int r = L->stage_sig_row[l];
    if (r < 0) continue;
    const hsa_signal_value_t v = hsa_signal_load_scacquire(L->stage_sig[l]);
    if (v > 0) continue;
    L->stage_sig_row[l] = -1;
    sluice_layer::StageRow& row = L->stage[r];
    --row.in_flight;
    if (v < 0) {
      L->stage_broken = true;
      row.state = kStageEmpty;
      row.local = -1;
      continue;
    }
    L->stage_h2d += (int64_t)L->stage_sig_bytes[l];
    SLUICE_HTRACE(29, L, 0, (int32_t)((L->stage_sig_bytes[l] >> 10) << 1 | (size_t)l));
    if (row.state == kStageEmpty && row.in_flight == 0) L->stage_dirty = true;  // free again
  }
  for (sluice_layer::StageRow& row : L->stage)
    if (row.state == kStageCopying && row.in_flight == 0 &&
        row.issued == stage_total(L, row.local)) {
      row.state = kStageReady;
      ++L->stage_filled;
    }
}

// Give the rows to the most selected experts the layer does not hold
// (count, then lower local id first).  A row keeps its expert while that
// one is still wanted; a row being filled for an expert no longer wanted
// stops, and is given out again once its chunks in flight landed.
void stage_choose(sluice_layer* L) {
  if (!L->stage_dirty) return;
  L->stage_dirty = false;
  const int n = (int)L->stage.size();
  int want[kMaxStageRows];
  int nw = 0;
  for (int loc = 0; loc < L->c.local_n; ++loc) {
    const uint32_t c = L->sel_count[loc];
    if (c == 0 || L->c.slot_of[loc] >= 0) continue;
    int pos = nw;
    while (pos > 0 && L->sel_count[want[pos - 1]] < c) --pos;
    if (pos >= n) continue;
    if (nw < n) ++nw;
    for (int j = nw - 1; j > pos; --j) want[j] = want[j - 1];
    want[pos] = loc;
  }
  bool covered[kMaxStageRows] = {}, keep[kMaxStageRows] = {};
  for (int r = 0; r < n; ++r) {
    const sluice_layer::StageRow& row = L->stage[r];
    for (int w = 0; w < nw && row.state != kStageEmpty; ++w)
      if (!covered[w] && row.local == want[w]) {
        covered[w] = keep[r] = true;
        break;
      }
  }
  int w = 0;
  for (int r = 0; r < n; ++r) {
    if (keep[r]) continue;
    while (w < nw && covered[w]) ++w;
    if (w >= nw) break;
    sluice_layer::StageRow& row = L->stage[r];
    if (row.state == kStageCopying) {
      row.state = kStageEmpty;
      row.local = -1;
    }
    if (row.in_flight > 0 || stage_busy(L, row)) continue;  // still written, or read
    row.local = want[w];
    row.state = kStageCopying;
    row.issued = 0;
    covered[w] = true;
  }
}

// The layer's row being filled whose expert is selected most often, or -1.
int stage_next_row(const sluice_layer* L) {
  int pick = -1;
  for (size_t r = 0; r < L->stage.size(); ++r) {
    const sluice_layer::StageRow& row = L->stage[r];
    if (row.state != kStageCopying || row.issued >= stage_total(L, row.local)) continue;
    if (pick < 0 || L->sel_count[row.local] > L->sel_count[L->stage[pick].local]) pick = (int)r;
  }
  return pick;
}

// Issue the next chunk of row r (being filled), on staging lane l (free).
// false if the copy could not be issued.
bool stage_issue(sluice_layer* L, const DeviceRes* R, int l, int r) {
  sluice_layer::StageRow& row = L->stage[r];
  size_t base = 0;  // the row's bytes: the staged params' rows one after the other
  for (size_t pi = 0; pi < L->params.size(); ++pi) {
    if (L->stage_dev[pi] == nullptr) continue;
    const ParamRows& p = L->params[pi];
    const bool cd = coded(p);
    const size_t bytes = cd ? (size_t)p.coded_len[row.local] : p.row_bytes;
    if (row.issued >= base + bytes) {
      base += bytes;
      continue;
    }
    const size_t in = row.issued - base;
    const size_t len = std::min(kStageChunk, bytes - in);
    char* dst = L->stage_dev[pi] + (size_t)r * L->stage_row_bytes[pi] + in;
    const char* src = (cd ? p.coded_base + (size_t)row.local * p.coded_stride
                          : p.host_base + (size_t)row.local * p.row_bytes) + in;
    const hsa_agent_t agent = cd ? p.coded_agent : p.host_agent;
    const hsa_agent_t from = agent.handle != 0 ? agent : R->cpu_agent;
    hsa_signal_store_relaxed(L->stage_sig[l], 1);
    if (hsa_amd_memory_async_copy_on_engine(dst, R->gpu_agent, src, from, len, 0, nullptr,
                                            L->stage_sig[l],
                                            (hsa_amd_sdma_engine_id_t)R->stage_engine[l],
                                            true) != HSA_STATUS_SUCCESS) {
      hsa_signal_store_relaxed(L->stage_sig[l], 0);
      L->stage_broken = true;
      row.state = kStageEmpty;
      row.local = -1;
      return false;
    }
    row.issued += len;
    ++row.in_flight;
    L->stage_sig_row[l] = r;
    L->stage_sig_bytes[l] = len;
    SLUICE_HTRACE(28, L, 0, (int32_t)((len >> 10) << 1 | (size_t)l));
    return true;
  }
  return false;
}

// Wait (bounded) until no staging chunk of the layer is in flight.
int stage_drain(sluice_layer* L) {
  for (int l = 0; l < kStageLanes; ++l)
    if (L->stage_sig_row[l] >= 0 && wait_signal(L->stage_sig[l]) == SLUICE_E_TIMEOUT)
      return SLUICE_E_TIMEOUT;
  stage_poll(L);
  return SLUICE_OK;
}

// Free the layer's staging rows (no chunk in flight: L->mu held, drained).
int stage_free(sluice_layer* L) {
  int rc = SLUICE_OK;
  for (char*& d : L->stage_dev)
    if (d != nullptr) {
      const hipError_t e = hipFree(d);
      if (e != hipSuccess) rc = (int)e;
      d = nullptr;
    }
  L->stage_dev.clear();
  L->stage_row_bytes.clear();
  L->stage.clear();
  L->stage_bytes = 0;
  return rc;
}

// Coded stores by the host rows they code: layers that stream from the
// same host rows (one host pool shared by several layers) share one coded
// store, freed with its last user.
struct CodedStore {
  const char* host_base;
  size_t row_bytes;
  int local_n;
  char* base;
  size_t stride;
  std::vector<uint32_t> len;
  hsa_agent_t agent;
  int users;
};
std::mutex g_coded_mu;
std::vector<CodedStore*> g_coded;

// Free the layer's coded host stores (L->mu held; no server serves it).
int codec_free(sluice_layer* L) {
  int rc = SLUICE_OK;
  std::lock_guard<std::mutex> lk(g_coded_mu);
  for (ParamRows& p : L->params) {
    if (p.coded_base != nullptr) {
      for (size_t i = 0; i < g_coded.size(); ++i) {
        CodedStore* cs = g_coded[i];
        if (cs->base != p.coded_base || --cs->users > 0) continue;
        const hipError_t e = hipHostFree(cs->base);
        if (e != hipSuccess) rc = (int)e;
        delete cs;
        g_coded.erase(g_coded.begin() + (long)i);
        break;
      }
    }
    p.coded_base = nullptr;
    p.coded_stride = 0;
    p.coded_len.clear();
    p.coded_agent = {};
  }
  L->codec_mask = 0;
  return rc;
}

// A record after the last one served has been posted (records are posted
// in stamp order, so looking at the next stamp's slot is enough).
bool record_pending(sluice_layer* L) {
  const int32_t next = next_stamp(L->done_stamp.load(std::memory_order_acquire));
  return rec_stamp(__atomic_load_n(&L->mb->rec[sluice_stamp::slot(next)].hdr,
                                   __ATOMIC_ACQUIRE)) == next;
}

// Serve one posted record of layer L.  block: wait (bounded) for it;
// `compute` (may be null) is polled for errors while waiting.
int serve_one(sluice_layer* L, bool fast_hit, bool block, hipStream_t compute) {
  GapMailbox* mb = L->mb;
  const int dev_status = __atomic_load_n(&mb->dev_status, __ATOMIC_ACQUIRE);
  if (dev_status != 0) return dev_status;  // a device wait failed earlier
  const int32_t want = next_stamp(L->host_stamp);
  GapRecord* rec = &mb->rec[sluice_stamp::slot(want)];
  uint64_t hdr = __atomic_load_n(&rec->hdr, __ATOMIC_ACQUIRE);
  double t0 = 0.0;
  if (rec_stamp(hdr) != want) {
    if (!block) return kNothing;
    t0 = now_s();
    unsigned spins = 0;
    while (rec_stamp(hdr = __atomic_load_n(&rec->hdr, __ATOMIC_ACQUIRE)) != want) {
      _mm_pause();
      if ((++spins & 4095u) == 0) {
        if (compute != nullptr) {
          hipError_t q = hipStreamQuery(compute);
          if (q != hipSuccess && q != hipErrorNotReady) return (int)q;
        }
        if (now_s() - t0 > gap_timeout_s()) return SLUICE_E_TIMEOUT;
      }
    }
  }
  // Copy the record out (each entry once its stamp shows: the device writes
  // the words in no particular order), then let the device reuse the mailbox.
  const uint32_t hi = (uint32_t)(hdr >> 32);
  const uint32_t cmask = (1u << kRecCountBits) - 1;
  const int n_uniq = (int)(hi & cmask);
  const int n_miss = (int)((hi >> kRecCountBits) & cmask);
  const bool waits = ((hi >> (2 * kRecCountBits)) & 1u) != 0;
  if (n_uniq > L->c.E) return SLUICE_E_STATE;
  L->uniq.resize(n_uniq);
  for (int i = 0; i < n_uniq; ++i) {
    uint64_t w = __atomic_load_n(&rec->ent[i], __ATOMIC_ACQUIRE);
    if (rec_stamp(w) != want) {
      if (t0 == 0.0) t0 = now_s();
      while (rec_stamp(w = __atomic_load_n(&rec->ent[i], __ATOMIC_ACQUIRE)) != want) {
        _mm_pause();
        if (now_s() - t0 > gap_timeout_s()) return SLUICE_E_TIMEOUT;
      }
    }
    L->uniq[i] = (int32_t)(w >> 32);
  }
  L->host_stamp = want;
  __atomic_store_n(&mb->ack_stamp, want, __ATOMIC_RELEASE);
  SLUICE_HTRACE(21, L, want, n_miss);

  std::lock_guard<std::mutex> lk(L->mu);
  L->streams.clear();
  bool map_write = false;
  // The device counts misses against the map it holds; only a standing map
  // holds every resident expert (a classic wave's map holds that wave's).
  const bool was_standing = L->c.map_is_standing;
  const int grc = L->c.gap(L->uniq.data(), n_uniq, fast_hit, L->streams, map_write);
  const int n_streams = (int)L->streams.size() / 2;
  stage_count(L);
  SLUICE_HTRACE(22, L, want, n_streams);
  int rc = SLUICE_OK;
  if (!waits) {
    // The device ran on with its map: the host must agree nothing changed.
    if (grc != 0 || n_streams != 0 || map_write || n_miss != 0) rc = SLUICE_E_STATE;
  } else if (grc == 0 && was_standing && n_streams != n_miss) {
    rc = SLUICE_E_STATE;
  } else if (n_streams > 0) {
    DeviceRes* R = nullptr;
    rc = device_res(L->device, &R);
    // A waiting gap whose bookkeeping succeeded is answered before its rows
    // land: the device installs the map at once and its expert product
    // computes the hit experts while the misses stream, waiting per filled
    // slot for the ready mark set below.  (On overflow the rows acquired
    // before it still stream, as in the reference, whose copies were issued
    // before the raise; the device map is left as it was, answered after.)
    const bool early = waits && grc == 0 && rc == SLUICE_OK &&
                       g_pipelined.load(std::memory_order_relaxed) != 0;
    // Coded stores are decoded only under a gap server that answers before
    // the rows land (the server's decode resources): the coded rows cross
    // the link into the server's ring in HBM and a decode job writes each
    // expert's rows into its slot, its last workgroup marking the slot
    // ready; otherwise every row streams as it is.
    CodecRes* C = early && rc == SLUICE_OK ? L->codec : nullptr;
    // rows copied per expert (the gap kernel copies the pulled ones itself)
    int n_copy = 0;
    for (const ParamRows& p : L->params) n_copy += !(early && p.rows_dev != nullptr);
    // Copy order: the misses whose expert is staged first, then the others
    // over the link.  A staged row serves only a gap answered before its
    // rows land, and its copy (HBM to HBM) runs as a kernel of the runtime:
    // the host waits for those copies before it answers, so no kernel ever
    // waits for a copy that itself needs CUs (the device runs only the
    // waiting gap kernel meanwhile).  Coded staged rows are decoded from the
    // row itself.
    L->order.clear();
    const bool from_stage = early && rc == SLUICE_OK && !L->stage.empty() &&
                            (C != nullptr || !has_coded(L));
    if (from_stage)
      for (int i = 0; i < n_streams; ++i)
        if (stage_ready_row(L, L->streams[2 * i]) >= 0) L->order.push_back(i);
    const int n_staged = (int)L->order.size();
    for (int i = 0; i < n_streams; ++i)
      if (n_staged == 0 || stage_ready_row(L, L->streams[2 * i]) < 0) L->order.push_back(i);
    const size_t n_sig = (size_t)n_streams * (size_t)n_copy;
    while (rc == SLUICE_OK && L->fill_sig.size() < n_sig) {
      hsa_signal_t sig{};
      if (hsa_signal_create(0, 0, nullptr, &sig) != HSA_STATUS_SUCCESS) rc = SLUICE_E_COPY;
      else L->fill_sig.push_back(sig);
    }
    L->sig_end.assign((size_t)n_streams, 0);
    L->srow_of.assign((size_t)n_streams, -1);
    L->ring_off.assign((size_t)n_streams, 0);
    L->use_id.assign((size_t)n_streams, 0);
    int whole = 0;  // experts (in copy order) whose copies were all issued
    int armed = 0;  // copies issued, each with its own signal
    // One copy with its own completion signal (engine 0: the runtime's
    // choice); false (rc set) if it failed to issue.
    auto copy = [&](void* dst, const void* src, hsa_agent_t from, size_t bytes, uint32_t eng) {
      int left = g_fail_after.load(std::memory_order_relaxed);
      while (left >= 0 && !g_fail_after.compare_exchange_weak(left, left - 1)) {
      }
      const hsa_signal_t sig = L->fill_sig[armed];
      hsa_signal_store_relaxed(sig, 1);
      const hsa_status_t st =
          left == 0 ? HSA_STATUS_ERROR
          : eng != 0
              ? hsa_amd_memory_async_copy_on_engine(dst, R->gpu_agent, src, from, bytes, 0, nullptr,
                                                    sig, (hsa_amd_sdma_engine_id_t)eng, true)
              : hsa_amd_memory_async_copy(dst, R->gpu_agent, src, from, bytes, 0, nullptr, sig);
      if (st != HSA_STATUS_SUCCESS) {
        hsa_signal_store_relaxed(sig, 0);
        rc = SLUICE_E_COPY;
        return false;
      }
      L->armed_copies = ++armed;
      return true;
    };
    // Wait for the j-th expert's copies (from signal *c on), then mark its
    // slot ready for this gap, or launch the decode that marks it.
    auto land = [&](int j, int* c) {
      int w = SLUICE_OK;
      for (; *c < L->sig_end[j] && w == SLUICE_OK; ++*c) w = wait_signal(L->fill_sig[*c]);
      if (w != SLUICE_OK) {
        if (rc == SLUICE_OK) rc = w;
        return false;
      }
      SLUICE_HTRACE(26, L, want, j);
      if (early) {
        const int i = L->order[j];
        const int slot = L->streams[2 * i + 1];
        if (C != nullptr) {
          unsigned long long seq = 0;
          const int srow = L->srow_of[j];
          w = launch_decode(L, C, L->streams[2 * i], slot, srow, L->ring_off[j], want, &seq);
          if (w != SLUICE_OK) {
            if (rc == SLUICE_OK) rc = w;
            return false;
          }
          if (L->use_id[j] != 0) ring_set(C, L->use_id[j], kUseLaunched, seq);
          if (srow >= 0) L->stage[srow].busy_seq = seq;
        } else {
          __atomic_store_n(&mb->slot_ready[slot], want, __ATOMIC_RELEASE);
        }
        SLUICE_HTRACE(27, L, want, j);
      }
      return true;
    };
    int landed = 0, c = 0;  // experts in copy order whose copies completed, their slots marked
    bool landing = true;    // no wait failed
    auto land_upto = [&](int n) {
      while (landing && landed < n) {
        if (land(landed, &c)) ++landed;
        else landing = false;
      }
    };
    // Room in the ring for the j-th expert's coded rows: while the live
    // regions leave none, land the oldest expert still landing (which
    // launches its decode), else wait for the oldest decode.
    auto ring_room = [&](int j, size_t need) {
      for (;;) {
        const int64_t id = ring_take(C, need, &L->ring_off[j]);
        if (id != 0) {
          L->use_id[j] = id;
          return true;
        }
        if (landed < whole) {
          land_upto(landed + 1);
          if (!landing) return false;
          continue;
        }
        // (no live region: the expert is larger than the ring, which the
        // server sized for the largest coded expert of its layers)
        const int w = C->uses.empty() ? SLUICE_E_STATE
                      : C->uses.front().state == kUseLaunched
                          ? codec_wait(C, C->uses.front().seq)
                          : SLUICE_E_STATE;
        if (w != SLUICE_OK) {
          if (rc == SLUICE_OK) rc = w;
          return false;
        }
      }
    };
    // Issue the copies of the j-th expert in copy order.
    auto issue = [&](int j) {
      const int i = L->order[j];
      const int local = L->streams[2 * i], slot = L->streams[2 * i + 1];
      const int srow = j < n_staged ? stage_ready_row(L, local) : -1;
      L->srow_of[j] = srow;
      if (C != nullptr && srow < 0) {
        size_t need = 0;
        for (const ParamRows& p : L->params) need += coded(p) ? ring_round(p.coded_len[local]) : 0;
        if (!ring_room(j, need)) return;
      }
      size_t at = L->ring_off[j];
      for (size_t pi = 0; rc == SLUICE_OK && pi < L->params.size(); ++pi) {
        const ParamRows& p = L->params[pi];
        L->bytes += (int64_t)p.row_bytes;
        if (early && p.rows_dev != nullptr) continue;  // the gap kernel copies these rows itself
        if (C != nullptr && coded(p)) {
          if (srow < 0) {
            const size_t len = p.coded_len[local];
            if (copy(C->ring + at, p.coded_base + (size_t)local * p.coded_stride,
                     p.coded_agent.handle != 0 ? p.coded_agent : R->cpu_agent, len,
                     R->engine[p.lane]))
              L->link_bytes += (int64_t)len;
            at += ring_round(len);
          }
        } else {
          char* dst = p.slot_base + (size_t)slot * p.row_bytes;
          if (srow >= 0) {
            copy(dst, L->stage_dev[pi] + (size_t)srow * L->stage_row_bytes[pi], R->gpu_agent,
                 p.row_bytes, 0);
          } else if (copy(dst, p.host_base + (size_t)local * p.row_bytes,
                          p.host_agent.handle != 0 ? p.host_agent : R->cpu_agent, p.row_bytes,
                          R->engine[p.lane])) {
            L->link_bytes += (int64_t)p.row_bytes;
          }
        }
        if (rc != SLUICE_OK) L->bytes -= (int64_t)p.row_bytes;
        if (j == n_staged && pi == 0) SLUICE_HTRACE(23, L, want, n_staged);
      }
      L->sig_end[j] = armed;
      if (rc != SLUICE_OK) return;
      whole = j + 1;
      if (srow >= 0) {
        ++L->stage_hits;
        L->stage_hit_bytes += (int64_t)link_bytes_of(L, local, C != nullptr);
      }
    };
    // The link is the bottleneck of a missing step: the staged experts and
    // the first expert over the link are queued, the staged ones landed,
    // then the device is answered (its resident experts then compute while
    // the rows stream), then the other experts queued.
    int j = 0;
    for (; rc == SLUICE_OK && j < n_staged; ++j) issue(j);
    if (rc == SLUICE_OK && j < n_streams) issue(j++);
    land_upto(std::min(whole, n_staged));
    // (a failure before the answer still answers the device: the map and
    // the fill list are the bookkeeping's; the slots are marked below)
    if (early) {
      respond(L, want, SLUICE_OK, n_streams);
      SLUICE_HTRACE(24, L, want, n_copy);
    }
    for (; rc == SLUICE_OK && j < n_streams; ++j) issue(j);
    SLUICE_HTRACE(25, L, want, armed);
    land_upto(whole);
    int marked = landed;  // streams whose slots are marked
    // every issued copy has completed (or the layer needs a resync, which
    // waits for them again)
    if (rc == SLUICE_OK || drain_copies(L) == SLUICE_OK) L->armed_copies = 0;
    if (rc != SLUICE_OK) {
      // A failed stream-in is reported to the caller (and, under the server,
      // raises the abort flag).  The device must not wait for rows that are
      // not coming, so the rest of the answered slots are marked too; and the
      // experts whose rows were not seen to land leave the slot cache, so
      // that no later gap takes them as hits.  The device map still holds
      // them until sluice_layer_gap_resync writes the host's.
      if (early)
        for (; marked < n_streams; ++marked)
          __atomic_store_n(&mb->slot_ready[L->streams[2 * L->order[marked] + 1]], want,
                           __ATOMIC_RELEASE);
      for (int j = landed; j < n_streams; ++j) (void)L->c.unfill(L->streams[2 * L->order[j] + 1]);
      // their ring regions are free once no copy writes them
      if (C != nullptr && L->armed_copies == 0)
        for (int j = landed; j < n_streams; ++j)
          if (L->use_id[j] != 0) ring_set(C, L->use_id[j], kUseDead, 0);
    }
    if (early) {
      L->done_stamp.store(want, std::memory_order_release);
      return rc;
    }
  }
  if (waits && rc == SLUICE_OK && grc != 0) rc = grc;
  if (waits) respond(L, want, rc, 0);
  L->done_stamp.store(want, std::memory_order_release);
  return rc;
}

// The params the gap kernel copies itself (sluice_layer_add_param).
PullRows pull_rows_of(const sluice_layer* L) {
  PullRows pull{};
  pull.rows = L->c.local_n;
  for (const ParamRows& p : L->params) {
    if (p.rows_dev == nullptr) continue;
    pull.vecs[pull.n] = (int)(p.row_bytes / 16);
    pull.src[pull.n] = (const u32x4_t*)p.rows_dev;
    pull.dst[pull.n] = (u32x4_t*)p.slot_base;
    ++pull.n;
  }
  return pull;
}

int launch_gap(sluice_layer* L, const int32_t* ids, int n, const void* hs_src, void* hs_dst,
               size_t hs_bytes, int32_t* plan, hipStream_t st) {
  if ((hs_bytes & 15) != 0 || ((uintptr_t)hs_src & 15) != 0 || ((uintptr_t)hs_dst & 15) != 0)
    return SLUICE_E_INVAL;
  if (hs_bytes > 0 && (hs_src == nullptr || hs_dst == nullptr)) return SLUICE_E_INVAL;
  const int E = L->c.E, S = L->c.S;
  int32_t* pending = L->dev_block + E + 3;
  const PullRows pull = pull_rows_of(L);
  hipLaunchKernelGGL(gap_kernel, dim3(1), dim3(kLookupThreads), 0, st, ids, n, L->map_dev,
                     L->dev_block, E, L->mb_dev, L->dev_block + E, pending, pending + S, S,
                     g_abort_dev, g_dev[L->device].bound_dev, (const u32x4_t*)hs_src, (u32x4_t*)hs_dst,
                     (int)(hs_bytes / 16), plan, pull);
  return (int)hipGetLastError();
}

}  // namespace

// ---------------------------------------------------------------------------
// Server thread: serves every registered layer's mailbox as records arrive.
// ---------------------------------------------------------------------------
struct sluice_gap_server {
  std::vector<sluice_layer*> layers;
  bool fast_hit = false;
  int device = 0;
  std::thread th;
  std::atomic<bool> stop{false};
  std::atomic<int> error{0};
  std::atomic<int64_t> served{0};
  // staging: the layer whose chunk each staging lane carries (nullptr:
  // free), the layer whose gap comes next, and whether the last look found
  // nothing to copy (no look again until a gap is served or a chunk lands)
  sluice_layer* stage_lane[kStageLanes] = {};
  size_t cursor = 0;
  bool stage_quiet = false;
  CodecRes* codec = nullptr;  // decode resources (layers with coded stores)
};

namespace {
// Smallest ring for coded rows; it holds at least two of the largest coded
// experts of the server's layers.
constexpr size_t kRingMin = 128u << 20;

int codec_res_destroy(CodecRes* C) {
  if (C == nullptr) return SLUICE_OK;
  int rc = SLUICE_OK;
  auto keep = [&](hipError_t e) {
    if (e != hipSuccess && rc == SLUICE_OK) rc = (int)e;
  };
  if (C->queue != nullptr) {
    // no decode job outlives its ring
    const int q = codec_sync(C->queue, gap_timeout_s());
    if (q != SLUICE_OK && rc == SLUICE_OK) rc = q;
  }
  if (C->ring != nullptr) keep(hipFree(C->ring));
  if (C->wg_count != nullptr) keep(hipFree(C->wg_count));
  if (C->done_host != nullptr) keep(hipHostFree(C->done_host));
  delete C;
  return rc;
}

// Decode resources on `device` with a ring of at least 2 * `largest` bytes.
int codec_res_create(int device, size_t largest, CodecRes** out) {
  *out = nullptr;
  int cur = 0;
  SLUICE_HIP_CHECK(hipGetDevice(&cur));
  if (cur != device) SLUICE_HIP_CHECK(hipSetDevice(device));
  CodecRes* C = new (std::nothrow) CodecRes();
  if (C == nullptr) {
    if (cur != device) (void)hipSetDevice(cur);
    return SLUICE_E_NOMEM;
  }
  C->device = device;
  C->ring_bytes = std::max(kRingMin, 2 * largest);
  DeviceRes* R = nullptr;
  int qrc = device_res(device, &R);
  if (qrc == SLUICE_OK) qrc = codec_queue(device, R->gpu_agent, R->cpu_agent, &C->queue);
  if (qrc != SLUICE_OK) {
    if (cur != device) (void)hipSetDevice(cur);
    delete C;
    return qrc;
  }
  hipError_t e = hipMalloc((void**)&C->wg_count, 256);
  if (e == hipSuccess) e = hipMemset(C->wg_count, 0, 256);
  void* h = nullptr;
  if (e == hipSuccess)
    e = hipHostMalloc(&h, 256, hipHostMallocCoherent | hipHostMallocMapped | hipHostMallocPortable);
  if (e == hipSuccess) {
    C->done_host = static_cast<unsigned long long*>(h);
    *C->done_host = 0;
    void* d = nullptr;
    e = hipHostGetDevicePointer(&d, h, 0);
    C->done_dev = static_cast<unsigned long long*>(d);
  }
  if (e == hipSuccess) e = hipMalloc((void**)&C->ring, C->ring_bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (cur != device) (void)hipSetDevice(cur);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // reported here, not by the caller's next call
    (void)codec_res_destroy(C);
    return (int)e;
  }
  *out = C;
  return SLUICE_OK;
}
}  // namespace

// One staging step, on a sweep that found no record: take in the chunks
// that landed, then put a chunk on each free staging lane, for the row
// whose expert its layer selects most often (every layer counts one gap
// per step, so the counts compare across layers; the link's idle time is
// the budget, so the likeliest hits go first).  A layer whose last
// stream-in failed to drain stages nothing.
static void stage_step(sluice_gap_server* S) {
  for (int l = 0; l < kStageLanes; ++l) {
    sluice_layer* L = S->stage_lane[l];
    if (L == nullptr || hsa_signal_load_relaxed(L->stage_sig[l]) > 0) continue;
    std::lock_guard<std::mutex> lk(L->mu);
    stage_poll(L);
    S->stage_lane[l] = nullptr;
    S->stage_quiet = false;
  }
  if (S->stage_quiet) return;
  const size_t n = S->layers.size();
  bool busy = false;
  for (int l = 0; l < kStageLanes; ++l) {
    if (S->stage_lane[l] != nullptr) {
      busy = true;
      continue;
    }
    sluice_layer* best = nullptr;
    int best_row = -1;
    for (size_t k = 0; k < n; ++k) {
      sluice_layer* L = S->layers[(S->cursor + k) % n];
      if (L->stage.empty() || L->stage_broken || L->armed_copies != 0) continue;
      if (L->codec == nullptr && has_coded(L)) continue;  // coded rows it could not decode
      if (L->stage_sig_row[l] >= 0 || (!L->stage_dirty && !stage_has_copy(L))) continue;
      std::lock_guard<std::mutex> lk(L->mu);
      stage_choose(L);
      const int r = stage_next_row(L);
      if (r >= 0 && (best == nullptr || L->sel_count[L->stage[r].local] >
                                            best->sel_count[best->stage[best_row].local])) {
        best = L;
        best_row = r;
      }
    }
    if (best != nullptr) {
      std::lock_guard<std::mutex> lk(best->mu);
      if (stage_issue(best, &g_dev[best->device], l, best_row)) {
        S->stage_lane[l] = best;
        busy = true;
      }
    }
  }
  if (!busy) S->stage_quiet = true;
}

// The server spins while gaps arrive (a decode step posts one per MoE layer,
// every ~0.1 ms); after kServerIdleS without a record it naps kServerNapUs
// between sweeps, so an idle engine does not hold a core.  The first gap
// after such a pause is served up to one nap (plus the wake-up) late.
constexpr double kServerIdleS = 5e-3;
constexpr int kServerNapUs = 50;

static void server_loop(sluice_gap_server* S) {
  (void)hipSetDevice(S->device);
  double last = now_s();
  unsigned idle = 0;
  while (!S->stop.load(std::memory_order_acquire)) {
    bool any = false;
    for (size_t i = 0; i < S->layers.size(); ++i) {
      sluice_layer* L = S->layers[i];
      const int rc = serve_one(L, S->fast_hit, false, nullptr);
      if (rc == kNothing) continue;
      any = true;
      S->cursor = (i + 1) % S->layers.size();
      S->stage_quiet = false;
      S->served.fetch_add(1, std::memory_order_relaxed);
      if (rc != SLUICE_OK) {
        int zero = 0;
        S->error.compare_exchange_strong(zero, rc);
        __atomic_store_n(g_abort_host, 1, __ATOMIC_RELEASE);
      }
    }
    if (any) {
      idle = 0;
      last = -1.0;  // read the clock again on the next idle sweep
      continue;
    }
    stage_step(S);
    _mm_pause();
    if ((++idle & 255u) != 0) continue;
    const double t = now_s();
    if (last < 0) last = t;
    if (t - last > kServerIdleS)
      std::this_thread::sleep_for(std::chrono::microseconds(kServerNapUs));
  }
}

extern "C" int sluice_layer_create(int E, int local_n, int num_slots, int protected_cap,
                                   const int32_t* local_of, int32_t* expert_map_dev,
                                   sluice_layer** out) {
  if (out == nullptr || E <= 0 || E > SLUICE_MAX_EXPERTS || local_n <= 0 || local_n > E ||
      num_slots <= 0 || num_slots > SLUICE_MAX_SLOTS || protected_cap < 0)
    return SLUICE_E_INVAL;
  sluice_layer* L = new (std::nothrow) sluice_layer();
  if (L == nullptr) return SLUICE_E_NOMEM;
  L->c.init(E, local_n, num_slots, protected_cap, local_of);
  L->map_dev = expert_map_dev;
  if (expert_map_dev != nullptr) {
    // Device resources are made here, never under graph capture.
    const int rc = layer_device_init(L);
    if (rc != SLUICE_OK) {
      delete L;
      return rc;
    }
  }
  *out = L;
  return SLUICE_OK;
}

extern "C" int sluice_layer_destroy(sluice_layer* L) {
  if (L == nullptr) return SLUICE_OK;
  if (L->server != nullptr) return SLUICE_E_STATE;
  int rc = SLUICE_OK;
  if (L->map_dev != nullptr && L->mb != nullptr) slotwait_unregister(L->map_dev);
  if (drain_copies(L) != SLUICE_OK) return SLUICE_E_STATE;  // copies still write its slots
  if (stage_drain(L) != SLUICE_OK) return SLUICE_E_STATE;   // chunks still write its staging rows
  for (hsa_signal_t sig : L->fill_sig) (void)hsa_signal_destroy(sig);
  for (hsa_signal_t sig : L->stage_sig)
    if (sig.handle != 0) (void)hsa_signal_destroy(sig);
  rc = stage_free(L);
  {
    const int crc = codec_free(L);
    if (rc == SLUICE_OK) rc = crc;
  }
  for (ParamRows& p : L->params)
    if (p.rows_dev != nullptr) {
      const hipError_t e = hipFree(p.rows_dev);
      if (e != hipSuccess) rc = (int)e;
      p.rows_dev = nullptr;
    }
  if (L->mb != nullptr) {
    hipError_t e = hipHostFree(L->mb);
    if (e != hipSuccess) rc = (int)e;
  }
  if (L->dev_block != nullptr) {
    hipError_t e = hipFree(L->dev_block);
    if (e != hipSuccess) rc = (int)e;
  }
  if (L->ids_host != nullptr) {
    hipError_t e = hipHostFree(L->ids_host);
    if (e != hipSuccess) rc = (int)e;
  }
  for (std::vector<hipEvent_t>* v : {&L->wave_ev, &L->copy_ev})
    for (hipEvent_t ev : *v) (void)hipEventDestroy(ev);
  if (L->pre_ev != nullptr) (void)hipEventDestroy(L->pre_ev);
  delete L;
  return rc;
}

namespace {
// [p, p + bytes) lies inside one allocation the HSA runtime knows (device
// memory, or host memory it allocated or locked): the SDMA engines copy
// from and to it directly, with no staging for pageable memory and no
// bounds check of their own.
bool known_range(const void* p, size_t bytes, hsa_agent_t* owner = nullptr) {
  hsa_amd_pointer_info_t info;
  memset(&info, 0, sizeof(info));
  info.size = sizeof(info);
  if (hsa_amd_pointer_info(p, &info, nullptr, nullptr, nullptr) != HSA_STATUS_SUCCESS) return false;
  if (owner != nullptr) *owner = info.agentOwner;
  if (info.type == HSA_EXT_POINTER_TYPE_UNKNOWN || bytes > info.sizeInBytes) return false;
  const uintptr_t a = (uintptr_t)p;
  for (const void* b : {info.hostBaseAddress, info.agentBaseAddress}) {
    const uintptr_t base = (uintptr_t)b;
    if (b != nullptr && a >= base && a - base <= info.sizeInBytes - bytes) return true;
  }
  return false;
}
}  // namespace

extern "C" int sluice_layer_add_param(sluice_layer* L, void* slot_base_dev, const void* host_base,
                                      size_t row_bytes) {
  if (L == nullptr || slot_base_dev == nullptr || host_base == nullptr || row_bytes == 0)
    return SLUICE_E_INVAL;
  // A layer with a device copies these rows with the SDMA engines: both
  // ranges must be allocations the runtime knows, whole.
  if (!L->stage.empty()) return SLUICE_E_STATE;  // staging rows are laid out over the params
  if (L->codec_mask != 0) return SLUICE_E_STATE;  // and the coded stores
  hsa_agent_t host_agent{};
  if (L->mb != nullptr &&
      (!known_range(host_base, row_bytes * (size_t)L->c.local_n, &host_agent) ||
       !known_range(slot_base_dev, row_bytes * (size_t)L->c.S)))
    return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> lk(L->mu);
  ParamRows row{};
  row.slot_base = (char*)slot_base_dev;
  row.host_base = (const char*)host_base;
  row.row_bytes = row_bytes;
  L->params.push_back(row);
  hsa_device_type_t host_type{};
  if (host_agent.handle != 0 &&
      hsa_agent_get_info(host_agent, HSA_AGENT_INFO_DEVICE, &host_type) == HSA_STATUS_SUCCESS &&
      host_type == HSA_DEVICE_TYPE_CPU)
    L->params.back().host_agent = host_agent;
  // Small rows are pulled by the gap kernel from a copy of all of them in
  // HBM (PullRows); a layer without a device keeps host copies.
  ParamRows& np = L->params.back();
  int n_pulled = 0;
  for (const ParamRows& q : L->params) n_pulled += q.rows_dev != nullptr;
  if (L->mb != nullptr && row_bytes <= kPullMaxRowBytes && row_bytes % 16 == 0 &&
      ((uintptr_t)slot_base_dev & 15) == 0 && n_pulled < kMaxPull) {
    const size_t all = row_bytes * (size_t)L->c.local_n;
    void* d = nullptr;
    hipError_t e = hipMalloc(&d, all);
    if (e == hipSuccess) e = hipMemcpy(d, host_base, all, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      if (d != nullptr) (void)hipFree(d);
      (void)hipGetLastError();  // reported here, not by the caller's next call
      L->params.pop_back();
      return (int)e;
    }
    np.rows_dev = (char*)d;
  }
  // Lanes: largest rows first, each to the lane with the fewest bytes so
  // far (bf16: w13 | w2; fp8: w13 | w2 + both scale rows).
  std::vector<int> order(L->params.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
    return L->params[a].row_bytes > L->params[b].row_bytes;
  });
  size_t load[kLanes] = {};
  L->lane_mask = 0;
  for (int i : order) {
    int best = 0;
    for (int l = 1; l < kLanes; ++l)
      if (load[l] < load[best]) best = l;
    L->params[i].lane = best;
    load[best] += L->params[i].row_bytes;
    L->lane_mask |= 1u << best;
  }
  return SLUICE_OK;
}

extern "C" int sluice_layer_pulled_params(sluice_layer* L) {
  if (L == nullptr) return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> lk(L->mu);
  int n = 0;
  for (const ParamRows& p : L->params) n += p.rows_dev != nullptr;
  return n;
}

extern "C" int sluice_layer_set_staging(sluice_layer* L, int rows) {
  if (L == nullptr || rows < 0 || rows > kMaxStageRows || L->mb == nullptr) return SLUICE_E_INVAL;
  if (L->server != nullptr) return SLUICE_E_STATE;
  DeviceRes* R = nullptr;
  const int drc = device_res(L->device, &R);
  if (drc != SLUICE_OK) return drc;
  std::lock_guard<std::mutex> lk(L->mu);
  if ((int)L->stage.size() == rows) return SLUICE_OK;  // as set (a restarted server keeps them)
  if (stage_drain(L) != SLUICE_OK) return SLUICE_E_TIMEOUT;
  int rc = stage_free(L);
  if (rc != SLUICE_OK || rows == 0) return rc;
  if (R->stage_engine[0] == 0) return SLUICE_E_INVAL;  // no copy engines free for staging
  for (hsa_signal_t& sig : L->stage_sig)
    if (sig.handle == 0 && hsa_signal_create(0, 0, nullptr, &sig) != HSA_STATUS_SUCCESS)
      return SLUICE_E_COPY;
  // the params the gap copies (the pulled ones come from their HBM copy),
  // coded where the store is coded
  size_t bytes = 0;
  L->stage_row_bytes.assign(L->params.size(), 0);
  for (size_t pi = 0; pi < L->params.size(); ++pi) {
    const ParamRows& p = L->params[pi];
    if (p.rows_dev != nullptr) continue;
    L->stage_row_bytes[pi] = coded(p) ? p.coded_stride : p.row_bytes;
    bytes += L->stage_row_bytes[pi];
  }
  if (bytes == 0) return SLUICE_OK;  // nothing to stage
  L->stage_dev.assign(L->params.size(), nullptr);
  for (size_t pi = 0; pi < L->params.size(); ++pi) {
    const ParamRows& p = L->params[pi];
    if (p.rows_dev != nullptr) continue;
    void* d = nullptr;
    const hipError_t e = hipMalloc(&d, L->stage_row_bytes[pi] * (size_t)rows);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // reported here, not by the caller's next call
      (void)stage_free(L);
      return (int)e;
    }
    L->stage_dev[pi] = (char*)d;
  }
  L->stage_bytes = bytes;
  L->stage.assign((size_t)rows, sluice_layer::StageRow{});
  L->sel_count.assign((size_t)L->c.local_n, 0);
  L->stage_gaps = 0;
  L->stage_dirty = false;
  L->stage_broken = false;
  return SLUICE_OK;
}

extern "C" int sluice_layer_stage_counters(const sluice_layer* Lc, int64_t* counters) {
  if (Lc == nullptr || counters == nullptr) return SLUICE_E_INVAL;
  sluice_layer* L = const_cast<sluice_layer*>(Lc);
  std::lock_guard<std::mutex> lk(L->mu);
  int ready = 0;
  for (const sluice_layer::StageRow& row : L->stage) ready += row.state == kStageReady;
  counters[0] = (int64_t)L->stage.size();
  counters[1] = ready;
  counters[2] = L->stage_filled;
  counters[3] = L->stage_h2d;
  counters[4] = L->stage_hits;
  counters[5] = L->stage_hit_bytes;
  return SLUICE_OK;
}

namespace {
// f(i) for every i in [0, n), on up to 16 host threads.
template <typename F>
void parallel_for(int n, F f) {
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const int nt = (int)std::min<unsigned>(std::min(hw, 16u), (unsigned)std::max(n, 1));
  std::atomic<int> next{0};
  auto work = [&] {
    for (int i; (i = next.fetch_add(1, std::memory_order_relaxed)) < n;) f(i);
  };
  std::vector<std::thread> th;
  for (int t = 1; t < nt; ++t) th.emplace_back(work);
  work();
  for (std::thread& t : th) t.join();
}
}  // namespace

extern "C" int sluice_layer_set_codec(sluice_layer* L, uint32_t bf16_params) {
  if (L == nullptr || L->mb == nullptr) return SLUICE_E_INVAL;
  if (L->server != nullptr) return SLUICE_E_STATE;
  std::lock_guard<std::mutex> lk(L->mu);
  if (bf16_params == L->codec_mask) return SLUICE_OK;  // as set (a restarted server keeps them)
  if (!L->stage.empty()) return SLUICE_E_STATE;        // staging rows are laid out over them
  int rc = codec_free(L);
  if (rc != SLUICE_OK || bf16_params == 0) return rc;
  const int local_n = L->c.local_n;
  int n_coded = 0;
  for (size_t pi = 0; pi < L->params.size() && pi < 32; ++pi) {
    ParamRows& p = L->params[pi];
    const size_t n = p.row_bytes / 2;
    if (!((bf16_params >> pi) & 1u) || p.rows_dev != nullptr || n_coded == kCodecMaxParts ||
        p.row_bytes % (2 * kCodecChunk) != 0 || n / kCodecChunk > 0xffffffffu ||
        ((uintptr_t)p.host_base & 1) != 0)
      continue;
    {  // the same host rows coded for another layer already
      std::lock_guard<std::mutex> lk2(g_coded_mu);
      CodedStore* hit = nullptr;
      for (CodedStore* cs : g_coded)
        if (cs->host_base == p.host_base && cs->row_bytes == p.row_bytes &&
            cs->local_n == local_n)
          hit = cs;
      if (hit != nullptr) {
        ++hit->users;
        p.coded_base = hit->base;
        p.coded_stride = hit->stride;
        p.coded_len = hit->len;
        p.coded_agent = hit->agent;
        ++n_coded;
        continue;
      }
    }
    const uint16_t* rows = reinterpret_cast<const uint16_t*>(p.host_base);
    std::vector<size_t> len((size_t)local_n);
    parallel_for(local_n, [&](int e) { len[e] = codec_coded_bytes(rows + (size_t)e * n, n); });
    const size_t mx = *std::max_element(len.begin(), len.end());
    // rows that code poorly (more than ~1 exponent in 8 escaped) stream as they are
    if (mx > p.row_bytes / 8 * 7 || mx > 0xffffffffu) continue;
    const size_t stride = ring_round(mx);
    void* buf = nullptr;
    const hipError_t e = hipHostMalloc(&buf, stride * (size_t)local_n, hipHostMallocPortable);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // reported here, not by the caller's next call
      (void)codec_free(L);
      return (int)e;
    }
    parallel_for(local_n, [&](int x) {
      codec_encode(rows + (size_t)x * n, n, static_cast<uint8_t*>(buf) + (size_t)x * stride);
    });
    p.coded_base = static_cast<char*>(buf);
    p.coded_stride = stride;
    p.coded_len.assign(len.begin(), len.end());
    hsa_agent_t owner{};
    hsa_device_type_t t{};
    if (known_range(buf, stride * (size_t)local_n, &owner) &&
        hsa_agent_get_info(owner, HSA_AGENT_INFO_DEVICE, &t) == HSA_STATUS_SUCCESS &&
        t == HSA_DEVICE_TYPE_CPU)
      p.coded_agent = owner;
    {
      std::lock_guard<std::mutex> lk2(g_coded_mu);
      g_coded.push_back(new CodedStore{p.host_base, p.row_bytes, local_n, p.coded_base,
                                       p.coded_stride, p.coded_len, p.coded_agent, 1});
    }
    ++n_coded;
  }
  L->codec_mask = bf16_params;
  return SLUICE_OK;
}

extern "C" int sluice_layer_codec_counters(const sluice_layer* Lc, int64_t* counters) {
  if (Lc == nullptr || counters == nullptr) return SLUICE_E_INVAL;
  sluice_layer* L = const_cast<sluice_layer*>(Lc);
  std::lock_guard<std::mutex> lk(L->mu);
  int64_t n = 0, rows = 0, coded_all = 0;
  for (const ParamRows& p : L->params) {
    if (!coded(p)) continue;
    ++n;
    rows += (int64_t)p.row_bytes;
    for (uint32_t b : p.coded_len) coded_all += b;
  }
  counters[0] = n;
  counters[1] = rows;
  counters[2] = coded_all;
  counters[3] = L->link_bytes;
  counters[4] = L->decodes;
  counters[5] = L->decodes_staged;
  return SLUICE_OK;
}

extern "C" int sluice_layer_pin(sluice_layer* L, int local, int debit_protected, int* slot_out) {
  if (L == nullptr) return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> lk(L->mu);
  const int s = L->c.pin(local, debit_protected != 0);
  if (slot_out) *slot_out = s;
  return s < 0 ? SLUICE_E_STATE : SLUICE_OK;
}

extern "C" int sluice_layer_gap_launch(sluice_layer* L, const int32_t* topk_ids, int n,
                                       const void* hs_src, void* hs_dst, size_t hs_bytes,
                                       int32_t* plan, sluice_stream_t stream) {
  if (L == nullptr || n < 0 || n > SLUICE_MAX_PAIRS || (n > 0 && topk_ids == nullptr))
    return SLUICE_E_INVAL;
  if (((uintptr_t)plan & 3) != 0) return SLUICE_E_INVAL;
  if (L->mb == nullptr || L->map_dev == nullptr) return SLUICE_E_STATE;
  return launch_gap(L, topk_ids, n, hs_src, hs_dst, hs_bytes, plan, (hipStream_t)stream);
}

extern "C" int sluice_layer_gap_serve(sluice_layer* L, int fast_hit, sluice_stream_t compute) {
  if (L == nullptr) return SLUICE_E_INVAL;
  if (L->mb == nullptr || L->server != nullptr) return SLUICE_E_STATE;
  return serve_one(L, fast_hit != 0, true, (hipStream_t)compute);
}

extern "C" int sluice_layer_gap(sluice_layer* L, const int32_t* topk_ids, int n, int fast_hit,
                                sluice_stream_t compute) {
  if (L == nullptr || n < 0 || n > SLUICE_MAX_PAIRS || (n > 0 && topk_ids == nullptr))
    return SLUICE_E_INVAL;
  if (L->mb == nullptr || L->map_dev == nullptr || L->server != nullptr) return SLUICE_E_STATE;
  int rc = launch_gap(L, topk_ids, n, nullptr, nullptr, 0, nullptr, (hipStream_t)compute);
  if (rc != SLUICE_OK) return rc;
  return serve_one(L, fast_hit != 0, true, (hipStream_t)compute);
}

extern "C" int sluice_gap_server_create(sluice_layer* const* layers, int n_layers, int fast_hit,
                                        sluice_gap_server** out) {
  if (out == nullptr || n_layers <= 0 || layers == nullptr) return SLUICE_E_INVAL;
  *out = nullptr;
  sluice_gap_server* S = new (std::nothrow) sluice_gap_server();
  if (S == nullptr) return SLUICE_E_NOMEM;
  for (int i = 0; i < n_layers; ++i) {
    sluice_layer* L = layers[i];
    if (L == nullptr || L->mb == nullptr || L->server != nullptr) {
      delete S;
      return L == nullptr ? SLUICE_E_INVAL : SLUICE_E_STATE;
    }
    for (sluice_layer* M : S->layers)
      if (M == L) {
        delete S;
        return SLUICE_E_INVAL;
      }
    S->layers.push_back(L);
  }
  S->fast_hit = fast_hit != 0;
  S->device = S->layers[0]->device;
  size_t largest = 0;  // coded rows of one expert, as they lie in the ring
  bool any_coded = false;
  for (sluice_layer* L : S->layers) {
    std::lock_guard<std::mutex> lk(L->mu);
    if (!has_coded(L)) continue;
    any_coded = true;
    for (int loc = 0; loc < L->c.local_n; ++loc) {
      size_t b = 0;
      for (const ParamRows& p : L->params) b += coded(p) ? ring_round(p.coded_len[loc]) : 0;
      largest = std::max(largest, b);
    }
  }
  // Without decode resources (no code object beside the library, no HSA
  // queue) the layers stream their uncoded rows, which stay registered.
  if (any_coded && codec_res_create(S->device, largest, &S->codec) != SLUICE_OK)
    S->codec = nullptr;
  for (sluice_layer* L : S->layers) {
    L->server = S;
    L->codec = has_coded(L) ? S->codec : nullptr;
  }
  try {
    S->th = std::thread(server_loop, S);
  } catch (...) {
    for (sluice_layer* L : S->layers) {
      L->server = nullptr;
      L->codec = nullptr;
    }
    (void)codec_res_destroy(S->codec);
    delete S;
    return SLUICE_E_NOMEM;
  }
  *out = S;
  return SLUICE_OK;
}

// Wait until every record posted so far has been served; returns the sticky
// error of the server, if any.  Call after the streams that launched gaps
// have been synchronised.
extern "C" int sluice_gap_server_drain(sluice_gap_server* S, double timeout_s) {
  if (S == nullptr) return SLUICE_E_INVAL;
  const double t0 = now_s();
  for (sluice_layer* L : S->layers) {
    for (;;) {
      const int dev_status = __atomic_load_n(&L->mb->dev_status, __ATOMIC_ACQUIRE);
      if (dev_status != 0) {
        int zero = 0;
        S->error.compare_exchange_strong(zero, dev_status);
        break;
      }
      if (!record_pending(L)) break;
      if (S->error.load() != 0) break;
      if (now_s() - t0 > timeout_s) return SLUICE_E_TIMEOUT;
      _mm_pause();
    }
  }
  // and the decodes those records launched
  if (S->codec != nullptr) {
    const unsigned long long seq = S->codec->launched.load(std::memory_order_acquire);
    while (codec_done(S->codec) < seq) {
      if (now_s() - t0 > timeout_s) return SLUICE_E_TIMEOUT;
      _mm_pause();
    }
  }
  return S->error.load();
}

extern "C" int sluice_gap_server_error(const sluice_gap_server* S) {
  return S == nullptr ? SLUICE_E_INVAL : S->error.load();
}

extern "C" int sluice_gap_server_destroy(sluice_gap_server* S) {
  if (S == nullptr) return SLUICE_OK;
  S->stop.store(true, std::memory_order_release);
  if (S->th.joinable()) S->th.join();
  for (sluice_layer* L : S->layers) {
    std::lock_guard<std::mutex> lk(L->mu);
    (void)stage_drain(L);  // no staging chunk outlives the server
    L->server = nullptr;
    L->codec = nullptr;
  }
  const int err = S->error.load();
  const int crc = codec_res_destroy(S->codec);  // waits for the decode jobs
  delete S;
  return err != SLUICE_OK ? err : crc;
}

extern "C" int sluice_gap_set_timeout(double seconds) {
  if (!(seconds >= 0.0) || seconds > 86400.0) return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> lk(g_dev_mu);
  g_timeout_set.store(seconds, std::memory_order_relaxed);
  // every device's bound word follows (the kernels read it when they wait);
  // no HIP call before any device was set up
  bool any = false;
  for (int d = 0; d < kMaxDevices; ++d) any = any || g_dev[d].bound_dev != nullptr;
  if (!any) return SLUICE_OK;
  int cur = -1;
  SLUICE_HIP_CHECK(hipGetDevice(&cur));
  int rc = SLUICE_OK;
  for (int d = 0; d < kMaxDevices && rc == SLUICE_OK; ++d) {
    if (g_dev[d].bound_dev == nullptr) continue;
    const long long ticks = bound_ticks(g_dev[d].clock_khz);
    hipError_t e = hipSetDevice(d);
    if (e == hipSuccess)
      e = hipMemcpy(g_dev[d].bound_dev, &ticks, sizeof(ticks), hipMemcpyHostToDevice);
    if (e != hipSuccess) rc = (int)e;
  }
  const hipError_t e = hipSetDevice(cur);
  if (rc == SLUICE_OK && e != hipSuccess) rc = (int)e;
  return rc;
}

extern "C" int sluice_gap_inject_copy_failure(int after) {
  g_fail_after.store(after < 0 ? -1 : after, std::memory_order_relaxed);
  return SLUICE_OK;
}

extern "C" int sluice_layer_unfill(sluice_layer* L, int slot) {
  if (L == nullptr || slot < 0 || slot >= L->c.S) return SLUICE_E_INVAL;
  if (L->server != nullptr) return SLUICE_E_STATE;
  std::lock_guard<std::mutex> lk(L->mu);
  return L->c.unfill(slot) ? SLUICE_OK : SLUICE_E_STATE;
}

extern "C" int sluice_gap_set_pipelined(int on) {
  if (on != 0 && on != 1) return SLUICE_E_INVAL;
  g_pipelined.store(on, std::memory_order_relaxed);
  return SLUICE_OK;
}

extern "C" int sluice_gap_abort(int set) {
  if (g_abort_host == nullptr) return SLUICE_OK;
  __atomic_store_n(g_abort_host, set ? 1 : 0, __ATOMIC_RELEASE);
  return SLUICE_OK;
}

// After an abort: once every stream that ran gap kernels is synchronised,
// clear the abort flag and line the host's stamps up with the device's, so
// the layers can be used again (their slot state is whatever the served
// records left; the aborted steps' outputs are invalid).  The device map
// may lag the host's slot cache (a device wait that ended after the host
// served the record, or fills dropped after a failed copy): the copy lanes
// are drained and the host's standing map is written to the device, which
// then holds the standing map again.
extern "C" int sluice_layer_gap_resync(sluice_layer* L) {
  if (L == nullptr || L->mb == nullptr || L->server != nullptr) return SLUICE_E_INVAL;
  DeviceRes* R = nullptr;
  const int rrc = device_res(L->device, &R);
  if (rrc != SLUICE_OK) return rrc;
  for (hipStream_t s : R->copy) SLUICE_HIP_CHECK(hipStreamSynchronize(s));
  {
    std::lock_guard<std::mutex> lk(L->mu);
    const int d = drain_copies(L);
    if (d != SLUICE_OK) return d;
    L->armed_copies = 0;
    const int ds = stage_drain(L);
    if (ds != SLUICE_OK) return ds;
    L->stage_broken = false;  // a failed chunk emptied its row; staging resumes
    L->stage_dirty = true;
  }
  int32_t dev_stamp = 0;
  SLUICE_HIP_CHECK(hipMemcpy(&dev_stamp, L->dev_block + L->c.E, sizeof(int32_t),
                             hipMemcpyDeviceToHost));
  std::lock_guard<std::mutex> lk(L->mu);
  {
    std::vector<int32_t> m((size_t)L->c.E);
    L->c.standing_map(m.data());
    SLUICE_HIP_CHECK(hipMemcpy(L->map_dev, m.data(), sizeof(int32_t) * m.size(),
                               hipMemcpyHostToDevice));
    const int32_t one = 1;  // the device's "standing map seen" word
    SLUICE_HIP_CHECK(hipMemcpy(L->dev_block + L->c.E + 1, &one, sizeof(int32_t),
                               hipMemcpyHostToDevice));
    L->c.map_is_standing = true;
    __atomic_store_n(&L->mb->standing, 1, __ATOMIC_RELEASE);
    // A gap the host answered early skipped the rows the device pulls; if
    // the device's wait ended before it read that answer, they never came.
    // Pull them again for every slot the cache holds.
    const PullRows pull = pull_rows_of(L);
    int nf = 0;
    for (int sl = 0; pull.n > 0 && sl < L->c.S; ++sl) {
      const int loc = L->c.expert_in_slot[sl];
      if (loc < 0) continue;
      L->mb->fill[nf] = sl;
      L->mb->fill_src[nf] = loc;
      ++nf;
    }
    L->mb->n_fill = 0;
    if (nf > 0) {
      hipLaunchKernelGGL(pull_slots_kernel, dim3(1), dim3(kLookupThreads), 0, nullptr, L->mb_dev,
                         nf, L->c.S, pull);
      SLUICE_HIP_CHECK(hipGetLastError());
      SLUICE_HIP_CHECK(hipStreamSynchronize(nullptr));
    }
  }
  L->host_stamp = dev_stamp;
  L->done_stamp.store(dev_stamp);
  __atomic_store_n(&L->mb->ack_stamp, dev_stamp, __ATOMIC_RELEASE);
  for (int i = 0; i < kRing; ++i) __atomic_store_n(&L->mb->rec[i].hdr, (uint64_t)0, __ATOMIC_RELEASE);
  __atomic_store_n(&L->mb->dev_status, 0, __ATOMIC_RELEASE);
  // no slot is left waiting for rows: the aborted gaps' rows are not coming
  const size_t n_pend = (size_t)L->c.S + 1 + L->c.S + 2 * (size_t)L->c.S;
  std::vector<int32_t> zero(n_pend, 0);
  SLUICE_HIP_CHECK(hipMemcpy(L->dev_block + L->c.E + 3, zero.data(), sizeof(int32_t) * n_pend,
                             hipMemcpyHostToDevice));
  return SLUICE_OK;
}

extern "C" int sluice_layer_gap_host(sluice_layer* L, const int32_t* ids, int n, int fast_hit,
                                     int32_t* streams, int max_streams, int* n_streams,
                                     int* map_written) {
  if (L == nullptr || n < 0 || (n > 0 && ids == nullptr)) return SLUICE_E_INVAL;
  if (L->server != nullptr) return SLUICE_E_STATE;
  std::lock_guard<std::mutex> lk(L->mu);
  // sorted(set(ids)) restricted to [0, E)
  std::vector<uint8_t> present(L->c.E, 0);
  for (int i = 0; i < n; ++i)
    if ((unsigned)ids[i] < (unsigned)L->c.E) present[ids[i]] = 1;
  std::vector<int32_t> uniq;
  for (int g = 0; g < L->c.E; ++g)
    if (present[g]) uniq.push_back(g);
  L->streams.clear();
  bool mw = false;
  const int rc = L->c.gap(uniq.data(), (int)uniq.size(), fast_hit != 0, L->streams, mw);
  const int ns = (int)L->streams.size() / 2;
  for (const ParamRows& p : L->params) L->bytes += (int64_t)ns * (int64_t)p.row_bytes;
  if (n_streams) *n_streams = ns;
  if (map_written) *map_written = mw ? 1 : 0;
  if (streams != nullptr) {
    if (ns > max_streams) return SLUICE_E_INVAL;
    for (int i = 0; i < 2 * ns; ++i) streams[i] = L->streams[i];
  }
  return rc;
}

// ---------------------------------------------------------------------------
// Classic (wave) step: run_moe + _run_waves (src/sluice/offloader.py:
// 1452-1765, 1846-1933) for steps the gap does not take (more tokens than
// the router-split envelope, prefill chunks).  plan: one host sync for the
// ids, then the bookkeeping; the caller then runs the expert product once
// per wave between classic_wave and classic_wave_done, which order the
// wave's map write and row copies around it.
// ---------------------------------------------------------------------------
namespace {

constexpr int kClassicMaxIds = 1 << 24;

int ensure_events(sluice_layer* L, size_t n) {
  for (std::vector<hipEvent_t>* v : {&L->wave_ev, &L->copy_ev}) {
    // copy_ev: one per wave and lane, [kLanes * w + lane]
    while (v->size() < (v == &L->copy_ev ? kLanes * n : n)) {
      hipEvent_t ev = nullptr;
      SLUICE_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
      v->push_back(ev);
    }
  }
  if (L->pre_ev == nullptr)
    SLUICE_HIP_CHECK(hipEventCreateWithFlags(&L->pre_ev, hipEventDisableTiming));
  return SLUICE_OK;
}

// Every used copy lane waits for `ev`.
int lanes_wait(const sluice_layer* L, DeviceRes* R, hipEvent_t ev) {
  for (int l = 0; l < kLanes; ++l)
    if (L->lane_mask >> l & 1u) SLUICE_HIP_CHECK(hipStreamWaitEvent(R->copy[l], ev, 0));
  return SLUICE_OK;
}

// Record evs[lane] on every used copy lane.
int lanes_record(const sluice_layer* L, DeviceRes* R, hipEvent_t* evs) {
  for (int l = 0; l < kLanes; ++l)
    if (L->lane_mask >> l & 1u) SLUICE_HIP_CHECK(hipEventRecord(evs[l], R->copy[l]));
  return SLUICE_OK;
}

// `st` waits for evs[lane] of every used copy lane.
int wait_lanes(const sluice_layer* L, hipStream_t st, hipEvent_t* evs) {
  for (int l = 0; l < kLanes; ++l)
    if (L->lane_mask >> l & 1u) SLUICE_HIP_CHECK(hipStreamWaitEvent(st, evs[l], 0));
  return SLUICE_OK;
}

// Row copies of wave w on the copy lanes (after whatever they wait on).
int issue_wave_copies(sluice_layer* L, int w, DeviceRes* R) {
  std::lock_guard<std::mutex> lk(L->mu);
  const slru::Wave& W = L->plan.waves[w];
  for (int i = 0; i < W.ns; ++i) {
    const int local = L->plan.streams[2 * (W.s0 + i)];
    const int slot = L->plan.streams[2 * (W.s0 + i) + 1];
    for (const ParamRows& p : L->params) {
      SLUICE_HIP_CHECK(hipMemcpyAsync(p.slot_base + (size_t)slot * p.row_bytes,
                                      p.host_base + (size_t)local * p.row_bytes, p.row_bytes,
                                      hipMemcpyHostToDevice, R->copy[p.lane]));
      L->bytes += (int64_t)p.row_bytes;
      L->link_bytes += (int64_t)p.row_bytes;
    }
  }
  return SLUICE_OK;
}

// A plan whose waves did not all run (the caller failed between waves)
// still owes the copies its bookkeeping assumed: issue them behind `st`.
int classic_flush(sluice_layer* L, hipStream_t st) {
  const int nW = (int)L->plan.waves.size();
  if (L->plan_copied < nW) {
    DeviceRes* R = nullptr;
    int rc = device_res(L->device, &R);
    if (rc) return rc;
    rc = ensure_events(L, (size_t)nW);
    if (rc) return rc;
    SLUICE_HIP_CHECK(hipEventRecord(L->pre_ev, st));
    rc = lanes_wait(L, R, L->pre_ev);
    if (rc) return rc;
    for (int w = L->plan_copied; w < nW; ++w) {
      rc = issue_wave_copies(L, w, R);
      if (rc) return rc;
    }
    hipEvent_t* evs = &L->copy_ev[kLanes * (nW - 1)];
    rc = lanes_record(L, R, evs);
    if (rc) return rc;
    rc = wait_lanes(L, st, evs);
    if (rc) return rc;
  }
  L->plan.clear();
  L->plan_next = L->plan_copied = 0;
  L->plan_in_wave = false;
  return SLUICE_OK;
}

// With a gap server attached: wait until every record this layer posted has
// been served, so the bookkeeping below does not race the server thread.
int wait_served(sluice_layer* L) {
  const double t0 = now_s();
  for (;;) {
    const int dev_status = __atomic_load_n(&L->mb->dev_status, __ATOMIC_ACQUIRE);
    if (dev_status != 0) return dev_status;
    if (L->server != nullptr) {
      const int err = sluice_gap_server_error(L->server);
      if (err != 0) return err;
    }
    if (!record_pending(L)) return SLUICE_OK;
    if (now_s() - t0 > gap_timeout_s()) return SLUICE_E_TIMEOUT;
    _mm_pause();
  }
}

void serialize_plan(const slru::Plan& P, std::vector<int32_t>& out) {
  out.clear();
  out.push_back((int32_t)P.waves.size());
  out.push_back(P.pipelined ? 1 : 0);
  for (const slru::Wave& W : P.waves) {
    out.push_back(W.np);
    out.insert(out.end(), P.pairs.begin() + 2 * W.p0, P.pairs.begin() + 2 * (W.p0 + W.np));
    out.push_back(W.ns);
    out.insert(out.end(), P.streams.begin() + 2 * W.s0, P.streams.begin() + 2 * (W.s0 + W.ns));
  }
}

bool classic_args_ok(int n, int T, const int32_t* ids, int spec_tokens) {
  if (n < 0 || T < 0 || n > kClassicMaxIds || spec_tokens < 0) return false;
  if (n > 0 && ids == nullptr) return false;
  if (T == 0) return n == 0;
  return n % T == 0;
}

}  // namespace

extern "C" int sluice_layer_classic_plan(sluice_layer* L, const int32_t* topk_ids, int n, int T,
                                         int nd, int ndec, int real_step, int spec_tokens,
                                         sluice_stream_t stream, int* n_waves) {
  if (L == nullptr || n_waves == nullptr || !classic_args_ok(n, T, topk_ids, spec_tokens))
    return SLUICE_E_INVAL;
  if (L->mb == nullptr || L->map_dev == nullptr) return SLUICE_E_STATE;
  hipStream_t st = (hipStream_t)stream;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  SLUICE_HIP_CHECK(hipStreamIsCapturing(st, &cs));
  if (cs != hipStreamCaptureStatusNone) return SLUICE_E_STATE;  // needs a host sync
  int rc = classic_flush(L, st);
  if (rc) return rc;
  if ((size_t)n > L->ids_cap) {
    if (L->ids_host != nullptr) SLUICE_HIP_CHECK(hipHostFree(L->ids_host));
    L->ids_host = nullptr;
    L->ids_cap = 0;
    size_t cap = 4096;
    while (cap < (size_t)n) cap *= 2;
    void* p = nullptr;
    SLUICE_HIP_CHECK(hipHostMalloc(&p, cap * sizeof(int32_t), hipHostMallocPortable));
    L->ids_host = static_cast<int32_t*>(p);
    L->ids_cap = cap;
  }
  // the one host sync of the step (src/sluice/offloader.py:1540)
  if (n > 0)
    SLUICE_HIP_CHECK(hipMemcpyAsync(L->ids_host, topk_ids, sizeof(int32_t) * (size_t)n,
                                    hipMemcpyDeviceToHost, st));
  SLUICE_HIP_CHECK(hipStreamSynchronize(st));
  if (L->server != nullptr) {
    rc = wait_served(L);
    if (rc) return rc;
  }
  {
    std::lock_guard<std::mutex> lk(L->mu);
    rc = L->c.classic(L->ids_host, n, T, nd, ndec, real_step != 0, spec_tokens, L->plan);
    if (rc) {
      L->plan.clear();
      return SLUICE_E_STATE;
    }
    ++L->classic_steps;
    L->classic_waves += (int64_t)L->plan.waves.size();
  }
  // the map stops being the standing map with the first wave's write
  __atomic_store_n(&L->mb->standing, 0, __ATOMIC_RELEASE);
  *n_waves = (int)L->plan.waves.size();
  return SLUICE_OK;
}

extern "C" int sluice_layer_classic_wave(sluice_layer* L, int wave, sluice_stream_t stream) {
  if (L == nullptr || wave < 0) return SLUICE_E_INVAL;
  const int nW = (int)L->plan.waves.size();
  if (wave >= nW || wave != L->plan_next || L->plan_in_wave) return SLUICE_E_STATE;
  hipStream_t st = (hipStream_t)stream;
  DeviceRes* R = nullptr;
  int rc = device_res(L->device, &R);
  if (rc) return rc;
  rc = ensure_events(L, (size_t)nW);
  if (rc) return rc;
  const slru::Wave& W = L->plan.waves[wave];
  if (wave == 0) {
    if (W.ns > 0) {
      // fills may overwrite a slot that earlier work on `st` reads
      SLUICE_HIP_CHECK(hipEventRecord(L->pre_ev, st));
      rc = lanes_wait(L, R, L->pre_ev);
      if (rc) return rc;
      rc = issue_wave_copies(L, 0, R);
      if (rc) return rc;
      rc = lanes_record(L, R, &L->copy_ev[0]);
      if (rc) return rc;
    }
    L->plan_copied = 1;
  }
  SlotTable tab;
  tab.n = L->c.S;
  for (int s = 0; s < L->c.S; ++s) tab.g[s] = -1;
  for (int i = 0; i < W.np; ++i) tab.g[L->plan.pairs[2 * (W.p0 + i) + 1]] = L->plan.pairs[2 * (W.p0 + i)];
  hipLaunchKernelGGL(map_refresh_kernel, dim3(1), dim3(256), 0, st, L->map_dev, L->c.E, tab,
                     L->dev_block + L->c.E + 1);
  SLUICE_HIP_CHECK(hipGetLastError());
  if (W.ns > 0) {
    rc = wait_lanes(L, st, &L->copy_ev[kLanes * wave]);
    if (rc) return rc;
  }
  L->plan_in_wave = true;
  return SLUICE_OK;
}

extern "C" int sluice_layer_classic_wave_done(sluice_layer* L, int wave, sluice_stream_t stream) {
  if (L == nullptr || wave < 0) return SLUICE_E_INVAL;
  const int nW = (int)L->plan.waves.size();
  if (wave >= nW || wave != L->plan_next || !L->plan_in_wave) return SLUICE_E_STATE;
  hipStream_t st = (hipStream_t)stream;
  SLUICE_HIP_CHECK(hipEventRecord(L->wave_ev[wave], st));
  L->plan_in_wave = false;
  L->plan_next = wave + 1;
  if (wave + 1 < nW) {
    // Wave w+1's rows go into slots the kernel of wave w-1 (ping-pong: the
    // other group was read by wave w) or of wave w (one group) read last;
    // wave 0 maps every slot it uses, so it is the floor (1893-1913).
    DeviceRes* R = nullptr;
    int rc = device_res(L->device, &R);
    if (rc) return rc;
    const int dep = L->plan.pipelined ? (wave > 0 ? wave - 1 : 0) : wave;
    rc = lanes_wait(L, R, L->wave_ev[dep]);
    if (rc) return rc;
    rc = issue_wave_copies(L, wave + 1, R);
    if (rc) return rc;
    rc = lanes_record(L, R, &L->copy_ev[kLanes * (wave + 1)]);
    if (rc) return rc;
    L->plan_copied = wave + 2;
  }
  return SLUICE_OK;
}

extern "C" int sluice_layer_classic_host(sluice_layer* L, const int32_t* ids, int n, int T, int nd,
                                         int ndec, int real_step, int spec_tokens, int* n_waves) {
  if (L == nullptr || !classic_args_ok(n, T, ids, spec_tokens)) return SLUICE_E_INVAL;
  if (L->server != nullptr) return SLUICE_E_STATE;
  std::lock_guard<std::mutex> lk(L->mu);
  const int rc = L->c.classic(ids, n, T, nd, ndec, real_step != 0, spec_tokens, L->plan);
  L->plan_next = L->plan_copied = (int)L->plan.waves.size();  // nothing to copy on the host
  L->plan_in_wave = false;
  if (rc) return SLUICE_E_STATE;
  ++L->classic_steps;
  L->classic_waves += (int64_t)L->plan.waves.size();
  for (const ParamRows& p : L->params)
    L->bytes += (int64_t)(L->plan.streams.size() / 2) * (int64_t)p.row_bytes;
  if (n_waves) *n_waves = (int)L->plan.waves.size();
  return SLUICE_OK;
}

extern "C" int sluice_layer_classic_plan_read(const sluice_layer* Lc, int32_t* out, int cap,
                                              int* len, int64_t* counters) {
  if (Lc == nullptr) return SLUICE_E_INVAL;
  sluice_layer* L = const_cast<sluice_layer*>(Lc);
  std::lock_guard<std::mutex> lk(L->mu);
  std::vector<int32_t> v;
  serialize_plan(L->plan, v);
  if (len) *len = (int)v.size();
  if (counters) {
    counters[0] = L->classic_steps;
    counters[1] = L->classic_waves;
  }
  if (out == nullptr) return SLUICE_OK;
  if ((int)v.size() > cap) return SLUICE_E_INVAL;
  for (size_t i = 0; i < v.size(); ++i) out[i] = v[i];
  return SLUICE_OK;
}

extern "C" int sluice_layer_set_policy(sluice_layer* L, int lfu, int count_experts) {
  if (L == nullptr) return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> lk(L->mu);
  L->c.lfu = lfu != 0;
  L->c.count = count_experts != 0;
  return SLUICE_OK;
}

extern "C" int sluice_layer_policy_state(const sluice_layer* Lc, int64_t* freq,
                                         int64_t* counts_decode, int64_t* counts_scan,
                                         int64_t* stats) {
  if (Lc == nullptr) return SLUICE_E_INVAL;
  sluice_layer* L = const_cast<sluice_layer*>(Lc);
  std::lock_guard<std::mutex> lk(L->mu);
  const slru::Cache& c = L->c;
  if (freq)
    for (int l = 0; l < c.local_n; ++l) freq[l] = c.freq[l];
  if (counts_decode)
    for (int g = 0; g < c.E; ++g) counts_decode[g] = c.cnt_decode[g];
  if (counts_scan)
    for (int g = 0; g < c.E; ++g) counts_scan[g] = c.cnt_scan[g];
  if (stats) {
    stats[0] = c.steps_small;
    stats[1] = c.steps_scan;
    stats[2] = c.lfu_steps;
  }
  return SLUICE_OK;
}

extern "C" int sluice_layer_step_stats(const sluice_layer* Lc, int64_t* out) {
  if (Lc == nullptr || out == nullptr) return SLUICE_E_INVAL;
  sluice_layer* L = const_cast<sluice_layer*>(Lc);
  std::lock_guard<std::mutex> lk(L->mu);
  const slru::Cache& c = L->c;
  const int64_t steps[2] = {c.steps_small, c.steps_scan};
  for (int k = 0; k < 2; ++k) {
    out[4 * k + 0] = steps[k];
    out[4 * k + 1] = c.cls_hits[k];
    out[4 * k + 2] = c.cls_misses[k];
    out[4 * k + 3] = c.cls_waves[k];
  }
  return SLUICE_OK;
}

extern "C" int sluice_layer_state(const sluice_layer* Lc, int32_t* slot_of, int32_t* expert_in_slot,
                                  int32_t* probation, int* n_probation, int32_t* protected_,
                                  int* n_protected, int32_t* free_slots, int* n_free,
                                  int64_t* counters) {
  if (Lc == nullptr) return SLUICE_E_INVAL;
  sluice_layer* L = const_cast<sluice_layer*>(Lc);
  std::lock_guard<std::mutex> lk(L->mu);
  const slru::Cache& c = L->c;
  if (slot_of)
    for (int l = 0; l < c.local_n; ++l) slot_of[l] = c.slot_of[l];
  if (expert_in_slot)
    for (int s = 0; s < c.S; ++s) expert_in_slot[s] = c.expert_in_slot[s];
  int i = 0;
  for (int s = c.lists[slru::kProbation].head; s >= 0; s = c.next[s], ++i)
    if (probation) probation[i] = s;
  if (n_probation) *n_probation = i;
  i = 0;
  for (int s = c.lists[slru::kProtected].head; s >= 0; s = c.next[s], ++i)
    if (protected_) protected_[i] = s;
  if (n_protected) *n_protected = i;
  if (free_slots)
    for (size_t j = 0; j < c.free_slots.size(); ++j) free_slots[j] = c.free_slots[j];
  if (n_free) *n_free = (int)c.free_slots.size();
  if (counters) {
    counters[0] = c.gaps;
    counters[1] = c.misses;
    counters[2] = c.fast_hits;
    counters[3] = c.map_writes;
    counters[4] = L->bytes & 0xffffffffLL;
    counters[5] = L->bytes >> 32;
    counters[6] = c.map_is_standing ? 1 : 0;
    counters[7] = c.protected_cap;
  }
  return SLUICE_OK;
}

extern "C" int sluice_layer_standing_map(const sluice_layer* Lc, int32_t* map_out) {
  if (Lc == nullptr || map_out == nullptr) return SLUICE_E_INVAL;
  sluice_layer* L = const_cast<sluice_layer*>(Lc);
  std::lock_guard<std::mutex> lk(L->mu);
  L->c.standing_map(map_out);
  return SLUICE_OK;
}

extern "C" int sluice_slot_lookup(const int32_t* ids, int n, const int32_t* expert_map,
                                  const int32_t* local_of, int E, sluice_gap_record* rec,
                                  int32_t stamp, sluice_stream_t stream) {
  if (n < 0 || E <= 0 || E > SLUICE_MAX_EXPERTS || rec == nullptr || (n > 0 && ids == nullptr))
    return SLUICE_E_INVAL;
  hipLaunchKernelGGL(slot_lookup_kernel, dim3(1), dim3(kLookupThreads), 0, (hipStream_t)stream,
                     ids, n, expert_map, local_of, E, rec, stamp);
  return (int)hipGetLastError();
}

extern "C" int sluice_map_refresh(int32_t* expert_map, int E, const int32_t* slot_global, int S,
                                  sluice_stream_t stream) {
  if (expert_map == nullptr || E <= 0 || E > SLUICE_MAX_EXPERTS || S < 0 || S > SLUICE_MAX_SLOTS ||
      (S > 0 && slot_global == nullptr))
    return SLUICE_E_INVAL;
  SlotTable tab;
  tab.n = S;
  for (int s = 0; s < S; ++s) tab.g[s] = slot_global[s];
  hipLaunchKernelGGL(map_refresh_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, expert_map, E,
                     tab, (int32_t*)nullptr);
  return (int)hipGetLastError();
}

extern "C" int sluice_copy_rows(void* const* dst, const void* const* src, const size_t* bytes, int n,
                                sluice_stream_t stream) {
  if (n < 0 || (n > 0 && (dst == nullptr || src == nullptr || bytes == nullptr)))
    return SLUICE_E_INVAL;
  for (int i = 0; i < n; ++i)
    SLUICE_HIP_CHECK(
        hipMemcpyAsync(dst[i], src[i], bytes[i], hipMemcpyHostToDevice, (hipStream_t)stream));
  return SLUICE_OK;
}

extern "C" int sluice_host_alloc(size_t bytes, void** out) {
  if (out == nullptr || bytes == 0) return SLUICE_E_INVAL;
  *out = nullptr;
  const hipError_t e = hipHostMalloc(out, bytes, hipHostMallocPortable);
  if (e != hipSuccess) {
    // the failure is reported here; clear it, or the runtime's sticky last
    // error would be reported again by the caller's next, unrelated call
    (void)hipGetLastError();
    *out = nullptr;
    return (int)e;
  }
  return SLUICE_OK;
}

extern "C" int sluice_host_free(void* p) {
  if (p == nullptr) return SLUICE_OK;
  SLUICE_HIP_CHECK(hipHostFree(p));
  return SLUICE_OK;
}

extern "C" int sluice_abi_version(void) { return SLUICE_ABI_VERSION; }

extern "C" const char* sluice_strerror(int code) {
  switch (code) {
    case SLUICE_OK: return "ok";
    case SLUICE_E_INVAL: return "invalid argument or shape outside kernel limits";
    case SLUICE_E_OVERFLOW:
      return "Sluice router-split: working set exceeds slots on a decode-sized step; raise SLUICE_SLOTS.";
    case SLUICE_E_TIMEOUT: return "a gap wait (host or device) reached its bound";
    case SLUICE_E_NOMEM: return "host allocation failed";
    case SLUICE_E_STATE: return "object used in a state it does not allow";
    case SLUICE_E_ABORTED: return "gap aborted after an earlier error";
    case SLUICE_E_SCRATCH:
      return "the call needs more scratch than sluice_fused_experts_bf16_noalloc holds "
             "(SLUICE_NOALLOC_SCRATCH_BYTES); use sluice_fused_experts_bf16 with a workspace";
    case SLUICE_E_COPY: return "a host-to-device row copy failed to issue or complete";
    default:
      if (code > 0) return hipGetErrorString((hipError_t)code);
      return "unknown sluice error";
  }
}

// ---------------------------------------------------------------------------
// Slot-wait registry: a streaming layer's expert map -> its slot-wait view
// (with its device's bound word, which the kernels read when they wait).
// ---------------------------------------------------------------------------
namespace {
struct WaitEntry {
  const int32_t* map;
  SlotWait w;
};
std::mutex g_wait_mu;
std::vector<WaitEntry> g_wait;
}  // namespace

void slotwait_register(const int32_t* map, const SlotWait& w) {
  std::lock_guard<std::mutex> lk(g_wait_mu);
  for (auto& e : g_wait)
    if (e.map == map) {
      e.w = w;
      return;
    }
  g_wait.push_back({map, w});
}

void slotwait_unregister(const int32_t* map) {
  std::lock_guard<std::mutex> lk(g_wait_mu);
  for (size_t i = 0; i < g_wait.size(); ++i)
    if (g_wait[i].map == map) {
      g_wait.erase(g_wait.begin() + (long)i);
      return;
    }
}

SlotWait slotwait_lookup(const int32_t* map) {
  std::lock_guard<std::mutex> lk(g_wait_mu);
  for (const auto& e : g_wait)
    if (e.map == map) return e.w;
  return SlotWait{};
}

// ---------------------------------------------------------------------------
// Gap timeline tracing (trace.h): the entry points of a -DSLUICE_TRACE build;
// SLUICE_E_STATE otherwise.
// ---------------------------------------------------------------------------
int trace_moe_read(unsigned long long* out, unsigned* n);  // moe.hip
int trace_moe_reset();

namespace {
#ifdef SLUICE_TRACE
// One thread writes its wall clock into mapped host memory every ~20 us; the
// host notes when each value appears.  The smallest host - device difference
// bounds the clocks' offset (to within the bus latency).
__global__ void trace_calib_kernel(unsigned long long* slot, int n) {
  for (int i = 0; i < n; ++i) {
    const unsigned long long t = wall_clock64();
    __hip_atomic_store(slot, ((unsigned long long)(i + 1) << 48) | (t & ((1ull << 48) - 1)),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const long long t0 = wall_clock64();
    while (wall_clock64() - t0 < 2000) __builtin_amdgcn_s_sleep(8);
  }
}
#endif
}  // namespace

extern "C" int sluice_trace_calibrate(int n, double* host_s, unsigned long long* dev_ticks) {
#ifdef SLUICE_TRACE
  if (n <= 0 || n > 100000 || host_s == nullptr || dev_ticks == nullptr) return SLUICE_E_INVAL;
  void* p = nullptr;
  SLUICE_HIP_CHECK(hipHostMalloc(&p, 256, hipHostMallocCoherent | hipHostMallocMapped));
  volatile unsigned long long* h = static_cast<volatile unsigned long long*>(p);
  *h = 0;
  void* dp = nullptr;
  hipStream_t st = nullptr;
  hipError_t e = hipHostGetDevicePointer(&dp, p, 0);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
  if (e != hipSuccess) {
    (void)hipHostFree(p);
    return (int)e;
  }
  hipLaunchKernelGGL(trace_calib_kernel, dim3(1), dim3(1), 0, st, (unsigned long long*)dp, n);
  int seen = 0;
  const double t0 = now_s();
  while (seen < n && now_s() - t0 < 10.0) {
    const unsigned long long v = *h;
    const int i = (int)(v >> 48);
    if (i > seen) {
      const double t = now_s();
      for (int j = seen; j < i - 1; ++j) {
        host_s[j] = -1.0;
        dev_ticks[j] = 0;
      }
      host_s[i - 1] = t;
      dev_ticks[i - 1] = v & ((1ull << 48) - 1);
      seen = i;
    }
  }
  e = hipStreamSynchronize(st);
  (void)hipStreamDestroy(st);
  (void)hipHostFree(p);
  return e != hipSuccess ? (int)e : seen;
#else
  (void)n;
  (void)host_s;
  (void)dev_ticks;
  return SLUICE_E_STATE;
#endif
}

extern "C" int sluice_trace_read(int which, void* out, unsigned* n) {
#ifdef SLUICE_TRACE
  if (n == nullptr) return SLUICE_E_INVAL;
  if (which == 0) return trace_dev_read(static_cast<unsigned long long*>(out), n);
  if (which == 1) return trace_moe_read(static_cast<unsigned long long*>(out), n);
  if (which == 2) {
    *n = g_trace_host_n.load();
    if (out != nullptr) memcpy(out, g_trace_host, sizeof(g_trace_host));
    return SLUICE_OK;
  }
  return SLUICE_E_INVAL;
#else
  (void)which;
  (void)out;
  (void)n;
  return SLUICE_E_STATE;
#endif
}

extern "C" int sluice_trace_reset(void) {
#ifdef SLUICE_TRACE
  int rc = trace_dev_reset();
  if (rc == SLUICE_OK) rc = trace_moe_reset();
  g_trace_host_n.store(0);
  return rc;
#else
  return SLUICE_E_STATE;
#endif
}
