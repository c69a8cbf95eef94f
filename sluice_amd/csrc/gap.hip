// a3-a8: the streaming gap on MI355X.
//
//   slot_lookup_kernel   ids -> sorted unique selected ids + miss count,
//                        published straight into host-mapped pinned memory
//                        (replaces topk_ids.to("cpu") + sorted(set(ids)),
//                        src/sluice/offloader.py:2406, 2427).
//   map_refresh_kernel   standing expert map from an S-entry table passed as
//                        a kernel argument (replaces _write_map's pinned
//                        staging + map_ev wait, offloader.py:2083-2123).
//   sluice_layer_*       the per-layer slot cache (slru::Cache) plus the gap
//                        driver: wait for the record, SLRU bookkeeping,
//                        hipMemcpyAsync of missing expert rows on a dedicated
//                        copy stream fenced by events both ways
//                        (offloader.py:2443-2464, 1979-1991, 2709-2723).
#include <immintrin.h>
#include <stdlib.h>
#include <time.h>

#include <mutex>
#include <vector>

#include "common.h"
#include "slru.h"

namespace {

constexpr int kLookupThreads = 256;

__global__ __launch_bounds__(kLookupThreads) void slot_lookup_kernel(
    const int32_t* __restrict__ ids, int n, const int32_t* __restrict__ map,
    const int32_t* __restrict__ local_of, int E, sluice_gap_record* rec,
    int32_t stamp) {
  __shared__ int present[SLUICE_MAX_EXPERTS];
  __shared__ int wcount[kLookupThreads / SLUICE_WAVE];
  __shared__ int wmiss[kLookupThreads / SLUICE_WAVE];
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
    for (int w = 0; w < kLookupThreads / SLUICE_WAVE; ++w) {
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

__global__ __launch_bounds__(256) void map_refresh_kernel(int32_t* __restrict__ map, int E,
                                                          SlotTable tab) {
  __shared__ int m[SLUICE_MAX_EXPERTS];
  for (int e = threadIdx.x; e < E; e += 256) m[e] = -1;
  __syncthreads();
  for (int s = threadIdx.x; s < tab.n; s += 256) {
    const int g = tab.g[s];
    if ((unsigned)g < (unsigned)E) m[g] = s;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) map[e] = m[e];
}

// Per-device resources shared by every layer: one copy stream (default
// priority) and the two fencing events.
struct DeviceRes {
  hipStream_t copy = nullptr;
  hipEvent_t ev_compute = nullptr;
  hipEvent_t ev_copy = nullptr;
};
constexpr int kMaxDevices = 64;
DeviceRes g_dev[kMaxDevices];
std::mutex g_dev_mu;

int device_res(int dev, DeviceRes** out) {
  if (dev < 0 || dev >= kMaxDevices) return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> lk(g_dev_mu);
  DeviceRes& r = g_dev[dev];
  if (r.copy == nullptr) {
    SLUICE_HIP_CHECK(hipStreamCreateWithFlags(&r.copy, hipStreamNonBlocking));
    SLUICE_HIP_CHECK(hipEventCreateWithFlags(&r.ev_compute, hipEventDisableTiming));
    SLUICE_HIP_CHECK(hipEventCreateWithFlags(&r.ev_copy, hipEventDisableTiming));
  }
  *out = &r;
  return SLUICE_OK;
}

double now_s() {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

double gap_timeout_s() {
  static double v = [] {
    const char* s = getenv("SLUICE_GAP_TIMEOUT_S");
    double t = s ? atof(s) : 60.0;
    return t > 0 ? t : 60.0;
  }();
  return v;
}

}  // namespace

struct ParamRows {
  char* slot_base;
  const char* host_base;
  size_t row_bytes;
};

struct sluice_layer {
  slru::Cache c;
  int32_t* map_dev = nullptr;
  std::vector<ParamRows> params;
  int device = -1;
  sluice_gap_record* rec = nullptr;  // host pointer (pinned, coherent, mapped)
  sluice_gap_record* rec_dev = nullptr;
  int32_t* local_of_dev = nullptr;
  int32_t stamp = 0;
  int64_t bytes = 0;
  std::vector<int> streams;
  std::vector<int32_t> table;
};

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
  L->table.assign(num_slots, -1);
  *out = L;
  return SLUICE_OK;
}

extern "C" int sluice_layer_destroy(sluice_layer* L) {
  if (L == nullptr) return SLUICE_OK;
  int rc = SLUICE_OK;
  if (L->rec != nullptr) {
    hipError_t e = hipHostFree(L->rec);
    if (e != hipSuccess) rc = (int)e;
  }
  if (L->local_of_dev != nullptr) {
    hipError_t e = hipFree(L->local_of_dev);
    if (e != hipSuccess) rc = (int)e;
  }
  delete L;
  return rc;
}

extern "C" int sluice_layer_add_param(sluice_layer* L, void* slot_base_dev, const void* host_base,
                                      size_t row_bytes) {
  if (L == nullptr || slot_base_dev == nullptr || host_base == nullptr || row_bytes == 0)
    return SLUICE_E_INVAL;
  L->params.push_back({(char*)slot_base_dev, (const char*)host_base, row_bytes});
  return SLUICE_OK;
}

extern "C" int sluice_layer_pin(sluice_layer* L, int local, int debit_protected, int* slot_out) {
  if (L == nullptr) return SLUICE_E_INVAL;
  const int s = L->c.pin(local, debit_protected != 0);
  if (slot_out) *slot_out = s;
  return s < 0 ? SLUICE_E_STATE : SLUICE_OK;
}

static int layer_device_init(sluice_layer* L) {
  if (L->rec != nullptr) return SLUICE_OK;
  SLUICE_HIP_CHECK(hipGetDevice(&L->device));
  void* p = nullptr;
  SLUICE_HIP_CHECK(hipHostMalloc(&p, sizeof(sluice_gap_record),
                                 hipHostMallocCoherent | hipHostMallocMapped));
  L->rec = (sluice_gap_record*)p;
  L->rec->stamp = 0;
  void* dp = nullptr;
  SLUICE_HIP_CHECK(hipHostGetDevicePointer(&dp, p, 0));
  L->rec_dev = (sluice_gap_record*)dp;
  SLUICE_HIP_CHECK(hipMalloc((void**)&L->local_of_dev, sizeof(int32_t) * L->c.E));
  std::vector<int32_t> lof(L->c.local_of.begin(), L->c.local_of.end());
  SLUICE_HIP_CHECK(hipMemcpy(L->local_of_dev, lof.data(), sizeof(int32_t) * L->c.E,
                             hipMemcpyHostToDevice));
  return SLUICE_OK;
}

extern "C" int sluice_layer_gap(sluice_layer* L, const int32_t* topk_ids, int n, int fast_hit,
                                sluice_stream_t compute) {
  if (L == nullptr || n < 0 || (n > 0 && topk_ids == nullptr)) return SLUICE_E_INVAL;
  if (L->map_dev == nullptr) return SLUICE_E_STATE;
  int rc = layer_device_init(L);
  if (rc) return rc;
  hipStream_t cs = (hipStream_t)compute;

  // 1. publish the step's selection into the host record.
  int32_t stamp = L->stamp + 1;
  if (stamp <= 0) stamp = 1;
  L->stamp = stamp;
  hipLaunchKernelGGL(slot_lookup_kernel, dim3(1), dim3(kLookupThreads), 0, cs, topk_ids, n,
                     L->map_dev, L->local_of_dev, L->c.E, L->rec_dev, stamp);
  SLUICE_HIP_CHECK(hipGetLastError());

  // 2. wait for it (bounded; the exactness anchor of the gap).
  volatile int32_t* sp = &L->rec->stamp;
  if (*sp != stamp) {
    const double t0 = now_s();
    unsigned spins = 0;
    while (__atomic_load_n((const int32_t*)sp, __ATOMIC_ACQUIRE) != stamp) {
      _mm_pause();
      if ((++spins & 4095u) == 0) {
        hipError_t q = hipStreamQuery(cs);
        if (q != hipSuccess && q != hipErrorNotReady) return (int)q;
        if (now_s() - t0 > gap_timeout_s()) return SLUICE_E_TIMEOUT;
      }
    }
  }
  __atomic_thread_fence(__ATOMIC_ACQUIRE);
  const int n_uniq = L->rec->n_uniq;
  if (n_uniq < 0 || n_uniq > L->c.E) return SLUICE_E_STATE;

  // 3. bookkeeping.
  L->streams.clear();
  bool map_write = false;
  const int grc = L->c.gap(L->rec->uniq, n_uniq, fast_hit != 0, L->streams, map_write);

  // 4. stream misses: copy stream waits for compute (the previous step's
  //    GEMM may still read a victim slot), then compute waits for the copies.
  const int n_streams = (int)L->streams.size() / 2;
  if (n_streams > 0) {
    DeviceRes* R = nullptr;
    rc = device_res(L->device, &R);
    if (rc) return rc;
    SLUICE_HIP_CHECK(hipEventRecord(R->ev_compute, cs));
    SLUICE_HIP_CHECK(hipStreamWaitEvent(R->copy, R->ev_compute, 0));
    for (int i = 0; i < n_streams; ++i) {
      const int local = L->streams[2 * i], slot = L->streams[2 * i + 1];
      for (const ParamRows& p : L->params) {
        SLUICE_HIP_CHECK(hipMemcpyAsync(p.slot_base + (size_t)slot * p.row_bytes,
                                        p.host_base + (size_t)local * p.row_bytes, p.row_bytes,
                                        hipMemcpyHostToDevice, R->copy));
        L->bytes += (int64_t)p.row_bytes;
      }
    }
    if (grc != 0) return grc;  // overflow: the reference raises before the compute wait
    SLUICE_HIP_CHECK(hipEventRecord(R->ev_copy, R->copy));
    SLUICE_HIP_CHECK(hipStreamWaitEvent(cs, R->ev_copy, 0));
  } else if (grc != 0) {
    return grc;
  }

  // 5. standing map.
  if (map_write) {
    SlotTable tab;
    tab.n = L->c.S;
    L->c.slot_globals(tab.g);
    hipLaunchKernelGGL(map_refresh_kernel, dim3(1), dim3(256), 0, cs, L->map_dev, L->c.E, tab);
    SLUICE_HIP_CHECK(hipGetLastError());
  }
  return SLUICE_OK;
}

extern "C" int sluice_layer_gap_host(sluice_layer* L, const int32_t* ids, int n, int fast_hit,
                                     int32_t* streams, int max_streams, int* n_streams,
                                     int* map_written) {
  if (L == nullptr || n < 0 || (n > 0 && ids == nullptr)) return SLUICE_E_INVAL;
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

extern "C" int sluice_layer_state(const sluice_layer* L, int32_t* slot_of, int32_t* expert_in_slot,
                                  int32_t* probation, int* n_probation, int32_t* protected_,
                                  int* n_protected, int32_t* free_slots, int* n_free,
                                  int64_t* counters) {
  if (L == nullptr) return SLUICE_E_INVAL;
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

extern "C" int sluice_layer_standing_map(const sluice_layer* L, int32_t* map_out) {
  if (L == nullptr || map_out == nullptr) return SLUICE_E_INVAL;
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
                     tab);
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
  SLUICE_HIP_CHECK(hipHostMalloc(out, bytes, hipHostMallocPortable));
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
    case SLUICE_E_TIMEOUT: return "timed out waiting for the device slot-lookup record";
    case SLUICE_E_NOMEM: return "host allocation failed";
    case SLUICE_E_STATE: return "object used in a state it does not allow";
    default:
      if (code > 0) return hipGetErrorString((hipError_t)code);
      return "unknown sluice error";
  }
}
