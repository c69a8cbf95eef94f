// Host side of the host store codec (codec.h): the encoder, run when a
// layer's store is coded, and the dispatch of decode jobs.
//
// The decode kernel (codec_kernel.hip) is built into its own code object,
// sluice_amd/codec_decode.hsaco, loaded here with the HSA loader and
// dispatched as AQL packets on a queue the library creates per device.  The
// jobs decode rows that an expert product may be waiting for; a HIP stream
// could share an in-order hardware queue with that product (HIP pools its
// queues once a process has more streams than GPU_MAX_HW_QUEUES) or, if it
// blocked, wait on the null stream's work, and the decode would then never
// start.  A queue of the library's own shares nothing.
#include <dlfcn.h>
#include <immintrin.h>
#include <stdio.h>
#include <string.h>
#include <time.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include <hsa/hsa_ext_amd.h>

#include "codec.h"
#include "common.h"

namespace {

// The first exponent of the window of kCodecWindow binades that holds most
// of the chunk's values other than zeros and subnormals (exponent 0, coded
// kCodecZero; the lowest such start on ties).
int chunk_base(const uint16_t* v) {
  uint32_t h[256] = {};
  for (size_t i = 0; i < kCodecChunk; ++i) ++h[(v[i] >> 7) & 0xff];
  h[0] = 0;
  uint32_t win = 0;
  for (int e = 0; e < (int)kCodecWindow; ++e) win += h[e];
  uint32_t best = win;
  int base = 0;
  for (int b = 1; b + (int)kCodecWindow <= 256; ++b) {
    win += h[b + kCodecWindow - 1] - h[b - 1];
    if (win > best) {
      best = win;
      base = b;
    }
  }
  return base;
}

double now_s() {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

}  // namespace

size_t codec_coded_bytes(const uint16_t* v, size_t n) {
  size_t esc = 0;
  for (size_t c = 0; c < n / kCodecChunk; ++c) {
    const uint16_t* x = v + c * kCodecChunk;
    const int b = chunk_base(x);
    for (size_t i = 0; i < kCodecChunk; ++i) {
      const uint32_t e = (x[i] >> 7) & 0xffu;
      esc += e != 0 && e - (uint32_t)b >= kCodecWindow;
    }
  }
  return codec_esc_off(n) + 4 * esc;
}

size_t codec_encode(const uint16_t* v, size_t n, uint8_t* out) {
  const size_t nc = n / kCodecChunk;
  uint8_t* sm = out;
  uint8_t* nib = out + n;
  uint8_t* base = out + codec_base_off(n);
  uint32_t* off = reinterpret_cast<uint32_t*>(out + codec_esc_off_off(n));
  uint32_t* esc = reinterpret_cast<uint32_t*>(out + codec_esc_off(n));
  memset(base + nc, 0, codec_pad4(nc) - nc);
  uint32_t ne = 0;
  for (size_t c = 0; c < nc; ++c) {
    const uint16_t* x = v + c * kCodecChunk;
    const int b = chunk_base(x);
    base[c] = (uint8_t)b;
    off[c] = ne;
    for (size_t i = 0; i < kCodecChunk; i += 2) {
      uint32_t code[2];
      for (int h = 0; h < 2; ++h) {
        const uint32_t w = x[i + h], e = (w >> 7) & 0xffu;
        sm[c * kCodecChunk + i + h] = (uint8_t)(((w >> 8) & 0x80u) | (w & 0x7fu));
        const uint32_t d = e - (uint32_t)b;
        code[h] = e == 0 ? kCodecZero : d < kCodecWindow ? d : kCodecEscape;
        if (code[h] == kCodecEscape) esc[ne++] = (uint32_t)(i + h) << 8 | e;
      }
      nib[(c * kCodecChunk + i) / 2] = (uint8_t)(code[0] | code[1] << 4);
    }
  }
  off[nc] = ne;
  return codec_esc_off(n) + 4 * (size_t)ne;
}

// ---------------------------------------------------------------------------
// Dispatch.
// ---------------------------------------------------------------------------
constexpr uint32_t kQueueSize = 1024;  // packets
constexpr int kArgSlots = 256;         // kernel-argument buffers, reused in turn
constexpr size_t kArgBytes = 256;      // per buffer (the job; checked against the code object)

struct CodecQueue {
  std::mutex mu;
  hsa_queue_t* q = nullptr;
  hsa_executable_t exe{};
  uint64_t kernel = 0;
  uint32_t kernarg_bytes = 0, group_bytes = 0, private_bytes = 0;
  char* args = nullptr;          // kArgSlots x kArgBytes, host memory the GPU reads
  hsa_signal_t sig[kArgSlots];   // completion of the job that last used each buffer
  uint64_t n = 0;                // jobs dispatched
  std::atomic<int> error{0};     // a queue error the runtime reported
};

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
CodecQueue* g_queue[kMaxDevices] = {};

void on_queue_error(hsa_status_t st, hsa_queue_t*, void* data) {
  static_cast<CodecQueue*>(data)->error.store(st == HSA_STATUS_SUCCESS ? SLUICE_E_COPY : (int)st);
}

hsa_status_t kernarg_pool(hsa_amd_memory_pool_t pool, void* data) {
  hsa_amd_segment_t seg;
  if (hsa_amd_memory_pool_get_info(pool, HSA_AMD_MEMORY_POOL_INFO_SEGMENT, &seg) !=
          HSA_STATUS_SUCCESS ||
      seg != HSA_AMD_SEGMENT_GLOBAL)
    return HSA_STATUS_SUCCESS;
  uint32_t flags = 0;
  if (hsa_amd_memory_pool_get_info(pool, HSA_AMD_MEMORY_POOL_INFO_GLOBAL_FLAGS, &flags) !=
      HSA_STATUS_SUCCESS)
    return HSA_STATUS_SUCCESS;
  if ((flags & HSA_AMD_MEMORY_POOL_GLOBAL_FLAG_KERNARG_INIT) == 0) return HSA_STATUS_SUCCESS;
  *static_cast<hsa_amd_memory_pool_t*>(data) = pool;
  return HSA_STATUS_INFO_BREAK;
}

// The code object beside this library: <dir of libsluice_hip*.so>/codec_decode.hsaco.
std::string code_object_path() {
  Dl_info info{};
  if (dladdr(reinterpret_cast<void*>(&code_object_path), &info) == 0 || info.dli_fname == nullptr)
    return "";
  std::string p = info.dli_fname;
  const size_t slash = p.rfind('/');
  return (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) +
         "/codec_decode.hsaco";
}

int open_queue(hsa_agent_t gpu, hsa_agent_t cpu, CodecQueue* Q) {
  const std::string path = code_object_path();
  FILE* f = path.empty() ? nullptr : fopen(path.c_str(), "rb");
  if (f == nullptr) return SLUICE_E_STATE;  // not built
  std::vector<char> blob;
  char buf[1 << 16];
  for (size_t r; (r = fread(buf, 1, sizeof(buf), f)) > 0;) blob.insert(blob.end(), buf, buf + r);
  fclose(f);
  hsa_code_object_reader_t reader{};
  if (hsa_code_object_reader_create_from_memory(blob.data(), blob.size(), &reader) !=
      HSA_STATUS_SUCCESS)
    return SLUICE_E_STATE;
  hsa_status_t st = hsa_executable_create_alt(HSA_PROFILE_FULL,
                                              HSA_DEFAULT_FLOAT_ROUNDING_MODE_DEFAULT, nullptr,
                                              &Q->exe);
  if (st == HSA_STATUS_SUCCESS)
    st = hsa_executable_load_agent_code_object(Q->exe, gpu, reader, nullptr, nullptr);
  if (st == HSA_STATUS_SUCCESS) st = hsa_executable_freeze(Q->exe, nullptr);
  (void)hsa_code_object_reader_destroy(reader);
  hsa_executable_symbol_t sym{};
  if (st == HSA_STATUS_SUCCESS)
    st = hsa_executable_get_symbol_by_name(Q->exe, "sluice_codec_decode_kernel.kd", &gpu, &sym);
  if (st == HSA_STATUS_SUCCESS)
    st = hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT,
                                        &Q->kernel);
  if (st == HSA_STATUS_SUCCESS)
    st = hsa_executable_symbol_get_info(
        sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_KERNARG_SEGMENT_SIZE, &Q->kernarg_bytes);
  if (st == HSA_STATUS_SUCCESS)
    st = hsa_executable_symbol_get_info(
        sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE, &Q->group_bytes);
  if (st == HSA_STATUS_SUCCESS)
    st = hsa_executable_symbol_get_info(
        sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE, &Q->private_bytes);
  if (st != HSA_STATUS_SUCCESS) return SLUICE_E_STATE;
  // the kernel reads exactly the job (no implicit arguments), and no stack
  if (Q->kernarg_bytes != sizeof(CodecJob) || Q->kernarg_bytes > kArgBytes ||
      Q->private_bytes != 0)
    return SLUICE_E_STATE;
  hsa_amd_memory_pool_t pool{};
  st = hsa_amd_agent_iterate_memory_pools(cpu, kernarg_pool, &pool);
  if ((st != HSA_STATUS_SUCCESS && st != HSA_STATUS_INFO_BREAK) || pool.handle == 0)
    return SLUICE_E_STATE;
  void* args = nullptr;
  if (hsa_amd_memory_pool_allocate(pool, kArgSlots * kArgBytes, 0, &args) != HSA_STATUS_SUCCESS)
    return SLUICE_E_NOMEM;
  Q->args = static_cast<char*>(args);
  memset(Q->args, 0, kArgSlots * kArgBytes);
  if (hsa_amd_agents_allow_access(1, &gpu, nullptr, args) != HSA_STATUS_SUCCESS)
    return SLUICE_E_STATE;
  for (hsa_signal_t& s : Q->sig)
    if (hsa_signal_create(0, 0, nullptr, &s) != HSA_STATUS_SUCCESS) return SLUICE_E_NOMEM;
  // default priority, one producer (Q->mu)
  if (hsa_queue_create(gpu, kQueueSize, HSA_QUEUE_TYPE_SINGLE, on_queue_error, Q, UINT32_MAX,
                       UINT32_MAX, &Q->q) != HSA_STATUS_SUCCESS)
    return SLUICE_E_STATE;
  return SLUICE_OK;
}

// Wait (bounded) for a completion signal to reach 0.
int wait_zero(hsa_signal_t s, double timeout_s, const CodecQueue* Q) {
  const double t0 = now_s();
  unsigned spins = 0;
  while (hsa_signal_load_scacquire(s) > 0) {
    _mm_pause();
    if ((++spins & 1023u) == 0) {
      if (Q->error.load() != 0) return Q->error.load();
      if (now_s() - t0 > timeout_s) return SLUICE_E_TIMEOUT;
    }
  }
  return SLUICE_OK;
}

constexpr double kArgWaitS = 20.0;

}  // namespace

int codec_queue(int device, hsa_agent_t gpu, hsa_agent_t cpu, CodecQueue** out) {
  if (device < 0 || device >= kMaxDevices || out == nullptr) return SLUICE_E_INVAL;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_queue[device] == nullptr) {
    CodecQueue* Q = new CodecQueue();
    const int rc = open_queue(gpu, cpu, Q);
    if (rc != SLUICE_OK) {
      // what was set up stays with the process (a failed set-up is rare and
      // leaves nothing the GPU still reads)
      return rc;
    }
    g_queue[device] = Q;
  }
  *out = g_queue[device];
  return SLUICE_OK;
}

int codec_dispatch(CodecQueue* Q, CodecJob& job) {
  size_t total = 0;
  for (int p = 0; p < job.n_part; ++p) total += job.part[p].n_chunk;
  if (Q == nullptr || job.n_part <= 0 || job.n_part > kCodecMaxParts || total == 0 ||
      total > 0xffffffffu || job.wg_count == nullptr)
    return SLUICE_E_INVAL;
  // a workgroup decodes 4 chunks per round
  job.n_wg = (uint32_t)std::min<size_t>((total + 3) / 4, kCodecMaxGrid);
  std::lock_guard<std::mutex> lk(Q->mu);
  if (Q->error.load() != 0) return Q->error.load();
  const int slot = (int)(Q->n % kArgSlots);
  // the buffer's last job has completed (it was dispatched kArgSlots jobs ago)
  int rc = wait_zero(Q->sig[slot], kArgWaitS, Q);
  if (rc != SLUICE_OK) return rc;
  hsa_queue_t* q = Q->q;
  // one producer (Q->mu): take the next packet slot once the packet
  // processor has consumed what lay there
  const uint64_t idx = hsa_queue_load_write_index_relaxed(q);
  const double t0 = now_s();
  while (idx - hsa_queue_load_read_index_scacquire(q) >= q->size) {
    _mm_pause();
    if (now_s() - t0 > kArgWaitS) return SLUICE_E_TIMEOUT;
  }
  char* args = Q->args + (size_t)slot * kArgBytes;
  memcpy(args, &job, sizeof(CodecJob));
  hsa_signal_store_relaxed(Q->sig[slot], 1);
  hsa_queue_store_write_index_relaxed(q, idx + 1);
  hsa_kernel_dispatch_packet_t* pkt =
      static_cast<hsa_kernel_dispatch_packet_t*>(q->base_address) + (idx & (q->size - 1));
  const uint16_t setup = 1u << HSA_KERNEL_DISPATCH_PACKET_SETUP_DIMENSIONS;
  pkt->workgroup_size_x = (uint16_t)kCodecThreads;
  pkt->workgroup_size_y = 1;
  pkt->workgroup_size_z = 1;
  pkt->reserved0 = 0;
  pkt->grid_size_x = job.n_wg * (uint32_t)kCodecThreads;
  pkt->grid_size_y = 1;
  pkt->grid_size_z = 1;
  pkt->private_segment_size = Q->private_bytes;
  pkt->group_segment_size = Q->group_bytes;
  pkt->kernel_object = Q->kernel;
  pkt->kernarg_address = args;
  pkt->reserved2 = 0;
  pkt->completion_signal = Q->sig[slot];
  // One job after the other (barrier bit: a job's last workgroup resets the
  // shared workgroup counter); system-scope fences: the rows were written
  // by SDMA engines, and the host reads the marks.
  const uint16_t header =
      (HSA_PACKET_TYPE_KERNEL_DISPATCH << HSA_PACKET_HEADER_TYPE) |
      (1u << HSA_PACKET_HEADER_BARRIER) |
      (HSA_FENCE_SCOPE_SYSTEM << HSA_PACKET_HEADER_SCACQUIRE_FENCE_SCOPE) |
      (HSA_FENCE_SCOPE_SYSTEM << HSA_PACKET_HEADER_SCRELEASE_FENCE_SCOPE);
  __atomic_store_n(reinterpret_cast<uint32_t*>(pkt), (uint32_t)header | ((uint32_t)setup << 16),
                   __ATOMIC_RELEASE);
  hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)idx);
  ++Q->n;
  return rc;
}

int codec_sync(CodecQueue* Q, double timeout_s) {
  if (Q == nullptr) return SLUICE_OK;
  std::lock_guard<std::mutex> lk(Q->mu);
  for (hsa_signal_t s : Q->sig) {
    const int rc = wait_zero(s, timeout_s, Q);
    if (rc != SLUICE_OK) return rc;
  }
  return Q->error.load();
}

namespace {
hsa_status_t first_cpu(hsa_agent_t a, void* data) {
  hsa_device_type_t t;
  if (hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS ||
      t != HSA_DEVICE_TYPE_CPU)
    return HSA_STATUS_SUCCESS;
  *static_cast<hsa_agent_t*>(data) = a;
  return HSA_STATUS_INFO_BREAK;
}
}  // namespace

extern "C" int sluice_codec_encode(const void* rows, size_t n, void* out, size_t cap,
                                   size_t* coded_bytes) {
  if (rows == nullptr || coded_bytes == nullptr || n == 0 || n % kCodecChunk != 0 ||
      ((uintptr_t)rows & 1) != 0 || ((uintptr_t)out & 3) != 0)
    return SLUICE_E_INVAL;
  const size_t need = codec_coded_bytes(static_cast<const uint16_t*>(rows), n);
  *coded_bytes = need;
  if (out == nullptr) return SLUICE_OK;
  if (cap < need) return SLUICE_E_INVAL;
  codec_encode(static_cast<const uint16_t*>(rows), n, static_cast<uint8_t*>(out));
  return SLUICE_OK;
}

extern "C" int sluice_codec_decode(const void* coded_dev, size_t n, size_t coded_bytes,
                                   void* out_dev, sluice_stream_t stream) {
  if (coded_dev == nullptr || out_dev == nullptr || n == 0 || n % kCodecChunk != 0 ||
      n / kCodecChunk > 0xffffffffu || coded_bytes < codec_esc_off(n) ||
      (coded_bytes - codec_esc_off(n)) % 4 != 0 || ((uintptr_t)coded_dev & 15) != 0 ||
      ((uintptr_t)out_dev & 15) != 0)
    return SLUICE_E_INVAL;
  int dev = 0;
  SLUICE_HIP_CHECK(hipGetDevice(&dev));
  if (hsa_init() != HSA_STATUS_SUCCESS) return SLUICE_E_COPY;  // counted: HIP holds one too
  hsa_amd_pointer_info_t info;
  memset(&info, 0, sizeof(info));
  info.size = sizeof(info);
  hsa_agent_t cpu{};
  const hsa_status_t it = hsa_iterate_agents(first_cpu, &cpu);
  if (hsa_amd_pointer_info(out_dev, &info, nullptr, nullptr, nullptr) != HSA_STATUS_SUCCESS ||
      info.type == HSA_EXT_POINTER_TYPE_UNKNOWN || cpu.handle == 0 ||
      (it != HSA_STATUS_SUCCESS && it != HSA_STATUS_INFO_BREAK))
    return SLUICE_E_INVAL;
  CodecQueue* Q = nullptr;
  int rc = codec_queue(dev, info.agentOwner, cpu, &Q);
  if (rc != SLUICE_OK) return rc;
  // the rows are read after the stream's work so far
  SLUICE_HIP_CHECK(hipStreamSynchronize((hipStream_t)stream));
  uint32_t* count = nullptr;
  SLUICE_HIP_CHECK(hipMalloc((void**)&count, sizeof(uint32_t)));
  rc = (int)hipMemset(count, 0, sizeof(uint32_t));
  if (rc == SLUICE_OK) rc = (int)hipDeviceSynchronize();
  if (rc == SLUICE_OK) {
    CodecJob job{};
    job.part[0] = {static_cast<const uint8_t*>(coded_dev), static_cast<uint16_t*>(out_dev),
                   (uint32_t)(n / kCodecChunk), codec_escapes(n, coded_bytes)};
    job.n_part = 1;
    job.wg_count = count;
    rc = codec_dispatch(Q, job);
    const int s = codec_sync(Q, 60.0);
    if (rc == SLUICE_OK) rc = s;
  }
  const hipError_t f = hipFree(count);
  if (rc == SLUICE_OK) rc = (int)f;
  return rc;
}
