// Lossless coding of a host store's bf16 rows (internal to libsluice_hip).
//
// The streamed gap is bound by the host link once its idle time is filled,
// so bytes that do not cross it are time saved.  A bf16 weight is sign (1),
// exponent (8) and mantissa (7) bits; the mantissa and sign carry close to
// 8 bits of information, the exponent of a weight matrix far fewer (2.5 bits
// for N(0, 0.02) values: nearly all lie within 14 consecutive binades).  A
// coded row keeps sign and mantissa whole and each exponent as a 4-bit
// code: its offset from a base chosen per chunk of kCodecChunk values (0 to
// 13), 14 for exponent 0 (zeros and subnormals), or 15 for an exponent
// outside [base, base + 13], kept in the chunk's escape list.  12 bits per
// value (0.75 of the row) plus the escapes; decoding gives the row's bytes
// back exactly.
//
// Layout of a coded row of n values (n a multiple of kCodecChunk, nc =
// n / kCodecChunk chunks):
//   [0, n)                 sm[i]  = sign(i) << 7 | mantissa(i)
//   [n, 1.5 n)             nib: value 2j in the low nibble of byte j, 2j+1 high
//   [1.5 n, +pad4(nc))     base exponent of each chunk
//   then (nc + 1) uint32   escape offsets: chunk c's escapes are [off[c], off[c+1])
//   then uint32 escapes    position in the chunk << 8 | exponent, ascending
#pragma once

#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <stddef.h>
#include <stdint.h>

constexpr size_t kCodecChunk = 2048;   // values per base exponent
constexpr int kCodecMaxParts = 4;      // coded rows one decode job writes
constexpr uint32_t kCodecWindow = 14;  // binades a chunk's base starts
constexpr uint32_t kCodecZero = 14;    // nibble of exponent 0 (zeros, subnormals)
constexpr uint32_t kCodecEscape = 15;  // nibble of an exponent outside the window
constexpr int kCodecThreads = 256;     // threads of a decode workgroup
constexpr uint32_t kCodecMaxGrid = 512;

__host__ __device__ inline size_t codec_pad4(size_t v) { return (v + 3) & ~(size_t)3; }
__host__ __device__ inline size_t codec_base_off(size_t n) { return n + n / 2; }
__host__ __device__ inline size_t codec_esc_off_off(size_t n) {
  return codec_base_off(n) + codec_pad4(n / kCodecChunk);
}
__host__ __device__ inline size_t codec_esc_off(size_t n) {
  return codec_esc_off_off(n) + 4 * (n / kCodecChunk + 1);
}

// One row to decode: n_chunk chunks of kCodecChunk values from src (a coded
// row in device memory holding n_esc escapes) to dst (n_chunk *
// kCodecChunk bf16 values).
struct CodecPart {
  const uint8_t* src;
  uint16_t* dst;
  uint32_t n_chunk;
  uint32_t n_esc;
};

// A decode job over n_wg workgroups: its parts, then (after every
// workgroup's stores) the last workgroup releases `stamp` into *ready
// (host-mapped; nullptr: none) and `seq` into *done (host-mapped; nullptr:
// none).  wg_count: a device word that is 0 when the job starts; the last
// workgroup sets it back to 0.
struct CodecJob {
  CodecPart part[kCodecMaxParts];
  int n_part;
  uint32_t n_wg;
  uint32_t* wg_count;
  int32_t* ready;
  int32_t stamp;
  unsigned long long* done;
  unsigned long long seq;
};

// Host side (codec.hip).
// Bytes of row v (n bf16 values, n % kCodecChunk == 0) coded.
size_t codec_coded_bytes(const uint16_t* v, size_t n);
// Code row v into out (4-byte aligned, codec_coded_bytes(v, n) bytes);
// returns them.
size_t codec_encode(const uint16_t* v, size_t n, uint8_t* out);
// Escapes of a coded row of n values that is `bytes` long.
inline uint32_t codec_escapes(size_t n, size_t bytes) {
  return (uint32_t)((bytes - codec_esc_off(n)) / 4);
}
// Decode jobs run on an HSA queue of the library's own per device
// (codec.hip), in dispatch order.
struct CodecQueue;
// The queue of `device` (created on first use; gpu: the device's agent,
// cpu: the host agent whose memory holds the kernel arguments).
int codec_queue(int device, hsa_agent_t gpu, hsa_agent_t cpu, CodecQueue** out);
// Dispatch a job (n_wg is set here, for its values).
int codec_dispatch(CodecQueue* q, CodecJob& job);
// Wait (bounded) until every job dispatched on q so far completed.
int codec_sync(CodecQueue* q, double timeout_s);
