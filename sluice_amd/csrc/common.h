// Shared device/host helpers for libsluice_hip (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sluice.h"

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

#define SLUICE_WAVE 64

// hipError_t values are positive; keep them as they are.
#define SLUICE_HIP_CHECK(expr)                 \
  do {                                         \
    hipError_t _e = (expr);                    \
    if (_e != hipSuccess) return (int)_e;      \
  } while (0)

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs; NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (SLUICE_WAVE - 1); }

// Number of lanes below this one whose bit is set in mask.
__device__ __forceinline__ int mask_rank(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ f32x4_t mfma16x16x32_bf16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x4_t ldg16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// Streaming (read-once) 16-byte load: nontemporal hint keeps expert weights
// from evicting the small activation tiles that are reused.
__device__ __forceinline__ u32x4_t ldg16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

// Wave-wide reductions on DPP: row_shr:1,2,4,8 leave each 16-lane row's
// result in its lane 15, row_bcast:15 and row_bcast:31 carry it into lane
// 63, which every lane then reads as a scalar.  Lanes a DPP step cannot
// source from take the identity.  (An xor-shuffle butterfly compiles to
// ds_bpermute round trips through LDS, several times slower per step.)
// Every lane gets the result.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t identity, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, CTRL, ROW_MASK, 0xf, false);
}

template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v, uint32_t identity, Op op) {
  v = op(v, dpp_mov<0x111, 0xf>(identity, v));
  v = op(v, dpp_mov<0x112, 0xf>(identity, v));
  v = op(v, dpp_mov<0x114, 0xf>(identity, v));
  v = op(v, dpp_mov<0x118, 0xf>(identity, v));
  v = op(v, dpp_mov<0x142, 0xa>(identity, v));
  v = op(v, dpp_mov<0x143, 0xc>(identity, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return wave_reduce_u32(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}

__device__ __forceinline__ float wave_max_f32(float v) {
  return __uint_as_float(wave_reduce_u32(__float_as_uint(v), 0xff800000u, [](uint32_t a,
                                                                              uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}

// Max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the same lane of
// each 16-lane row), in every lane: v_permlane32_swap and v_permlane16_swap
// of a value with itself hand each lane both halves of the exchange.
__device__ __forceinline__ float rows4_max(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t m = __float_as_uint(fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1])));
  const auto b = __builtin_amdgcn_permlane16_swap(m, m, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows4_sum(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t m = __float_as_uint(__uint_as_float(a[0]) + __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(m, m, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  return __uint_as_float(wave_reduce_u32(__float_as_uint(v), 0u, [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
}
