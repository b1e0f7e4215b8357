// Shared device helpers for the omnia HIP kernels (gfx950, wave64).
//
// bf16 travels as raw 16-bit patterns (uint16_t) through every interface; arithmetic
// widens to fp32 by a shift and narrows with round-to-nearest-even through the
// hardware convert (`v_cvt_pk_bf16_f32`, selected from a plain `(__bf16)` cast).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "omnia_hip.h"

namespace omnia {

constexpr int kWave = 64;

// Native 16-byte vector (clang ext_vector), usable with the nontemporal builtins.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}

__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __uint_as_float(packed & 0xFFFF0000u);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t bits) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits.
__device__ __forceinline__ uint16_t f32_to_bf16(float value) {
  __bf16 narrowed = static_cast<__bf16>(value);
  return __builtin_bit_cast(uint16_t, narrowed);
}

// Two fp32 values -> one packed pair, `lo` in the low half (the lower address).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) |
         (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// fp32 value rounded to bf16 and widened back: one bf16 rounding step.
__device__ __forceinline__ float round_bf16(float value) {
  return bf16_to_f32(f32_to_bf16(value));
}

// Eight bf16 values held in one 16-byte vector, unpacked to fp32.
__device__ __forceinline__ void unpack8(const u32x4& v, float out[8]) {
  out[0] = bf16_lo(v.x); out[1] = bf16_hi(v.x);
  out[2] = bf16_lo(v.y); out[3] = bf16_hi(v.y);
  out[4] = bf16_lo(v.z); out[5] = bf16_hi(v.z);
  out[6] = bf16_lo(v.w); out[7] = bf16_hi(v.w);
}

__device__ __forceinline__ u32x4 pack8(const float in[8]) {
  u32x4 v;
  v.x = pack_bf16(in[0], in[1]);
  v.y = pack_bf16(in[2], in[3]);
  v.z = pack_bf16(in[4], in[5]);
  v.w = pack_bf16(in[6], in[7]);
  return v;
}

// Butterfly sum over groups of `width` consecutive lanes (width a power of two <= 64).
// Every lane of a group ends with the group's total.
template <int width>
__device__ __forceinline__ float group_sum(float value) {
#pragma unroll
  for (int offset = width / 2; offset > 0; offset >>= 1) {
    value += __shfl_xor(value, offset, kWave);
  }
  return value;
}

template <typename T>
__device__ __forceinline__ T load_nt(const T* ptr) {
  return __builtin_nontemporal_load(ptr);
}

template <typename T>
__device__ __forceinline__ void store_nt(T* ptr, const T& value) {
  __builtin_nontemporal_store(value, ptr);
}

}  // namespace omnia
