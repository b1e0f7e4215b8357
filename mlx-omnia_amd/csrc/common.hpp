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
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));  // 4 bf16 MFMA operand
typedef short s16x8 __attribute__((ext_vector_type(8)));

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

// fp64 -> bf16 bits, round to nearest even, for values in the normal bf16 range; zero,
// subnormals, infinities and NaN go through fp32 (a double rounding is possible only in
// the subnormal tail, reached for sigmoid arguments below about -87).
__device__ __forceinline__ uint32_t f64_to_bf16(double value) {
  const uint64_t bits = __builtin_bit_cast(uint64_t, value);
  const uint32_t sign = static_cast<uint32_t>(bits >> 48) & 0x8000u;
  const int exponent = static_cast<int>((bits >> 52) & 0x7FF) - 1023;
  if (exponent < -126 || exponent > 127) return f32_to_bf16(static_cast<float>(value));
  const uint64_t mantissa = bits & ((uint64_t{1} << 52) - 1);
  const uint64_t rest = mantissa & ((uint64_t{1} << 45) - 1);
  constexpr uint64_t kHalf = uint64_t{1} << 44;
  uint32_t magnitude = (static_cast<uint32_t>(exponent + 127) << 7) |
                       static_cast<uint32_t>(mantissa >> 45);
  if (rest > kHalf || (rest == kHalf && (magnitude & 1u))) ++magnitude;
  return sign | magnitude;
}

// Two fp32 values -> one packed bf16 pair (RNE), `lo` in the low half (the lower
// address): a single v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2 pair = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(pair, bf16x2));
}

// Rounds two fp32 values to bf16 in one conversion and widens them back.
__device__ __forceinline__ void round_pair(float& lo, float& hi) {
  const uint32_t packed = pack_bf16(lo, hi);
  lo = bf16_lo(packed);
  hi = bf16_hi(packed);
}

// fp32 value rounded to bf16 and widened back: one bf16 rounding step.
__device__ __forceinline__ float round_bf16(float value) {
  return bf16_to_f32(f32_to_bf16(value));
}

// The bits of a bf16 value an epilogue needs (a residual, a projection bias), loaded at
// a kernel's start together with its other loads, instead of after its last wait or
// barrier where it would be one more dependent round trip: src[index], or any[0] (which
// must be a valid bf16 address) when `src` is null, the caller then ignoring it. The
// load is unconditional and the caller widens the bits where it uses them: a select on
// the value would let the compiler sink the load into a branch and wait on it there.
__device__ __forceinline__ uint32_t early_bf16_bits(const uint16_t* src, int64_t index, const uint16_t* any) {
  const bool have = src != nullptr;
  return (have ? src : any)[have ? index : 0];
}

// A workgroup barrier ordering LDS traffic only. __syncthreads() also drains each wave's
// outstanding global loads and stores (its fence waits for vmcnt(0)); this one lets them
// stay in flight across it, for barriers that guard LDS data alone (no wave reads global
// memory another wave of the workgroup wrote).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// XCD-aware block order. The part hands workgroups to its 8 XCDs in turn (workgroup b
// to XCD b % 8), and each XCD has its own L2. This maps them so that each XCD takes one
// contiguous run of blocks (the first blocks % 8 XCDs one more than the others), which
// keeps the cache lines neighbouring blocks share (quantization scales, for instance) in
// one L2 instead of fetching them from HBM for two. A bijection on [0, blocks) for any
// count, so every block is still computed exactly once.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_contiguous_block(int b, int blocks) {
  const int xcd = b % kXcds, k = b / kXcds;
  return xcd * (blocks / kXcds) + min(xcd, blocks % kXcds) + k;
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
template <int width, typename T>
__device__ __forceinline__ T group_sum(T value) {
#pragma unroll
  for (int offset = width / 2; offset > 0; offset >>= 1) {
    value += __shfl_xor(value, offset, kWave);
  }
  return value;
}

// Cross-lane moves inside a 16-lane DPP row (no LDS traffic). Every control used here
// (row rotations, mirrors, quad permutations) gives each lane a source inside its row, so
// bound_ctrl changes nothing; set, it lets the compiler fold the move into the consuming
// VALU op (v_add_f32_dpp and the like).
template <int ctrl>
__device__ __forceinline__ uint32_t dpp(uint32_t value) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(value), ctrl, 0xF, 0xF, true));
}
constexpr int kRowRor1 = 0x121, kRowRor2 = 0x122, kRowRor4 = 0x124, kRowRor8 = 0x128;

// Sum over the 16 lanes of each DPP row; every lane ends with the same value (each
// rotation step adds two operands that the partner lane adds in swapped order).
__device__ __forceinline__ double row16_sum(double value) {
#define OMNIA_ROW_STEP(ctrl)                                                          \
  {                                                                                   \
    const uint64_t bits = __builtin_bit_cast(uint64_t, value);                        \
    const uint32_t lo = dpp<ctrl>(static_cast<uint32_t>(bits));                       \
    const uint32_t hi = dpp<ctrl>(static_cast<uint32_t>(bits >> 32));                 \
    value += __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);      \
  }
  OMNIA_ROW_STEP(kRowRor8)
  OMNIA_ROW_STEP(kRowRor4)
  OMNIA_ROW_STEP(kRowRor2)
  OMNIA_ROW_STEP(kRowRor1)
#undef OMNIA_ROW_STEP
  return value;
}

// Cross-row steps of a wave reduction (gfx950): with the same value in both operands,
// v_permlane16_swap hands each lane the value of the same column in the paired 16-lane
// row (rows 0-1, 2-3), v_permlane32_swap that of the other 32-lane half. Both lanes of a
// pair get the same two dwords: the first from the lower lane (row 0 or 2, half 0), the
// second from the upper one (checked on MI355X with a one-wave probe of lane ids).
__device__ __forceinline__ void row_pair(uint32_t v, uint32_t& a, uint32_t& b) {
  const auto swapped = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  a = swapped[0];
  b = swapped[1];
}
__device__ __forceinline__ void half_pair(uint32_t v, uint32_t& a, uint32_t& b) {
  const auto swapped = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  a = swapped[0];
  b = swapped[1];
}

constexpr int kQuadSwap1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kQuadSwap2 = 0x4E;  // quad_perm [2, 3, 0, 1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

// fp64 sum over the wave, the same in every lane.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v = row16_sum(v);
  uint32_t lo_a, lo_b, hi_a, hi_b;
  const uint64_t bits = __builtin_bit_cast(uint64_t, v);
  row_pair(static_cast<uint32_t>(bits), lo_a, lo_b);
  row_pair(static_cast<uint32_t>(bits >> 32), hi_a, hi_b);
  v = __builtin_bit_cast(double, (static_cast<uint64_t>(hi_a) << 32) | lo_a) +
      __builtin_bit_cast(double, (static_cast<uint64_t>(hi_b) << 32) | lo_b);
  const uint64_t bits2 = __builtin_bit_cast(uint64_t, v);
  half_pair(static_cast<uint32_t>(bits2), lo_a, lo_b);
  half_pair(static_cast<uint32_t>(bits2 >> 32), hi_a, hi_b);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi_a) << 32) | lo_a) +
         __builtin_bit_cast(double, (static_cast<uint64_t>(hi_b) << 32) | lo_b);
}

// fp32 sum over the wave, the same in every lane: row rotations (each lane of a pair adds
// the same two operands), then the two cross-row swaps.
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += __uint_as_float(dpp<kRowRor8>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor4>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor1>(__float_as_uint(v)));
  uint32_t a, b;
  row_pair(__float_as_uint(v), a, b);
  v = __uint_as_float(a) + __uint_as_float(b);
  half_pair(__float_as_uint(v), a, b);
  return __uint_as_float(a) + __uint_as_float(b);
}

// fp32 maximum over the wave, the same in every lane.
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, __uint_as_float(dpp<kRowRor8>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp<kRowRor4>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp<kRowRor2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp<kRowRor1>(__float_as_uint(v))));
  uint32_t a, b;
  row_pair(__float_as_uint(v), a, b);
  v = fmaxf(__uint_as_float(a), __uint_as_float(b));
  half_pair(__float_as_uint(v), a, b);
  return fmaxf(__uint_as_float(a), __uint_as_float(b));
}

// Sum over each 16-lane DPP row, the same in each of its lanes.
__device__ __forceinline__ float octet_sum(float v) {
  v += __uint_as_float(dpp<kQuadSwap1>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kQuadSwap2>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowMirror>(__float_as_uint(v)));
  return v;
}

// A row's sum over a group of kLanes consecutive lanes (16, 32 or 64), in every lane of
// the group: the 16-lane DPP rows of the group pair up first (rows 0 + 1, then + rows
// 2 + 3), then the butterfly inside each row. A lane holding no term holds +0.
template <int kLanes>
__device__ __forceinline__ float group_row_sum(float v) {
  static_assert(kLanes == 16 || kLanes == 32 || kLanes == 64, "16, 32 or 64 lanes");
  if constexpr (kLanes >= 32) {
    uint32_t lo, hi;
    row_pair(__float_as_uint(v), lo, hi);
    v = __uint_as_float(lo) + __uint_as_float(hi);
  }
  if constexpr (kLanes == 64) {
    uint32_t lo, hi;
    half_pair(__float_as_uint(v), lo, hi);
    v = __uint_as_float(lo) + __uint_as_float(hi);
  }
  return octet_sum(v);
}

// c + a.lo * b.lo + a.hi * b.hi over two packed bf16 pairs (v_dot2_f32_bf16), fp32.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}

// Pins a loaded value where it stands: an empty asm that reads it, so the load is issued
// (and waited on) here. Without it, a load whose only use sits under a later branch on a
// kernel argument (a store past the end skipped) is moved into that branch, and the
// branch's own scalar round trip for the argument then comes before the load's addresses
// can be formed: two scalar round trips ahead of the first load instead of one.
template <typename T>
__device__ __forceinline__ void keep_loaded(const T& value) {
  asm volatile("" ::"v"(value));
}

template <typename T>
__device__ __forceinline__ T load_nt(const T* ptr) {
  return __builtin_nontemporal_load(ptr);
}

template <typename T>
__device__ __forceinline__ void store_nt(T* ptr, const T& value) {
  __builtin_nontemporal_store(value, ptr);
}

// sin and cos of x in fp64, for |x| < kSinCosFastLimit (2^25). Argument reduction by pi/2
// after Cody and Waite ("Software Manual for the Elementary Functions", 1980): pi/2 is
// split into C1 + C2 + C3 (27 significant bits each) + C4, so k * Ci is exact for
// |k| < 2^26 and x - k * C1 is exact (Sterbenz); each later step rounds once relative to
// its own result, so the reduced argument r (|r| <= pi/4 plus a rounding margin) carries
// a relative error of a few fp64 ulps even when x lies close to a multiple of pi/2.
// sin r and cos r are their Taylor series to r^17 and r^18 (the first omitted terms are
// below 1e-19 at |r| = 0.79), evaluated by Horner's rule; the quadrant k mod 4 then picks
// and signs them. NaN in gives NaN out.
constexpr double kSinCosFastLimit = 0x1p25;

// The reduction and the two series: sin r and cos r, and k (an integer-valued double).
__device__ __forceinline__ double sin_cos_reduced(double x, double& sin_r, double& cos_r) {
  constexpr double kTwoOverPi = 0x1.45f306dc9c883p-1;
  constexpr double kC1 = 0x1.921fb54000000p+0;
  constexpr double kC2 = 0x1.10b4610000000p-30;
  constexpr double kC3 = 0x1.a626330000000p-58;
  constexpr double kC4 = 0x1.45c06e0e68948p-86;
  const double k = __builtin_rint(x * kTwoOverPi);
  double r = __builtin_fma(-k, kC1, x);
  r = __builtin_fma(-k, kC2, r);
  r = __builtin_fma(-k, kC3, r);
  r = __builtin_fma(-k, kC4, r);
  const double r2 = r * r;
  // (-1)^n / (2n+1)! for n = 8 .. 1, and (-1)^n / (2n)! for n = 9 .. 1, as doubles.
  double ps = 0x1.952c77030ad4ap-49;
  ps = __builtin_fma(ps, r2, -0x1.ae7f3e733b81fp-41);
  ps = __builtin_fma(ps, r2, 0x1.6124613a86d09p-33);
  ps = __builtin_fma(ps, r2, -0x1.ae64567f544e4p-26);
  ps = __builtin_fma(ps, r2, 0x1.71de3a556c734p-19);
  ps = __builtin_fma(ps, r2, -0x1.a01a01a01a01ap-13);
  ps = __builtin_fma(ps, r2, 0x1.1111111111111p-7);
  ps = __builtin_fma(ps, r2, -0x1.5555555555555p-3);
  sin_r = __builtin_fma(ps * r2, r, r);
  double pc = -0x1.6827863b97d97p-53;
  pc = __builtin_fma(pc, r2, 0x1.ae7f3e733b81fp-45);
  pc = __builtin_fma(pc, r2, -0x1.93974a8c07c9dp-37);
  pc = __builtin_fma(pc, r2, 0x1.1eed8eff8d898p-29);
  pc = __builtin_fma(pc, r2, -0x1.27e4fb7789f5cp-22);
  pc = __builtin_fma(pc, r2, 0x1.a01a01a01a01ap-16);
  pc = __builtin_fma(pc, r2, -0x1.6c16c16c16c17p-10);
  pc = __builtin_fma(pc, r2, 0x1.5555555555555p-5);
  pc = __builtin_fma(pc, r2, -0x1.0000000000000p-1);
  cos_r = __builtin_fma(pc, r2, 1.0);
  return k;
}

__device__ __forceinline__ void sin_cos_fp64(double x, double& sin_x, double& cos_x) {
  double sin_r, cos_r;
  const double k = sin_cos_reduced(x, sin_r, cos_r);
  const int quadrant = static_cast<int>(static_cast<int64_t>(k) & 3);
  sin_x = quadrant == 0 ? sin_r : quadrant == 1 ? cos_r : quadrant == 2 ? -sin_r : -cos_r;
  cos_x = quadrant == 0 ? cos_r : quadrant == 1 ? -sin_r : quadrant == 2 ? -cos_r : sin_r;
}

// The same values with the quadrant applied by selects alone (no branch, no conversion):
// k + 1.5 * 2^52 holds k mod 2^32 in its low word (two's complement for negative k), for
// any k, so lanes past the limit (whose values the caller replaces) stay well defined.
// Odd k swaps sin and cos; the signs follow bit 1 of k (sin) and of k + 1 (cos).
__device__ __forceinline__ void sin_cos_fp64_selects(double x, double& sin_x, double& cos_x) {
  double sin_r, cos_r;
  const double k = sin_cos_reduced(x, sin_r, cos_r);
  const uint32_t quadrant = static_cast<uint32_t>(__builtin_bit_cast(uint64_t, k + 0x1.8p52));
  const bool swap = (quadrant & 1u) != 0;
  const double s = swap ? cos_r : sin_r;
  const double c = swap ? sin_r : cos_r;
  sin_x = (quadrant & 2u) != 0 ? -s : s;
  cos_x = ((quadrant + 1u) & 2u) != 0 ? -c : c;
}

}  // namespace omnia
