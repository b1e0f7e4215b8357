// The rotary angle atlas: fp32 rows [cos(theta_0..P-1) || sin(theta_0..P-1)] for a run of
// positions, built on the device.
//
// Arithmetic (the fp64 build of tests/test_kernel_qk_norm_rope.py:51-66 that the table
// kernels are tested against; the frequencies also carry the YaRN table of
// models/laguna/layers/attention.py:196-222 as 1 / freqs):
//   theta = pos * f_i in fp64 (f_i the caller's fp64 frequencies, for the plain rope
//   exp(-ln(base) * i / P)), cos and sin in fp64, each rounded once to fp32.
// The caller computes the frequencies once on the host, so every device and the host
// start from the same fp64 values.
//
// The fp32 order (omnia_rope_angle_atlas_fp32): the op chain of models/laguna/layers/
// attention.py:236-243, `theta = arange(rows, fp32)[:, None] / inverse[None, :]` with
// `inverse = base ** (arange(0, D, 2) / D)` in fp32 (or the YaRN table), then cos and
// sin of that fp32 angle. Each fp32 operation is the correctly rounded one: the quotient
// is formed in fp64 from the two fp32 operands and rounded once to fp32 (fp64 carries
// more than 2 * 24 + 2 bits, so this double rounding is innocuous for a quotient), and
// cos and sin of the fp32 angle are evaluated in fp64 and rounded once. The caller
// computes the fp32 `inverse` row once on the host.
//
// sin and cos: for |theta| < 2^25 (every position below about 3.3e7 at a frequency of at
// most 1), the Cody-Waite reduction and Taylor series of sin_cos_fp64 (common.hpp); above,
// and for a non-finite angle, the device library's fp64 sincos.
//
// Layout, no division: a thread computes V consecutive pairs of one row (V = 4 when P is a
// multiple of 4 and the table rows and the frequencies are 16-byte aligned: one 16-byte
// store for its cosines and one for its sines; else V = 1). A workgroup of 256 threads is `lanes` threads across
// (the power of two >= P / V, at most 64) by 256 / lanes rows; blockIdx.x is the row
// block and blockIdx.y the run of 64 V pairs. Each row is [cos(theta_0..P-1) ||
// sin(theta_0..P-1)] (the reference's atlas, models/laguna/layers/attention.py:236-243).
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kAtlasBlock = 256;
typedef double f64x2 __attribute__((ext_vector_type(2)));

// sin and cos of the thread's V angles: the Cody-Waite path for all of them, with no
// branch; then, only where some lane holds an angle at or past the limit (or NaN), the
// library's sincos in place of those.
template <int V>
__device__ __forceinline__ void atlas_sin_cos(const double (&theta)[V], double (&s)[V], double (&c)[V]) {
  bool slow = false;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    sin_cos_fp64_selects(theta[j], s[j], c[j]);
    slow |= !(__builtin_fabs(theta[j]) < kSinCosFastLimit);
  }
  if (__builtin_expect(slow, 0)) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      if (!(__builtin_fabs(theta[j]) < kSinCosFastLimit)) sincos(theta[j], &s[j], &c[j]);
    }
  }
}

// (row, first pair) of this thread, or false past the grid's edge (P is a multiple of V).
template <int V>
__device__ __forceinline__ bool atlas_entry(int pairs, int64_t rows, int64_t& row, int& i) {
  row = static_cast<int64_t>(blockIdx.x) * blockDim.y + threadIdx.y;
  i = (static_cast<int>(blockIdx.y) * kWave + static_cast<int>(threadIdx.x)) * V;
  return row < rows && i < pairs;
}

// The V angles of the thread: fp64 (theta = position * frequency) or the fp32 order
// (theta = fp32(fp32(position) / inverse), the quotient formed in fp64 and rounded once).
template <int V, bool kFp32Order>
__device__ __forceinline__ void atlas_angles(const void* frequencies, int i, int64_t position,
                                             double (&theta)[V]) {
  if constexpr (kFp32Order) {
    const float* inverse = static_cast<const float*>(frequencies) + i;
    float f[V];
    if constexpr (V == 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(inverse);
      f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
    } else {
      f[0] = inverse[0];
    }
    const double p = static_cast<double>(static_cast<float>(position));   // arange in fp32
#pragma unroll
    for (int j = 0; j < V; ++j) theta[j] = static_cast<double>(static_cast<float>(p / static_cast<double>(f[j])));
  } else {
    const double* f = static_cast<const double*>(frequencies) + i;
    const double p = static_cast<double>(position);
    if constexpr (V == 4) {
      const f64x2 lo = *reinterpret_cast<const f64x2*>(f);
      const f64x2 hi = *reinterpret_cast<const f64x2*>(f + 2);
      theta[0] = p * lo.x; theta[1] = p * lo.y; theta[2] = p * hi.x; theta[3] = p * hi.y;
    } else {
      theta[0] = p * f[0];
    }
  }
}

template <int V, bool kFp32Order>
__global__ __launch_bounds__(kAtlasBlock) void rope_atlas_kernel(const void* __restrict__ frequencies,
                                                                 int pairs, int64_t first,
                                                                 int64_t rows, float* __restrict__ atlas,
                                                                 int64_t stride) {
  int64_t row;
  int i;
  if (!atlas_entry<V>(pairs, rows, row, i)) return;
  double theta[V];
  atlas_angles<V, kFp32Order>(frequencies, i, first + row, theta);
  double sd[V], cd[V];
  atlas_sin_cos<V>(theta, sd, cd);
  float c[V], s[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    c[j] = static_cast<float>(cd[j]);
    s[j] = static_cast<float>(sd[j]);
  }
  float* out = atlas + row * stride + i;
  if constexpr (V == 4) {
    *reinterpret_cast<f32x4*>(out) = f32x4{c[0], c[1], c[2], c[3]};
    *reinterpret_cast<f32x4*>(out + pairs) = f32x4{s[0], s[1], s[2], s[3]};
  } else {
    out[0] = c[0];
    out[pairs] = s[0];
  }
}

// The workgroup shape and grid for `pairs` columns by `rows` rows, V pairs per thread.
struct AtlasLaunch {
  dim3 grid, block;
};

AtlasLaunch atlas_launch(int64_t pairs, int64_t rows, int v) {
  const int64_t across = (pairs + v - 1) / v;
  int lanes = 1;
  while (lanes < across && lanes < kWave) lanes *= 2;
  const int per_block = kAtlasBlock / lanes;
  return AtlasLaunch{dim3(static_cast<unsigned>((rows + per_block - 1) / per_block),
                          static_cast<unsigned>((across + kWave - 1) / kWave)),
                     dim3(static_cast<unsigned>(lanes), static_cast<unsigned>(per_block))};
}

// Four pairs per thread when every row's cosine and sine halves start 16-byte aligned and
// the frequencies can be read as 16-byte vectors.
int atlas_width(const void* frequencies, int64_t pairs, const float* atlas, int64_t stride) {
  return pairs % 4 == 0 && stride % 4 == 0 && aligned16(atlas) && aligned16(frequencies) ? 4 : 1;
}

template <bool kFp32Order>
int32_t launch_atlas(const void* frequencies, int64_t pairs, int64_t first, int64_t rows,
                     float* atlas, int64_t stride, hipStream_t stream) {
  const int v = atlas_width(frequencies, pairs, atlas, stride);
  const AtlasLaunch launch = atlas_launch(pairs, rows, v);
  if (v == 4) {
    rope_atlas_kernel<4, kFp32Order><<<launch.grid, launch.block, 0, stream>>>(
        frequencies, static_cast<int>(pairs), first, rows, atlas, stride);
  } else {
    rope_atlas_kernel<1, kFp32Order><<<launch.grid, launch.block, 0, stream>>>(
        frequencies, static_cast<int>(pairs), first, rows, atlas, stride);
  }
  return launched("rope_angle_atlas");
}

int32_t check_atlas(int64_t pairs, int64_t first, int64_t rows, int64_t stride) {
  OMNIA_REQUIRE(pairs > 0 && pairs <= 4096, "rope_angle_atlas: pairs must be in [1, 4096]");
  OMNIA_REQUIRE(first >= 0 && rows >= 0 && first + rows <= (int64_t{1} << 40),
                "rope_angle_atlas: bad position range");
  OMNIA_REQUIRE(stride >= 2 * pairs, "rope_angle_atlas: row stride smaller than 2 * pairs");
  OMNIA_REQUIRE(rows * pairs < (int64_t{1} << 40), "rope_angle_atlas: too many entries");
  OMNIA_REQUIRE(atlas_launch(pairs, rows, 1).grid.x < (1u << 31), "rope_angle_atlas: too many rows");
  return 0;
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_rope_angle_atlas_fp32(const float* inverse_frequencies, int64_t pairs,
                                               int64_t first, int64_t rows, float* atlas,
                                               int64_t stride, hipStream_t stream) {
  using namespace omnia;
  int32_t rc = check_atlas(pairs, first, rows, stride);
  if (rc != 0 || rows == 0) return rc;
  OMNIA_REQUIRE(inverse_frequencies && atlas, "rope_angle_atlas: null pointer");
  rc = check_device(stream);
  if (rc != 0) return rc;
  return launch_atlas<true>(inverse_frequencies, pairs, first, rows, atlas, stride, stream);
}

extern "C" int32_t omnia_rope_angle_atlas(const double* frequencies, int64_t pairs, int64_t first,
                                          int64_t rows, float* atlas, int64_t stride,
                                          hipStream_t stream) {
  using namespace omnia;
  int32_t rc = check_atlas(pairs, first, rows, stride);
  if (rc != 0 || rows == 0) return rc;
  OMNIA_REQUIRE(frequencies && atlas, "rope_angle_atlas: null pointer");
  rc = check_device(stream);
  if (rc != 0) return rc;
  return launch_atlas<false>(frequencies, pairs, first, rows, atlas, stride, stream);
}
