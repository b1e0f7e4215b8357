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
// Layout: one thread per (position, pair); a workgroup covers 256 consecutive entries of
// the row-major [rows, P] grid, and each thread writes its cosine at column i and its
// sine at column P + i of the row (the reference's atlas, models/laguna/layers/
// attention.py:236-243).
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kAtlasBlock = 256;

__global__ __launch_bounds__(kAtlasBlock) void rope_atlas_kernel(const double* __restrict__ frequencies,
                                                                 int pairs, int64_t first,
                                                                 int64_t rows, float* __restrict__ atlas,
                                                                 int64_t stride) {
  const int64_t entry = static_cast<int64_t>(blockIdx.x) * kAtlasBlock + threadIdx.x;
  if (entry >= rows * pairs) return;
  const int64_t row = entry / pairs;
  const int i = static_cast<int>(entry % pairs);
  const double theta = static_cast<double>(first + row) * frequencies[i];
  double s, c;
  sincos(theta, &s, &c);
  float* out = atlas + row * stride;
  out[i] = static_cast<float>(c);
  out[pairs + i] = static_cast<float>(s);
}

__global__ __launch_bounds__(kAtlasBlock) void rope_atlas_fp32_kernel(const float* __restrict__ inverse,
                                                                      int pairs, int64_t first,
                                                                      int64_t rows, float* __restrict__ atlas,
                                                                      int64_t stride) {
  const int64_t entry = static_cast<int64_t>(blockIdx.x) * kAtlasBlock + threadIdx.x;
  if (entry >= rows * pairs) return;
  const int64_t row = entry / pairs;
  const int i = static_cast<int>(entry % pairs);
  const float position = static_cast<float>(first + row);   // arange in fp32
  const float theta = static_cast<float>(static_cast<double>(position) / static_cast<double>(inverse[i]));
  double s, c;
  sincos(static_cast<double>(theta), &s, &c);
  float* out = atlas + row * stride;
  out[i] = static_cast<float>(c);
  out[pairs + i] = static_cast<float>(s);
}

int32_t check_atlas(int64_t pairs, int64_t first, int64_t rows, int64_t stride) {
  OMNIA_REQUIRE(pairs > 0 && pairs <= 4096, "rope_angle_atlas: pairs must be in [1, 4096]");
  OMNIA_REQUIRE(first >= 0 && rows >= 0 && first + rows <= (int64_t{1} << 40),
                "rope_angle_atlas: bad position range");
  OMNIA_REQUIRE(stride >= 2 * pairs, "rope_angle_atlas: row stride smaller than 2 * pairs");
  OMNIA_REQUIRE(rows * pairs < (int64_t{1} << 40), "rope_angle_atlas: too many entries");
  OMNIA_REQUIRE((rows * pairs + kAtlasBlock - 1) / kAtlasBlock < (int64_t{1} << 31),
                "rope_angle_atlas: too many rows");
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
  const int64_t blocks = (rows * pairs + kAtlasBlock - 1) / kAtlasBlock;
  rope_atlas_fp32_kernel<<<static_cast<unsigned>(blocks), kAtlasBlock, 0, stream>>>(
      inverse_frequencies, static_cast<int>(pairs), first, rows, atlas, stride);
  return launched("rope_angle_atlas");
}

extern "C" int32_t omnia_rope_angle_atlas(const double* frequencies, int64_t pairs, int64_t first,
                                          int64_t rows, float* atlas, int64_t stride,
                                          hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(pairs > 0 && pairs <= 4096, "rope_angle_atlas: pairs must be in [1, 4096]");
  OMNIA_REQUIRE(first >= 0 && rows >= 0 && first + rows <= (int64_t{1} << 40),
                "rope_angle_atlas: bad position range");
  OMNIA_REQUIRE(stride >= 2 * pairs, "rope_angle_atlas: row stride smaller than 2 * pairs");
  OMNIA_REQUIRE(rows * pairs < (int64_t{1} << 40), "rope_angle_atlas: too many entries");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(frequencies && atlas, "rope_angle_atlas: null pointer");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const int64_t blocks = (rows * pairs + kAtlasBlock - 1) / kAtlasBlock;
  OMNIA_REQUIRE(blocks < (int64_t{1} << 31), "rope_angle_atlas: too many rows");
  rope_atlas_kernel<<<static_cast<unsigned>(blocks), kAtlasBlock, 0, stream>>>(
      frequencies, static_cast<int>(pairs), first, rows, atlas, stride);
  return launched("rope_angle_atlas");
}
