// Residual add + RMSNorm over rows of bf16 (config: T x 2560).
//
// Arithmetic (rounding points of core/kernels/add_norm/rows.py:65-79, which are
// mx.fast.rms_norm's):
//   s_i = bf16(x_i + b_i)
//   inv = 1 / sqrt(sum_i s_i^2 / H + eps)          (fp32, IEEE sqrt and divide)
//   n_i = bf16(w_i * bf16(s_i * inv))
// The sum of squares is accumulated in fp64 (each square of a bf16 value is exact in
// fp32) and rounded once to fp32, so it is the correctly rounded fp32 sum whatever the
// lane order: the result does not depend on how the row is split across lanes.
//
// Layout, by the number of rows:
// - from 4096 rows, one wave64 per row. Lane l owns the 16-byte vectors l, l+64,
//   l+128, ... of the row, so every load and store instruction of the wave covers 1 KiB
//   of contiguous memory, and the sum of squares is a butterfly over the wave;
// - below that, one workgroup per row with one 16-byte vector per lane (5 waves at
//   H = 2560): a grid of one wave per row would leave each CU a wave or two, each
//   waiting out its loads and then a long serial sum. The waves' partial sums meet in
//   LDS, added in wave order, so every wave gets the same total.
// Either way all loads of x and the branch are issued before any math, and both
// outputs are written in the same pass: each tensor crosses HBM exactly once. The norm
// weight (H * 2 bytes) is shared by every row and stays in L2.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kMaxVectorsPerLane = 16;  // hidden <= 64 lanes * 16 vectors * 8 = 8192

template <int VPL>
__global__ __launch_bounds__(256) void add_rms_norm_kernel(
    const u32x4* __restrict__ x, const u32x4* __restrict__ branch,
    const u32x4* __restrict__ weight, u32x4* __restrict__ summed,
    u32x4* __restrict__ normalized, int64_t rows, int vecs, float hidden, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;  // whole wave leaves together; no barrier follows
  const int64_t base = row * vecs;

  // Every load goes out before any arithmetic, with no branch among them (a load in a
  // divergent branch makes the compiler wait on it): a lane past the row's end re-reads
  // the row's last vector and adds nothing to the sum. The weight vectors come with them
  // up to 8 per lane; wider rows read them in the output loop rather than spill.
  constexpr bool kWeightFirst = VPL <= 8;
  u32x4 xv[VPL], bv[VPL], wv[kWeightFirst ? VPL : 1];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int v = min(lane + i * kWave, vecs - 1);
    xv[i] = load_nt(x + base + v);
    bv[i] = load_nt(branch + base + v);
    if constexpr (kWeightFirst) wv[i] = weight[v];
  }
  __builtin_amdgcn_sched_barrier(0);

  float s[VPL][8];
  double acc = 0.0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const bool in_row = lane + i * kWave < vecs;
    float a[8], b[8];
    unpack8(xv[i], a);
    unpack8(bv[i], b);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s[i][j] = round_bf16(a[j] + b[j]);
      acc += in_row ? static_cast<double>(s[i][j] * s[i][j]) : 0.0;
    }
  }
  acc = wave_sum_f64(acc);
  const float inv = 1.0f / sqrtf(static_cast<float>(acc) / hidden + eps);

#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int v = lane + i * kWave;
    if (v < vecs) {
      float w[8], n[8];
      if constexpr (kWeightFirst) unpack8(wv[i], w);
      else unpack8(weight[v], w);
#pragma unroll
      for (int j = 0; j < 8; ++j) n[j] = w[j] * round_bf16(s[i][j] * inv);
      store_nt(summed + base + v, pack8(s[i]));
      store_nt(normalized + base + v, pack8(n));
    }
  }
}

// One row per workgroup, one 16-byte vector per lane (vector threadIdx.x of the row).
__global__ __launch_bounds__(1024) void add_rms_norm_row_kernel(
    const u32x4* __restrict__ x, const u32x4* __restrict__ branch,
    const u32x4* __restrict__ weight, u32x4* __restrict__ summed,
    u32x4* __restrict__ normalized, int vecs, float hidden, float eps) {
  __shared__ double partial[1024 / kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * vecs;
  const bool in_row = static_cast<int>(threadIdx.x) < vecs;
  // A lane past the row's end re-reads the row's last vector and adds nothing.
  const int v = in_row ? static_cast<int>(threadIdx.x) : vecs - 1;
  const u32x4 xv = load_nt(x + base + v);
  const u32x4 bv = load_nt(branch + base + v);
  const u32x4 wv = weight[v];
  __builtin_amdgcn_sched_barrier(0);

  float a[8], b[8];
  unpack8(xv, a);
  unpack8(bv, b);
  uint32_t words[4];
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    words[j / 2] = pack_bf16(a[j] + b[j], a[j + 1] + b[j + 1]);
    const double lo = bf16_lo(words[j / 2]), hi = bf16_hi(words[j / 2]);
    acc = __builtin_fma(lo, lo, acc);   // exact squares
    acc = __builtin_fma(hi, hi, acc);
  }
  acc = wave_sum_f64(in_row ? acc : 0.0);
  if (lane == 0) partial[wave] = acc;
  __syncthreads();  // no store is outstanding yet
  double total = 0.0;
  for (int w = 0; w < waves; ++w) total += partial[w];  // wave order, in every wave
  const float inv = 1.0f / sqrtf(static_cast<float>(total) / hidden + eps);

  if (in_row) {
    const u32x4 sv = u32x4{words[0], words[1], words[2], words[3]};
    float s[8], w[8], n[8];
    unpack8(sv, s);
    unpack8(wv, w);
#pragma unroll
    for (int j = 0; j < 8; ++j) n[j] = w[j] * round_bf16(s[j] * inv);
    store_nt(summed + base + v, sv);
    store_nt(normalized + base + v, pack8(n));
  }
}

template <int VPL>
void launch(int waves_per_block, int64_t blocks, hipStream_t stream, const u32x4* x,
            const u32x4* b, const u32x4* w, u32x4* s, u32x4* n, int64_t rows, int vecs,
            float hidden, float eps) {
  add_rms_norm_kernel<VPL><<<dim3(static_cast<unsigned>(blocks)),
                             dim3(waves_per_block * kWave), 0, stream>>>(
      x, b, w, s, n, rows, vecs, hidden, eps);
}

using Launcher = void (*)(int, int64_t, hipStream_t, const u32x4*, const u32x4*,
                          const u32x4*, u32x4*, u32x4*, int64_t, int, float, float);

constexpr Launcher kLaunchers[kMaxVectorsPerLane] = {
    launch<1>,  launch<2>,  launch<3>,  launch<4>,  launch<5>,  launch<6>,
    launch<7>,  launch<8>,  launch<9>,  launch<10>, launch<11>, launch<12>,
    launch<13>, launch<14>, launch<15>, launch<16>};

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_add_rms_norm(const uint16_t* x, const uint16_t* branch,
                                      const uint16_t* weight, uint16_t* summed,
                                      uint16_t* normalized, int64_t rows, int64_t hidden,
                                      float eps, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0, "add_rms_norm: rows must be >= 0");
  OMNIA_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= 8 * kWave * kMaxVectorsPerLane,
                "add_rms_norm: hidden must be a multiple of 8 in [8, 8192]");
  OMNIA_REQUIRE(rows < (int64_t{1} << 31), "add_rms_norm: too many rows");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(x && branch && weight && summed && normalized,
                "add_rms_norm: null pointer");
  OMNIA_REQUIRE(aligned16(x) && aligned16(branch) && aligned16(weight) &&
                    aligned16(summed) && aligned16(normalized),
                "add_rms_norm: pointers must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;

  const int vecs = static_cast<int>(hidden / 8);
  const int vpl = (vecs + kWave - 1) / kWave;
  if (rows < 4096) {  // one workgroup per row, one vector per lane
    add_rms_norm_row_kernel<<<dim3(static_cast<unsigned>(rows)), dim3(vpl * kWave), 0, stream>>>(
        reinterpret_cast<const u32x4*>(x), reinterpret_cast<const u32x4*>(branch),
        reinterpret_cast<const u32x4*>(weight), reinterpret_cast<u32x4*>(summed),
        reinterpret_cast<u32x4*>(normalized), vecs, static_cast<float>(hidden), eps);
    return launched("add_rms_norm");
  }
  const int waves_per_block = 4;
  const int64_t blocks = (rows + waves_per_block - 1) / waves_per_block;
  kLaunchers[vpl - 1](waves_per_block, blocks, stream,
                      reinterpret_cast<const u32x4*>(x),
                      reinterpret_cast<const u32x4*>(branch),
                      reinterpret_cast<const u32x4*>(weight),
                      reinterpret_cast<u32x4*>(summed), reinterpret_cast<u32x4*>(normalized),
                      rows, vecs, static_cast<float>(hidden), eps);
  return launched("add_rms_norm");
}
