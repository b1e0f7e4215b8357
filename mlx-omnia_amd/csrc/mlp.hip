// Dense SwiGLU MLP of a one-token step, bf16 weights, in two dispatches: the gate||up
// projection with the SwiGLU applied, then the down projection with the residual added.
//
// Arithmetic (core/kernels/mlp/dense.py:34-147,222-246, the reference's `DenseMlp`):
//   gate_up_swiglu:  g = bf16(sum_h x_h W[n, h]),  u = bf16(sum_h x_h W[I + n, h])   (fp32 sums)
//                    e = bf16(exp(|g|)), den = bf16(1 + e), y = bf16(1 / den)
//                    sig = g < 0 ? y : bf16(1 - y)
//                    act[n] = bf16(bf16(g * sig) * u)
//   down_residual:   out[n] = bf16(residual[n] + bf16(sum_i act_i D[n, i]))          (fp32 sum)
// Every step of the activation is a bf16 value computed in fp32 and rounded once (RNE),
// the "stable exp(|g|) branch form" the reference writes with `bfloat` temporaries. The
// fp32 sums' order is free (the reference's is a 4-wide lane sweep and a simd tree).
//
// Layout. The fused weight is [2I, H] with the gate rows first, the down weight [H, I],
// both row-major. gate_up_swiglu: a wave owns one output element n and streams its gate
// and up rows together; lane l owns the 16-byte vectors l, l + 64, ... of a row, so one
// load instruction covers 1 KiB of contiguous memory (x is read alongside, from L2). Each
// sum is a wave reduction (DPP row rotations, then permlane swaps); lane 0 runs the
// activation chain and stores. One pair per wave measured 16.1 us at H = 2560, I = 9728,
// against 16.5 us for two and 18.2 us for four. down_residual: one
// workgroup per output row, whose two waves each take half of the contraction in steps of
// 10 vectors per lane (at I = 9728 one step holds a wave's whole half in flight) and
// combine their sums through LDS. The activation is read with ordinary loads and stays in
// L2 (I * 2 bytes); the weight streams with nontemporal loads. Measured at H = 2560,
// I = 9728: 9.8 us, against 12.4 us for two rows per wave in 8-vector steps and 11.0 us
// for one wave per row.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kMaxVectorsPerLane = 16;  // gate_up: hidden <= 8192 (x held in registers)
constexpr int kDownSplit = 2;           // down: waves sharing one output row
constexpr int kDownChunk = 10;          // down: vectors per lane per step of the contraction

__device__ __forceinline__ float wave_total(float v) {
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

// The reference's bf16 SwiGLU step for step (core/kernels/mlp/dense.py:86-96): every
// temporary is a bf16 value.
__device__ __forceinline__ uint16_t swiglu_bf16_steps(float gate_sum, float up_sum) {
  const float g = round_bf16(gate_sum);
  const float u = round_bf16(up_sum);
  const float e = round_bf16(expf(fabsf(g)));
  const float den = round_bf16(1.0f + e);
  const float y = round_bf16(1.0f / den);
  const float sig = g < 0.0f ? y : round_bf16(1.0f - y);
  const float silu = round_bf16(g * sig);
  return f32_to_bf16(silu * u);
}

struct GateUpArgs {
  const u32x4* x;     // [H / 8]
  const u32x4* w;     // [2I, H / 8]
  uint16_t* out;      // [I]
  int inner;
  int vecs;           // H / 8
};

// The arguments as scalars (GateUpArgs field by field): gfx950 preloads a kernel's leading
// scalar and pointer arguments into SGPRs at wave launch, so the first loads go out with
// no scalar round trip ahead of them.
template <int VPL>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void dense_gate_up_swiglu_kernel(
    const u32x4* x, const u32x4* w, uint16_t* out, int inner, int vecs) {
  const GateUpArgs a{x, w, out, inner, vecs};
  const int lane = threadIdx.x % kWave;
  const int n = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;  // this wave's output
  if (n >= a.inner) return;  // whole wave; no barrier follows
  u32x4 xv[VPL], gv[VPL], uv[VPL];
  const u32x4* gate_row = a.w + static_cast<int64_t>(n) * a.vecs;
  const u32x4* up_row = a.w + (static_cast<int64_t>(a.inner) + n) * a.vecs;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int v = lane + i * kWave;
    xv[i] = gv[i] = uv[i] = u32x4{0u, 0u, 0u, 0u};
    if (v < a.vecs) {
      xv[i] = a.x[v];
      gv[i] = load_nt(gate_row + v);
      uv[i] = load_nt(up_row + v);
    }
  }
  float gate = 0.0f, up = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    float xf[8], gf[8], uf[8];
    unpack8(xv[i], xf);
    unpack8(gv[i], gf);
    unpack8(uv[i], uf);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      gate = __builtin_fmaf(xf[j], gf[j], gate);
      up = __builtin_fmaf(xf[j], uf[j], up);
    }
  }
  gate = wave_total(gate);
  up = wave_total(up);
  if (lane == 0) a.out[n] = swiglu_bf16_steps(gate, up);
}

struct DownArgs {
  const u32x4* act;          // [I / 8]
  const u32x4* w;            // [H, I / 8]
  const uint16_t* residual;  // [H]
  uint16_t* out;             // [H]
  int hidden;
  int vecs;                  // I / 8
};

// One workgroup per output row; its kDownSplit waves take consecutive slices of the
// contraction, kDownChunk vectors per lane per step, and leave their sums in LDS.
// The struct argument stays: the same arguments as preloaded scalars measured 0.1 us
// slower (9.72 -> 9.81 us at the decode shape).
__global__ __launch_bounds__(kDownSplit * kWave) void dense_down_residual_kernel(DownArgs a) {
  __shared__ float partial[kDownSplit];
  const int lane = threadIdx.x % kWave;
  const int part = threadIdx.x / kWave;
  const int row = blockIdx.x;  // the grid is exactly `hidden` workgroups
  // The residual, loaded ahead of the row (every thread reads the same value; thread 0
  // uses it after the barrier).
  const uint16_t resid_raw = a.residual[row];
  const int per = (a.vecs + kDownSplit - 1) / kDownSplit;
  const int lo = part * per;
  const int hi = min(a.vecs, lo + per);
  const u32x4* wrow = a.w + static_cast<int64_t>(row) * a.vecs;
  float acc = 0.0f;
  for (int base = lo; base < hi; base += kDownChunk * kWave) {
    u32x4 xv[kDownChunk], wv[kDownChunk];
#pragma unroll
    for (int i = 0; i < kDownChunk; ++i) {
      const int v = base + lane + i * kWave;
      xv[i] = u32x4{0u, 0u, 0u, 0u};
      wv[i] = u32x4{0u, 0u, 0u, 0u};
      if (v < hi) {
        xv[i] = a.act[v];
        wv[i] = load_nt(wrow + v);
      }
    }
#pragma unroll
    for (int i = 0; i < kDownChunk; ++i) {
      float xf[8], wf[8];
      unpack8(xv[i], xf);
      unpack8(wv[i], wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(xf[j], wf[j], acc);
    }
  }
  acc = wave_total(acc);
  if (lane == 0) partial[part] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = partial[0];
#pragma unroll
    for (int p = 1; p < kDownSplit; ++p) sum += partial[p];
    a.out[row] = f32_to_bf16(bf16_to_f32(resid_raw) + round_bf16(sum));
  }
}

template <int VPL>
void launch_gate_up(const GateUpArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.inner + kWavesPerBlock - 1) / kWavesPerBlock));
  dense_gate_up_swiglu_kernel<VPL><<<grid, kWavesPerBlock * kWave, 0, stream>>>(a.x, a.w, a.out, a.inner,
                                                                               a.vecs);
}

using GateUpLauncher = void (*)(const GateUpArgs&, hipStream_t);
constexpr GateUpLauncher kGateUpLaunchers[kMaxVectorsPerLane] = {
    launch_gate_up<1>,  launch_gate_up<2>,  launch_gate_up<3>,  launch_gate_up<4>,
    launch_gate_up<5>,  launch_gate_up<6>,  launch_gate_up<7>,  launch_gate_up<8>,
    launch_gate_up<9>,  launch_gate_up<10>, launch_gate_up<11>, launch_gate_up<12>,
    launch_gate_up<13>, launch_gate_up<14>, launch_gate_up<15>, launch_gate_up<16>};

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_dense_gate_up_swiglu(const uint16_t* x, const uint16_t* fused_weight,
                                              int64_t hidden, int64_t inner, uint16_t* activated,
                                              hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= 8 * kWave * kMaxVectorsPerLane,
                "dense_gate_up_swiglu: hidden must be a multiple of 8 in [8, 8192]");
  OMNIA_REQUIRE(inner > 0 && inner < (int64_t{1} << 24), "dense_gate_up_swiglu: bad inner size");
  OMNIA_REQUIRE(x && fused_weight && activated, "dense_gate_up_swiglu: null pointer");
  OMNIA_REQUIRE(aligned16(x) && aligned16(fused_weight),
                "dense_gate_up_swiglu: x and the weight must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const int vecs = static_cast<int>(hidden / 8);
  GateUpArgs a{reinterpret_cast<const u32x4*>(x), reinterpret_cast<const u32x4*>(fused_weight),
               activated, static_cast<int>(inner), vecs};
  kGateUpLaunchers[(vecs + kWave - 1) / kWave - 1](a, stream);
  return launched("dense_gate_up_swiglu");
}

extern "C" int32_t omnia_dense_down_residual(const uint16_t* activated, const uint16_t* down_weight,
                                             const uint16_t* residual, int64_t hidden,
                                             int64_t inner, uint16_t* out, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(hidden > 0 && hidden < (int64_t{1} << 24), "dense_down_residual: bad hidden size");
  OMNIA_REQUIRE(inner > 0 && inner % 8 == 0 && inner < (int64_t{1} << 24),
                "dense_down_residual: inner must be a positive multiple of 8");
  OMNIA_REQUIRE(activated && down_weight && residual && out, "dense_down_residual: null pointer");
  OMNIA_REQUIRE(aligned16(activated) && aligned16(down_weight),
                "dense_down_residual: the activation and the weight must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  DownArgs a{reinterpret_cast<const u32x4*>(activated), reinterpret_cast<const u32x4*>(down_weight),
             residual, out, static_cast<int>(hidden), static_cast<int>(inner / 8)};
  dense_down_residual_kernel<<<dim3(static_cast<unsigned>(hidden)), kDownSplit * kWave, 0, stream>>>(a);
  return launched("dense_down_residual");
}
