// Routed expert MLP of a one-token step, dense bf16 weights: the gate/up projection of the
// chosen experts and the down projection with the SwiGLU and the routing combine fused.
//
// Arithmetic (the dense bindings core/kernels/gate_up/dense.py:21-135 and
// core/kernels/down_combine/dense.py:21-117, "blocked" layout: gate and up block-
// concatenated on the output axis, the activation computed by the down half):
//   gate_up:  y[j, n] = bf16(sum_h x_h * W_gu[c_j, n, h])           n < 2I, fp32 sum
//   down:     a_i    = g_i / (1 + exp(-g_i)) * u_i   (fp32, g = y[j, i], u = y[j, I + i])
//             d[j, n] = bf16(fp32(sum_i a_i * W_dn[c_j, n, i]) * w_j)   fp32 sum
//             out[n]  = bf16(bf16(sum_j d[j, n]) + residual[n])    (sum over j in order)
// matching the reference's `(T)(t * scale)` per expert, then `routed.sum(axis=0) +
// residual` in bf16 ops. The fp32 sums' order is free (the reference's own is a float4
// lane sweep and a simd reduction). An expert id outside [0, experts) contributes a zero
// row: the kernels never read outside the weight stack.
//
// Layout. gate_up: a wave streams kRowsPerWave (2) rows of one chosen expert; lane l owns the
// 16-byte vectors l, l + 64, ... of a row (a row of H bf16 is H / 8 vectors), so each
// load instruction covers 1 KiB of contiguous memory and a wave keeps 2 rows x 4 KiB in
// flight at H = 2048. x is read once per wave (L2-resident). Each row's fp32 sum is a
// wave reduction in vector registers (DPP and permlane swaps).
// down: a workgroup owns kDownRows output rows and has one wave per chosen expert; the
// wave computes its expert's activation once (the lane's slice of I, kept in registers)
// and reuses it for all the rows. Lanes l and l + 32 own the same slice of I, so each
// evaluates half of its elements and the two swap results. Half-waves then take one row
// each (32 lanes x 16-byte vectors over I), reduce it, scale and round it, and leave it
// in LDS; after a barrier one lane per row adds the experts in order and the residual.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kRowsPerWave = 2;         // gate_up rows per wave (4: 10.2 us, 2: 9.6 us, 1: 10.4 us at the config)
constexpr int kDownRows = 4;            // down output rows per workgroup (8: 7.1 us, 4: 6.9 us, 2: 7.5 us)
constexpr int kMaxVectorsPerLane = 16;  // gate_up: hidden <= 8192
constexpr int kMaxDownVectors = 8;      // down: inner <= 2048 (the activation slice stays in registers)
constexpr int kMaxSlots = 16;           // chosen experts per token (down: one wave each)
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float fsum_row16(float v) {
  v += __uint_as_float(dpp<kRowRor8>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor4>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor1>(__float_as_uint(v)));
  return v;
}

// Sum over each 32-lane half of the wave, the same in every lane of the half.
__device__ __forceinline__ float fsum_half(float v) {
  v = fsum_row16(v);
  uint32_t a, b;
  row_pair(__float_as_uint(v), a, b);
  return __uint_as_float(a) + __uint_as_float(b);
}

// Sum over the wave, the same in every lane.
__device__ __forceinline__ float fsum_wave(float v) {
  v = fsum_half(v);
  uint32_t a, b;
  half_pair(__float_as_uint(v), a, b);
  return __uint_as_float(a) + __uint_as_float(b);
}

struct GateUpArgs {
  const u32x4* x;        // [H / 8]
  const uint16_t* w;     // [experts, rows, H]
  const int32_t* chosen; // [k]
  uint16_t* out;         // [k, rows]
  int64_t experts;
  int rows;              // 2 * inner
  int vecs;              // H / 8
  int k;
  int waves_per_slot;
};

// The arguments as scalars (GateUpArgs field by field, 14 dwords): gfx950 preloads a
// kernel's leading scalar and pointer arguments into SGPRs at wave launch (14 dwords at
// most), so the first loads go out with no scalar round trip ahead of them.
template <int VPL>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void moe_gate_up_kernel(
    const u32x4* x, const uint16_t* weight, const int32_t* chosen, int64_t experts, int rows,
    int vecs, int k, int waves_per_slot, uint16_t* out) {
  const GateUpArgs a{x, weight, chosen, out, experts, rows, vecs, k, waves_per_slot};
  const int lane = threadIdx.x % kWave;
  // Uniform, so the slot's expert id is a scalar load, waited on without the
  // activation loads issued beside it.
  const int wave = __builtin_amdgcn_readfirstlane(
      static_cast<int>(blockIdx.x * kWavesPerBlock + threadIdx.x / kWave));
  const int slot = wave / a.waves_per_slot;
  if (slot >= a.k) return;  // whole wave; no barrier follows
  const int row0 = (wave - slot * a.waves_per_slot) * kRowsPerWave;
  const int64_t expert = a.chosen[slot];
  const bool valid = expert >= 0 && expert < a.experts;  // wave-uniform
  const u32x4* w = reinterpret_cast<const u32x4*>(a.w) +
                   (valid ? expert : 0) * a.rows * static_cast<int64_t>(a.vecs);
  // Rows in flight together: all four while the vectors fit the register budget.
  constexpr int kGroup = VPL <= 8 ? kRowsPerWave : 1;
  u32x4 xv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {   // branch-free: a lane past the row reads its last vector
    const int v = lane + i * kWave;
    const u32x4 loaded = a.x[min(v, a.vecs - 1)];
    xv[i] = v < a.vecs ? loaded : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int r0 = 0; r0 < kRowsPerWave; r0 += kGroup) {
    u32x4 wv[kGroup][VPL];
#pragma unroll
    for (int r = 0; r < kGroup; ++r) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int v = lane + i * kWave;
        wv[r][i] = u32x4{0u, 0u, 0u, 0u};
        if (valid && row0 + r0 + r < a.rows && v < a.vecs) {
          wv[r][i] = load_nt(w + static_cast<int64_t>(row0 + r0 + r) * a.vecs + v);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kGroup; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float xf[8], wf[8];
        unpack8(xv[i], xf);
        unpack8(wv[r][i], wf);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(xf[j], wf[j], acc);
      }
      acc = fsum_wave(acc);
      if (lane == 0 && row0 + r0 + r < a.rows) {
        a.out[static_cast<int64_t>(slot) * a.rows + row0 + r0 + r] = f32_to_bf16(acc);
      }
    }
  }
}

struct DownArgs {
  const uint16_t* act;      // [k, 2 * inner]: gate || up
  const uint16_t* w;        // [experts, hidden, inner]
  const int32_t* chosen;    // [k]
  const float* weights;     // [k]
  const uint16_t* residual; // [hidden] or null
  uint16_t* out;            // [hidden]
  int64_t experts;
  int hidden;
  int inner;
  int vecs;                 // inner / 8
  int k;
};

// The arguments as scalars, those the first loads need first (14 dwords; inner is
// 8 * vecs): gfx950 preloads a kernel's leading scalar and pointer arguments into SGPRs
// at wave launch, so the first loads go out with no scalar round trip ahead of them; k and
// `out`, needed by the epilogue, are loaded meanwhile.
template <int VPL>
__global__ __launch_bounds__(kMaxSlots * kWave) void moe_down_kernel(
    const uint16_t* act_in, const uint16_t* weight, const int32_t* chosen, const float* weights,
    const uint16_t* residual, int64_t experts, int hidden, int vecs, int k, uint16_t* out) {
  const DownArgs a{act_in, weight, chosen, weights, residual, out, experts, hidden, 8 * vecs, vecs, k};
  __shared__ float partial[kMaxSlots][kDownRows];
  const int lane = threadIdx.x % kWave;
  // One wave per chosen expert (blockDim = k waves); uniform, so its routing entries
  // are scalar loads.
  const int slot = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int half = lane / 32;
  const int hl = lane % 32;
  const int row_base = blockIdx.x * kDownRows;
  const int64_t expert = a.chosen[slot];
  const bool valid = expert >= 0 && expert < a.experts;  // wave-uniform
  const float scale = a.weights[slot];
  // The residual of the output row this thread writes at the end (rows past the last
  // read the last).
  const uint32_t resid = early_bf16_bits(
      a.residual, min(row_base + static_cast<int>(threadIdx.x % kDownRows), a.hidden - 1), a.act);

  // The lane's slice of the pair block (elements (hl + 32 i) * 8 + j of I) is loaded
  // first, then the first group of weight rows; the activation is computed while the
  // weight loads are in flight (vector-memory results are counted in issue order, so the
  // wait for the block leaves the weight loads outstanding). With an even VPL the upper
  // half of the wave loads its vectors rotated by VPL / 2 (slot i holds vector
  // i + VPL / 2, modulo VPL), so the half of the elements it activates sits at the same
  // indices as the lower half's: no per-lane select between array elements, which the
  // compiler folded into one lane-dependent index and moved the arrays to scratch memory.
  constexpr bool kRotated = VPL % 2 == 0;
  const int rotation = kRotated ? half * (VPL / 2) : 0;
  u32x4 gate_raw[VPL], up_raw[VPL];
  {
    const uint16_t* gate = a.act + static_cast<int64_t>(slot) * 2 * a.inner;
    const uint16_t* up = gate + a.inner;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int slot_vector = i + rotation < VPL ? i + rotation : i + rotation - VPL;
      const int v = hl + slot_vector * 32;
      const bool in = v < a.vecs;
      gate_raw[i] = in ? *reinterpret_cast<const u32x4*>(gate + v * 8) : u32x4{0u, 0u, 0u, 0u};
      up_raw[i] = in ? *reinterpret_cast<const u32x4*>(up + v * 8) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  const u32x4* w = reinterpret_cast<const u32x4*>(a.w) +
                   (valid ? expert : 0) * a.hidden * static_cast<int64_t>(a.vecs);
  // Row pairs in flight together: all of the workgroup's while the vectors fit the
  // 128-register budget of a 16-wave workgroup.
  constexpr int kGroupWanted = VPL <= 4 ? 4 : (VPL <= 6 ? 2 : 1);
  constexpr int kGroup = kGroupWanted < kDownRows / 2 ? kGroupWanted : kDownRows / 2;
  auto load_group = [&](int p0, u32x4 (&wv)[kGroup][VPL]) {
#pragma unroll
    for (int p = 0; p < kGroup; ++p) {
      const int n = row_base + (p0 + p) * 2 + half;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int v = hl + i * 32;
        wv[p][i] = u32x4{0u, 0u, 0u, 0u};
        if (valid && n < a.hidden && v < a.vecs) wv[p][i] = load_nt(w + static_cast<int64_t>(n) * a.vecs + v);
      }
    }
  };
  u32x4 wv[kGroup][VPL];
  load_group(0, wv);
  // Both halves of the wave hold the same slice; each computes half of it (flat
  // elements [half * 4 VPL, (half + 1) * 4 VPL)) and the halves swap results.
  float act[VPL][8];
  {
    float g[VPL * 8], u[VPL * 8];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      unpack8(gate_raw[i], g + i * 8);
      unpack8(up_raw[i], u + i * 8);
    }
    constexpr int kHalf = VPL * 4;
#pragma unroll
    for (int f = 0; f < kHalf; ++f) {
      const float gf = kRotated ? g[f] : (half ? g[f + kHalf] : g[f]);
      const float uf = kRotated ? u[f] : (half ? u[f + kHalf] : u[f]);
      // exp(-g) as v_exp_f32 of -g log2(e), the division as v_rcp_f32: a few ulps in fp32,
      // far below the bf16 rounding of the projection they feed.
      const float mine = gf * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gf * kLog2e)) * uf;
      uint32_t lower, upper;  // the lower half's value and the upper half's
      half_pair(__float_as_uint(mine), lower, upper);
      act[f / 8][f % 8] = __uint_as_float(lower);
      act[(f + kHalf) / 8][(f + kHalf) % 8] = __uint_as_float(upper);
    }
  }
#pragma unroll
  for (int p0 = 0; p0 < kDownRows / 2; p0 += kGroup) {
    if (p0 > 0) load_group(p0, wv);
#pragma unroll
    for (int p = 0; p < kGroup; ++p) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float wf[8];
        unpack8(wv[p][i], wf);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(act[i][j], wf[j], acc);
      }
      acc = fsum_half(acc);
      if (hl == 0) {
        partial[slot][(p0 + p) * 2 + half] = valid ? bf16_to_f32(f32_to_bf16(acc * scale)) : 0.0f;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < kDownRows) {
    const int n = row_base + threadIdx.x;
    if (n < a.hidden) {
      float sum = 0.0f;
      for (int j = 0; j < a.k; ++j) sum += partial[j][threadIdx.x];
      float out = round_bf16(sum);
      if (a.residual != nullptr) out = out + bf16_to_f32(resid);
      a.out[n] = f32_to_bf16(out);
    }
  }
}

template <int VPL>
void launch_gate_up(const GateUpArgs& a, hipStream_t stream) {
  const int64_t waves = static_cast<int64_t>(a.k) * a.waves_per_slot;
  const dim3 grid(static_cast<unsigned>((waves + kWavesPerBlock - 1) / kWavesPerBlock));
  moe_gate_up_kernel<VPL><<<grid, kWavesPerBlock * kWave, 0, stream>>>(
      a.x, a.w, a.chosen, a.experts, a.rows, a.vecs, a.k, a.waves_per_slot, a.out);
}

template <int VPL>
void launch_down(const DownArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.hidden + kDownRows - 1) / kDownRows));
  moe_down_kernel<VPL><<<grid, a.k * kWave, 0, stream>>>(a.act, a.w, a.chosen, a.weights, a.residual,
                                                         a.experts, a.hidden, a.vecs, a.k, a.out);
}

using GateUpLauncher = void (*)(const GateUpArgs&, hipStream_t);
constexpr GateUpLauncher kGateUpLaunchers[kMaxVectorsPerLane] = {
    launch_gate_up<1>,  launch_gate_up<2>,  launch_gate_up<3>,  launch_gate_up<4>,
    launch_gate_up<5>,  launch_gate_up<6>,  launch_gate_up<7>,  launch_gate_up<8>,
    launch_gate_up<9>,  launch_gate_up<10>, launch_gate_up<11>, launch_gate_up<12>,
    launch_gate_up<13>, launch_gate_up<14>, launch_gate_up<15>, launch_gate_up<16>};

using DownLauncher = void (*)(const DownArgs&, hipStream_t);
constexpr DownLauncher kDownLaunchers[kMaxDownVectors] = {
    launch_down<1>, launch_down<2>, launch_down<3>, launch_down<4>,
    launch_down<5>, launch_down<6>, launch_down<7>, launch_down<8>};

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_moe_gate_up(const uint16_t* x, const uint16_t* weight, int64_t experts,
                                     int64_t rows, int64_t hidden, const int32_t* chosen,
                                     int64_t k, uint16_t* out, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(experts > 0 && experts < (int64_t{1} << 20), "moe_gate_up: bad expert count");
  OMNIA_REQUIRE(rows > 0 && rows < (int64_t{1} << 24), "moe_gate_up: bad row count");
  OMNIA_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= 8 * kWave * kMaxVectorsPerLane,
                "moe_gate_up: hidden must be a multiple of 8 in [8, 8192]");
  OMNIA_REQUIRE(k >= 0 && k <= 1024, "moe_gate_up: k must be in [0, 1024]");
  if (k == 0) return 0;
  OMNIA_REQUIRE(x && weight && chosen && out, "moe_gate_up: null pointer");
  OMNIA_REQUIRE(aligned16(x) && aligned16(weight), "moe_gate_up: x and weight must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const int vecs = static_cast<int>(hidden / 8);
  GateUpArgs a{reinterpret_cast<const u32x4*>(x), weight, chosen, out, experts,
               static_cast<int>(rows), vecs, static_cast<int>(k),
               static_cast<int>((rows + kRowsPerWave - 1) / kRowsPerWave)};
  kGateUpLaunchers[(vecs + kWave - 1) / kWave - 1](a, stream);
  return launched("moe_gate_up");
}

extern "C" int32_t omnia_moe_down_combine(const uint16_t* act, const uint16_t* weight,
                                          int64_t experts, int64_t hidden, int64_t inner,
                                          const int32_t* chosen, const float* weights,
                                          int64_t k, const uint16_t* residual, uint16_t* out,
                                          hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(experts > 0 && experts < (int64_t{1} << 20), "moe_down_combine: bad expert count");
  OMNIA_REQUIRE(hidden > 0 && hidden < (int64_t{1} << 24), "moe_down_combine: bad hidden size");
  OMNIA_REQUIRE(inner > 0 && inner % 8 == 0 && inner <= 8 * 32 * kMaxDownVectors,
                "moe_down_combine: inner must be a multiple of 8 in [8, 2048]");
  OMNIA_REQUIRE(k > 0 && k <= kMaxSlots, "moe_down_combine: k must be in [1, 16]");
  OMNIA_REQUIRE(act && weight && chosen && weights && out, "moe_down_combine: null pointer");
  OMNIA_REQUIRE(aligned16(act) && aligned16(weight),
                "moe_down_combine: act and weight must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const int vecs = static_cast<int>(inner / 8);
  DownArgs a{act, weight, chosen, weights, residual, out, experts, static_cast<int>(hidden),
             static_cast<int>(inner), vecs, static_cast<int>(k)};
  kDownLaunchers[(vecs + 31) / 32 - 1](a, stream);
  return launched("moe_down_combine");
}
