// Gated activations: SwiGLU and the DeltaNet gate-softplus.
//
// SwiGLU (core/layers.py:249-250,284-287 `gate * mx.sigmoid(gate) * up`, three bf16
// ops, each rounding its result):
//   s = bf16(sigmoid(g)),  t = bf16(g * s),  y = bf16(t * u)
// s is the correctly rounded bf16 of the sigmoid of the bf16 input. It is evaluated in
// fp32 from the hardware 2^x with the exponent split into a high part and its exact
// residual (error <= ~5 fp32 ulp); when that value lies within 16 fp32 ulp of a bf16
// rounding midpoint (about one element in 2000), or |g| > 80, the sigmoid is
// recomputed in fp64 and rounded straight from fp64, behind one branch per vector and
// out of line, so the common path stays at the streaming-copy speed. g * s and t * u are products of
// two bf16 values, exact in fp32, so y is fully determined: the kernel is bit-exact
// against any correctly rounded restatement of the chain.
//
// Gate-softplus (models/qwen3_5/layers/deltanet.py:222-224):
//   dt = f32(a) + dt_bias;  g = -exp(A_log) * softplus(dt)       all fp32
// with softplus = mx.logaddexp(dt, 0) = max + log1p(exp(min - max)) and its inf/NaN
// arms (the lowering core/kernels/qmv/softplus.py:64-76 restates). Each fp32 step is
// evaluated in fp64 and rounded once, so it is correctly rounded; the data (a [T, 32]
// bf16) is small and the extra fp64 work is hidden behind memory latency.
//
// Layout: 16-byte vectors of 8 bf16; SwiGLU streams the flat array (or row-strided
// views, e.g. the two halves of a fused [T, 2I] projection) with one vector per lane,
// the pattern measured fastest for a streaming copy on MI355X.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kBlock = 256;

// sigmoid(g) in fp32 from the hardware 2^x, the exponent split into a high part and
// its exact residual: within about 5 fp32 ulp of the true value. `hard` is set when
// that is not enough to decide the bf16 rounding: the value lies within 16 fp32 ulp of
// a bf16 rounding midpoint, or |g| > 80 (or g is NaN).
__device__ __forceinline__ float sigmoid_fast(float g, bool& hard) {
  constexpr float kLog2e = 1.44269502162933349609375f;       // fp32(log2 e)
  constexpr float kLog2eLo = 1.925963033500011079101241e-8f;  // log2 e - kLog2e
  constexpr float kLn2 = 0.693147180559945309417232f;
  const float a = fabsf(g);
  const float xh = -a * kLog2e;
  const float xl = __builtin_fmaf(-a, kLog2eLo, __builtin_fmaf(-a, kLog2e, -xh));
  const float p = __builtin_amdgcn_exp2f(xh);
  const float e = __builtin_fmaf(p, xl * kLn2, p);              // exp(-|g|)
  const float s = (g >= 0.0f ? 1.0f : e) * __builtin_amdgcn_rcpf(1.0f + e);
  const uint32_t low = __float_as_uint(s) & 0xFFFFu;
  hard = !(a <= 80.0f) || low - 0x7FF0u <= 0x20u;
  return s;
}

// The correctly rounded bf16 of sigmoid(g) (as fp32), from fp64.
__device__ __attribute__((noinline)) float sigmoid_exact(float g) {
  const double ed = exp(-static_cast<double>(fabsf(g)));
  const double sd = (g >= 0.0f ? 1.0 : ed) / (1.0 + ed);
  return bf16_to_f32(static_cast<uint16_t>(f64_to_bf16(sd)));
}

__device__ __forceinline__ u32x4 swiglu8(const u32x4& gate, const u32x4& up) {
  float g[8], u[8], s[8], y[8];
  unpack8(gate, g);
  unpack8(up, u);
  uint32_t hard_mask = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    bool hard;
    s[j] = sigmoid_fast(g[j], hard);
    hard_mask |= static_cast<uint32_t>(hard) << j;
  }
  // About one element in 2000 needs the fp64 evaluation; one branch per vector.
  if (hard_mask != 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (hard_mask & (1u << j)) s[j] = sigmoid_exact(g[j]);  // already a bf16 value
    }
  }
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    round_pair(s[j], s[j + 1]);
    float t0 = g[j] * s[j], t1 = g[j + 1] * s[j + 1];
    round_pair(t0, t1);
    y[j] = t0 * u[j];
    y[j + 1] = t1 * u[j + 1];
  }
  return pack8(y);
}

// Contiguous gate, up and out: one vector per lane over the flat array.
__global__ __launch_bounds__(kBlock) void swiglu_flat_kernel(const u32x4* __restrict__ gate,
                                                             const u32x4* __restrict__ up,
                                                             u32x4* __restrict__ out,
                                                             int64_t vectors) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= vectors) return;
  const u32x4 g = load_nt(gate + i);
  const u32x4 u = load_nt(up + i);
  store_nt(out + i, swiglu8(g, u));
}

// Row-strided gate and up (e.g. halves of a fused projection), contiguous out.
__global__ __launch_bounds__(kBlock) void swiglu_rows_kernel(const uint16_t* __restrict__ gate,
                                                             int64_t gate_stride,
                                                             const uint16_t* __restrict__ up,
                                                             int64_t up_stride,
                                                             uint16_t* __restrict__ out,
                                                             int64_t rows, uint32_t row_vectors) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= rows * row_vectors) return;
  const int64_t r = i / row_vectors;
  const int64_t c = (i - r * row_vectors) * 8;
  const u32x4 g = load_nt(reinterpret_cast<const u32x4*>(gate + r * gate_stride + c));
  const u32x4 u = load_nt(reinterpret_cast<const u32x4*>(up + r * up_stride + c));
  store_nt(reinterpret_cast<u32x4*>(out + r * row_vectors * 8 + c), swiglu8(g, u));
}

// softplus(dt) as mx.logaddexp(dt, 0): max + log1p(exp(min - max)), each fp32 step
// correctly rounded (evaluated in fp64, rounded once).
__device__ __forceinline__ float softplus_f32(float dt) {
  const float maxval = dt > 0.0f ? dt : 0.0f;
  const float minval = dt > 0.0f ? 0.0f : dt;
  if (minval == -__builtin_huge_valf() || maxval == __builtin_huge_valf()) return maxval;
  const float r1 = static_cast<float>(exp(static_cast<double>(minval - maxval)));
  const float r2 = static_cast<float>(log1p(static_cast<double>(r1)));
  return maxval + r2;
}

__device__ __forceinline__ float gate_softplus1(float a, float a_log, float dt_bias) {
  const float dt = a + dt_bias;
  const float decay = -static_cast<float>(exp(static_cast<double>(a_log)));
  return decay * softplus_f32(dt);
}

// Even head count, 4-byte aligned rows: one pair of heads per lane. The tensor is small
// (1.5 MB at the config) and each element carries fp64 transcendentals, so the grid is
// spread wide rather than vectorised deep, and nothing divides: a block of kBlock threads
// is 2^lane_bits head pairs (the power of two >= heads / 2, at most kBlock) by the rest
// in rows, block b taking row block b / column_blocks and pair block b % column_blocks.
// With at most kDecayHeads heads, the block holds -exp(A_log) of every head in LDS,
// computed once per block rather than once per element (one fp64 exp of three).
struct SoftplusArgs {
  const uint16_t* a;
  int64_t a_stride;
  const float* a_log;
  const float* dt_bias;
  float* out;
  int64_t rows;
  int heads;
  int lane_bits;
  unsigned column_blocks;
};

constexpr int kDecayHeads = kBlock;

__device__ __forceinline__ void softplus_block(const SoftplusArgs& p, unsigned b, float* decay) {
  const int head_pairs = p.heads / 2;
  const bool cached = p.heads <= kDecayHeads;   // then column_blocks == 1
  unsigned row_block = b, column_block = 0;
  if (p.column_blocks > 1) {   // block-uniform
    row_block = b / p.column_blocks;
    column_block = b - row_block * p.column_blocks;
  }
  const int pair = static_cast<int>(column_block << p.lane_bits) + static_cast<int>(threadIdx.x & ((1u << p.lane_bits) - 1));
  const int64_t row = static_cast<int64_t>(row_block) * (kBlock >> p.lane_bits) + (threadIdx.x >> p.lane_bits);
  const bool live = pair < head_pairs && row < p.rows;
  // Every load first, with no branch among them (a thread past the end reads the last
  // pair and leaves before any store): A_log for the decay table first, so that its
  // wait leaves the others in flight while the table's fp64 exps run.
  const int h = min(pair, head_pairs - 1) * 2;
  const int64_t r = min(row, p.rows - 1);
  const float table_log = p.a_log[min(static_cast<int>(threadIdx.x), p.heads - 1)];
  const f32x2 bb = *reinterpret_cast<const f32x2*>(p.dt_bias + h);
  const uint32_t x = *reinterpret_cast<const uint32_t*>(p.a + r * p.a_stride + h);
  __builtin_amdgcn_sched_barrier(0);   // the loads in this order, ahead of the arithmetic
  // `out` taken now: where it is an argument past the preloaded ones, its load otherwise
  // went out at the store, one scalar round trip at the end.
  asm volatile("" ::"s"(p.out));
  if (cached && static_cast<int>(threadIdx.x) < p.heads) {
    decay[threadIdx.x] = -static_cast<float>(exp(static_cast<double>(table_log)));
  }
  lds_barrier();   // the table is LDS; the loads above stay in flight
  if (!live) return;
  f32x2 o;
  if (cached) {  // the same fp32 steps as gate_softplus1
    o = f32x2{decay[h] * softplus_f32(bf16_lo(x) + bb.x), decay[h + 1] * softplus_f32(bf16_hi(x) + bb.y)};
  } else {
    const f32x2 la = *reinterpret_cast<const f32x2*>(p.a_log + h);
    o = f32x2{gate_softplus1(bf16_lo(x), la.x, bb.x), gate_softplus1(bf16_hi(x), la.y, bb.y)};
  }
  *reinterpret_cast<f32x2*>(p.out + r * p.heads + h) = o;
}

// The arguments as scalars, `out` last: gfx950 preloads a kernel's leading scalar and
// pointer arguments into SGPRs at wave launch (14 dwords at most), so every input load
// goes out with no scalar round trip ahead of it; `out`, needed only by the store, is
// loaded meanwhile.
__global__ __launch_bounds__(kBlock) void gate_softplus_kernel(
    const uint16_t* a, int64_t a_stride, const float* a_log, const float* dt_bias, int64_t rows,
    int heads, int lane_bits, unsigned column_blocks, float* out) {
  __shared__ float decay[kDecayHeads];
  softplus_block(SoftplusArgs{a, a_stride, a_log, dt_bias, out, rows, heads, lane_bits, column_blocks},
                 blockIdx.x, decay);
}

// Any head count or alignment: one element per lane.
__global__ __launch_bounds__(kBlock) void gate_softplus_scalar_kernel(
    const uint16_t* __restrict__ a, int64_t a_stride, const float* __restrict__ a_log,
    const float* __restrict__ dt_bias, float* __restrict__ out, int64_t rows, int heads) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= rows * heads) return;
  const int64_t r = i / heads;
  const int h = static_cast<int>(i - r * heads);
  out[i] = gate_softplus1(bf16_to_f32(a[r * a_stride + h]), a_log[h], dt_bias[h]);
}

unsigned blocks_for(int64_t items) {
  return static_cast<unsigned>((items + kBlock - 1) / kBlock);
}

// The gate-softplus grid over rows x heads / 2 pairs (heads even, positive).
struct SoftplusGrid {
  int lane_bits;
  unsigned column_blocks;
  int64_t blocks;
};

SoftplusGrid softplus_grid(int64_t rows, int64_t heads) {
  const int64_t pairs = heads / 2;
  int bits = 0;
  while ((int64_t{1} << bits) < pairs && (1 << bits) < kBlock) ++bits;
  const int64_t column_blocks = (pairs + (int64_t{1} << bits) - 1) >> bits;
  const int64_t rows_per_block = kBlock >> bits;
  return SoftplusGrid{bits, static_cast<unsigned>(column_blocks),
                      (rows + rows_per_block - 1) / rows_per_block * column_blocks};
}

// Both gated activations of a layer in one grid (the SwiGLU and the gate-softplus of
// configs[3]): blocks [0, softplus_blocks) run the gate-softplus, one pair of heads per
// lane as gate_softplus_kernel does; the rest stream the SwiGLU, one vector per lane as
// swiglu_flat_kernel / swiglu_rows_kernel do. The gate-softplus blocks come first, so
// their fp64 work runs beside the SwiGLU stream rather than after its last blocks.
struct GatedArgs {
  const uint16_t* gate;
  int64_t gate_stride;
  const uint16_t* up;
  int64_t up_stride;
  uint16_t* y;
  int64_t rows;
  uint32_t row_vectors;
  int64_t vectors;
  SoftplusArgs softplus;
  unsigned softplus_blocks;
};

template <bool kFlat>
__global__ __launch_bounds__(kBlock) void gated_activations_kernel(GatedArgs p) {
  if (blockIdx.x < p.softplus_blocks) {  // block-uniform
    __shared__ float decay[kDecayHeads];
    softplus_block(p.softplus, blockIdx.x, decay);
    return;
  }
  const int64_t i = static_cast<int64_t>(blockIdx.x - p.softplus_blocks) * kBlock + threadIdx.x;
  if (i >= p.vectors) return;
  if constexpr (kFlat) {
    const u32x4 g = load_nt(reinterpret_cast<const u32x4*>(p.gate) + i);
    const u32x4 u = load_nt(reinterpret_cast<const u32x4*>(p.up) + i);
    store_nt(reinterpret_cast<u32x4*>(p.y) + i, swiglu8(g, u));
  } else {
    const int64_t r = i / p.row_vectors;
    const int64_t c = (i - r * p.row_vectors) * 8;
    const u32x4 g = load_nt(reinterpret_cast<const u32x4*>(p.gate + r * p.gate_stride + c));
    const u32x4 u = load_nt(reinterpret_cast<const u32x4*>(p.up + r * p.up_stride + c));
    store_nt(reinterpret_cast<u32x4*>(p.y + r * p.row_vectors * 8 + c), swiglu8(g, u));
  }
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_swiglu(const uint16_t* gate, int64_t gate_stride, const uint16_t* up,
                                int64_t up_stride, uint16_t* out, int64_t rows,
                                int64_t inner, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && inner > 0 && inner % 8 == 0,
                "swiglu: inner must be a positive multiple of 8");
  OMNIA_REQUIRE(gate_stride >= inner && up_stride >= inner && gate_stride % 8 == 0 &&
                    up_stride % 8 == 0,
                "swiglu: row strides must be >= inner and multiples of 8");
  OMNIA_REQUIRE(rows * (inner / 8) < (int64_t{1} << 40), "swiglu: too large");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(gate && up && out, "swiglu: null pointer");
  OMNIA_REQUIRE(aligned16(gate) && aligned16(up) && aligned16(out),
                "swiglu: pointers must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const int64_t vectors = rows * (inner / 8);
  OMNIA_REQUIRE(vectors / kBlock < (int64_t{1} << 31), "swiglu: grid too large");
  if (gate_stride == inner && up_stride == inner) {
    swiglu_flat_kernel<<<blocks_for(vectors), kBlock, 0, stream>>>(
        reinterpret_cast<const u32x4*>(gate), reinterpret_cast<const u32x4*>(up),
        reinterpret_cast<u32x4*>(out), vectors);
  } else {
    OMNIA_REQUIRE(inner / 8 < (int64_t{1} << 31), "swiglu: rows too wide");
    swiglu_rows_kernel<<<blocks_for(vectors), kBlock, 0, stream>>>(
        gate, gate_stride, up, up_stride, out, rows, static_cast<uint32_t>(inner / 8));
  }
  return launched("swiglu");
}

extern "C" int32_t omnia_gate_softplus(const uint16_t* a, int64_t a_stride, const float* a_log,
                                       const float* dt_bias, float* out, int64_t rows,
                                       int64_t heads, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && heads > 0 && heads <= (int64_t{1} << 20),
                "gate_softplus: bad heads");
  OMNIA_REQUIRE(a_stride >= heads, "gate_softplus: row stride smaller than heads");
  OMNIA_REQUIRE(rows * heads < (int64_t{1} << 40), "gate_softplus: too large");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(a && a_log && dt_bias && out, "gate_softplus: null pointer");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const auto aligned = [](const void* p, uintptr_t n) {
    return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0;
  };
  const bool paired = heads % 2 == 0 && a_stride % 2 == 0 && aligned(a, 4) &&
                      aligned(a_log, 8) && aligned(dt_bias, 8) && aligned(out, 8);
  if (paired) {
    const SoftplusGrid grid = softplus_grid(rows, heads);
    OMNIA_REQUIRE(grid.blocks < (int64_t{1} << 31), "gate_softplus: grid too large");
    gate_softplus_kernel<<<static_cast<unsigned>(grid.blocks), kBlock, 0, stream>>>(
        a, a_stride, a_log, dt_bias, rows, static_cast<int>(heads), grid.lane_bits, grid.column_blocks,
        out);
  } else {
    gate_softplus_scalar_kernel<<<blocks_for(rows * heads), kBlock, 0, stream>>>(
        a, a_stride, a_log, dt_bias, out, rows, static_cast<int>(heads));
  }
  return launched("gate_softplus");
}

extern "C" int32_t omnia_gated_activations(const uint16_t* gate, int64_t gate_stride,
                                           const uint16_t* up, int64_t up_stride, uint16_t* y,
                                           int64_t rows, int64_t inner, const uint16_t* a,
                                           int64_t a_stride, const float* a_log,
                                           const float* dt_bias, float* g, int64_t a_rows,
                                           int64_t heads, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && inner > 0 && inner % 8 == 0,
                "gated_activations: inner must be a positive multiple of 8");
  OMNIA_REQUIRE(gate_stride >= inner && up_stride >= inner && gate_stride % 8 == 0 &&
                    up_stride % 8 == 0,
                "gated_activations: row strides must be >= inner and multiples of 8");
  OMNIA_REQUIRE(rows * (inner / 8) < (int64_t{1} << 40), "gated_activations: too large");
  OMNIA_REQUIRE(inner / 8 < (int64_t{1} << 31), "gated_activations: rows too wide");
  OMNIA_REQUIRE(a_rows >= 0 && heads > 0 && heads % 2 == 0 && heads <= (int64_t{1} << 20),
                "gated_activations: heads must be even and positive");
  OMNIA_REQUIRE(a_stride >= heads && a_stride % 2 == 0,
                "gated_activations: a's row stride must be even and >= heads");
  OMNIA_REQUIRE(a_rows * heads < (int64_t{1} << 40), "gated_activations: a too large");
  if (rows == 0 && a_rows == 0) return 0;
  OMNIA_REQUIRE(rows == 0 || (gate && up && y), "gated_activations: null SwiGLU pointer");
  OMNIA_REQUIRE(a_rows == 0 || (a && a_log && dt_bias && g),
                "gated_activations: null gate-softplus pointer");
  OMNIA_REQUIRE(aligned16(gate) && aligned16(up) && aligned16(y),
                "gated_activations: SwiGLU pointers must be 16-byte aligned");
  const auto aligned = [](const void* p, uintptr_t n) {
    return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0;
  };
  OMNIA_REQUIRE(aligned(a, 4) && aligned(a_log, 8) && aligned(dt_bias, 8) && aligned(g, 8),
                "gated_activations: a must be 4-byte and A_log, dt_bias, g 8-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const int64_t vectors = rows * (inner / 8);
  const SoftplusGrid softplus = softplus_grid(a_rows, heads);
  const int64_t softplus_blocks = a_rows == 0 ? 0 : softplus.blocks;
  const int64_t swiglu_blocks = (vectors + kBlock - 1) / kBlock;
  OMNIA_REQUIRE(softplus_blocks + swiglu_blocks < (int64_t{1} << 31),
                "gated_activations: grid too large");
  const GatedArgs p{gate, gate_stride, up, up_stride, y, rows, static_cast<uint32_t>(inner / 8),
                    vectors,
                    SoftplusArgs{a, a_stride, a_log, dt_bias, g, a_rows, static_cast<int>(heads),
                                 softplus.lane_bits, softplus.column_blocks},
                    static_cast<unsigned>(softplus_blocks)};
  const dim3 grid(static_cast<unsigned>(softplus_blocks + swiglu_blocks));
  if (gate_stride == inner && up_stride == inner) {
    gated_activations_kernel<true><<<grid, kBlock, 0, stream>>>(p);
  } else {
    gated_activations_kernel<false><<<grid, kBlock, 0, stream>>>(p);
  }
  return launched("gated_activations");
}
