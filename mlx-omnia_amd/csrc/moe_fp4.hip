// Routed expert MLP of a one-token step over FP4 expert stacks (MLX's
// `QuantizedSwitchLinear`, modes "mxfp4" and "nvfp4"): gate/up with its activation, then
// down/combine, the interleaved layout of the reference's mxfp4 and nvfp4 kernels.
//
// Formats (core/layers.py:164-197): weight [E, rows, in / 8] uint32, two e2m1 codes per
// byte, the low nibble first (value j is nibble j of the row), and
// - mxfp4 (core/kernels/shared/mxfp4.py:8-32): scales [E, rows, in / 32] uint8, an e8m0
//   exponent per 32 values, applied as the fp32 whose bit pattern is `byte << 23`; the
//   projection's own bias [E, rows] bf16;
// - nvfp4 (core/kernels/shared/nvfp4/qmoe.py:8-50): scales [E, rows, in / 16] uint8, a
//   signed e4m3 per 16 values decoded as mlx decodes it (0x7F and 0xFF are +-480, not
//   NaN); no bias.
//
// Arithmetic:
//   gate_up: r = sum over groups of s * sum_j x_j v_j (fp32, any order); rows 2n and
//     2n + 1 are output n's gate and up.
//     mxfp4 (core/kernels/gate_up/mxfp4.py:24-65): g = T(r_gate + b_gate),
//       u = T(r_up + b_up); g = T(min(g, limit)), u = T(clamp(u, -limit, limit));
//       sig = T(1 / (1 + exp(-1.702 g))); y = T(T(g * sig) * T(u + 1)).
//     nvfp4 (core/kernels/gate_up/nvfp4.py:24-68): g = T(r_gate), u = T(r_up);
//       sig = T(1 / (1 + exp(-g))); y = T(T(g * sig) * u).
//     Each operation in fp32.
//   down_combine (core/kernels/down_combine/mxfp4.py:16-58, nvfp4.py:16-61): t the same
//     dot product over the activation row of the slot; acc = sum over slots in order of
//     T(fp32(T(t + b) * w)) in fp32 (b = 0 for nvfp4); y = T(fp32(T(acc) + residual)).
// An expert id outside [0, experts) gives zero rows.
//
// Decoding is gfx950's own: v_cvt_scalef32_pk_bf16_fp4 turns the two e2m1 codes of a
// byte into a bf16 pair (low nibble first; checked on the box for every byte value), so
// one conversion and one v_dot2_f32_bf16 take two weights against the activations in
// memory order. A lane takes 32 values at a time: 16 bytes of codes and one e8m0 byte, or
// two e4m3 bytes read as one 16-bit load; each group's dot product is scaled once in fp32.
//
// Both kernels issue every load of a lane (codes, the scale bits into a register of their
// own, the activations) before any arithmetic and with no branch among the loads: a load
// inside a divergent branch, or a scale byte packed beside another, makes the compiler
// wait on it, one memory round trip per chunk.
//
// The packed NVFP4 form of down_combine (core/kernels/down_combine/nvfp4_packed.py) adds an
// unrouted slot, several tokens per dispatch and a bf16 epilogue; it is described at its
// kernel below.
//
// gate_up: a wave owns kPairsPerWave gate/up pairs of one slot and streams them together,
// 64 lanes across each row; lane p runs pair p's activation. down_combine: a workgroup
// owns kDownRows output rows with one wave per slot, 64 lanes across each row and the
// slot's activations held once for all of them; the slots' terms meet in LDS and are
// summed in slot order.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kChunk = 32;                // values per lane per step: 16 bytes of codes
constexpr int kPairsPerWave = 2;          // gate_up: gate/up pairs per wave
constexpr int kGateWaves = 4;             // gate_up: waves per workgroup
constexpr int kGateBatch = 2;             // gate_up: 64-chunk trips whose loads go out together
constexpr int kDownRows = 4;              // down: output rows per workgroup, each wave's share
constexpr int kMaxInner = 4096;           // down: at most two 64-chunk steps per lane
constexpr int kMaxDownSteps = kMaxInner / (kChunk * kWave);
constexpr int kMaxDownSlots = 16;

enum class Fp4 { kMx, kNv };

// The e8m0 group scale as the reference applies it: the fp32 with exponent field `byte`.
__device__ __forceinline__ float e8m0(uint32_t byte) { return __uint_as_float(byte << 23); }

// The e4m3 group scale as mlx decodes it: sign, 4 exponent bits (bias 7), 3 mantissa bits;
// exponent 0 is subnormal (m / 8 * 2^-6) and the all-ones codes are +-480. A normal code's
// 7 magnitude bits shifted to the top of an fp32's exponent and mantissa, with the
// exponent rebased by 127 - 7, give 2^(e - 7) (1 + m / 8) exactly.
__device__ __forceinline__ float e4m3(uint32_t byte) {
  const uint32_t mag = byte & 0x7Fu;
  const float normal = __uint_as_float((mag << 20) + (120u << 23));
  const float subnormal = static_cast<float>(mag) * 0x1p-9f;
  const float v = mag < 8u ? subnormal : normal;
  return __uint_as_float(__float_as_uint(v) | ((byte & 0x80u) << 24));
}

// The e2m1 codes of byte B of a word as a bf16 pair, low nibble first.
template <int B>
__device__ __forceinline__ uint32_t fp4_pair(uint32_t word) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, 1.0f, B));
}

// sum_j x_j v_j over 8 values: one word of codes against 4 bf16 activation pairs.
__device__ __forceinline__ float word_dot(uint32_t word, const u32x4& x, float acc) {
  acc = dot2_bf16(fp4_pair<0>(word), x.x, acc);
  acc = dot2_bf16(fp4_pair<1>(word), x.y, acc);
  acc = dot2_bf16(fp4_pair<2>(word), x.z, acc);
  return dot2_bf16(fp4_pair<3>(word), x.w, acc);
}

// acc plus one 32-value chunk's scaled dot product: one e8m0 group, or two e4m3 groups of
// 16 (the low scale byte is the first group's).
template <Fp4 F>
__device__ __forceinline__ float chunk_value(uint32_t s, const u32x4& w, const u32x4 (&x)[4], float acc) {
  if constexpr (F == Fp4::kMx) {
    float d = word_dot(w.x, x[0], 0.0f);
    d = word_dot(w.y, x[1], d);
    d = word_dot(w.z, x[2], d);
    d = word_dot(w.w, x[3], d);
    return __builtin_fmaf(e8m0(s), d, acc);
  } else {
    const float lo = word_dot(w.y, x[1], word_dot(w.x, x[0], 0.0f));
    const float hi = word_dot(w.w, x[3], word_dot(w.z, x[2], 0.0f));
    return __builtin_fmaf(e4m3(s >> 8), hi, __builtin_fmaf(e4m3(s & 0xFFu), lo, acc));
  }
}

// The scale bits of one chunk: [rows, in / 32] bytes (mxfp4) or [rows, in / 32] 16-bit
// pairs of bytes (nvfp4), at the chunk's index.
template <Fp4 F>
__device__ __forceinline__ uint32_t load_scales(const void* scales, int64_t at) {
  if constexpr (F == Fp4::kMx) return static_cast<const uint8_t*>(scales)[at];
  else return static_cast<const uint16_t*>(scales)[at];
}

struct Stack {
  const u32x4* weight;     // [experts, rows, in / 32] chunks of 16 bytes
  const void* scales;      // per chunk: one e8m0 byte or two e4m3 bytes
  const uint16_t* bias;    // [experts, rows] bf16, or null
};

// ---- gate_up ------------------------------------------------------------------------

struct GateUpArgs {
  const uint16_t* x;       // [hidden]
  Stack stack;             // [experts, 2 * inner, ...]
  const int32_t* chosen;   // [slots]; null when `keys` routes
  const uint32_t* keys;    // [experts] ordinal keys (ascending = better), or null
  uint16_t* out;           // [slots, inner]
  int64_t experts;
  int hidden;
  int inner;
  float limit;             // mxfp4: +inf for no clamp
};

constexpr int kMaxOrdinalExperts = 1024;   // keys per lane: at most 16

// (hi, lo) = the smaller of itself and (ohi, olo), as one 64-bit unsigned value.
__device__ __forceinline__ void min_u64(uint32_t& hi, uint32_t& lo, uint32_t ohi, uint32_t olo) {
  const bool take = ohi < hi || (ohi == hi && olo < lo);
  hi = take ? ohi : hi;
  lo = take ? olo : lo;
}

template <int kCtrl>
__device__ __forceinline__ void min_dpp_step(uint32_t& hi, uint32_t& lo) {
  min_u64(hi, lo, dpp<kCtrl>(hi), dpp<kCtrl>(lo));
}

// Minimum over the wave of a 64-bit value, the same in every lane: DPP steps inside each
// 16-lane row (quad swaps, half-row and row mirrors), then the two cross-row swaps, all in
// vector registers.
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  uint32_t hi = static_cast<uint32_t>(v >> 32), lo = static_cast<uint32_t>(v);
  min_dpp_step<kQuadSwap1>(hi, lo);
  min_dpp_step<kQuadSwap2>(hi, lo);
  min_dpp_step<kRowHalfMirror>(hi, lo);
  min_dpp_step<kRowMirror>(hi, lo);
  uint32_t ha, hb, la, lb;
  row_pair(hi, ha, hb);
  row_pair(lo, la, lb);
  hi = ha;
  lo = la;
  min_u64(hi, lo, hb, lb);
  half_pair(hi, ha, hb);
  half_pair(lo, la, lb);
  hi = ha;
  lo = la;
  min_u64(hi, lo, hb, lb);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// The expert in rank `slot` of the ordinal keys (ascending, equal keys to the lower index,
// the sort's rule of core/kernels/gate_up/kernel.py:23-36): slot + 1 rounds of a wave
// argmin over (key, index), each removing its winner. Every wave of the slot computes it.
// kKeys keys per lane (expert lane + 64 j), loaded at a clamped index with no branch (a
// load in a branch makes the compiler wait on it) by ordinal_keys, ranked by
// ordinal_expert; an index past the last is never chosen.
template <int kKeys>
__device__ __forceinline__ void ordinal_keys(const uint32_t* keys, int experts, int lane, uint32_t (&raw)[kKeys]) {
#pragma unroll
  for (int j = 0; j < kKeys; ++j) raw[j] = keys[min(lane + kWave * j, experts - 1)];
}

template <int kKeys>
__device__ __forceinline__ int ordinal_expert(const uint32_t (&raw)[kKeys], int experts, int slot, int lane) {
  uint64_t mine[kKeys];
#pragma unroll
  for (int j = 0; j < kKeys; ++j) {
    const int e = lane + kWave * j;
    mine[j] = e < experts ? (static_cast<uint64_t>(raw[j]) << 32) | static_cast<uint32_t>(e) : ~uint64_t{0};
  }
  uint64_t best = ~uint64_t{0};
  for (int round = 0; round <= slot; ++round) {   // slot < experts: bounded
    uint64_t local = mine[0];
#pragma unroll
    for (int j = 1; j < kKeys; ++j) local = mine[j] < local ? mine[j] : local;
    best = wave_min_u64(local);
#pragma unroll
    for (int j = 0; j < kKeys; ++j) mine[j] = mine[j] == best ? ~uint64_t{0} : mine[j];
  }
  return static_cast<int>(static_cast<uint32_t>(best));
}

// kTrips > 0: hidden / 32 chunks span exactly kTrips 64-lane trips; 0: any number of trips.
// kKeys > 0: the slot's expert comes from the ordinal keys (kKeys per lane), not `chosen`.
template <Fp4 F, int kTrips, int kKeys = 0>
__device__ __forceinline__ void gate_up_body(const GateUpArgs& a) {
  const int lane = threadIdx.x % kWave;
  const int slot = blockIdx.y;
  const int pair0 = (blockIdx.x * kGateWaves + threadIdx.x / kWave) * kPairsPerWave;
  // No early exit: a branch on the size made it a scalar round trip of its own ahead of
  // the other arguments' (two before the first load). A wave past the last pair computes
  // the last one and stores nothing.
  const bool wave_live = pair0 < a.inner;
  const int first_pair = wave_live ? pair0 : a.inner - 1;
  const int pairs = min(kPairsPerWave, a.inner - first_pair);
  const int stored = wave_live ? pairs : 0;
  uint16_t* out = a.out + static_cast<int64_t>(slot) * a.inner + first_pair;
  constexpr int kBatch = kTrips > 0 ? kTrips : kGateBatch;
  const int chunks = a.hidden / kChunk;
  // With the expert read from `chosen`, the first batch's chunks of x, which do not depend
  // on it, are loaded before it is known, so their round trip overlaps the id's. (With the
  // expert ranked from the ordinal keys here, x loaded ahead of the ranking measured no
  // faster, and x stays with the codes.)
  constexpr bool kEarlyX = kKeys == 0;
  // The id is read through the vector path (every lane reads the same word), ahead of x:
  // vector loads return in order, so waiting for it waits for nothing issued after it,
  // where a scalar read went out only after the kernel's argument loads had returned.
  int zero = 0;
  asm volatile("" : "+v"(zero));   // a zero the compiler cannot see as uniform
  int chosen_v = 0;
  if constexpr (kEarlyX) chosen_v = a.chosen[slot + zero];
  u32x4 x_first[kBatch][4];
  if constexpr (kEarlyX) {
#pragma unroll
    for (int h = 0; h < kBatch; ++h) {
      const int c = min(lane + h * kWave, chunks - 1);
#pragma unroll
      for (int j = 0; j < 4; ++j) x_first[h][j] = reinterpret_cast<const u32x4*>(a.x + c * kChunk)[j];
    }
    __builtin_amdgcn_sched_barrier(0);   // the x loads ahead of the wait for the id
  }
  uint32_t key_bits[kKeys > 0 ? kKeys : 1];
  if constexpr (kKeys > 0) {
    ordinal_keys<kKeys>(a.keys, static_cast<int>(a.experts), lane, key_bits);
    __builtin_amdgcn_sched_barrier(0);   // the keys' loads ahead of the wait below
  }
  // The stack's pointers, `out` and the limit, taken here, ahead of the branch on the id:
  // the compiler otherwise loaded each at its first use, the pointers behind the branch
  // (one more scalar round trip ahead of the codes) and the others at the store.
  asm volatile("" ::"s"(a.stack.weight), "s"(a.stack.scales), "s"(a.stack.bias), "s"(a.out));
  if constexpr (F == Fp4::kMx) asm volatile("" ::"s"(a.limit));
  int expert;
  if constexpr (kKeys > 0) expert = ordinal_expert<kKeys>(key_bits, static_cast<int>(a.experts), slot, lane);
  else expert = __builtin_amdgcn_readfirstlane(chosen_v);
  if (expert < 0 || expert >= a.experts) {
    if (lane < stored) out[lane] = 0;
    return;
  }
  constexpr int kRows = 2 * kPairsPerWave;
  const int rows = 2 * pairs;
  const int64_t row0 = static_cast<int64_t>(expert) * 2 * a.inner + 2 * static_cast<int64_t>(first_pair);
  // The projection bias of the pair this lane activates (its gate and up rows), loaded
  // ahead of the codes.
  uint32_t gate_bias_bits = 0, up_bias_bits = 0;
  if constexpr (F == Fp4::kMx) {
    const int64_t at = row0 + 2 * min(lane, pairs - 1);
    gate_bias_bits = early_bf16_bits(a.stack.bias, at, a.x);
    up_bias_bits = early_bf16_bits(a.stack.bias, at + 1, a.x);
  }
  const int trips = kTrips > 0 ? kTrips : (chunks + kWave - 1) / kWave;
  float r[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) r[i] = 0.0f;
  // kBatch trips' loads are issued before their arithmetic, with no branch among them: a
  // lane past the row's end re-reads the last chunk and drops the term, and a row past
  // the wave's last pair re-reads the pair's last row (that sum is never stored).
  for (int t0 = 0; t0 < trips; t0 += kBatch) {
    u32x4 w[kBatch][kRows];
    uint32_t s[kBatch][kRows];
    u32x4 x[kBatch][4];
#pragma unroll
    for (int h = 0; h < kBatch; ++h) {
      const int c = min(lane + (t0 + h) * kWave, chunks - 1);
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        const int64_t at = (row0 + min(i, rows - 1)) * chunks + c;
        w[h][i] = load_nt(a.stack.weight + at);
        s[h][i] = load_scales<F>(a.stack.scales, at);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[h][j] = kEarlyX && t0 == 0 ? x_first[h][j] : reinterpret_cast<const u32x4*>(a.x + c * kChunk)[j];
      }
    }
    __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the arithmetic
#pragma unroll
    for (int h = 0; h < kBatch; ++h) {
      const bool in_row = lane + (t0 + h) * kWave < chunks;
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        const float term = chunk_value<F>(s[h][i], w[h][i], x[h], r[i]);
        r[i] = in_row ? term : r[i];
      }
    }
  }
  // Lane p takes pair p's sums and runs its activation.
  float gate_sum = 0.0f, up_sum = 0.0f;
#pragma unroll
  for (int p = 0; p < kPairsPerWave; ++p) {
    const float gp = wave_sum_f32(r[2 * p]);
    const float up = wave_sum_f32(r[2 * p + 1]);
    gate_sum = lane == p ? gp : gate_sum;
    up_sum = lane == p ? up : up_sum;
  }
  if (lane >= stored) return;
  if constexpr (F == Fp4::kMx) {
    float gate_bias = 0.0f, up_bias = 0.0f;
    if (a.stack.bias != nullptr) {
      gate_bias = bf16_to_f32(gate_bias_bits);
      up_bias = bf16_to_f32(up_bias_bits);
    }
    float g = round_bf16(gate_sum + gate_bias);
    float u = round_bf16(up_sum + up_bias);
    if (a.limit < __builtin_inff()) {
      g = round_bf16(fminf(g, a.limit));
      u = round_bf16(fminf(fmaxf(u, -a.limit), a.limit));
    }
    const float sig = round_bf16(1.0f / (1.0f + expf(-1.702f * g)));
    const float act = round_bf16(g * sig);
    out[lane] = f32_to_bf16(act * round_bf16(u + 1.0f));
  } else {
    const float g = round_bf16(gate_sum);
    const float u = round_bf16(up_sum);
    const float sig = round_bf16(1.0f / (1.0f + expf(-g)));
    const float act = round_bf16(g * sig);
    out[lane] = f32_to_bf16(act * u);
  }
}

// The arguments the first loads need come first, as scalars (copies of GateUpArgs fields,
// which replace the struct's own): gfx950 preloads a kernel's leading scalar and pointer
// arguments into SGPRs at wave launch, so the id's, the keys' and x's loads go out with
// no scalar round trip ahead of them, and the rest of GateUpArgs is loaded while they are
// in flight.
#define OMNIA_GATE_UP_LEADING                                                              \
  const uint16_t *x, const int32_t *chosen, const uint32_t *keys, int64_t experts, int hidden, \
      int inner, GateUpArgs a
#define OMNIA_GATE_UP_REPLACE \
  a.x = x;                    \
  a.chosen = chosen;          \
  a.keys = keys;              \
  a.experts = experts;        \
  a.hidden = hidden;          \
  a.inner = inner

template <int kTrips>
__global__ __launch_bounds__(kGateWaves * kWave) void moe_gate_up_mxfp4_kernel(OMNIA_GATE_UP_LEADING) {
  OMNIA_GATE_UP_REPLACE;
  gate_up_body<Fp4::kMx, kTrips>(a);
}

template <int kTrips, int kKeys>
__global__ __launch_bounds__(kGateWaves * kWave) void moe_gate_up_nvfp4_kernel(OMNIA_GATE_UP_LEADING) {
  OMNIA_GATE_UP_REPLACE;
  gate_up_body<Fp4::kNv, kTrips, kKeys>(a);
}

#define OMNIA_GATE_UP_ARGS a.x, a.chosen, a.keys, a.experts, a.hidden, a.inner, a

template <int kKeys>
void launch_nvfp4_gate_up(int64_t trips, dim3 grid, dim3 block, hipStream_t stream, const GateUpArgs& a) {
  if (trips == 1) moe_gate_up_nvfp4_kernel<1, kKeys><<<grid, block, 0, stream>>>(OMNIA_GATE_UP_ARGS);
  else if (trips == 2) moe_gate_up_nvfp4_kernel<2, kKeys><<<grid, block, 0, stream>>>(OMNIA_GATE_UP_ARGS);
  else moe_gate_up_nvfp4_kernel<0, kKeys><<<grid, block, 0, stream>>>(OMNIA_GATE_UP_ARGS);
}

// ---- down_combine -------------------------------------------------------------------

struct DownArgs {
  const uint16_t* act;      // [slots, inner]
  Stack stack;              // [experts, hidden, ...]
  const int32_t* chosen;    // [slots]
  const float* weights;     // [slots]
  const uint16_t* residual; // [hidden] or null
  uint16_t* out;            // [hidden]
  int64_t experts;
  int hidden;
  int inner;
  int slots;
};

// kLanes lanes run across each row (64, or 32 for short rows: the wave's two halves then
// take rows h and h + 2); kSteps = ceil(inner / (32 * kLanes)) chunks per lane.
template <Fp4 F, int kSteps, int kLanes = kWave>
__device__ __forceinline__ void down_body(const DownArgs& a, int blocks,
                                          float (&partial)[kMaxDownSlots][kDownRows]) {
  constexpr int kHalves = kWave / kLanes;            // row groups per wave
  constexpr int kRowsPerGroup = kDownRows / kHalves;
  const int lane = threadIdx.x % kWave;
  const int part = lane % kLanes;
  const int group = lane / kLanes;
  // One wave per slot.
  const int slot = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int row_base = xcd_contiguous_block(blockIdx.x, blocks) * kDownRows;
  const int rows = min(kDownRows, a.hidden - row_base);
  const int chunks = a.inner / kChunk;
  // The slot's routing entries (expert id and weight) first, through the vector path
  // (every lane of the wave reads the same word): vector loads return in order, so waiting
  // for them waits for nothing issued after them, where scalar reads went out only after
  // the kernel's argument loads had returned. Then the residual of the output row this
  // thread writes (rows past the last read the last).
  const int slot_lanes = static_cast<int>(threadIdx.x / kWave);
  const int chosen_v = a.chosen[slot_lanes];
  const float route_weight_v = a.weights[slot_lanes];
  const uint32_t resid = early_bf16_bits(
      a.residual, row_base + min(static_cast<int>(threadIdx.x % kDownRows), rows - 1), a.act);
  // The slot's activations (shared by the group's rows), which do not depend on the
  // expert: loaded before the expert id is waited on, so their round trip overlaps the
  // id's. A lane past the row's last chunk re-reads that chunk.
  const uint16_t* x = a.act + static_cast<int64_t>(slot) * a.inner;
  u32x4 xv[kSteps][4];
#pragma unroll
  for (int h = 0; h < kSteps; ++h) {
    const int c = min(part + kLanes * h, chunks - 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[h][j] = reinterpret_cast<const u32x4*>(x + c * kChunk)[j];
  }
  __builtin_amdgcn_sched_barrier(0);   // the activation loads ahead of the wait for the id
  // The stack's pointers, `out` and the slot count, taken here with the id: the compiler
  // otherwise loaded each at its first use, the pointers behind the id's wait (one more
  // scalar round trip ahead of the codes) and the others at the combine.
  asm volatile("" ::"s"(a.stack.weight), "s"(a.stack.scales), "s"(a.stack.bias), "s"(a.out), "s"(a.slots));
  const int expert = __builtin_amdgcn_readfirstlane(chosen_v);
  const float route_weight = __builtin_bit_cast(
      float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, route_weight_v)));
  const bool valid = expert >= 0 && expert < a.experts;   // uniform over the wave
  const int64_t row0 = static_cast<int64_t>(valid ? expert : 0) * a.hidden + row_base;
  // The projection bias of the row lane i takes, loaded ahead of the codes.
  const uint32_t bias = early_bf16_bits(a.stack.bias, row0 + min(lane, rows - 1), a.act);
  float t[kRowsPerGroup];
#pragma unroll
  for (int q = 0; q < kRowsPerGroup; ++q) t[q] = 0.0f;
  if (valid) {
    // Every code and scale load is issued before any arithmetic, with no branch among
    // them: a lane past the row's last chunk re-reads that chunk and drops the term, and
    // a row past the last one re-reads the last (its sum is never used).
    u32x4 w[kSteps][kRowsPerGroup];
    uint32_t s[kSteps][kRowsPerGroup];
#pragma unroll
    for (int h = 0; h < kSteps; ++h) {
      const int c = min(part + kLanes * h, chunks - 1);
#pragma unroll
      for (int q = 0; q < kRowsPerGroup; ++q) {
        const int64_t at = (row0 + min(group + kHalves * q, rows - 1)) * chunks + c;
        w[h][q] = load_nt(a.stack.weight + at);
        s[h][q] = load_scales<F>(a.stack.scales, at);
      }
    }
    __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the arithmetic
#pragma unroll
    for (int h = 0; h < kSteps; ++h) {
      const bool in_row = part + kLanes * h < chunks;
#pragma unroll
      for (int q = 0; q < kRowsPerGroup; ++q) {
        const float term = chunk_value<F>(s[h][q], w[h][q], xv[h], t[q]);
        t[q] = in_row ? term : t[q];
      }
    }
  }
  // Lane i takes row i's sum (row g + kHalves q is group g's q-th). With two groups, one
  // permlane32 swap hands every lane both groups' sums.
  float mine = 0.0f;
#pragma unroll
  for (int q = 0; q < kRowsPerGroup; ++q) {
    if constexpr (kLanes == kWave) {
      const float total = wave_sum_f32(t[q]);
      mine = lane == q ? total : mine;
    } else {
      float v = t[q];
      v += __uint_as_float(dpp<kQuadSwap1>(__float_as_uint(v)));
      v += __uint_as_float(dpp<kQuadSwap2>(__float_as_uint(v)));
      v += __uint_as_float(dpp<kRowHalfMirror>(__float_as_uint(v)));
      v += __uint_as_float(dpp<kRowMirror>(__float_as_uint(v)));
      uint32_t lo, hi;
      row_pair(__float_as_uint(v), lo, hi);
      const float group_total = __uint_as_float(lo) + __uint_as_float(hi);
      uint32_t g0, g1;
      half_pair(__float_as_uint(group_total), g0, g1);
      mine = lane == kHalves * q ? __uint_as_float(g0) : mine;
      mine = lane == kHalves * q + 1 ? __uint_as_float(g1) : mine;
    }
  }
  if (lane < rows) {
    float term = 0.0f;
    if (valid) {
      const float b = a.stack.bias != nullptr ? bf16_to_f32(bias) : 0.0f;
      term = round_bf16(round_bf16(mine + b) * route_weight);
    }
    partial[slot][lane] = term;
  }
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < rows) {
    const int n = row_base + threadIdx.x;
    float sum = 0.0f;
    for (int j = 0; j < a.slots; ++j) sum += partial[j][threadIdx.x];
    float out = round_bf16(sum);
    if (a.residual != nullptr) out = out + bf16_to_f32(resid);
    a.out[n] = f32_to_bf16(out);
  }
}

// As in the gate/up kernels, the arguments the first loads need come first, as scalars
// (copies of DownArgs fields, which replace the struct's own, and the grid size),
// preloaded into SGPRs at wave launch.
#define OMNIA_DOWN_LEADING                                                                  \
  const uint16_t *act, const int32_t *chosen, const float *weights, const uint16_t *residual, \
      int64_t experts, int hidden, int inner, int blocks, DownArgs a
#define OMNIA_DOWN_REPLACE \
  a.act = act;             \
  a.chosen = chosen;       \
  a.weights = weights;     \
  a.residual = residual;   \
  a.experts = experts;     \
  a.hidden = hidden;       \
  a.inner = inner

template <int kSteps>
__global__ __launch_bounds__(kMaxDownSlots * kWave) void moe_down_mxfp4_kernel(OMNIA_DOWN_LEADING) {
  __shared__ float partial[kMaxDownSlots][kDownRows];
  OMNIA_DOWN_REPLACE;
  down_body<Fp4::kMx, kSteps>(a, blocks, partial);
}

template <int kSteps, int kLanes>
__global__ __launch_bounds__(kMaxDownSlots * kWave) void moe_down_nvfp4_kernel(OMNIA_DOWN_LEADING) {
  __shared__ float partial[kMaxDownSlots][kDownRows];
  OMNIA_DOWN_REPLACE;
  down_body<Fp4::kNv, kSteps, kLanes>(a, blocks, partial);
}

#define OMNIA_DOWN_ARGS \
  a.act, a.chosen, a.weights, a.residual, a.experts, a.hidden, a.inner, static_cast<int>(grid.x), a

// ---- down_combine with the unrouted slot (the packed NVFP4 form) --------------------
//
// core/kernels/down_combine/nvfp4_packed.py:38-138: every token's routed down
// projections, the unrouted (shared) stack's, the routing sum and the residual in one
// dispatch, for any number of tokens. Slot s < top_k runs expert chosen[t, s] over
// act[t, s]; slot top_k runs the shared stack over act[t, top_k], unweighted. The scale
// plane is the checkpoint's group-16 plane, which equals the reference's halved plane
// with its patch restored wherever that plane is accepted (its certificate is the
// caller's to check). The epilogue is bf16 at every step, in slot order:
//   d_s = T(dot_s); total = T(T(d_s * T(w_s)) + total) over s < top_k;
//   y = T(residual + T(total + d_top_k)), each operation in fp32.

constexpr int kSharedRows = 8;         // output rows per workgroup
constexpr int kSharedWaves = 16;       // slot s runs on wave s % 16
constexpr int kMaxSharedSlots = 32;    // top_k + 1

struct SharedDownArgs {
  const uint16_t* act;        // [tokens, top_k + 1, inner]
  Stack routed;               // [experts, hidden, ...]
  Stack shared;               // [hidden, ...]
  const int32_t* chosen;      // [tokens, top_k]
  const float* weights;       // [tokens, top_k]
  const uint16_t* residual;   // [tokens, hidden]
  uint16_t* out;              // [tokens, hidden]
  int64_t experts;
  int hidden;
  int inner;
  int top_k;
};

// kLanes lanes run across each row (16, 32 or 64: the fewest that give each lane one
// 32-value chunk), so a wave holds kWave / kLanes row groups, each taking every
// (kWave / kLanes)-th row of the workgroup with the slot's activation chunk loaded once.
// The arguments the first loads need come first, as scalars (copies of SharedDownArgs
// fields, which replace the struct's own, and the grid's width), preloaded into SGPRs at
// wave launch.
template <int kLanes>
__global__ __launch_bounds__(kSharedWaves * kWave) void moe_down_nvfp4_shared_kernel(
    const uint16_t* act, const int32_t* chosen, const float* weights, const uint16_t* residual,
    int64_t experts, int hidden, int inner, int top_k, int blocks, SharedDownArgs a) {
  a.act = act;
  a.chosen = chosen;
  a.weights = weights;
  a.residual = residual;
  a.experts = experts;
  a.hidden = hidden;
  a.inner = inner;
  a.top_k = top_k;
  constexpr int kGroups = kWave / kLanes;
  constexpr int kRowsPerGroup = kSharedRows / kGroups;
  __shared__ float term[kMaxSharedSlots][kSharedRows];
  __shared__ float route_weight[kMaxSharedSlots];
  const int lane = threadIdx.x % kWave;
  const int part = lane % kLanes;
  const int group = lane / kLanes;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int waves = min(a.top_k + 1, kSharedWaves);   // the launch's block: no argument load
  const int64_t token = blockIdx.y;
  const int row_base = xcd_contiguous_block(blockIdx.x, blocks) * kSharedRows;
  int zero = 0;
  asm volatile("" : "+v"(zero));   // a zero the compiler cannot see as uniform
  const int rows = min(kSharedRows, a.hidden - row_base);
  const int slots = a.top_k + 1;
  const int chunks = a.inner / kChunk;
  const int c = min(part, chunks - 1);   // a lane past the row's end re-reads its last chunk
  const bool in_row = part < chunks;
  // The epilogue's operands, loaded ahead of the codes: the residual of the output row
  // this thread writes (rows past the last read the last), and the token's routing
  // weights, thread j holding weight j (kept in LDS for the epilogue).
  const uint16_t resid_raw =
      a.residual[token * a.hidden + row_base + min(static_cast<int>(threadIdx.x % kSharedRows), rows - 1)];
  const float my_weight =   // no routed slots: the weights may be null
      a.top_k > 0 ? a.weights[token * a.top_k + min(static_cast<int>(threadIdx.x % kMaxSharedSlots), a.top_k - 1)]
                  : 0.0f;
  for (int slot = wave; slot < slots; slot += waves) {   // uniform over the wave
    // Every load (the activation chunk, each row's codes and scale bits) goes out before
    // any arithmetic, with no branch among them; a row past the last re-reads the last.
    // The expert id first, through the vector path (every lane reads the same word; the
    // shared slot reads the first word of act instead, as `chosen` may be null): vector
    // loads return in order, so waiting for it waits for nothing issued after it. Then
    // the chunk: it does not depend on the expert, so its round trip overlaps the id's.
    const bool shared = slot == a.top_k;
    const int32_t* ids = shared ? reinterpret_cast<const int32_t*>(a.act) : a.chosen;
    const int chosen_v = ids[(shared ? 0 : token * a.top_k + slot) + zero];
    const u32x4* x = reinterpret_cast<const u32x4*>(
        a.act + (token * slots + slot) * a.inner + static_cast<int64_t>(c) * kChunk);
    u32x4 xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[j] = x[j];
    __builtin_amdgcn_sched_barrier(0);   // the chunk's loads ahead of the wait for the id
    // The stack field by field (selecting the struct itself selected its address in the
    // argument segment and loaded the fields from there, behind the id's wait).
    Stack stack;
    stack.weight = shared ? a.shared.weight : a.routed.weight;
    stack.scales = shared ? a.shared.scales : a.routed.scales;
    asm volatile("" ::"s"(stack.weight), "s"(stack.scales), "s"(a.out));   // `out` too, not at the store
    const int expert = shared ? 0 : __builtin_amdgcn_readfirstlane(chosen_v);
    const bool valid = shared || (expert >= 0 && expert < a.experts);
    const int64_t row0 = (shared ? 0 : static_cast<int64_t>(valid ? expert : 0) * a.hidden) + row_base;
    u32x4 w[kRowsPerGroup];
    uint32_t s[kRowsPerGroup];
#pragma unroll
    for (int q = 0; q < kRowsPerGroup; ++q) {
      const int64_t at = (row0 + min(group + kGroups * q, rows - 1)) * chunks + c;
      w[q] = load_nt(stack.weight + at);
      s[q] = load_scales<Fp4::kNv>(stack.scales, at);
    }
    __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the arithmetic
    float mine = 0.0f;
#pragma unroll
    for (int q = 0; q < kRowsPerGroup; ++q) {
      const float t = in_row ? chunk_value<Fp4::kNv>(s[q], w[q], xv, 0.0f) : 0.0f;
      const float total = group_row_sum<kLanes>(t);
      mine = part == q ? total : mine;
    }
    const int row = group + kGroups * part;
    if (part < kRowsPerGroup && row < rows) term[slot][row] = valid ? round_bf16(mine) : 0.0f;
  }
  if (static_cast<int>(threadIdx.x) < a.top_k) route_weight[threadIdx.x] = my_weight;
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < rows) {
    const int r = threadIdx.x;
    const int64_t n = token * a.hidden + row_base + r;
    float total = 0.0f;
    for (int j = 0; j < a.top_k; ++j) {
      const float weight = round_bf16(route_weight[j]);
      total = round_bf16(round_bf16(term[j][r] * weight) + total);
    }
    const float joined = round_bf16(total + term[a.top_k][r]);
    a.out[n] = f32_to_bf16(bf16_to_f32(resid_raw) + joined);
  }
}

// Host side: shape checks and launches shared by both formats.

int32_t launch_gate_up(Fp4 format, const char* name, const uint16_t* x, const uint32_t* weight,
                       const void* scales, const uint16_t* bias, int64_t experts, int64_t hidden,
                       int64_t inner, const int32_t* chosen, const uint32_t* keys, int64_t slots, float limit,
                       uint16_t* out, hipStream_t stream) {
  OMNIA_REQUIRE(experts > 0 && experts < (int64_t{1} << 20), std::string(name) + ": bad expert count");
  OMNIA_REQUIRE(hidden > 0 && hidden % kChunk == 0 && hidden <= 16384,
                std::string(name) + ": hidden must be a multiple of 32 in [32, 16384]");
  OMNIA_REQUIRE(inner > 0 && inner < (int64_t{1} << 24), std::string(name) + ": bad inner size");
  OMNIA_REQUIRE(slots >= 0 && slots <= 1024, std::string(name) + ": slots must be in [0, 1024]");
  OMNIA_REQUIRE(!(limit < 0.0f), std::string(name) + ": the limit must be non-negative (+inf: none)");
  if (slots == 0) return 0;
  OMNIA_REQUIRE(x && weight && scales && (chosen || keys) && out, std::string(name) + ": null pointer");
  OMNIA_REQUIRE(keys == nullptr || (format == Fp4::kNv && experts <= kMaxOrdinalExperts && slots <= experts),
                std::string(name) + ": ordinal routing takes at most 1024 experts and top_k <= experts");
  OMNIA_REQUIRE(aligned16(x) && aligned16(weight), std::string(name) + ": x and weight must be 16-byte aligned");
  OMNIA_REQUIRE(format == Fp4::kMx || reinterpret_cast<uintptr_t>(scales) % 2 == 0,
                std::string(name) + ": the scales must be 2-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  GateUpArgs a{x, Stack{reinterpret_cast<const u32x4*>(weight), scales, bias}, chosen, keys, out, experts,
               static_cast<int>(hidden), static_cast<int>(inner), limit};
  const int64_t waves = (inner + kPairsPerWave - 1) / kPairsPerWave;
  const dim3 grid(static_cast<unsigned>((waves + kGateWaves - 1) / kGateWaves), static_cast<unsigned>(slots));
  const dim3 block(kGateWaves * kWave);
  const int64_t trips = (hidden / kChunk + kWave - 1) / kWave;
  if (format == Fp4::kMx) {
    if (trips == 1) moe_gate_up_mxfp4_kernel<1><<<grid, block, 0, stream>>>(OMNIA_GATE_UP_ARGS);
    else if (trips == 2) moe_gate_up_mxfp4_kernel<2><<<grid, block, 0, stream>>>(OMNIA_GATE_UP_ARGS);
    else moe_gate_up_mxfp4_kernel<0><<<grid, block, 0, stream>>>(OMNIA_GATE_UP_ARGS);
  } else if (keys == nullptr) {
    launch_nvfp4_gate_up<0>(trips, grid, block, stream, a);
  } else if (experts <= 2 * kWave) {
    launch_nvfp4_gate_up<2>(trips, grid, block, stream, a);
  } else if (experts <= 4 * kWave) {
    launch_nvfp4_gate_up<4>(trips, grid, block, stream, a);
  } else {
    launch_nvfp4_gate_up<kMaxOrdinalExperts / kWave>(trips, grid, block, stream, a);
  }
  return launched(name);
}

int32_t launch_down(Fp4 format, const char* name, const uint16_t* act, const uint32_t* weight,
                    const void* scales, const uint16_t* bias, int64_t experts, int64_t hidden,
                    int64_t inner, const int32_t* chosen, const float* weights, int64_t slots,
                    const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  OMNIA_REQUIRE(experts > 0 && experts < (int64_t{1} << 20), std::string(name) + ": bad expert count");
  OMNIA_REQUIRE(hidden > 0 && hidden < (int64_t{1} << 24), std::string(name) + ": bad hidden size");
  OMNIA_REQUIRE(inner > 0 && inner % kChunk == 0 && inner <= kMaxInner,
                std::string(name) + ": inner must be a multiple of 32 in [32, 4096]");
  OMNIA_REQUIRE(slots > 0 && slots <= kMaxDownSlots, std::string(name) + ": slots must be in [1, 16]");
  OMNIA_REQUIRE(act && weight && scales && chosen && weights && out, std::string(name) + ": null pointer");
  OMNIA_REQUIRE(aligned16(act) && aligned16(weight), std::string(name) + ": act and weight must be 16-byte aligned");
  OMNIA_REQUIRE(format == Fp4::kMx || reinterpret_cast<uintptr_t>(scales) % 2 == 0,
                std::string(name) + ": the scales must be 2-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  DownArgs a{act, Stack{reinterpret_cast<const u32x4*>(weight), scales, bias}, chosen, weights, residual, out,
             experts, static_cast<int>(hidden), static_cast<int>(inner), static_cast<int>(slots)};
  const dim3 grid(static_cast<unsigned>((hidden + kDownRows - 1) / kDownRows));
  const dim3 block(static_cast<unsigned>(slots * kWave));
  static_assert(kMaxDownSteps == 2 && kDownRows == 4, "one instantiation per step count");
  const bool one = inner <= kChunk * kWave;
  if (format == Fp4::kMx) {
    if (one) moe_down_mxfp4_kernel<1><<<grid, block, 0, stream>>>(OMNIA_DOWN_ARGS);
    else moe_down_mxfp4_kernel<2><<<grid, block, 0, stream>>>(OMNIA_DOWN_ARGS);
  } else if (inner <= kChunk * kWave / 2) {   // at most 32 chunks: 32 lanes per row
    moe_down_nvfp4_kernel<1, kWave / 2><<<grid, block, 0, stream>>>(OMNIA_DOWN_ARGS);
  } else if (one) {
    moe_down_nvfp4_kernel<1, kWave><<<grid, block, 0, stream>>>(OMNIA_DOWN_ARGS);
  } else {
    moe_down_nvfp4_kernel<2, kWave><<<grid, block, 0, stream>>>(OMNIA_DOWN_ARGS);
  }
  return launched(name);
}

int32_t launch_down_shared(const uint16_t* act, const uint32_t* weight, const uint8_t* scales,
                           int64_t experts, const uint32_t* shared_weight, const uint8_t* shared_scales,
                           int64_t hidden, int64_t inner, const int32_t* chosen, const float* weights,
                           int64_t tokens, int64_t top_k, const uint16_t* residual, uint16_t* out,
                           hipStream_t stream) {
  const char* name = "moe_down_combine_nvfp4_shared";
  OMNIA_REQUIRE(experts > 0 && experts < (int64_t{1} << 20), std::string(name) + ": bad expert count");
  OMNIA_REQUIRE(hidden > 0 && hidden < (int64_t{1} << 24), std::string(name) + ": bad hidden size");
  OMNIA_REQUIRE(inner > 0 && inner % kChunk == 0 && inner <= kChunk * kWave,
                std::string(name) + ": inner must be a multiple of 32 in [32, 2048]");
  OMNIA_REQUIRE(top_k >= 0 && top_k < kMaxSharedSlots, std::string(name) + ": top_k must be in [0, 31]");
  OMNIA_REQUIRE(tokens >= 0 && tokens <= 65535, std::string(name) + ": tokens must be in [0, 65535]");
  if (tokens == 0) return 0;
  OMNIA_REQUIRE(act && weight && scales && shared_weight && shared_scales && residual && out &&
                    (top_k == 0 || (chosen && weights)),
                std::string(name) + ": null pointer");
  OMNIA_REQUIRE(aligned16(act) && aligned16(weight) && aligned16(shared_weight),
                std::string(name) + ": act and the weights must be 16-byte aligned");
  OMNIA_REQUIRE(reinterpret_cast<uintptr_t>(scales) % 2 == 0 && reinterpret_cast<uintptr_t>(shared_scales) % 2 == 0,
                std::string(name) + ": the scales must be 2-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  SharedDownArgs a{act,
                   Stack{reinterpret_cast<const u32x4*>(weight), scales, nullptr},
                   Stack{reinterpret_cast<const u32x4*>(shared_weight), shared_scales, nullptr},
                   chosen, weights, residual, out, experts, static_cast<int>(hidden), static_cast<int>(inner),
                   static_cast<int>(top_k)};
  const dim3 grid(static_cast<unsigned>((hidden + kSharedRows - 1) / kSharedRows), static_cast<unsigned>(tokens));
  const int64_t waves = top_k + 1 < kSharedWaves ? top_k + 1 : kSharedWaves;   // the kernel assumes this
  const dim3 block(static_cast<unsigned>(waves * kWave));
  const int64_t chunks = inner / kChunk;
  if (chunks <= 16) moe_down_nvfp4_shared_kernel<16><<<grid, block, 0, stream>>>(
        a.act, a.chosen, a.weights, a.residual, a.experts, a.hidden, a.inner, a.top_k,
        static_cast<int>(grid.x), a);
  else if (chunks <= 32) moe_down_nvfp4_shared_kernel<32><<<grid, block, 0, stream>>>(
        a.act, a.chosen, a.weights, a.residual, a.experts, a.hidden, a.inner, a.top_k,
        static_cast<int>(grid.x), a);
  else moe_down_nvfp4_shared_kernel<64><<<grid, block, 0, stream>>>(
        a.act, a.chosen, a.weights, a.residual, a.experts, a.hidden, a.inner, a.top_k,
        static_cast<int>(grid.x), a);
  return launched(name);
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_moe_down_combine_nvfp4_shared(
    const uint16_t* act, const uint32_t* weight, const uint8_t* scales, int64_t experts,
    const uint32_t* shared_weight, const uint8_t* shared_scales, int64_t hidden, int64_t inner,
    const int32_t* chosen, const float* weights, int64_t tokens, int64_t top_k, const uint16_t* residual,
    uint16_t* out, hipStream_t stream) {
  return omnia::launch_down_shared(act, weight, scales, experts, shared_weight, shared_scales, hidden, inner,
                                   chosen, weights, tokens, top_k, residual, out, stream);
}

extern "C" int32_t omnia_moe_gate_up_mxfp4(const uint16_t* x, const uint32_t* weight, const uint8_t* scales,
                                           const uint16_t* bias, int64_t experts, int64_t hidden,
                                           int64_t inner, const int32_t* chosen, int64_t slots,
                                           float limit, uint16_t* out, hipStream_t stream) {
  return omnia::launch_gate_up(omnia::Fp4::kMx, "moe_gate_up_mxfp4", x, weight, scales, bias, experts, hidden,
                               inner, chosen, nullptr, slots, limit, out, stream);
}

extern "C" int32_t omnia_moe_down_combine_mxfp4(const uint16_t* act, const uint32_t* weight,
                                                const uint8_t* scales, const uint16_t* bias,
                                                int64_t experts, int64_t hidden, int64_t inner,
                                                const int32_t* chosen, const float* weights,
                                                int64_t slots, const uint16_t* residual, uint16_t* out,
                                                hipStream_t stream) {
  return omnia::launch_down(omnia::Fp4::kMx, "moe_down_combine_mxfp4", act, weight, scales, bias, experts,
                            hidden, inner, chosen, weights, slots, residual, out, stream);
}

extern "C" int32_t omnia_moe_gate_up_nvfp4(const uint16_t* x, const uint32_t* weight, const uint8_t* scales,
                                           int64_t experts, int64_t hidden, int64_t inner,
                                           const int32_t* chosen, int64_t slots, uint16_t* out,
                                           hipStream_t stream) {
  return omnia::launch_gate_up(omnia::Fp4::kNv, "moe_gate_up_nvfp4", x, weight, scales, nullptr, experts, hidden,
                               inner, chosen, nullptr, slots, __builtin_inff(), out, stream);
}

extern "C" int32_t omnia_moe_gate_up_nvfp4_ordinal(const uint16_t* x, const uint32_t* weight,
                                                   const uint8_t* scales, int64_t experts, int64_t hidden,
                                                   int64_t inner, const uint32_t* keys, int64_t top_k,
                                                   uint16_t* out, hipStream_t stream) {
  return omnia::launch_gate_up(omnia::Fp4::kNv, "moe_gate_up_nvfp4_ordinal", x, weight, scales, nullptr, experts,
                               hidden, inner, nullptr, keys, top_k, __builtin_inff(), out, stream);
}

extern "C" int32_t omnia_moe_down_combine_nvfp4(const uint16_t* act, const uint32_t* weight,
                                                const uint8_t* scales, int64_t experts, int64_t hidden,
                                                int64_t inner, const int32_t* chosen, const float* weights,
                                                int64_t slots, const uint16_t* residual, uint16_t* out,
                                                hipStream_t stream) {
  return omnia::launch_down(omnia::Fp4::kNv, "moe_down_combine_nvfp4", act, weight, scales, nullptr, experts,
                            hidden, inner, chosen, weights, slots, residual, out, stream);
}
