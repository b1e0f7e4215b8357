// Routed expert MLP of a one-token step over affine-quantized expert stacks (MLX's
// `QuantizedSwitchLinear`, mode "affine"): gate/up with the SwiGLU applied, then
// down/combine, the interleaved layout of the reference's affine kernels.
//
// Format (core/layers.py:164-197; decoded as core/kernels/shared/affine.py:9-58 reads it):
// a row is one little-endian bit stream of `bits`-wide values (value j at bit j * bits,
// straddling two words at 3, 5 and 6 bits), packed in uint32 words; scales and biases are
// bf16 per group of `group` values; w = scale * q + bias.
//
// Arithmetic:
//   gate_up (core/kernels/gate_up/affine.py:24-95): per row r = sum over groups of
//     scale * sum_j x_j q_j + bias * sum_j x_j (fp32, any order); rows 2n and 2n + 1 are
//     the gate and up of output n; g = T(r_gate), u = T(r_up), clamped when a limit is
//     declared (gate capped above, up clipped both ways);
//     y = T(T(g * T(1 / (1 + exp(-g)))) * u), each operation in fp32.
//   down_combine (core/kernels/down_combine/affine.py:17-70): t_e the same dot product over
//     the activation row of slot e; acc = sum over slots in order of T(fp32(T(t_e) * w_e))
//     in fp32; y = T(fp32(T(acc) + residual)).
// With a shared expert declared, the last slot reads the shared leaf, on its own width and
// group (gate_up/affine.py:36-49, down_combine/affine.py:29-44); its index is not read.
// An expert id outside [0, experts) gives zero rows.
//
// Decoding. A lane takes 32 consecutive values of a row at a time: `bits` words, one
// quantization group (groups are multiples of 32). For widths up to 6, a value q OR-ed
// into the bf16 pattern of 128.0 (0x4300) is the bf16 value 128 + q exactly (the bf16 step
// at 128 is 1), so two values go into one `v_dot2_f32_bf16` against a pair of activations;
// the 128 * sum(x) this adds comes back out through the bias term:
// scale * dot + (bias - 128 * scale) * sum(x). At 4 bits a word's pairs are its nibble
// fields i and i + 4 (mask 0x000F000F), at 2 bits fields i and i + 8, so the activations
// are paired to match once per lane; at 3, 5 and 6 bits consecutive values pair up. At 8
// bits the bytes convert to fp32 (exact), whose high halves are their bf16 values.
//
// gate_up: a wave owns kPairsPerWave gate/up pairs of one slot (consecutive rows of the
// interleaved matrix) and streams them together; x is read per 32-value chunk from L2, and
// lane p runs pair p's activation. down_combine: a workgroup owns kDownRows output rows
// with one wave per slot; 16, 32 or 64 lanes run across each row (the fewest that cover
// its chunks, one chunk per lane), so each lane loads its chunk of the slot's activations
// once for all the rows of its lane group; the slots' terms meet in LDS and are summed in
// slot order.
// Both issue a lane's loads (words, scale and bias bits each in a register of its own, the
// activations) before the arithmetic, with no branch among them: a scale packed beside
// another or a load inside a divergent branch makes the compiler wait on each load, one
// round trip per chunk. The down kernel is compiled per lane count, so a lane issues no
// load past the row's end, and its row sums associate exactly as a 16-lane row summing a
// lane's chunks in order would.
// Measured at Qwen3-30B-A3B's routed MLP, 4 bits, groups of 64, one call: gate_up with 2
// pairs per wave 6.0 us (before the load issue was fixed: 4 pairs 7.6, 8 pairs 8.7, 1 pair
// 6.6 against 6.1 for 2). down, A/B on one box: 16 lanes per row, each lane loading its
// chunks' activations for its one row, 5.6 us; 32 lanes per row at inner 768 with the
// activations held once for the lane group's rows, 5.1 us at 4 rows per workgroup, 5.0 at
// 8 (6.5 at 16), bit-identical outputs.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kChunk = 32;                // values per lane per step (`bits` words)
constexpr int kPairsPerWave = 2;          // gate_up: gate/up pairs per wave
constexpr int kGateWaves = 4;             // gate_up: waves per workgroup
constexpr int kDownRows = 8;              // down: output rows per workgroup
constexpr int kMaxInner = 1536;           // down: at most 48 chunks, one per lane
constexpr int kMaxDownSlots = 16;         // down: one wave per slot
constexpr uint32_t kMagic = 0x43004300u;  // the bf16 pair (128, 128)
constexpr uint32_t kOnes = 0x3F803F80u;   // the bf16 pair (1, 1)

struct Leaf {
  const uint32_t* weight;  // [experts, rows, in * bits / 32], or [rows, ...] when shared
  const uint16_t* scales;  // [experts, rows, in / group]
  const uint16_t* biases;
  int bits;
  int group;
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) { return dot2_bf16(a, b, c); }

// Value j of a 32-value chunk held in B words (j is a constant once unrolled).
template <int B>
__device__ __forceinline__ uint32_t field(const uint32_t (&w)[B], int j) {
  const int bit = j * B;
  const int d = bit >> 5;
  const int s = bit & 31;
  uint32_t v = w[d] >> s;
  if (s + B > 32) v |= w[d + 1] << (32 - s);
  return v & ((1u << B) - 1u);
}

// The chunk's B words, nontemporal (each weight byte is read once per step).
template <int B>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t (&w)[B]) {
  if constexpr (B == 4 || B == 8) {
#pragma unroll
    for (int i = 0; i < B / 4; ++i) {
      const u32x4 v = load_nt(reinterpret_cast<const u32x4*>(p) + i);
      w[4 * i] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
  } else if constexpr (B == 2 || B == 6) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int i = 0; i < B / 2; ++i) {
      const u32x2 v = load_nt(reinterpret_cast<const u32x2*>(p) + i);
      w[2 * i] = v.x;
      w[2 * i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < B; ++i) w[i] = load_nt(p + i);
  }
}

// A lane's 32 activations (16 bf16 pairs in memory order) paired the way the B-bit
// decoder pairs its values, and their fp32 sum.
template <int B>
__device__ __forceinline__ float pair_x(const u32x4 (&raw)[4], uint32_t (&xq)[16]) {
  uint32_t xp[16];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xp[4 * i] = raw[i].x;
    xp[4 * i + 1] = raw[i].y;
    xp[4 * i + 2] = raw[i].z;
    xp[4 * i + 3] = raw[i].w;
  }
#pragma unroll
  for (int m = 0; m < 16; ++m) sum = dot2(xp[m], kOnes, sum);
  constexpr int kSpan = B == 4 ? 8 : B == 2 ? 16 : 0;  // values per word
  if constexpr (kSpan != 0) {
    // Word d's pair i is values (kSpan d + i, kSpan d + i + kSpan / 2).
#pragma unroll
    for (int d = 0; d < 32 / kSpan; ++d) {
#pragma unroll
      for (int i = 0; i < kSpan / 2; ++i) {
        const uint32_t a = xp[(kSpan * d + i) / 2];
        const uint32_t b = xp[(kSpan * d + i + kSpan / 2) / 2];
        xq[kSpan / 2 * d + i] = (i % 2 == 0) ? ((a & 0xFFFFu) | (b << 16)) : ((a >> 16) | (b & 0xFFFF0000u));
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < 16; ++m) xq[m] = xp[m];
  }
  return sum;
}

// sum_j x_j (q_j + offset) over one chunk; offset is 128 below 8 bits, 0 at 8.
template <int B>
__device__ __forceinline__ float chunk_dot(const uint32_t (&w)[B], const uint32_t (&xq)[16]) {
  float acc = 0.0f;
  if constexpr (B == 4) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = dot2(((w[d] >> (4 * i)) & 0x000F000Fu) | kMagic, xq[4 * d + i], acc);
    }
  } else if constexpr (B == 2) {
#pragma unroll
    for (int d = 0; d < 2; ++d) {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = dot2(((w[d] >> (2 * i)) & 0x00030003u) | kMagic, xq[8 * d + i], acc);
    }
  } else if constexpr (B == 8) {
#pragma unroll
    for (int d = 0; d < 8; ++d) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float lo = static_cast<float>((w[d] >> (16 * h)) & 0xFFu);
        const float hi = static_cast<float>((w[d] >> (16 * h + 8)) & 0xFFu);
        const uint32_t pair = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
        acc = dot2(pair, xq[2 * d + h], acc);
      }
    }
  } else {
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const uint32_t pair = field<B>(w, 2 * p) | (field<B>(w, 2 * p + 1) << 16) | kMagic;
      acc = dot2(pair, xq[p], acc);
    }
  }
  return acc;
}

// The chunk's contribution scale * sum(x q) + bias * sum(x), from chunk_dot's value.
template <int B>
__device__ __forceinline__ float chunk_term(float dot, float xsum, uint32_t scale_bits, uint32_t bias_bits) {
  const float s = __uint_as_float(scale_bits << 16);   // bf16 bits, zero-extended
  const float b = __uint_as_float(bias_bits << 16);
  const float shifted = B == 8 ? b : b - 128.0f * s;
  return __builtin_fmaf(s, dot, shifted * xsum);
}

__device__ __forceinline__ bool uses_shared(const Leaf& shared, int slot, int slots) {
  return shared.weight != nullptr && slot == slots - 1;
}

// The slot's leaf, field by field: selecting the struct itself selected its address in the
// argument segment and loaded the fields from there, one more dependent scalar round trip.
__device__ __forceinline__ Leaf pick_leaf(const Leaf& shared, const Leaf& routed, bool use_shared) {
  Leaf leaf;
  leaf.weight = use_shared ? shared.weight : routed.weight;
  leaf.scales = use_shared ? shared.scales : routed.scales;
  leaf.biases = use_shared ? shared.biases : routed.biases;
  leaf.bits = use_shared ? shared.bits : routed.bits;
  leaf.group = use_shared ? shared.group : routed.group;
  return leaf;
}

// ---- gate_up ------------------------------------------------------------------------

struct GateUpArgs {
  const uint16_t* x;       // [hidden]
  Leaf routed;             // [experts, 2 * inner, hidden * bits / 32]
  Leaf shared;             // [2 * inner, ...]; weight null when none is declared
  const int32_t* chosen;   // [slots]
  uint16_t* out;           // [slots, inner]
  int64_t experts;
  int hidden;
  int inner;
  int slots;
  float limit;             // +inf: no clamp
};

// The lane's chunk of x for trip `trip` (lanes past the row's end re-read the last chunk).
__device__ __forceinline__ void load_x_chunk(const GateUpArgs& a, int lane, int trip, u32x4 (&raw)[4]) {
  const int c = min(lane + kWave * trip, a.hidden / kChunk - 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) raw[i] = reinterpret_cast<const u32x4*>(a.x + c * kChunk)[i];
}

// `first` holds the lane's chunk of x for trip 0, loaded by the caller before it read the
// expert id (x does not depend on it).
template <int B>
__device__ __forceinline__ void gate_up_rows(const GateUpArgs& a, const Leaf& leaf, int64_t row0, int rows,
                                             int lane, const u32x4 (&first)[4], float (&r)[2 * kPairsPerWave]) {
  const int chunks = a.hidden / kChunk;
  const int64_t words = static_cast<int64_t>(a.hidden) * B / 32;
  const int groups = a.hidden / leaf.group;
  const int trips = (chunks + kWave - 1) / kWave;   // uniform over the wave
  for (int trip = 0; trip < trips; ++trip) {
    // Every load of the trip goes out before its arithmetic, with no branch among them:
    // a lane past the row's end re-reads the last chunk and drops the term, and a row
    // past the wave's last pair re-reads the pair's last row (that sum is never stored).
    const int c = min(lane + kWave * trip, chunks - 1);
    u32x4 raw[4];
    if (trip == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) raw[i] = first[i];
    } else {
      load_x_chunk(a, lane, trip, raw);
    }
    uint32_t w[2 * kPairsPerWave][B];
    uint32_t sb[2 * kPairsPerWave], bb[2 * kPairsPerWave];
#pragma unroll
    for (int i = 0; i < 2 * kPairsPerWave; ++i) {
      const int64_t row = row0 + min(i, rows - 1);
      load_words<B>(leaf.weight + row * words + static_cast<int64_t>(c) * B, w[i]);
      const int64_t g = row * groups + (c * kChunk) / leaf.group;
      sb[i] = leaf.scales[g];
      bb[i] = leaf.biases[g];
    }
    __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the arithmetic
    uint32_t xq[16];
    const float xsum = pair_x<B>(raw, xq);
    const bool in_row = lane + kWave * trip < chunks;
#pragma unroll
    for (int i = 0; i < 2 * kPairsPerWave; ++i) {
      const float term = r[i] + chunk_term<B>(chunk_dot<B>(w[i], xq), xsum, sb[i], bb[i]);
      r[i] = in_row ? term : r[i];
    }
  }
}

// The arguments the first loads need come first, as scalars (copies of GateUpArgs fields):
// gfx950 preloads a kernel's leading scalar and pointer arguments into SGPRs at wave
// launch, so the id's and x's loads go out with no scalar round trip ahead of them, and
// GateUpArgs is loaded while they are in flight (5.43 -> 5.29 us at the decode shape).
__global__ __launch_bounds__(kGateWaves * kWave) void moe_gate_up_affine_kernel(
    const uint16_t* x, const int32_t* chosen_ids, int hidden, int inner, GateUpArgs a) {
  const int lane = threadIdx.x % kWave;
  const int slot = blockIdx.y;
  const int pair0 = (blockIdx.x * kGateWaves + threadIdx.x / kWave) * kPairsPerWave;
  // No early exit: a branch on the size made it a scalar round trip of its own ahead of
  // the other arguments' (two before the first load). A wave past the last pair computes
  // the last one and stores nothing.
  const bool wave_live = pair0 < inner;
  const int first_pair = wave_live ? pair0 : inner - 1;
  const int pairs = min(kPairsPerWave, inner - first_pair);
  const int stored = wave_live ? pairs : 0;
  // The expert id, then the lane's first chunk of x, which does not depend on it: the
  // chunk's round trip overlaps the id's. The id is read through the vector path (every
  // lane reads the same word): a scalar read was sunk by the compiler into the branch that
  // uses it, behind the wait for GateUpArgs, while vector loads return in order, so
  // waiting for the id waits for nothing issued after it.
  int zero = 0;
  asm volatile("" : "+v"(zero));   // a zero the compiler cannot see as uniform
  const int chosen_v = chosen_ids[slot + zero];
  u32x4 first[4];
  {
    const int c = min(lane, hidden / kChunk - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) first[i] = reinterpret_cast<const u32x4*>(x + c * kChunk)[i];
  }
  __builtin_amdgcn_sched_barrier(0);   // the chunk's loads ahead of the wait for the id
  const int chosen = __builtin_amdgcn_readfirstlane(chosen_v);
  const bool shared = uses_shared(a.shared, slot, a.slots);
  const Leaf leaf = pick_leaf(a.shared, a.routed, shared);
  // Every GateUpArgs field the rest of the kernel uses, taken here together: one wait,
  // overlapping the id's and x's round trips (each was otherwise loaded at its first use,
  // the leaf's behind the id's wait and `out`'s and the limit's at the store).
  asm volatile("" ::"s"(leaf.weight), "s"(leaf.scales), "s"(leaf.biases), "s"(leaf.bits), "s"(leaf.group),
               "s"(a.out), "s"(a.experts), "s"(a.limit));
  uint16_t* out = a.out + static_cast<int64_t>(slot) * a.inner + first_pair;
  int64_t row0 = 2 * static_cast<int64_t>(first_pair);
  if (!shared) {
    if (chosen < 0 || chosen >= a.experts) {
      if (lane < stored) out[lane] = 0;
      return;
    }
    row0 += static_cast<int64_t>(chosen) * 2 * a.inner;
  }
  float r[2 * kPairsPerWave];
#pragma unroll
  for (int i = 0; i < 2 * kPairsPerWave; ++i) r[i] = 0.0f;
  switch (leaf.bits) {  // wave-uniform
    case 2: gate_up_rows<2>(a, leaf, row0, 2 * pairs, lane, first, r); break;
    case 3: gate_up_rows<3>(a, leaf, row0, 2 * pairs, lane, first, r); break;
    case 4: gate_up_rows<4>(a, leaf, row0, 2 * pairs, lane, first, r); break;
    case 5: gate_up_rows<5>(a, leaf, row0, 2 * pairs, lane, first, r); break;
    case 6: gate_up_rows<6>(a, leaf, row0, 2 * pairs, lane, first, r); break;
    default: gate_up_rows<8>(a, leaf, row0, 2 * pairs, lane, first, r); break;
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
  float g = round_bf16(gate_sum);
  float u = round_bf16(up_sum);
  if (a.limit < __builtin_inff()) {
    g = fminf(g, a.limit);
    u = fminf(fmaxf(u, -a.limit), a.limit);
  }
  const float den = 1.0f + expf(-g);
  const float sig = round_bf16(1.0f / den);
  const float act = round_bf16(g * sig);
  if (lane < stored) out[lane] = f32_to_bf16(act * u);
}

// ---- down_combine -------------------------------------------------------------------

struct DownArgs {
  const uint16_t* act;      // [slots, inner]
  Leaf routed;              // [experts, hidden, inner * bits / 32]
  Leaf shared;              // [hidden, ...]; weight null when none is declared
  const int32_t* chosen;    // [slots]
  const float* weights;     // [slots]
  const uint16_t* residual; // [hidden] or null
  uint16_t* out;            // [hidden]
  int64_t experts;
  int hidden;
  int inner;
  int slots;
};

// The terms of one lane group's rows (rows group, group + kGroups, ... of the workgroup's
// kDownRows) for the lane's chunk `part` of the slot's activation row (`raw`, loaded by the
// caller): every weight load (each row's words, scale and bias bits in registers of their
// own) goes out before any arithmetic, with no branch among them; the activations are
// paired while the rows arrive, and each row is summed as soon as its own words are in. A
// lane past the row's last chunk re-reads that chunk and drops the term, and a row past
// the last one re-reads the last (its sum is never used).
template <int B, int kLanes>
__device__ __forceinline__ void down_terms(const DownArgs& a, const Leaf& leaf, int64_t row_first,
                                           int rows, int group, int part, const u32x4 (&raw)[4],
                                           float (&t)[kDownRows * kLanes / kWave]) {
  constexpr int kGroups = kWave / kLanes;
  constexpr int kRowsPerGroup = kDownRows / kGroups;
  const int chunks = a.inner / kChunk;
  const int64_t words = static_cast<int64_t>(a.inner) * B / 32;
  const int groups = a.inner / leaf.group;
  const int c = min(part, chunks - 1);
  uint32_t w[kRowsPerGroup][B];
  uint32_t sb[kRowsPerGroup], bb[kRowsPerGroup];
#pragma unroll
  for (int q = 0; q < kRowsPerGroup; ++q) {
    const int64_t row = row_first + min(group + kGroups * q, rows - 1);
    load_words<B>(leaf.weight + row * words + static_cast<int64_t>(c) * B, w[q]);
    const int64_t g = row * groups + (c * kChunk) / leaf.group;
    sb[q] = leaf.scales[g];
    bb[q] = leaf.biases[g];
  }
  __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the arithmetic
  uint32_t xq[16];
  const float xsum = pair_x<B>(raw, xq);
  const bool in_row = part < chunks;
#pragma unroll
  for (int q = 0; q < kRowsPerGroup; ++q) {
    const float term = 0.0f + chunk_term<B>(chunk_dot<B>(w[q], xq), xsum, sb[q], bb[q]);
    t[q] = in_row ? term : 0.0f;
  }
}

// One wave per slot; kLanes lanes across each row (16, 32 or 64: the fewest that cover
// the row's chunks), so each lane holds one activation chunk for the rows of its group.
template <int kLanes>
// As in the gate/up kernel, the arguments the first loads need come first, as scalars
// (copies of DownArgs fields and the grid size), preloaded into SGPRs at wave launch
// (4.57 -> 4.36 us at the decode shape).
__global__ __launch_bounds__(kMaxDownSlots * kWave) void moe_down_affine_kernel(
    const uint16_t* act, const int32_t* chosen_ids, const float* route_weights,
    const uint16_t* residual, int inner, int hidden, int blocks, DownArgs a) {
  constexpr int kGroups = kWave / kLanes;
  constexpr int kRowsPerGroup = kDownRows / kGroups;
  __shared__ float partial[kMaxDownSlots][kDownRows];
  const int lane = threadIdx.x % kWave;
  // One wave per slot.
  const int slot = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int row_base = xcd_contiguous_block(blockIdx.x, blocks) * kDownRows;
  const int rows = min(kDownRows, hidden - row_base);
  const int group = lane / kLanes;
  const int part = lane % kLanes;
  // The slot's routing entries (weight and expert id) first, through the vector path
  // (every lane of the wave reads the same word): vector loads return in order, so waiting
  // for them waits for nothing issued after them. As scalar reads, the compiler issued
  // them after DownArgs' loads and waited for those first (one register was shared). Then
  // the residual of the output row this thread writes (rows past the last read the last).
  const int slot_lanes = static_cast<int>(threadIdx.x / kWave);
  const float route_weight_v = route_weights[slot_lanes];
  const int chosen_v = chosen_ids[slot_lanes];
  const uint32_t resid = early_bf16_bits(
      residual, row_base + min(static_cast<int>(threadIdx.x % kDownRows), rows - 1), act);
  // The slot's activation chunk, which does not depend on the id: its round trip overlaps
  // the id's.
  u32x4 raw[4];
  {
    const int c = min(part, inner / kChunk - 1);
    const uint16_t* x = act + static_cast<int64_t>(slot) * inner + c * kChunk;
#pragma unroll
    for (int j = 0; j < 4; ++j) raw[j] = reinterpret_cast<const u32x4*>(x)[j];
  }
  __builtin_amdgcn_sched_barrier(0);   // the chunk's loads ahead of the wait for the id
  const int chosen = __builtin_amdgcn_readfirstlane(chosen_v);
  const float route_weight = __builtin_bit_cast(
      float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, route_weight_v)));
  // The leaf, and every other DownArgs field the kernel uses, taken together so that one
  // wait covers DownArgs' loads (each was otherwise loaded at its first use, `out` and the
  // slot count at the combine).
  const bool shared = uses_shared(a.shared, slot, a.slots);
  const Leaf leaf = pick_leaf(a.shared, a.routed, shared);
  const int64_t experts = a.experts;
  asm volatile("" ::"s"(chosen), "s"(leaf.weight), "s"(leaf.scales), "s"(leaf.biases), "s"(leaf.bits),
               "s"(leaf.group), "s"(experts), "s"(a.out), "s"(a.slots));
  __builtin_amdgcn_sched_barrier(0);
  // Selects, no branch (a branch would let the compiler sink the id's read into it).
  const bool routed_ok = chosen >= 0 && chosen < experts;   // uniform over the wave
  const bool valid = shared || routed_ok;
  const int64_t row_first = row_base + static_cast<int64_t>(!shared && routed_ok ? chosen : 0) * a.hidden;
  float t[kRowsPerGroup];
#pragma unroll
  for (int q = 0; q < kRowsPerGroup; ++q) t[q] = 0.0f;
  if (valid) {
    switch (leaf.bits) {  // wave-uniform
      case 2: down_terms<2, kLanes>(a, leaf, row_first, rows, group, part, raw, t); break;
      case 3: down_terms<3, kLanes>(a, leaf, row_first, rows, group, part, raw, t); break;
      case 4: down_terms<4, kLanes>(a, leaf, row_first, rows, group, part, raw, t); break;
      case 5: down_terms<5, kLanes>(a, leaf, row_first, rows, group, part, raw, t); break;
      case 6: down_terms<6, kLanes>(a, leaf, row_first, rows, group, part, raw, t); break;
      default: down_terms<8, kLanes>(a, leaf, row_first, rows, group, part, raw, t); break;
    }
  }
#pragma unroll
  for (int q = 0; q < kRowsPerGroup; ++q) {
    const float sum = group_row_sum<kLanes>(t[q]);
    const int row = group + kGroups * q;
    if (part == 0) partial[slot][row] = valid ? round_bf16(round_bf16(sum) * route_weight) : 0.0f;
  }
  __syncthreads();
  if (threadIdx.x < kDownRows && row_base + static_cast<int>(threadIdx.x) < a.hidden) {
    const int n = row_base + threadIdx.x;
    float sum = 0.0f;
    for (int j = 0; j < a.slots; ++j) sum += partial[j][threadIdx.x];
    float out = round_bf16(sum);
    if (a.residual != nullptr) out = out + bf16_to_f32(resid);
    a.out[n] = f32_to_bf16(out);
  }
}

bool valid_format(int64_t bits, int64_t group) {
  return (bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8) &&
         (group == 32 || group == 64 || group == 128);
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_moe_gate_up_affine(
    const uint16_t* x, const uint32_t* weight, const uint16_t* scales, const uint16_t* biases,
    int64_t experts, int64_t hidden, int64_t inner, int64_t bits, int64_t group_size,
    const int32_t* chosen, int64_t slots, float limit, const uint32_t* shared_weight,
    const uint16_t* shared_scales, const uint16_t* shared_biases, int64_t shared_bits,
    int64_t shared_group_size, uint16_t* out, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(experts > 0 && experts < (int64_t{1} << 20), "moe_gate_up_affine: bad expert count");
  OMNIA_REQUIRE(hidden > 0 && hidden % kChunk == 0 && hidden <= 16384,
                "moe_gate_up_affine: hidden must be a multiple of 32 in [32, 16384]");
  OMNIA_REQUIRE(inner > 0 && inner < (int64_t{1} << 24), "moe_gate_up_affine: bad inner size");
  OMNIA_REQUIRE(valid_format(bits, group_size) && hidden % group_size == 0,
                "moe_gate_up_affine: bits must be 2, 3, 4, 5, 6 or 8 and the group 32, 64 or 128, dividing hidden");
  OMNIA_REQUIRE(slots >= 0 && slots <= 1024, "moe_gate_up_affine: slots must be in [0, 1024]");
  OMNIA_REQUIRE(!(limit < 0.0f), "moe_gate_up_affine: the limit must be non-negative (+inf: none)");
  if (slots == 0) return 0;
  OMNIA_REQUIRE(x && weight && scales && biases && chosen && out, "moe_gate_up_affine: null pointer");
  OMNIA_REQUIRE(aligned16(x) && aligned16(weight), "moe_gate_up_affine: x and weight must be 16-byte aligned");
  if (shared_weight != nullptr) {
    OMNIA_REQUIRE(shared_scales && shared_biases, "moe_gate_up_affine: shared leaf without scales or biases");
    OMNIA_REQUIRE(valid_format(shared_bits, shared_group_size) && hidden % shared_group_size == 0,
                  "moe_gate_up_affine: bad shared width or group");
    OMNIA_REQUIRE(aligned16(shared_weight), "moe_gate_up_affine: the shared weight must be 16-byte aligned");
  }
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  GateUpArgs a{x,
               Leaf{weight, scales, biases, static_cast<int>(bits), static_cast<int>(group_size)},
               Leaf{shared_weight, shared_scales, shared_biases, static_cast<int>(shared_bits),
                    static_cast<int>(shared_group_size)},
               chosen, out, experts, static_cast<int>(hidden), static_cast<int>(inner),
               static_cast<int>(slots), limit};
  const int64_t waves = (inner + kPairsPerWave - 1) / kPairsPerWave;
  const dim3 grid(static_cast<unsigned>((waves + kGateWaves - 1) / kGateWaves), static_cast<unsigned>(slots));
  moe_gate_up_affine_kernel<<<grid, kGateWaves * kWave, 0, stream>>>(a.x, a.chosen, a.hidden, a.inner, a);
  return launched("moe_gate_up_affine");
}

extern "C" int32_t omnia_moe_down_combine_affine(
    const uint16_t* act, const uint32_t* weight, const uint16_t* scales, const uint16_t* biases,
    int64_t experts, int64_t hidden, int64_t inner, int64_t bits, int64_t group_size,
    const int32_t* chosen, const float* weights, int64_t slots, const uint16_t* residual,
    const uint32_t* shared_weight, const uint16_t* shared_scales, const uint16_t* shared_biases,
    int64_t shared_bits, int64_t shared_group_size, uint16_t* out, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(experts > 0 && experts < (int64_t{1} << 20), "moe_down_combine_affine: bad expert count");
  OMNIA_REQUIRE(hidden > 0 && hidden < (int64_t{1} << 24), "moe_down_combine_affine: bad hidden size");
  OMNIA_REQUIRE(inner > 0 && inner % kChunk == 0 && inner <= kMaxInner,
                "moe_down_combine_affine: inner must be a multiple of 32 in [32, 1536]");
  OMNIA_REQUIRE(valid_format(bits, group_size) && inner % group_size == 0,
                "moe_down_combine_affine: bits must be 2, 3, 4, 5, 6 or 8 and the group 32, 64 or 128, dividing inner");
  OMNIA_REQUIRE(slots > 0 && slots <= kMaxDownSlots, "moe_down_combine_affine: slots must be in [1, 16]");
  OMNIA_REQUIRE(act && weight && scales && biases && chosen && weights && out,
                "moe_down_combine_affine: null pointer");
  OMNIA_REQUIRE(aligned16(act) && aligned16(weight), "moe_down_combine_affine: act and weight must be 16-byte aligned");
  if (shared_weight != nullptr) {
    OMNIA_REQUIRE(shared_scales && shared_biases, "moe_down_combine_affine: shared leaf without scales or biases");
    OMNIA_REQUIRE(valid_format(shared_bits, shared_group_size) && inner % shared_group_size == 0,
                  "moe_down_combine_affine: bad shared width or group");
    OMNIA_REQUIRE(aligned16(shared_weight), "moe_down_combine_affine: the shared weight must be 16-byte aligned");
  }
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  DownArgs a{act,
             Leaf{weight, scales, biases, static_cast<int>(bits), static_cast<int>(group_size)},
             Leaf{shared_weight, shared_scales, shared_biases, static_cast<int>(shared_bits),
                  static_cast<int>(shared_group_size)},
             chosen, weights, residual, out, experts, static_cast<int>(hidden),
             static_cast<int>(inner), static_cast<int>(slots)};
  const dim3 grid(static_cast<unsigned>((hidden + kDownRows - 1) / kDownRows));
  const dim3 block(static_cast<unsigned>(slots * kWave));
  static_assert(kMaxInner / kChunk <= kWave, "a row's chunks fit one wave");
  const int64_t chunks = inner / kChunk;
  if (chunks <= 16) {
    moe_down_affine_kernel<16><<<grid, block, 0, stream>>>(
        a.act, a.chosen, a.weights, a.residual, a.inner, a.hidden, static_cast<int>(grid.x), a);
  } else if (chunks <= 32) {
    moe_down_affine_kernel<32><<<grid, block, 0, stream>>>(
        a.act, a.chosen, a.weights, a.residual, a.inner, a.hidden, static_cast<int>(grid.x), a);
  } else {
    moe_down_affine_kernel<64><<<grid, block, 0, stream>>>(
        a.act, a.chosen, a.weights, a.residual, a.inner, a.hidden, static_cast<int>(grid.x), a);
  }
  return launched("moe_down_combine_affine");
}
