// Per-head q/k RMSNorm + half-split rotary, one dispatch for every head of a segment.
//
// Arithmetic (core/kernels/qkv_rope/qk_norm_rope.py:21-24,120-140,295-308; the norm
// rounds as mx.fast.rms_norm does):
//   inv  = 1 / sqrt(sum_d x_d^2 / D + eps)   (sum in fp64, rounded once to fp32)
//   n_d  = bf16(w_d * bf16(x_d * inv))
//   for p < P:  a = bf16(n_p * bf16(mscale)),  b = bf16(n_{p+P} * bf16(mscale))
//               out_p     = bf16(a * cos_p - b * sin_p)
//               out_{p+P} = bf16(a * sin_p + b * cos_p)
//   for 2P <= d < D:  out_d = n_d                     (partial-rotary tail)
// (cos_p, sin_p) come either from a caller's fp32 table row `offset + t`
// (`omnia_qk_norm_rope`), or are derived in-kernel exactly as
// core/kernels/qkv_rope/epilogue.py:57-63 derives them (`omnia_rope_epilogue`):
//   angle_p = f32(pos) * exp2(-(p / P) * log2(base)),  with cos/sin of that fp32 angle.
// In-kernel, exp2, cos and sin are evaluated in fp64 (sin_cos_fp64, common.hpp) and rounded
// once to fp32, i.e. correctly rounded for all practical purposes (the reference's Metal code uses
// fast::cos/sin, which no other machine reproduces bit for bit).
//
// Layout (wave64): a head of D bf16 is G = D/8 lanes x one 16-byte vector, so one
// wave instruction covers a "slot" of 64/G heads (4 at D=128). A wave owns a few slots
// (`slots_per_wave`, 2 for prefill) of the q heads or of the k heads of one token, so
// its norm weight, input row and output base are wave-uniform; it issues all its head
// loads before any arithmetic and loads its eight (cos, sin) pairs once (L2-resident:
// every wave of a token reads the same 512-byte row). There is no LDS and no barrier:
// measured on MI355X, a per-token workgroup that stages the row in LDS behind a
// barrier runs slower than these independent waves, and so do waves owning a whole
// token (fewer, longer waves leave HBM idle in the ramp and the tail).
// The rotary partner of element p is element p+P, on lane `lane ^ (P/8)` of the same
// head group: one cross-lane exchange of four packed dwords. The per-head sum of
// squares is a butterfly inside the G-lane group. No LDS and no barrier.
// Input is token-major with a row stride (so q and k can be read straight out of a
// fused qkv projection); output is head-major [heads, T, D], the layout attention
// consumes (qk_norm_rope.py:163-175).
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kWavesPerBlock = 4;
// Below this many waves at eight pairs per lane, the full-rotary kernel runs four.
constexpr int64_t kNarrowWaves = 2048;

struct RopeArgs {
  const uint16_t* queries_in;
  const uint16_t* keys_in;
  const uint16_t* query_weight;
  const uint16_t* key_weight;
  const float* cos_table;
  const float* sin_table;
  uint16_t* queries_out;
  uint16_t* keys_out;
  int64_t length;
  int64_t query_stride;  // elements between consecutive tokens of the q input
  int64_t key_stride;
  int64_t table_stride;  // floats between consecutive table rows
  int64_t offset;        // position of token 0
  int query_heads;
  int kv_heads;
  int pairs;             // P
  int q_parts;           // waves per token on the q heads
  int k_parts;           // waves per token on the k heads
  float eps;
  float mscale;
  float log2_base;
};

// cos/sin of the in-kernel angle for pair `pair` at `position` (epilogue.py:57-63),
// evaluated in fp64 and rounded once to fp32.
__device__ __forceinline__ void derived_angle(int pair, int pairs, int64_t position,
                                              float log2_base, float& c, float& s) {
  const float d = static_cast<float>(pair) / static_cast<float>(pairs);
  const float exponent = -d * log2_base;
  const float frequency = static_cast<float>(exp2(static_cast<double>(exponent)));
  const float angle = static_cast<float>(position) * frequency;
  double sd, cd;
  sin_cos_fp64(static_cast<double>(angle), sd, cd);
  c = static_cast<float>(cd);
  s = static_cast<float>(sd);
}

// Sum over the G lanes of each head group.
template <int G>
__device__ __forceinline__ double head_sum(double value) {
  if constexpr (G == 16) {
    return row16_sum(value);
  } else {
    return group_sum<G>(value);
  }
}

// Sum over groups of G consecutive lanes (G = 4, 8 or 16) by DPP steps inside each
// 16-lane row: quad swaps, then the half-row mirror, then the row mirror. Both lanes of
// each exchange add the same two operands, so every lane of a group ends with the same
// total.
template <int G>
__device__ __forceinline__ double dpp_group_sum(double value) {
#define OMNIA_DPP_STEP(ctrl)                                                          \
  {                                                                                   \
    const uint64_t bits = __builtin_bit_cast(uint64_t, value);                        \
    const uint32_t lo = dpp<ctrl>(static_cast<uint32_t>(bits));                       \
    const uint32_t hi = dpp<ctrl>(static_cast<uint32_t>(bits >> 32));                 \
    value += __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);      \
  }
  static_assert(G == 4 || G == 8 || G == 16, "group of 4, 8 or 16 lanes");
  OMNIA_DPP_STEP(kQuadSwap1)
  OMNIA_DPP_STEP(kQuadSwap2)
  if constexpr (G >= 8) OMNIA_DPP_STEP(kRowHalfMirror)
  if constexpr (G == 16) OMNIA_DPP_STEP(kRowMirror)
#undef OMNIA_DPP_STEP
  return value;
}

// The partner half of each rotary pair, `pair_lanes` lanes away inside the head.
template <int G, bool FULL>
__device__ __forceinline__ uint32_t partner(uint32_t value, int pair_lanes) {
  if constexpr (G == 16 && FULL) {
    return dpp<kRowRor8>(value);  // pair_lanes == 8: the other half of the DPP row
  } else {
    return static_cast<uint32_t>(__shfl_xor(static_cast<int>(value), pair_lanes, kWave));
  }
}

// SPW: slots per wave. FULL: 2P == D (every lane rotates). SCALED: mscale != 1 (the
// bf16 pre-scale round trip is applied; at mscale == 1 it is the identity and is
// skipped). EXACT: both head counts are multiples of the heads per slot, so no lane of
// any slot is idle.
template <int D, int SPW, bool TABLE, bool FULL, bool SCALED, bool EXACT>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void qk_norm_rope_kernel(RopeArgs a) {
  constexpr int G = D / 8;          // lanes per head
  constexpr int kHeadsPerSlot = kWave / G;
  const int lane = threadIdx.x % kWave;
  const int parts = a.q_parts + a.k_parts;
  // A 32-bit division (the launch keeps the unit count below 2^32): a 64-bit one is a long
  // instruction sequence ahead of every wave's first load.
  const uint32_t unit = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  const int64_t t = unit / static_cast<uint32_t>(parts);
  if (t >= a.length) return;  // whole wave leaves together; no barrier follows
  const int part = static_cast<int>(unit - static_cast<uint32_t>(t) * static_cast<uint32_t>(parts));
  const bool is_query = part < a.q_parts;  // wave-uniform
  const int heads = is_query ? a.query_heads : a.kv_heads;
  const int slots = (heads + kHeadsPerSlot - 1) / kHeadsPerSlot;
  const int slot_begin = (is_query ? part : part - a.q_parts) * SPW;
  const int slot_end = min(slots, slot_begin + SPW);
  const int64_t position = a.offset + t;
  const int g = lane % G;               // lane within its head
  const int head_in_slot = lane / G;
  const int pair_lanes = a.pairs / 8;   // lanes holding the first rotary half
  const bool rotary = FULL || g < 2 * pair_lanes;
  const bool first_half = g < pair_lanes;
  const int base = rotary ? (first_half ? g : g - pair_lanes) * 8 : 0;

  // This lane's eight (cos, sin) pairs. With the sine negated on first-half lanes, both
  // halves rotate as own * cos + partner * sin:
  //   first half:  a*cos - b*sin   (own = a, partner = b)
  //   second half: a*sin + b*cos = b*cos + a*sin   (own = b, partner = a)
  // which are the reference's expressions term for term (negation and the order of
  // the two addends do not change an IEEE result).
  float c[8], s[8];
  if constexpr (TABLE) {
    f32x4 c0 = {}, c1 = {}, s0 = {}, s1 = {};
    if (rotary) {
      const float* crow = a.cos_table + position * a.table_stride + base;
      const float* srow = a.sin_table + position * a.table_stride + base;
      c0 = *reinterpret_cast<const f32x4*>(crow);
      c1 = *reinterpret_cast<const f32x4*>(crow + 4);
      s0 = *reinterpret_cast<const f32x4*>(srow);
      s1 = *reinterpret_cast<const f32x4*>(srow + 4);
    }
    c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w;
    c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
    s[0] = s0.x; s[1] = s0.y; s[2] = s0.z; s[3] = s0.w;
    s[4] = s1.x; s[5] = s1.y; s[6] = s1.z; s[7] = s1.w;
  } else {
    // Lane i derives pairs i and i+64; lanes then fetch the pairs they rotate.
    float cl = 0.0f, sl = 0.0f, ch = 0.0f, sh = 0.0f;
    if (lane < a.pairs) derived_angle(lane, a.pairs, position, a.log2_base, cl, sl);
    if (D == 256 && lane + kWave < a.pairs) {
      derived_angle(lane + kWave, a.pairs, position, a.log2_base, ch, sh);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int pair = base + j;
      const float lo_c = __shfl(cl, pair % kWave, kWave);
      const float lo_s = __shfl(sl, pair % kWave, kWave);
      if (D == 256) {
        const float hi_c = __shfl(ch, pair % kWave, kWave);
        const float hi_s = __shfl(sh, pair % kWave, kWave);
        c[j] = pair < kWave ? lo_c : hi_c;
        s[j] = pair < kWave ? lo_s : hi_s;
      } else {
        c[j] = lo_c;
        s[j] = lo_s;
      }
    }
  }
  float w[8];
  unpack8(*(reinterpret_cast<const u32x4*>(is_query ? a.query_weight : a.key_weight) + g), w);

  // Head loads go out after the table row and weight loads: vector-memory results are
  // counted in issue order, so the first slot's arithmetic then waits only for the
  // row, the weight and its own head, while the later heads are still in flight.
  const uint16_t* in = (is_query ? a.queries_in + t * a.query_stride
                                 : a.keys_in + t * a.key_stride) + head_in_slot * D + g * 8;
  u32x4 raw[SPW];
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    const int slot = slot_begin + i;
    raw[i] = u32x4{0u, 0u, 0u, 0u};
    if (slot < slot_end && (EXACT || slot * kHeadsPerSlot + head_in_slot < heads)) {
      raw[i] = load_nt(reinterpret_cast<const u32x4*>(in + slot * kHeadsPerSlot * D));
    }
  }

#pragma unroll
  for (int j = 0; j < 8; ++j) s[j] = first_half ? -s[j] : s[j];

  uint16_t* out = (is_query ? a.queries_out : a.keys_out) + (head_in_slot * a.length + t) * D + g * 8;
  const int64_t out_slot = static_cast<int64_t>(kHeadsPerSlot) * a.length * D;

#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    const int slot = slot_begin + i;
    if (slot >= slot_end) break;  // uniform across the wave
    float x[8];
    unpack8(raw[i], x);
    double sumsq = 0.0;
#pragma unroll
    for (int j = 0; j < 8; ++j) sumsq += static_cast<double>(x[j] * x[j]);
    sumsq = head_sum<G>(sumsq);
    const float inv =
        1.0f / sqrtf(static_cast<float>(sumsq) / static_cast<float>(D) + a.eps);

    // n = bf16(w * bf16(x * inv)), two elements per conversion.
    float n[8];
    uint32_t packed[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      float lo = x[j] * inv, hi = x[j + 1] * inv;
      round_pair(lo, hi);
      packed[j / 2] = pack_bf16(w[j] * lo, w[j + 1] * hi);
      n[j] = bf16_lo(packed[j / 2]);
      n[j + 1] = bf16_hi(packed[j / 2]);
    }
    float other[8];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const uint32_t theirs = partner<G, FULL>(packed[j / 2], pair_lanes);
      other[j] = bf16_lo(theirs);
      other[j + 1] = bf16_hi(theirs);
    }
    float own[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) own[j] = n[j];
    if constexpr (SCALED) {
      const float mscale = round_bf16(a.mscale);
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        own[j] *= mscale; own[j + 1] *= mscale;
        other[j] *= mscale; other[j + 1] *= mscale;
        round_pair(own[j], own[j + 1]);
        round_pair(other[j], other[j + 1]);
      }
    }
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float rotated = own[j] * c[j] + other[j] * s[j];
      o[j] = FULL ? rotated : (rotary ? rotated : n[j]);
    }
    if (EXACT || slot * kHeadsPerSlot + head_in_slot < heads) {
      store_nt(reinterpret_cast<u32x4*>(out + slot * out_slot), pack8(o));
    }
  }
}

// The 16-byte or 8-byte vectors of PPL bf16 values (PPL / 2 words), loaded and stored as
// one instruction.
template <int W> struct WordVector;
template <> struct WordVector<4> { using T = u32x4; };
template <> struct WordVector<2> { using T = uint32_t __attribute__((ext_vector_type(2))); };

template <int W, bool NT>
__device__ __forceinline__ void load_words(const uint16_t* p, uint32_t (&out)[W]) {
  using T = typename WordVector<W>::T;
  const T v = NT ? load_nt(reinterpret_cast<const T*>(p)) : *reinterpret_cast<const T*>(p);
#pragma unroll
  for (int i = 0; i < W; ++i) out[i] = v[i];
}

template <int W>
__device__ __forceinline__ void store_words(uint16_t* p, const uint32_t (&in)[W]) {
  using T = typename WordVector<W>::T;
  T v;
#pragma unroll
  for (int i = 0; i < W; ++i) v[i] = in[i];
  store_nt(reinterpret_cast<T*>(p), v);
}

// Full-rotary layout (2P == D): each lane owns PPL rotary pairs (p, p + P), p = PPL g ..
// PPL g + PPL - 1 of one head, read as one vector from each half (16 bytes at PPL = 8,
// 8 bytes at PPL = 4). A head is then G = P / PPL lanes (8 at D = 128, PPL = 8) and one
// wave instruction covers 64 / G heads; each wave owns one such slot of the q heads or
// of the k heads of one token. Each lane holds both halves of its pairs, so the
// rotation needs no cross-lane exchange, and the per-head sum of squares is a DPP
// reduction over G lanes. Measured on MI355X at the prefill shape, this beats the
// partner-exchange layout by about 3%. Small grids take PPL = 4 (the launch's choice).
//
// Which waves run together decides how the transposed output [heads, T, D] is written.
// Token by token (the derived-angle form), the waves in flight write 256-byte pieces
// of every head plane at once. With a table (slot-major), a workgroup's four waves take
// four consecutive tokens of one slot and consecutive workgroups the next four, so the
// waves in flight write long runs of the same eight head planes: 16.78 against 17.14 us
// at the prefill shape (T = 4096, 32 + 8 heads), the decode step 2.65 against 2.75 us.
// The derived-angle form measured no gain from it.
//
// kLead: the form whose arguments for the input loads arrive preloaded (the leading-
// argument kernel below): the inputs' loads go out first, ahead of any wait for RopeArgs.
// Otherwise the weights go out first, then the inputs, once RopeArgs has arrived.
template <int D, int PPL, bool TABLE, bool SCALED, bool EXACT, bool kLead>
__device__ __forceinline__ void pairs_body(const RopeArgs& a, const uint16_t* queries_in,
                                           const uint16_t* keys_in, int64_t length,
                                           int64_t query_stride, int64_t key_stride, int q_parts,
                                           int query_heads, int kv_heads) {
  constexpr int P = D / 2;
  constexpr int G = P / PPL;                 // lanes per head
  constexpr int W = PPL / 2;                 // words per half
  constexpr int kHeadsPerSlot = kWave / G;
  static_assert(PPL == 8 || PPL == 4, "eight or four pairs per lane");
  const int lane = threadIdx.x % kWave;
  const int parts = q_parts + a.k_parts;   // one slot per wave
  int64_t t;
  int part;
  if constexpr (TABLE) {
    // Slot-major on a 2-D grid (x fastest: the same order as one dimension of slot *
    // groups + group, with no division): workgroup (g, slot) takes tokens 4 g + wave.
    part = static_cast<int>(blockIdx.y);
    t = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  } else {
    // A 32-bit division (the launch keeps the unit count below 2^32): a 64-bit one is a
    // long instruction sequence ahead of every wave's first load.
    const uint32_t unit = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    t = unit / static_cast<uint32_t>(parts);
    part = static_cast<int>(unit - static_cast<uint32_t>(t) * static_cast<uint32_t>(parts));
  }
  // No early exit: a wave past the last token (in the last token group only) computes the
  // last token's values and stores nothing. With a branch here the compiler loaded the
  // length alone, waited for it, and only then loaded the other arguments: two dependent
  // scalar round trips ahead of the first vector load instead of one.
  const bool token_live = t < length;
  t = token_live ? t : length - 1;
  const bool is_query = part < q_parts;   // wave-uniform
  const int heads = is_query ? query_heads : kv_heads;
  const int slot = is_query ? part : part - q_parts;
  const int g = lane % G;
  const int head = slot * kHeadsPerSlot + lane / G;
  const bool live = EXACT || head < heads;
  const int base = g * PPL;                  // first pair of this lane

  // Every load goes out before any arithmetic, in the order the arithmetic needs them
  // (vector-memory results are counted in issue order): the weights and the head's two
  // halves (the halves first in the kLead form), then the table row, with no branch among
  // them (a load in a branch makes the compiler wait on it). A lane of a head past the
  // last reads the last head and is zeroed afterwards.
  uint32_t wraw1[W], wraw2[W], first[W], second[W];
  int64_t position;
  if constexpr (kLead) {
    const int head_read = live ? head : heads - 1;
    const uint16_t* in = (is_query ? queries_in + t * query_stride
                                   : keys_in + t * key_stride) + head_read * D + base;
    load_words<W, true>(in, first);
    load_words<W, true>(in + P, second);
    __builtin_amdgcn_sched_barrier(0);   // the inputs' loads ahead of any wait for RopeArgs
    position = a.offset + t;
    const uint16_t* weight = is_query ? a.query_weight : a.key_weight;
    load_words<W, false>(weight + base, wraw1);
    load_words<W, false>(weight + P + base, wraw2);
  } else {
    position = a.offset + t;
    const uint16_t* weight = is_query ? a.query_weight : a.key_weight;
    load_words<W, false>(weight + base, wraw1);
    load_words<W, false>(weight + P + base, wraw2);
    const int head_read = live ? head : heads - 1;
    const uint16_t* in = (is_query ? queries_in + t * query_stride
                                   : keys_in + t * key_stride) + head_read * D + base;
    load_words<W, true>(in, first);
    load_words<W, true>(in + P, second);
  }
  f32x4 ct[PPL / 4], st[PPL / 4];
  if constexpr (TABLE) {
    const float* crow = a.cos_table + position * a.table_stride + base;
    const float* srow = a.sin_table + position * a.table_stride + base;
#pragma unroll
    for (int i = 0; i < PPL / 4; ++i) ct[i] = *reinterpret_cast<const f32x4*>(crow + 4 * i);
#pragma unroll
    for (int i = 0; i < PPL / 4; ++i) st[i] = *reinterpret_cast<const f32x4*>(srow + 4 * i);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!live) {
#pragma unroll
    for (int i = 0; i < W; ++i) first[i] = second[i] = 0u;
  }

  float c[PPL], s[PPL];
  if constexpr (TABLE) {
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      c[j] = ct[j / 4][j % 4];
      s[j] = st[j / 4][j % 4];
    }
  } else {
    // Lane i derives pairs i and i + 64; lanes then fetch the pairs they rotate.
    float cl = 0.0f, sl = 0.0f, ch = 0.0f, sh = 0.0f;
    if (lane < P) derived_angle(lane, P, position, a.log2_base, cl, sl);
    if (P > kWave && lane + kWave < P) derived_angle(lane + kWave, P, position, a.log2_base, ch, sh);
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const int pair = base + j;
      const float lo_c = __shfl(cl, pair % kWave, kWave);
      const float lo_s = __shfl(sl, pair % kWave, kWave);
      if constexpr (P > kWave) {
        const float hi_c = __shfl(ch, pair % kWave, kWave);
        const float hi_s = __shfl(sh, pair % kWave, kWave);
        c[j] = pair < kWave ? lo_c : hi_c;
        s[j] = pair < kWave ? lo_s : hi_s;
      } else {
        c[j] = lo_c;
        s[j] = lo_s;
      }
    }
  }
  float w1[PPL], w2[PPL], x1[PPL], x2[PPL];
#pragma unroll
  for (int i = 0; i < W; ++i) {
    w1[2 * i] = bf16_lo(wraw1[i]); w1[2 * i + 1] = bf16_hi(wraw1[i]);
    w2[2 * i] = bf16_lo(wraw2[i]); w2[2 * i + 1] = bf16_hi(wraw2[i]);
    x1[2 * i] = bf16_lo(first[i]); x1[2 * i + 1] = bf16_hi(first[i]);
    x2[2 * i] = bf16_lo(second[i]); x2[2 * i + 1] = bf16_hi(second[i]);
  }
  // x * x is exact in fp64 (and in fp32), so one fma per element gives the same sum as
  // the square rounded to fp32 and added in fp64, in two instructions instead of three.
  double sumsq = 0.0;
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const double d1 = static_cast<double>(x1[j]);
    const double d2 = static_cast<double>(x2[j]);
    sumsq = __builtin_fma(d1, d1, sumsq);
    sumsq = __builtin_fma(d2, d2, sumsq);
  }
  sumsq = dpp_group_sum<G>(sumsq);
  const float inv = 1.0f / sqrtf(static_cast<float>(sumsq) / static_cast<float>(D) + a.eps);

  // n = bf16(w * bf16(x * inv)); with mscale != 1, the rotary inputs are
  // bf16(n * bf16(mscale)).
  float n1[PPL], n2[PPL];
#pragma unroll
  for (int j = 0; j < PPL; j += 2) {
    float a0 = x1[j] * inv, a1 = x1[j + 1] * inv;
    float b0 = x2[j] * inv, b1 = x2[j + 1] * inv;
    round_pair(a0, a1);
    round_pair(b0, b1);
    n1[j] = w1[j] * a0;
    n1[j + 1] = w1[j + 1] * a1;
    n2[j] = w2[j] * b0;
    n2[j + 1] = w2[j + 1] * b1;
    round_pair(n1[j], n1[j + 1]);
    round_pair(n2[j], n2[j + 1]);
  }
  if constexpr (SCALED) {
    const float mscale = round_bf16(a.mscale);
#pragma unroll
    for (int j = 0; j < PPL; j += 2) {
      n1[j] *= mscale; n1[j + 1] *= mscale;
      n2[j] *= mscale; n2[j + 1] *= mscale;
      round_pair(n1[j], n1[j + 1]);
      round_pair(n2[j], n2[j + 1]);
    }
  }
  // out_p = bf16(x1 * cos - x2 * sin), out_{p+P} = bf16(x1 * sin + x2 * cos).
  uint32_t o1[W], o2[W];
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const int j = 2 * i;
    o1[i] = pack_bf16(n1[j] * c[j] - n2[j] * s[j], n1[j + 1] * c[j + 1] - n2[j + 1] * s[j + 1]);
    o2[i] = pack_bf16(n1[j] * s[j] + n2[j] * c[j], n1[j + 1] * s[j + 1] + n2[j + 1] * c[j + 1]);
  }
  if (live && token_live) {
    uint16_t* out = (is_query ? a.queries_out : a.keys_out) + (head * length + t) * D + base;
    store_words<W>(out, o1);
    store_words<W>(out + P, o2);
  }
}

template <int D, int PPL, bool TABLE, bool SCALED, bool EXACT>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void qk_norm_rope_pairs_kernel(RopeArgs a) {
  pairs_body<D, PPL, TABLE, SCALED, EXACT, false>(a, a.queries_in, a.keys_in, a.length, a.query_stride,
                                                  a.key_stride, a.q_parts, a.query_heads, a.kv_heads);
}

// The decode step's form (four pairs per lane): the arguments the input loads need come
// first, as scalars (copies of RopeArgs fields), which gfx950 preloads into SGPRs at wave
// launch, so the inputs' loads go out with no scalar round trip ahead of them: 2.43 ->
// 2.34 us at the decode step. At eight pairs per lane the same form measured slower: the
// prefill headline 16.34 -> 16.41 us and the derived-angle epilogue 17.0 -> 18.6 us.
template <int D, int PPL, bool TABLE, bool SCALED, bool EXACT>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void qk_norm_rope_pairs_lead_kernel(
    const uint16_t* queries_in, const uint16_t* keys_in, int64_t length, int64_t query_stride,
    int64_t key_stride, int q_parts, int query_heads, int kv_heads, RopeArgs a) {
  pairs_body<D, PPL, TABLE, SCALED, EXACT, true>(a, queries_in, keys_in, length, query_stride, key_stride,
                                                 q_parts, query_heads, kv_heads);
}

template <int D, int PPL, bool TABLE, bool SCALED>
void launch_pairs(const RopeArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  constexpr int kHeadsPerSlot = kWave * PPL / (D / 2);
  const bool exact = a.query_heads % kHeadsPerSlot == 0 && a.kv_heads % kHeadsPerSlot == 0;
  if constexpr (PPL == 4) {
#define OMNIA_LEAD_ARGS \
  a.queries_in, a.keys_in, a.length, a.query_stride, a.key_stride, a.q_parts, a.query_heads, a.kv_heads, a
    if (exact) qk_norm_rope_pairs_lead_kernel<D, PPL, TABLE, SCALED, true><<<grid, block, 0, stream>>>(OMNIA_LEAD_ARGS);
    else qk_norm_rope_pairs_lead_kernel<D, PPL, TABLE, SCALED, false><<<grid, block, 0, stream>>>(OMNIA_LEAD_ARGS);
#undef OMNIA_LEAD_ARGS
  } else if (exact) {
    qk_norm_rope_pairs_kernel<D, PPL, TABLE, SCALED, true><<<grid, block, 0, stream>>>(a);
  } else {
    qk_norm_rope_pairs_kernel<D, PPL, TABLE, SCALED, false><<<grid, block, 0, stream>>>(a);
  }
}

template <int D, int SPW, bool TABLE, bool FULL, bool SCALED>
void launch_exact(const RopeArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  constexpr int kHeadsPerSlot = kWave / (D / 8);
  if (a.query_heads % kHeadsPerSlot == 0 && a.kv_heads % kHeadsPerSlot == 0) {
    qk_norm_rope_kernel<D, SPW, TABLE, FULL, SCALED, true><<<grid, block, 0, stream>>>(a);
  } else {
    qk_norm_rope_kernel<D, SPW, TABLE, FULL, SCALED, false><<<grid, block, 0, stream>>>(a);
  }
}

template <int D, int SPW, bool TABLE>
void launch_variant(const RopeArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  const bool full = 2 * a.pairs == D;
  const bool scaled = a.mscale != 1.0f;
  if (!TABLE || (full && !scaled)) {
    launch_exact<D, SPW, TABLE, true, false>(a, grid, block, stream);
  } else if (full) {
    launch_exact<D, SPW, TABLE, true, true>(a, grid, block, stream);
  } else if (!scaled) {
    launch_exact<D, SPW, TABLE, false, false>(a, grid, block, stream);
  } else {
    launch_exact<D, SPW, TABLE, false, true>(a, grid, block, stream);
  }
}

template <int D, bool TABLE>
void launch_spw(const RopeArgs& a, int spw, dim3 grid, dim3 block, hipStream_t stream) {
  switch (spw) {
    case 1: launch_variant<D, 1, TABLE>(a, grid, block, stream); break;
    case 2: launch_variant<D, 2, TABLE>(a, grid, block, stream); break;
    default: launch_variant<D, 4, TABLE>(a, grid, block, stream); break;
  }
}

// Slots per wave: measured on MI355X at the prefill shape (q [4096,32,128], k
// [4096,8,128]), two slots per wave beat one (more per-wave overhead) and four or
// eight (fewer waves in flight during ramp and tail); short segments drop to one so the
// grid still covers the chip.
int slots_per_wave(int64_t length, int q_slots, int k_slots) {
  int spw = 2;
  constexpr int64_t kTargetWaves = 8192;
  if (length * ((q_slots + 1) / 2 + (k_slots + 1) / 2) < kTargetWaves) spw = 1;
  return spw;
}

// `spw` <= 0 picks the slots per wave; the sweep harness passes 1, 2 or 4 explicitly.
template <bool TABLE>
int32_t launch(RopeArgs a, int head_dim, hipStream_t stream, const char* name, int spw = 0) {
  if (2 * a.pairs == head_dim) {  // full rotary: the pair-owning layout, one slot per wave
    // Eight pairs per lane; four where a grid of eight would leave the chip mostly idle
    // (fewer than kNarrowWaves waves: the decode rows), so that each wave's serial chain
    // is half as long and twice as many waves share the work. D = 256 keeps eight (a
    // head of 32 lanes would need a cross-row sum).
    const int wide_slot = kWave / (head_dim / 16);
    const int64_t wide_waves = a.length * ((a.query_heads + wide_slot - 1) / wide_slot +
                                           (a.kv_heads + wide_slot - 1) / wide_slot);
    const bool narrow = head_dim <= 128 && wide_waves < kNarrowWaves;
    const int heads_per_slot = narrow ? wide_slot / 2 : wide_slot;  // heads of 2G lanes
    a.q_parts = (a.query_heads + heads_per_slot - 1) / heads_per_slot;
    a.k_parts = (a.kv_heads + heads_per_slot - 1) / heads_per_slot;
    // With a table, every workgroup holds four tokens of one slot (the kernel's mapping),
    // grid (token groups, slots); without, the 1-D grid of units, fewer than 2^32.
    const int64_t groups = (a.length + kWavesPerBlock - 1) / kWavesPerBlock;
    const int64_t waves = a.length * (a.q_parts + a.k_parts);
    const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
    OMNIA_REQUIRE(groups < (int64_t{1} << 31) && blocks < (int64_t{1} << 30),
                  std::string(name) + ": too many tokens x heads");
    const dim3 grid = TABLE ? dim3(static_cast<unsigned>(groups), static_cast<unsigned>(a.q_parts + a.k_parts))
                            : dim3(static_cast<unsigned>(blocks));
    const dim3 block(kWavesPerBlock * kWave);
    const bool scaled = TABLE && a.mscale != 1.0f;
#define OMNIA_PAIRS(D, PPL)                                                   \
  (scaled ? launch_pairs<D, PPL, TABLE, true>(a, grid, block, stream)         \
          : launch_pairs<D, PPL, TABLE, false>(a, grid, block, stream))
    switch (head_dim) {
      case 64: narrow ? OMNIA_PAIRS(64, 4) : OMNIA_PAIRS(64, 8); break;
      case 128: narrow ? OMNIA_PAIRS(128, 4) : OMNIA_PAIRS(128, 8); break;
      case 256: OMNIA_PAIRS(256, 8); break;
      default: return fail(-EINVAL, std::string(name) + ": head_dim must be 64, 128 or 256");
    }
#undef OMNIA_PAIRS
    return launched(name);
  }
  const int heads_per_slot = kWave / (head_dim / 8);
  const int q_slots = (a.query_heads + heads_per_slot - 1) / heads_per_slot;
  const int k_slots = (a.kv_heads + heads_per_slot - 1) / heads_per_slot;
  if (spw <= 0) spw = slots_per_wave(a.length, q_slots, k_slots);
  spw = spw >= 4 ? 4 : spw;
  a.q_parts = (q_slots + spw - 1) / spw;
  a.k_parts = (k_slots + spw - 1) / spw;
  const int64_t waves = a.length * (a.q_parts + a.k_parts);
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  OMNIA_REQUIRE(blocks < (int64_t{1} << 30), std::string(name) + ": too many tokens x heads");
  const dim3 grid(static_cast<unsigned>(blocks));
  const dim3 block(kWavesPerBlock * kWave);
  switch (head_dim) {
    case 64: launch_spw<64, TABLE>(a, spw, grid, block, stream); break;
    case 128: launch_spw<128, TABLE>(a, spw, grid, block, stream); break;
    case 256: launch_spw<256, TABLE>(a, spw, grid, block, stream); break;
    default: return fail(-EINVAL, std::string(name) + ": head_dim must be 64, 128 or 256");
  }
  return launched(name);
}

bool power_of_two(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int32_t check_common(const char* name, int64_t length, int64_t query_heads, int64_t kv_heads,
                     int64_t head_dim, int64_t pairs, int64_t query_stride,
                     int64_t key_stride) {
  const std::string n(name);
  OMNIA_REQUIRE(length >= 0 && length < (int64_t{1} << 31), n + ": bad length");
  OMNIA_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
                n + ": head_dim must be 64, 128 or 256");
  OMNIA_REQUIRE(query_heads > 0 && kv_heads > 0 && query_heads + kv_heads <= 4096,
                n + ": bad head counts");
  OMNIA_REQUIRE(pairs >= 8 && pairs % 8 == 0 && power_of_two(pairs / 8) && 2 * pairs <= head_dim,
                n + ": rotary_pairs must be 8 * 2^k with 2 * rotary_pairs <= head_dim");
  OMNIA_REQUIRE(query_stride >= query_heads * head_dim && query_stride % 8 == 0,
                n + ": query row stride too small or not a multiple of 8");
  OMNIA_REQUIRE(key_stride >= kv_heads * head_dim && key_stride % 8 == 0,
                n + ": key row stride too small or not a multiple of 8");
  return 0;
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_qk_norm_rope(
    const uint16_t* raw_queries, int64_t query_stride, const uint16_t* raw_keys,
    int64_t key_stride, const uint16_t* query_weight, const uint16_t* key_weight,
    const float* cos_table, const float* sin_table, int64_t table_stride,
    int64_t table_rows, int64_t offset, uint16_t* queries, uint16_t* keys, int64_t length,
    int64_t query_heads, int64_t kv_heads, int64_t head_dim, int64_t rotary_pairs,
    float eps, float mscale, hipStream_t stream) {
  using namespace omnia;
  int32_t rc = check_common("qk_norm_rope", length, query_heads, kv_heads, head_dim,
                            rotary_pairs, query_stride, key_stride);
  if (rc != 0) return rc;
  OMNIA_REQUIRE(table_stride >= rotary_pairs && table_stride % 4 == 0,
                "qk_norm_rope: table stride must be >= rotary_pairs and a multiple of 4");
  OMNIA_REQUIRE(offset >= 0 && offset + length <= table_rows,
                "qk_norm_rope: rows offset .. offset + length must lie inside the table");
  if (length == 0) return 0;
  OMNIA_REQUIRE(raw_queries && raw_keys && query_weight && key_weight && cos_table &&
                    sin_table && queries && keys,
                "qk_norm_rope: null pointer");
  OMNIA_REQUIRE(aligned16(raw_queries) && aligned16(raw_keys) && aligned16(query_weight) &&
                    aligned16(key_weight) && aligned16(cos_table) && aligned16(sin_table) &&
                    aligned16(queries) && aligned16(keys),
                "qk_norm_rope: pointers must be 16-byte aligned");
  rc = check_device(stream);
  if (rc != 0) return rc;
  RopeArgs a{raw_queries, raw_keys, query_weight, key_weight, cos_table, sin_table,
             queries, keys, length, query_stride, key_stride, table_stride, offset,
             static_cast<int>(query_heads), static_cast<int>(kv_heads),
             static_cast<int>(rotary_pairs), 1, 1, eps, mscale, 0.0f};
  return launch<true>(a, static_cast<int>(head_dim), stream, "qk_norm_rope");
}

extern "C" int32_t omnia_rope_epilogue(const uint16_t* fused, int64_t fused_stride,
                                       const uint16_t* query_weight,
                                       const uint16_t* key_weight, int64_t offset,
                                       uint16_t* queries, uint16_t* keys, int64_t length,
                                       int64_t query_heads, int64_t kv_heads,
                                       int64_t head_dim, float log2_base, float eps,
                                       hipStream_t stream) {
  using namespace omnia;
  int32_t rc = check_common("rope_epilogue", length, query_heads, kv_heads, head_dim,
                            head_dim / 2, fused_stride, fused_stride);
  if (rc != 0) return rc;
  OMNIA_REQUIRE(fused_stride >= (query_heads + 2 * kv_heads) * head_dim,
                "rope_epilogue: fused row narrower than q + k + v");
  OMNIA_REQUIRE(offset >= 0 && offset + length <= (int64_t{1} << 24),
                "rope_epilogue: positions must stay below 2^24 (exact in fp32)");
  if (length == 0) return 0;
  OMNIA_REQUIRE(fused && query_weight && key_weight && queries && keys,
                "rope_epilogue: null pointer");
  OMNIA_REQUIRE(aligned16(fused) && aligned16(query_weight) && aligned16(key_weight) &&
                    aligned16(queries) && aligned16(keys),
                "rope_epilogue: pointers must be 16-byte aligned");
  rc = check_device(stream);
  if (rc != 0) return rc;
  RopeArgs a{fused, fused + query_heads * head_dim, query_weight, key_weight, nullptr,
             nullptr, queries, keys, length, fused_stride, fused_stride, 0, offset,
             static_cast<int>(query_heads), static_cast<int>(kv_heads),
             static_cast<int>(head_dim / 2), 1, 1, eps, 1.0f, log2_base};
  return launch<false>(a, static_cast<int>(head_dim), stream, "rope_epilogue");
}
