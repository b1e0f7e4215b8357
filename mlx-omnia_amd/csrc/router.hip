// MoE routing: softmax -> top-k -> renormalise, and the fused residual join + router.
//
// Selection (core/kernels/route/default.py:44-69 and models/qwen3/layers/moe.py:34-42,
// with the lowest-index tie rule of core/kernels/route/ordinal.py:1-27): the k experts
// with the largest bf16 logits, in descending order, an exact tie going to the lower
// expert index. Softmax is monotone, so this is the order of the softmax
// probabilities. Weights: p = softmax(logits) in fp32, renormalised over the kept
// experts, w_j = p_j / sum_i p_i. The full softmax denominator cancels in that ratio,
// so the kernels evaluate w_j = exp(l_j - l_1) / sum_i exp(l_i - l_1) over the k kept
// logits (l_1 the largest), the same quantity to within fp32 rounding.
//
// Keys: each logit becomes a 32-bit key, an order-preserving map of its bf16 bits
// (sign flip for positives, all bits for negatives, -0 folded onto +0, NaN below
// everything, so a NaN logit ranks last as core/kernels/route/ordinal.py:37-47 ranks a
// NaN score) in the high half and 0xFFFF - expert in the low half. Unsigned key order
// is then descending logit with the lower index first on ties; k rounds of a wave-wide
// max extract the winners.
//
// Sigmoid routing with a correction bias (core/kernels/route/ordinal.py:200-286,
// `router_tournament`): score = sigmoid(x) of the float32 logit, correctly rounded (the
// stable form y = 1 / (1 + exp|x|), x < 0 ? y : 1 - y, in fp64, rounded once); key =
// ordinal(-(score + bias)) with the sum in fp32 and `ordinal` the map of ordinal.py:
// 37-47 (ascending unsigned order = ascending float order, +-0 one value, NaN above
// everything). The k smallest keys win, lower expert first on equal keys; the weights
// are the winners' unbiased scores over their fp32 sum taken in winner order. The fused
// router's sigmoid form (core/kernels/route/residual.py:109-115) emits the exact bf16
// logits and these keys, and optionally the selection.
//
// Fused kernel (core/kernels/route/residual.py:117-299 is the one-token precedent;
// config: x, residual [4096, 2048], router [128, 2048], k = 8): a workgroup of 16
// waves owns 16 tokens.
//   1. residual add + RMSNorm, one row per wave (arithmetic of add_rms_norm.hip),
//      writing summed and normalized, keeping the bf16 normalized tile [16, H] in LDS
//      and the Euclidean norm of each normalized row;
//   2. logits[16, E] = tile x W^T on v_mfma_f32_16x16x32_bf16, each wave owning one
//      16-expert tile over a slice of H (E = 128: two halves). W is read in the packed
//      layout omnia_pack_router_weight writes: the 16 x 32 B-operand block of one MFMA
//      is 1 KiB in lane order, so each load instruction of a wave reads 1 KiB of
//      contiguous memory (eight whole cache lines) and a wave's walk over its slice is
//      one contiguous stream. Each MFMA sums its 32 products with a zero accumulator;
//      the step results are added with ordinary fp32 adds, and the slices' partials
//      meet in LDS;
//   3. per token: the bf16 rounding of each logit, made exact. With A = ||n|| ||W_e||
//      (Cauchy-Schwarz: A >= sum |n_k W_ek|), the fp32 logit L is within
//      delta = (62 + chain + slices - 1) * 2^-24 * A (+1% and a tiny absolute floor for
//      subnormal flushes) of the exact dot product: each MFMA's internal sum of 32
//      products carries at most 31 roundings, each counted at a full ulp, and each fp32
//      add on an element's path (the chain: in-order adds inside a group of step
//      results, then a tree over the groups) and of a slice partial one half-ulp
//      rounding. When [L - delta, L + delta] rounds to
//      one bf16 value, that value is the correctly rounded logit; otherwise the logit is
//      recomputed as an fp64 dot product from the LDS tile and W (the products of two
//      bf16 values are exact in fp32) and rounded once. Recomputed are the unsure
//      logits whose upper bound could reach the top k (all of them when the logits or
//      the keys are written out), so the selection, the weights and any emitted logit
//      equal those of the correctly rounded logits. Then the selection and the weights
//      above. In the sigmoid form the bounds go through bounds of the sigmoid (below)
//      to bounds of each ordinal key, which is monotone in the logit.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {


constexpr int kTileTokens = 16;   // MFMA M
constexpr int kWaves = 16;        // one row per wave in phases 1 and 3
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxTopK = 64;

__device__ __forceinline__ uint32_t order16(uint32_t bits) {
  if ((bits & 0x7FFFu) > 0x7F80u) return 0u;       // NaN below everything (-inf is 0x7F)
  if (bits == 0x8000u) bits = 0u;                  // -0 == +0
  return (bits & 0x8000u) ? (~bits & 0xFFFFu) : (bits | 0x8000u);
}

__device__ __forceinline__ uint32_t unorder16(uint32_t ordinal) {
  return (ordinal & 0x8000u) ? (ordinal & 0x7FFFu) : (~ordinal & 0xFFFFu);
}

__device__ __forceinline__ uint32_t route_key(uint32_t logit_bits, int expert) {
  return (order16(logit_bits) << 16) | (0xFFFFu - static_cast<uint32_t>(expert));
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Maximum over the wave, left in every lane: DPP steps inside each 16-lane row (quad
// swaps, half-row and row mirrors), then the two cross-row swaps. Everything stays in
// vector registers; no LDS and no scalar round trip on the dependency chain.
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
  v = umax(v, dpp<kQuadSwap1>(v));
  v = umax(v, dpp<kQuadSwap2>(v));
  v = umax(v, dpp<kRowHalfMirror>(v));
  v = umax(v, dpp<kRowMirror>(v));
  uint32_t a, b;
  row_pair(v, a, b);
  v = umax(a, b);
  half_pair(v, a, b);
  return umax(a, b);
}

// Sum over the wave, the same in every lane (each step adds the same two operands on
// both lanes of a pair, so every lane computes the identical fp32 result).
__device__ __forceinline__ float wave_sum(float v) {
  v += __uint_as_float(dpp<kQuadSwap1>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kQuadSwap2>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowMirror>(__float_as_uint(v)));
  uint32_t a, b;
  row_pair(__float_as_uint(v), a, b);
  v = __uint_as_float(a) + __uint_as_float(b);
  half_pair(__float_as_uint(v), a, b);
  return __uint_as_float(a) + __uint_as_float(b);
}

// Extracts the top k of the wave's keys (V per lane; keys are distinct, 0 is below every
// real key). Each lane first sorts its keys (descending); a round then takes the wave
// maximum of the lanes' first keys, and the lane holding it shifts its keys up. Lane
// j < k ends with the j-th winner; returns the k-th (uniform). `keys` is consumed.
template <int V>
__device__ __forceinline__ uint32_t select_topk(uint32_t (&keys)[V], int k, int lane,
                                                uint32_t& chosen) {
#pragma unroll
  for (int i = 0; i < V; ++i) {  // insertion sort of V <= 4 keys
#pragma unroll
    for (int j = V - 1; j > i; --j) {
      const uint32_t hi = umax(keys[j - 1], keys[j]);
      const uint32_t lo = keys[j - 1] ^ keys[j] ^ hi;
      keys[j - 1] = hi;
      keys[j] = lo;
    }
  }
  chosen = 0;
  uint32_t best = 0;
  for (int j = 0; j < k; ++j) {
    best = wave_max(keys[0]);
    const bool take = keys[0] == best;
#pragma unroll
    for (int v = 0; v + 1 < V; ++v) keys[v] = take ? keys[v + 1] : keys[v];
    keys[V - 1] = take ? 0u : keys[V - 1];
    chosen = lane == j ? best : chosen;
  }
  return best;
}

__device__ __forceinline__ float key_logit(uint32_t key) {
  return bf16_to_f32(static_cast<uint16_t>(unorder16(key >> 16)));
}

// Writes the winners' indices and renormalised softmax weights from lanes 0..k-1.
__device__ __forceinline__ void write_winners(uint32_t chosen, int k, int lane,
                                              int32_t* indices, float* weights) {
  const float top = key_logit(static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(chosen), 0)));
  const float e = lane < k ? expf(key_logit(chosen) - top) : 0.0f;
  const float total = wave_sum(e);
  if (lane < k) {
    indices[lane] = static_cast<int32_t>(0xFFFFu - (chosen & 0xFFFFu));
    weights[lane] = e / total;
  }
}

// The final top k of a row whose selection on bounds was refined, ranked among its
// contenders only: the experts whose upper-bound key reaches `threshold` (the k-th
// best lower-bound key). Every expert of the exact top k is one of them, since its
// exact key is at least the k-th exact key, which is at least the threshold. There are
// about k contenders; they are packed into the first lanes through `slots` (64 words of
// LDS owned by this wave), each counts the contenders with a larger exact key (keys
// are distinct), and the winners land in rank order: lane j < k holds the j-th
// winner's key, as select_topk leaves it. Returns false (nothing written) when the
// contenders do not fit one wave.
template <int V>
__device__ __forceinline__ bool rank_contenders(const uint32_t (&exact)[V], const uint32_t (&upper)[V],
                                                uint32_t threshold, int k, int lane, uint32_t* slots,
                                                uint32_t& chosen) {
  uint64_t mask[V];
  int count = 0;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    mask[v] = __ballot(upper[v] >= threshold);
    count += __popcll(mask[v]);
  }
  if (count > kWave || count < k) return false;   // uniform
  int base = 0;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if (upper[v] >= threshold) {
      const int at = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                static_cast<uint32_t>(mask[v] >> 32),
                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask[v]), 0)));
      slots[at] = exact[v];
    }
    base += __popcll(mask[v]);
  }
  __builtin_amdgcn_wave_barrier();
  const uint32_t key = lane < count ? slots[lane] : 0u;
  int rank = 0;
  for (int j = 0; j < count; ++j) {   // uniform
    rank += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), j)) > key ? 1 : 0;
  }
  __builtin_amdgcn_wave_barrier();
  if (lane < count && rank < k) slots[rank] = key;
  __builtin_amdgcn_wave_barrier();
  chosen = lane < k ? slots[lane] : 0u;
  return true;
}

// ---- sigmoid scores, ordinal keys and their selection ---------------------------------

// Correctly rounded fp32 sigmoid of an fp32 value.
__device__ __forceinline__ float sigmoid_rounded(float x) {
  const double y = 1.0 / (1.0 + exp(fabs(static_cast<double>(x))));
  return static_cast<float>(x < 0.0f ? y : 1.0 - y);
}

// lo <= sigmoid_rounded(x) <= hi from the hardware's single-precision 2^y (v_exp_f32) and
// 1/y (v_rcp_f32), each within a few ulps; x * log2(e) rounded to fp32 moves exp(-x) by
// at most |x| 2^-24 of itself. All of it stays below (|x| + 6) 2^-24 of the value, and the
// slack taken is (1 + |x|) 2^-16 of it plus 2^-100 (where exp(-x) overflows, the true
// value is below 2^-127). For the selection on bounds only: a wider interval costs
// recomputations, never a different result.
__device__ __forceinline__ void sigmoid_bounds(float x, float& lo, float& hi) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
  const float s = __builtin_amdgcn_rcpf(1.0f + e);
  const float slack = s * (0x1p-16f * (1.0f + fabsf(x))) + 0x1p-100f;
  lo = fmaxf(s - slack, 0.0f);   // a NaN slack (s = 0 at x = -inf) leaves [0, 1]
  hi = fminf(s + slack, 1.0f);
}

// ordinal.py:37-47 `router_key_ordinal`.
__device__ __forceinline__ uint32_t ordinal_of(float key) {
  const uint32_t bits = __float_as_uint(key);
  const uint32_t magnitude = bits & 0x7FFFFFFFu;
  if (magnitude > 0x7F800000u) return 0xFFFFFFFFu;
  if (magnitude == 0u) return 0x80000000u;
  return (bits & 0x80000000u) ? ~bits : (bits ^ 0x80000000u);
}

// The k smallest ordinal keys of one wave's row (V per lane: expert lane + 64 v; lanes
// past `experts` hold nothing), lower expert first on equal keys; writes the experts and
// the winners' scores over their fp32 sum in winner order. Each round takes the lanes'
// best (largest ~key, then largest 0xFFFF - expert) in two wave maxima and reads the
// winner's score from the lane that holds it.
template <int V>
__device__ __forceinline__ void ordinal_topk_write(const uint32_t (&keys)[V], const float (&scores)[V],
                                                   int experts, int k, int lane,
                                                   int32_t* indices, float* weights) {
  uint32_t hi[V], lo[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int e = lane + v * kWave;
    hi[v] = e < experts ? ~keys[v] : 0u;   // a NaN key (0xFFFFFFFF) still beats a
    lo[v] = e < experts ? 0xFFFFu - static_cast<uint32_t>(e) : 0u;  // padded slot
  }
  float total = 0.0f, mine = 0.0f;
  int my_expert = 0;
  for (int j = 0; j < k; ++j) {
    uint32_t bh = 0u, bl = 0u;
    float bs = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const bool better = hi[v] > bh || (hi[v] == bh && lo[v] > bl);
      bh = better ? hi[v] : bh;
      bl = better ? lo[v] : bl;
      bs = better ? scores[v] : bs;
    }
    const uint32_t top_hi = wave_max(bh);
    const uint32_t top_lo = wave_max(bh == top_hi ? bl : 0u);
    const int expert = __builtin_amdgcn_readfirstlane(static_cast<int>(0xFFFFu - top_lo));
    const int owner = expert % kWave;
    const float score = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bs), owner));
    total = score + total;
    if (lane == owner) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if (lane + v * kWave == expert) {
          hi[v] = 0u;
          lo[v] = 0u;
        }
      }
    }
    if (lane == j) {
      my_expert = expert;
      mine = score;
    }
  }
  if (lane < k) {
    indices[lane] = my_expert;
    weights[lane] = mine / total;
  }
}

// The sigmoid form's tail for row `row`, from its exact bf16 logits (V per lane, expert
// lane + 64 v; `experts` of them): scores, ordinal keys (written to keys[row] when keys
// is given) and the selection (to indices[row] and weights[row], when indices is given).
// The row addresses are formed where they are stored, so no pointer stays live.
template <int V>
__device__ __forceinline__ void sigmoid_finish(const uint32_t (&bits)[V], const float (&bias)[V],
                                               int experts, int k, int lane, uint32_t* keys,
                                               int32_t* indices, float* weights, int64_t row) {
  uint32_t key_of[V];
  float scores[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    scores[v] = sigmoid_rounded(bf16_to_f32(static_cast<uint16_t>(bits[v])));
    key_of[v] = ordinal_of(-(scores[v] + bias[v]));
    if (keys && lane + v * kWave < experts) keys[row * experts + lane + v * kWave] = key_of[v];
  }
  if (indices) ordinal_topk_write<V>(key_of, scores, experts, k, lane, indices + row * k, weights + row * k);
}

// The sigmoid form's last step when it only selects. The contenders are the experts whose
// best-case key reaches the threshold of the bounds: every winner is one, and by now each
// has its exact logit. They are packed into the first lanes through `slots` (64 words of
// this wave's own). Each lane takes one contender's exact score and key and ranks it among
// the others, (key, expert) ascending. The first k write their expert and their score over
// the winners' fp32 sum, taken in winner order, as ordinal_topk_write does. Too many
// contenders (keys tied everywhere, NaN keys) or too few go to sigmoid_finish.
template <int V>
__device__ __forceinline__ void sigmoid_select_contenders(const uint32_t (&bits)[V], const uint32_t (&upper)[V],
                                                          uint32_t threshold, const float (&bias)[V],
                                                          int experts, int k, int lane,
                                                          int32_t* indices, float* weights, int64_t row,
                                                          uint32_t* slots, const float* bias_table) {
  uint64_t mask[V];
  int count = 0;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    mask[v] = __ballot(upper[v] >= threshold);
    count += __popcll(mask[v]);
  }
  if (count > kWave || count < k) {   // uniform
    sigmoid_finish<V>(bits, bias, experts, k, lane, nullptr, indices, weights, row);
    return;
  }
  int base = 0;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if (upper[v] >= threshold) {
      const int at = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                static_cast<uint32_t>(mask[v] >> 32),
                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask[v]), 0)));
      slots[at] = (static_cast<uint32_t>(lane + v * kWave) << 16) | (bits[v] & 0xFFFFu);
    }
    base += __popcll(mask[v]);
  }
  __builtin_amdgcn_wave_barrier();
  uint32_t key = 0xFFFFFFFFu;
  int expert = 0xFFFF;
  float score = 0.0f;
  if (lane < count) {
    const uint32_t slot = slots[lane];
    expert = static_cast<int>(slot >> 16);
    score = sigmoid_rounded(bf16_to_f32(static_cast<uint16_t>(slot & 0xFFFFu)));
    key = ordinal_of(-(score + bias_table[expert]));
  }
  int rank = 0;
  for (int j = 0; j < count; ++j) {   // uniform
    const uint32_t other = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), j));
    const int other_expert = __builtin_amdgcn_readlane(expert, j);
    rank += (other < key || (other == key && other_expert < expert)) ? 1 : 0;
  }
  const bool winner = lane < count && rank < k;
  float total = 0.0f;
  for (int r = 0; r < k; ++r) {   // uniform
    const uint64_t who = __ballot(winner && rank == r);
    const int owner = static_cast<int>(__builtin_ctzll(who));
    total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(score), owner)) + total;
  }
  if (winner) {
    indices[row * k + rank] = expert;
    weights[row * k + rank] = score / total;
  }
}

// ---- sigmoid + bias -> ordinal keys -> top-k over given logits: one wave per row ----

template <int V, bool kF32>
__global__ __launch_bounds__(256) void sigmoid_topk_kernel(const void* __restrict__ logits,
                                                           int64_t stride,
                                                           const float* __restrict__ bias,
                                                           int64_t rows, int experts, int k,
                                                           uint32_t* __restrict__ keys_out,
                                                           int32_t* __restrict__ indices,
                                                           float* __restrict__ weights) {
  __shared__ uint32_t slots[4][kWave];  // the contenders of each wave's row
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (row >= rows) return;
  // Every load first, from a clamped index and with no branch (a load in a branch is
  // waited on there, one round trip per value); lanes past the experts then drop theirs.
  float x[V], b[V];
  uint32_t raw[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int e = min(lane + v * kWave, experts - 1);
    if constexpr (kF32) {
      x[v] = static_cast<const float*>(logits)[row * stride + e];
    } else {
      raw[v] = static_cast<const uint16_t*>(logits)[row * stride + e];
      x[v] = bf16_to_f32(static_cast<uint16_t>(raw[v]));
    }
    b[v] = bias[e];
  }
  // `weights` (past the 14 preloaded argument dwords) taken now, while the loads are in
  // flight: the compiler otherwise loaded it at the store, a scalar round trip at the end.
  asm volatile("" ::"s"(weights));
  if constexpr (!kF32) {
    if (!keys_out && indices && experts == V * kWave) {  // uniform
      // Selection only, every lane an expert: select on the hardware sigmoid's bounds,
      // then rank the contenders (about k) on their exact scores, as the fused router's
      // sigmoid form does. The k-th best worst-case key is the threshold; every expert
      // of the exact top k has its best-case key at or above it.
      uint32_t worst[V], best[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        float lo, hi;
        sigmoid_bounds(x[v], lo, hi);
        worst[v] = ~ordinal_of(-(lo + b[v]));   // inverted: larger is better
        best[v] = ~ordinal_of(-(hi + b[v]));
      }
      uint32_t chosen = 0;
      const uint32_t threshold = select_topk<V>(worst, k, lane, chosen);
      sigmoid_select_contenders<V>(raw, best, threshold, b, experts, k, lane, indices, weights, row,
                                   slots[threadIdx.x / kWave], bias);
      return;
    }
  }
  uint32_t keys[V];
  float scores[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int e = lane + v * kWave;
    const float score = sigmoid_rounded(x[v]);
    const uint32_t key = ordinal_of(-(score + b[v]));
    keys[v] = e < experts ? key : 0xFFFFFFFFu;
    scores[v] = e < experts ? score : 0.0f;
    if (keys_out && e < experts) keys_out[row * experts + e] = key;
  }
  if (indices) ordinal_topk_write<V>(keys, scores, experts, k, lane, indices + row * k, weights + row * k);
}

// Writes the winners' indices and their softmax probabilities over the whole row (no
// renormalisation over the kept experts): p_j = exp(l_j - l_1) / sum_e exp(l_e - l_1),
// l_1 the largest logit, the denominator summed over every expert of the row.
template <int V>
__device__ __forceinline__ void write_winners_unnormalised(uint32_t chosen, const uint16_t (&raw)[V],
                                                           int experts, int k, int lane,
                                                           int32_t* indices, float* weights) {
  const float top = key_logit(static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(chosen), 0)));
  float part = 0.0f;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const float e = expf(bf16_to_f32(raw[v]) - top);
    part += lane + v * kWave < experts ? e : 0.0f;
  }
  const float total = wave_sum(part);
  if (lane < k) {
    indices[lane] = static_cast<int32_t>(0xFFFFu - (chosen & 0xFFFFu));
    weights[lane] = expf(key_logit(chosen) - top) / total;
  }
}

// ---- softmax -> top-k over given bf16 logits: one wave per row --------------------
//
// kNormalize: the kept probabilities renormalised over themselves (write_winners), or
// the probabilities themselves (write_winners_unnormalised). kShared: the row holds one
// more logit after the routed ones, the shared expert's; slot k gets index `experts`
// and weight sigmoid(logit), correctly rounded to fp32. The output row is k + kShared
// slots long. The shared slots of a workgroup's four rows are computed by one of its
// waves, four lanes at once (the wave rotates with the workgroup, so that the waves
// carrying them spread over the SIMDs): the fp64 sigmoid is one instruction stream
// however many lanes run it, and one per row had cost every wave that stream.
template <int V, bool kNormalize, bool kShared>
__global__ __launch_bounds__(256) void softmax_topk_kernel(const uint16_t* __restrict__ logits,
                                                           int64_t stride, int64_t rows,
                                                           int experts, int k,
                                                           int32_t* __restrict__ indices,
                                                           float* __restrict__ weights) {
  const int lane = threadIdx.x % kWave;
  const int wave = static_cast<int>(threadIdx.x / kWave);
  const int64_t first_row = static_cast<int64_t>(blockIdx.x) * 4;
  const int64_t row = first_row + wave;
  const int slots = k + (kShared ? 1 : 0);
  const bool owner = kShared && wave == static_cast<int>(blockIdx.x % 4);   // wave-uniform
  // Every load first, from clamped indices and with no branch (a load in a branch makes
  // the compiler wait on it at once): the row's logits (lanes past the experts then drop
  // theirs; a row past the last reads the last) and the shared logits of the workgroup's
  // rows, lane j < 4 holding row first_row + j's.
  const int64_t load_row = min(row, rows - 1);
  uint16_t raw[V];
#pragma unroll
  for (int v = 0; v < V; ++v) raw[v] = logits[load_row * stride + min(lane + v * kWave, experts - 1)];
  const int64_t shared_row = min(first_row + min(lane, 3), rows - 1);
  const uint16_t shared_raw = kShared ? logits[shared_row * stride + experts] : uint16_t{0};
  // The owner's sigmoids now, before any store of the wave is in flight (a wait behind a
  // store would wait for the store too).
  float shared_weight = 0.0f;
  if (owner) shared_weight = sigmoid_rounded(bf16_to_f32(shared_raw));
  if (row < rows) {   // wave-uniform; the owner of a short last workgroup still writes
    uint32_t keys[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e = lane + v * kWave;
      const uint32_t key = route_key(raw[v], e);
      keys[v] = e < experts ? key : 0u;
    }
    uint32_t chosen;
    select_topk<V>(keys, k, lane, chosen);
    if (kNormalize) {
      write_winners(chosen, k, lane, indices + row * slots, weights + row * slots);
    } else {
      write_winners_unnormalised<V>(chosen, raw, experts, k, lane, indices + row * slots,
                                    weights + row * slots);
    }
  }
  if (owner && lane < 4 && first_row + lane < rows) {
    indices[shared_row * slots + k] = experts;
    weights[shared_row * slots + k] = shared_weight;
  }
}

// ---- packed router weight --------------------------------------------------------
//
// Layout written by omnia_pack_router_weight for W [E, H] bf16 (E a multiple of 16, H of
// 32): blocks of 16 experts x 32 k of 1 KiB each; block (tile, step) starts at element
// (tile * H / 32 + step) * 512 and holds, at l * 8 + j, W[tile * 16 + l % 16]
// [step * 32 + (l / 16) * 8 + j] for l < 64, j < 8: lane l's B operand of
// v_mfma_f32_16x16x32_bf16. After the E * H values: E fp32 row norms ||W_e||_2, each
// rounded up (an upper bound of the exact norm); then W again, row-major, for the
// exact recomputation of single logits (a row is 4 KiB of contiguous memory there,
// where the operand blocks would scatter it over 256 cache lines).

__host__ __device__ constexpr int64_t packed_weight_elements(int64_t experts, int64_t hidden) {
  return experts * hidden;
}
// Element offset of the row-major copy: after the blocks and the norms (2 bf16 slots
// per fp32 norm).
__host__ __device__ constexpr int64_t packed_rows_offset(int64_t experts, int64_t hidden) {
  return experts * hidden + 2 * experts;
}
__host__ __device__ constexpr int64_t packed_bytes(int64_t experts, int64_t hidden) {
  return (packed_rows_offset(experts, hidden) + experts * hidden) * 2;
}

// The next fp32 value above a finite non-negative x (x itself if x is +inf).
__device__ __forceinline__ float bump_up(float x) {
  return x < __builtin_inff() ? __uint_as_float(__float_as_uint(x) + 1u) : x;
}

// Upper bound, in fp32, of sqrt(sum), sum >= 0 given in fp64.
__device__ __forceinline__ float norm_upper(double sum) {
  return bump_up(static_cast<float>(sqrt(sum) * (1.0 + 0x1p-40)));
}

constexpr int kPackBlock = 256;

// Blocks [0, chunk_blocks) move one 16-byte chunk per thread; the rest compute one row
// norm per wave.
__global__ __launch_bounds__(kPackBlock) void pack_router_kernel(const u32x4* __restrict__ w,
                                                                 u32x4* __restrict__ packed,
                                                                 float* __restrict__ norms,
                                                                 u32x4* __restrict__ rows,
                                                                 int experts, int hidden,
                                                                 int chunk_blocks) {
  const int chunks = experts * hidden / 8;
  if (static_cast<int>(blockIdx.x) < chunk_blocks) {
    const int o = blockIdx.x * kPackBlock + threadIdx.x;
    if (o >= chunks) return;
    const int block = o / 64, l = o % 64;
    const int tile = block / (hidden / 32), step = block % (hidden / 32);
    const int64_t src = (static_cast<int64_t>(tile * 16 + l % 16) * hidden + step * 32 + (l / 16) * 8) / 8;
    packed[o] = w[src];
    rows[o] = w[o];
    return;
  }
  const int lane = threadIdx.x % kWave;
  const int e = (blockIdx.x - chunk_blocks) * (kPackBlock / kWave) + threadIdx.x / kWave;
  if (e >= experts) return;  // whole wave
  double sum = 0.0;
  for (int c = lane; c < hidden / 8; c += kWave) {
    float v[8];
    unpack8(w[static_cast<int64_t>(e) * (hidden / 8) + c], v);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double d = v[j];  // squared in fp64: no overflow for any finite bf16
      sum = __builtin_fma(d, d, sum);
    }
  }
  sum = wave_sum_f64(sum);
  if (lane == 0) norms[e] = norm_upper(sum);
}

// ---- fused residual add + RMSNorm + router projection + top-k ---------------------

// Correctly rounded bf16 bits of two logits sum_k n_k * W_ek at once, by one wave, from
// normalized rows in LDS and experts' rows of W (the second pair may repeat the first):
// the products of two bf16 values are exact in fp32 and are summed in fp64. Both rows'
// loads are in flight together.
template <int VPL>
__device__ __forceinline__ void exact_logits(const uint16_t* n_row0, const uint16_t* n_row1,
                                             const uint16_t* w_row0, const uint16_t* w_row1,
                                             int lane, uint32_t& bits0, uint32_t& bits1) {
  u32x4 w0[VPL], w1[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int h0 = (lane + i * kWave) * 8;
    w0[i] = *reinterpret_cast<const u32x4*>(w_row0 + h0);
    w1[i] = *reinterpret_cast<const u32x4*>(w_row1 + h0);
  }
  double acc0 = 0.0, acc1 = 0.0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int h0 = (lane + i * kWave) * 8;
    float n0[8], n1[8], a[8], b[8];
    unpack8(*reinterpret_cast<const u32x4*>(n_row0 + h0), n0);
    unpack8(*reinterpret_cast<const u32x4*>(n_row1 + h0), n1);
    unpack8(w0[i], a);
    unpack8(w1[i], b);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc0 += static_cast<double>(n0[j] * a[j]);
      acc1 += static_cast<double>(n1[j] * b[j]);
    }
  }
  bits0 = f64_to_bf16(wave_sum_f64(acc0));
  bits1 = f64_to_bf16(wave_sum_f64(acc1));
}

// The exact logits of tasks[lo, hi) (each task r * E + e: token r of the tile, expert e),
// by one wave, when every unsure logit is wanted (logits or keys written). The tasks of a
// token are contiguous in the list, so the wave holds the current token's normalized row
// in fp64 registers and widens it again only when the token changes; each expert's row of
// W is loaded one task ahead, so the next load overlaps this sum. Each logit is summed
// in the order exact_logits sums it (per lane over the row's 16-byte pieces, then the
// wave: fma(n, w, acc) adds the exact product n * w as acc + n * w does), so the bits are
// the same; lane 0 writes them to exact_bits[task].
template <int VPL, int E>
__device__ __forceinline__ void exact_task_run(const uint16_t* tile, int row_pitch,
                                               const uint16_t* weight_rows, const uint16_t* tasks,
                                               int lo, int hi, int lane, uint32_t* exact_bits) {
  constexpr int H = 512 * VPL;
  if (lo >= hi) return;  // wave-uniform
  double nd[VPL][8];
  int row = -1;
  int task = __builtin_amdgcn_readfirstlane(static_cast<int>(tasks[lo]));
  u32x4 cur[VPL], next[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    cur[i] = *reinterpret_cast<const u32x4*>(weight_rows + static_cast<int64_t>(task % E) * H +
                                             (lane + i * kWave) * 8);
  }
  for (int c = lo; c < hi; ++c) {   // uniform
    // The next task's row of W, or this one's again after the last (in bounds, unused).
    const int following = __builtin_amdgcn_readfirstlane(static_cast<int>(tasks[c + 1 < hi ? c + 1 : c]));
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      next[i] = *reinterpret_cast<const u32x4*>(weight_rows + static_cast<int64_t>(following % E) * H +
                                                (lane + i * kWave) * 8);
    }
    const int r = task / E;
    if (r != row) {  // uniform: the token changed
      row = r;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float n[8];
        unpack8(*reinterpret_cast<const u32x4*>(tile + r * row_pitch + (lane + i * kWave) * 8), n);
#pragma unroll
        for (int j = 0; j < 8; ++j) nd[i][j] = static_cast<double>(n[j]);
      }
    }
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float w[8];
      unpack8(cur[i], w);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = __builtin_fma(nd[i][j], static_cast<double>(w[j]), acc);
    }
    const uint32_t exact = f64_to_bf16(wave_sum_f64(acc));
    if (lane == 0) exact_bits[task] = exact;
#pragma unroll
    for (int i = 0; i < VPL; ++i) cur[i] = next[i];
    task = following;
  }
}

struct RouterArgs {
  const u32x4* x;
  const u32x4* branch;
  const u32x4* norm_weight;
  const uint16_t* packed;         // W in operand blocks
  const float* weight_norms;      // ||W_e||, rounded up
  const uint16_t* weight_rows;    // W row-major
  u32x4* summed;
  u32x4* normalized;
  uint16_t* logits;               // [T, E] bf16, optional
  int32_t* indices;               // [T, k]; optional in the sigmoid form
  float* weights;                 // [T, k]
  const float* bias;              // [E] fp32: the sigmoid form; null: softmax
  uint32_t* keys;                 // [T, E] ordinal keys (sigmoid form), optional
  int64_t rows;
  int k;
  float eps;
#ifdef OMNIA_PHASE_CLOCKS
  uint64_t* clocks;               // [workgroups, 16 waves, kClockSlots] or null
#endif
};

// Phase clocks: a diagnostic build (-DOMNIA_PHASE_CLOCKS, libomnia_router_clocks.so)
// records the 100 MHz wall clock (s_memrealtime) at the phase boundaries of the H = 2048
// kernel, one vector store per wave from lane 0, into a buffer set with
// omnia_router_phase_clocks_set. The product library compiles the marks to nothing.
constexpr int kClockSlots = 10;
#ifdef OMNIA_PHASE_CLOCKS
#define OMNIA_CLOCK(args, wave, lane, slot)                                                   \
  do {                                                                                        \
    if ((lane) == 0 && (args).clocks != nullptr)                                              \
      (args).clocks[(static_cast<int64_t>(blockIdx.x) * kWaves + (wave)) * kClockSlots + (slot)] = \
          static_cast<uint64_t>(wall_clock64());                                              \
  } while (0)
#else
#define OMNIA_CLOCK(args, wave, lane, slot) \
  do {                                      \
  } while (0)
#endif

template <int VPL, int E>
struct FusedShape {
  static constexpr int H = 512 * VPL;
  static constexpr int kTiles = E / 16;             // 16-expert MFMA tiles
  static constexpr int kSlices = kWaves / kTiles;   // waves sharing one tile, over H
  static constexpr int kSlice = H / kSlices;
  static constexpr int kSteps = kSlice / 32;        // MFMAs per wave
  static constexpr int kRowPitch = H + 8;           // bf16; the pad staggers LDS banks
  // LDS: the normalized tile, the logits [16][E] (reused for the recomputed bits), the
  // row norms, the task count (padded to 16 bytes) and the task list [16 * E] of uint16.
  static constexpr size_t kLds = static_cast<size_t>(kTileTokens) * kRowPitch * 2 +
                                 static_cast<size_t>(kTileTokens) * E * 4 + kTileTokens * 4 +
                                 16 + static_cast<size_t>(kTileTokens) * E * 2;
  // |L - exact| <= kDelta * A + kFloor (see the file comment): 31 full-ulp roundings
  // inside each MFMA (62 half-ulps), one half-ulp per step add and per slice add; 1%
  // covers the rounding of A, delta and L +- delta. The floor covers products that
  // leave the fp32 normal range.
  // The walk adds each block of kUnroll step results in order (kUnroll - 1 adds), the
  // kOuter block sums in a binary tree (log2 kOuter levels), then the slices.
  static constexpr int kUnroll = 8;
  static constexpr int kOuter = kSlice / (32 * kUnroll);
  static constexpr int kLevels = kOuter == 16 ? 4 : kOuter == 8 ? 3 : kOuter == 4 ? 2 : 1;
  static constexpr float kDelta = (62.0f + (kUnroll - 1) + kLevels + kSlices - 1) * 1.01f / 16777216.0f;
  static_assert(kOuter == (1 << kLevels), "a power-of-two number of step blocks");
  static_assert(H <= 8192, "the absolute floor assumes H <= 2^13");
  static_assert(E % 16 == 0 && kWaves % kTiles == 0 && kSlice % 256 == 0, "shape");
};
// Absolute part of the bound, per unit of ||n|| + ||W_e|| + 1: an MFMA that flushed
// subnormal bf16 inputs or fp32 products would lose at most H * 2^-126 times those.
constexpr float kDeltaFloor = 0x1p-113f;


template <int VPL, int E>
__global__ __launch_bounds__(kThreads) void residual_rms_router_kernel(RouterArgs a) {
  using S = FusedShape<VPL, E>;
  constexpr int H = S::H, kTiles = S::kTiles, kSlices = S::kSlices, kSlice = S::kSlice;
  constexpr int kRowPitch = S::kRowPitch;
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* tile = reinterpret_cast<uint16_t*>(smem);
  float* logit_tile = reinterpret_cast<float*>(smem + kTileTokens * kRowPitch * 2);  // [token][expert]
  float* row_norm = logit_tile + kTileTokens * E;                                      // ||n_t||, rounded up
  int* task_count = reinterpret_cast<int*>(row_norm + kTileTokens);
  uint16_t* tasks = reinterpret_cast<uint16_t*>(task_count + 4);                      // token * E + expert
  if (threadIdx.x == 0) *task_count = 0;  // ordered before phase 3 by the barriers below

  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kTileTokens;
  constexpr int V = E / kWave;  // experts per lane in phase 3
  float weight_norm[V];         // loaded now, used in phase 3
#pragma unroll
  for (int v = 0; v < V; ++v) weight_norm[v] = a.weight_norms[lane + v * kWave];
  float bias[V];                // the sigmoid form's correction bias, loaded with them
#pragma unroll
  for (int v = 0; v < V; ++v) bias[v] = a.bias ? a.bias[lane + v * kWave] : 0.0f;

  // The walk of phase 2 over W: wave w owns expert tile w % kTiles over slice w / kTiles
  // of H, in kOuter blocks of kUnroll steps. Each workgroup starts at a different block,
  // so the workgroups of an XCD do not all read the same W lines at once (the order of
  // the step adds changes per workgroup; the error bound does not).
  constexpr int kUnroll = S::kUnroll;
  constexpr int kOuter = S::kOuter;
  const int start = static_cast<int>(blockIdx.x % kOuter);
  const uint16_t* brow =
      a.packed + (static_cast<int64_t>(wave % kTiles) * (H / 32) + (wave / kTiles) * (kSlice / 32)) * 512 +
      lane * 8;
  u32x4 next[kUnroll];
  // At H = 2048 the first block's loads go out now, ahead of phase 1, whose row loads
  // take the HBM stream: the 8 KiB per wave arrive while the CU's L1 is otherwise idle
  // (23.0 us against 24.4 us at [4096, 2048], E = 128). At H = 4096 the rows leave no
  // registers for them.
  constexpr bool kEarlyWalk = VPL <= 4;
  if constexpr (kEarlyWalk) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      next[u] = *reinterpret_cast<const u32x4*>(brow + (start * kUnroll + u) * 512);
    }
  }

  // Phase 1: residual add + RMSNorm of row `wave`.
  {
    const int r = wave;
    const int64_t t = first + r;
    // Every load before any arithmetic and none in a branch: a row past the last reads
    // the last row (in bounds) and is zeroed.
    const int64_t tl = t < a.rows ? t : a.rows - 1;
    u32x4 xv[VPL], bv[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      xv[i] = load_nt(a.x + tl * (H / 8) + lane + i * kWave);
      bv[i] = load_nt(a.branch + tl * (H / 8) + lane + i * kWave);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (t >= a.rows) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) xv[i] = bv[i] = u32x4{0u, 0u, 0u, 0u};
    }
    // s = bf16(x + b) is formed twice (for the sum of squares, then for the outputs)
    // rather than kept: at H = 4096 the rows alone fill half the register budget.
    double sumsq = 0.0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float xf[8], bf[8];
      unpack8(xv[i], xf);
      unpack8(bv[i], bf);
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        float lo = xf[j] + bf[j], hi = xf[j + 1] + bf[j + 1];
        round_pair(lo, hi);
        sumsq += static_cast<double>(lo * lo);
        sumsq += static_cast<double>(hi * hi);
      }
    }
    sumsq = wave_sum_f64(sumsq);
    const float inv = 1.0f / sqrtf(static_cast<float>(sumsq) / static_cast<float>(H) + a.eps);
    double nsq = 0.0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float xf[8], bf[8], w[8], s[8], n[8];
      unpack8(xv[i], xf);
      unpack8(bv[i], bf);
      unpack8(a.norm_weight[lane + i * kWave], w);  // L2-resident, shared by every row
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        s[j] = xf[j] + bf[j];
        s[j + 1] = xf[j + 1] + bf[j + 1];
        round_pair(s[j], s[j + 1]);
        float lo = s[j] * inv, hi = s[j + 1] * inv;
        round_pair(lo, hi);
        n[j] = w[j] * lo;
        n[j + 1] = w[j + 1] * hi;
        round_pair(n[j], n[j + 1]);
        const double n0 = n[j], n1 = n[j + 1];  // squared in fp64: no overflow
        nsq = __builtin_fma(n0, n0, nsq);
        nsq = __builtin_fma(n1, n1, nsq);
      }
      const u32x4 packed = pack8(n);
      const int v = lane + i * kWave;
      *reinterpret_cast<u32x4*>(tile + r * kRowPitch + v * 8) =
          t < a.rows ? packed : u32x4{0u, 0u, 0u, 0u};
      if (t < a.rows) {
        store_nt(a.summed + t * (H / 8) + v, pack8(s));
        store_nt(a.normalized + t * (H / 8) + v, packed);
      }
    }
    nsq = wave_sum_f64(nsq);
    if (lane == 0) row_norm[r] = t < a.rows ? norm_upper(nsq) : 0.0f;
  }
  __syncthreads();

  // Phase 2: logits = tile x W^T. Lane l feeds row (token) l % 16 of A and column
  // (expert) l % 16 of B, both over k = (l / 16) * 8 .. + 8 of each 32-wide step.
  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  {
    const f32x4 zero = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int slice = wave / kTiles;
    const uint16_t* arow = tile + (lane % 16) * kRowPitch + slice * kSlice + (lane / 16) * 8;
    if constexpr (!kEarlyWalk) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        next[u] = *reinterpret_cast<const u32x4*>(brow + (start * kUnroll + u) * 512);
      }
    }
    // Each block's kUnroll step results are added in order into its group sum (the first
    // is a copy), and the kOuter group sums meet in a binary tree: level j holds the
    // pending sum of 2^j groups until its partner arrives.
    f32x4 level[S::kLevels];
    for (int step = 0; step < kOuter; ++step) {
      const int s0 = (start + step) % kOuter;
      const int s1 = (start + step + 1) % kOuter;
      u32x4 b[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        b[u] = next[u];
        if (step + 1 < kOuter) {
          next[u] = *reinterpret_cast<const u32x4*>(brow + (s1 * kUnroll + u) * 512);
        }
      }
      f32x4 group;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const u32x4 av = *reinterpret_cast<const u32x4*>(arow + (s0 * kUnroll + u) * 32);
        const f32x4 part = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, b[u]), zero, 0, 0, 0);
        if (u == 0) {
          group = part;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) group[j] = group[j] + part[j];
        }
      }
      // Carry the group into the tree, as a binary counter on `step`.
#pragma unroll
      for (int lv = 0; lv < S::kLevels; ++lv) {
        if ((step >> lv) & 1) {
#pragma unroll
          for (int j = 0; j < 4; ++j) group[j] = level[lv][j] + group[j];
        } else {
          level[lv] = group;
          break;
        }
      }
      if (step == kOuter - 1) acc = group;   // every level paired: the whole slice
    }
  }
  // D layout: lane l holds column (expert) l % 16, rows (tokens) (l / 16) * 4 + i. The
  // slices add their partials in turn.
  {
    const int e = (wave % kTiles) * 16 + lane % 16;
    const int slice = wave / kTiles;
#pragma unroll 1
    for (int turn = 0; turn < kSlices; ++turn) {
      if (slice == turn) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int at = ((lane / 16) * 4 + i) * E + e;
          logit_tile[at] = turn == 0 ? acc[i] : logit_tile[at] + acc[i];
        }
      }
      __syncthreads();
    }
  }

  // Phase 3: exact bf16 logits where they decide anything, then the selection; one
  // token per wave. The logits that need an exact recomputation are pooled over the
  // workgroup and shared out among all its waves, so the workgroup waits for about one
  // recomputation whichever token needs them.
  const int r = wave;
  const int64_t t = first + r;
  const bool active = t < a.rows;  // wave-uniform; inactive waves still meet the barriers
  const bool emit = a.logits != nullptr;
  const bool sigmoid = a.bias != nullptr;
  // Every logit exact (no selection on the bounds) when logits or keys are written out.
  const bool exact_all = emit || (sigmoid && a.keys != nullptr);
  const float n_norm = row_norm[r];
  uint32_t bits[V], upper[V], keys[V];
  bool unsure[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int e = lane + v * kWave;
    const float logit = logit_tile[r * E + e];
    const float w_norm = weight_norm[v];
    const float delta = S::kDelta * (n_norm * w_norm) + kDeltaFloor * (n_norm + w_norm + 1.0f);
    const uint32_t lo = f32_to_bf16(logit - delta);
    const uint32_t hi = f32_to_bf16(logit + delta);
    bits[v] = lo;
    unsure[v] = lo != hi;
    if (sigmoid) {
      // The ordinal key falls as the logit rises: the worst key comes from the lower
      // bound, the best from the upper. Inverted, so that select_topk's largest are the
      // best (ties take one round together, which only lowers the threshold).
      float worst, best, unused;
      sigmoid_bounds(bf16_to_f32(static_cast<uint16_t>(lo)), worst, unused);
      sigmoid_bounds(bf16_to_f32(static_cast<uint16_t>(hi)), unused, best);
      keys[v] = ~ordinal_of(-(worst + bias[v]));
      upper[v] = ~ordinal_of(-(best + bias[v]));
    } else {
      keys[v] = route_key(lo, e);
      upper[v] = route_key(hi, e);
    }
  }
  // Select on the lower bounds. A certain logit's lower bound is its value; an unsure
  // logit whose upper bound stays below the k-th selected key cannot be selected. If
  // every selected logit is certain and no unsure one can reach the k-th, this
  // selection is final.
  uint32_t chosen = 0;
  uint32_t threshold = 0xFFFFFFFFu;
  if (active && !exact_all) threshold = select_topk<V>(keys, a.k, lane, chosen);
  bool need[V];
  bool refined = false;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    need[v] = active && unsure[v] && (exact_all || upper[v] >= threshold);
    const uint64_t mask = __ballot(need[v]);
    if (mask != 0) {  // wave-uniform
      refined = true;
      int base = 0;
      if (lane == 0) base = atomicAdd(task_count, __popcll(mask));
      base = __builtin_amdgcn_readfirstlane(base);
      const int below = __builtin_amdgcn_mbcnt_hi(
          static_cast<uint32_t>(mask >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
      if (need[v]) tasks[base + below] = static_cast<uint16_t>(r * E + lane + v * kWave);
    }
  }
  __syncthreads();
  // The recomputations, two per wave per pass; results overwrite the logits in LDS,
  // which are no longer read.
  uint32_t* exact_bits = reinterpret_cast<uint32_t*>(logit_tile);
  const int count = *task_count;
  for (int i = 2 * wave; i < count; i += 2 * kWaves) {  // wave-uniform
    const int task0 = tasks[i];
    const int task1 = i + 1 < count ? tasks[i + 1] : task0;
    uint32_t exact0, exact1;
    exact_logits<VPL>(tile + (task0 / E) * kRowPitch, tile + (task1 / E) * kRowPitch,
                      a.weight_rows + static_cast<int64_t>(task0 % E) * H,
                      a.weight_rows + static_cast<int64_t>(task1 % E) * H, lane, exact0, exact1);
    if (lane == 0) {
      exact_bits[task0] = exact0;
      exact_bits[task1] = exact1;
    }
  }
  __syncthreads();
  if (!active) return;  // no barrier follows
  if (refined) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (need[v]) bits[v] = exact_bits[r * E + lane + v * kWave];
    }
  }
  if (emit) {
#pragma unroll
    for (int v = 0; v < V; ++v) a.logits[t * E + lane + v * kWave] = static_cast<uint16_t>(bits[v]);
  }
  if (sigmoid) {   // the contenders' ranking (split kernel) would spill registers here
    sigmoid_finish<V>(bits, bias, E, a.k, lane, a.keys, a.indices, a.weights, t);
    return;
  }
  if (refined || exact_all) {
#pragma unroll
    for (int v = 0; v < V; ++v) keys[v] = route_key(bits[v], lane + v * kWave);
    select_topk<V>(keys, a.k, lane, chosen);   // ranking the contenders spills here
  }
  write_winners(chosen, a.k, lane, a.indices + t * a.k, a.weights + t * a.k);
}

template <int VPL, int E>
int32_t launch_fused(const RouterArgs& a, hipStream_t stream) {
  constexpr size_t lds = FusedShape<VPL, E>::kLds;
  // The attribute belongs to the kernel on the current device; set it on each call
  // (a cheap host-side call) rather than caching per process.
  const hipError_t status = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&residual_rms_router_kernel<VPL, E>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (status != hipSuccess) {
    return fail(-1, std::string("residual_rms_router: LDS attribute: ") + hipGetErrorString(status));
  }
  const dim3 grid(static_cast<unsigned>((a.rows + kTileTokens - 1) / kTileTokens));
  residual_rms_router_kernel<VPL, E><<<grid, kThreads, lds, stream>>>(a);
  return launched("residual_rms_router");
}

// ---- H = 2048: the same arithmetic with the phases overlapped by wave roles --------
//
// Every CU holds one 16-token workgroup at the config (4096 tokens, 256 CUs), so the
// phases cannot overlap across workgroups; here they overlap inside one. Waves
// [0, kRowWaves) are row waves: phase 1 for two token rows each. Waves [kRowWaves, 16)
// are walkers: at launch they load the first kRing blocks of their share of W (from L2)
// into registers, while the rows stream from HBM, then run the MFMA walk.
// Where the summed and normalized rows are stored decides where HBM's time goes. In
// the selection-only form at E = 128 (kDeferStores) the row waves keep both rows in LDS
// and store them only once the walk is done: the launch's reads then have HBM to
// themselves (the last tile completes about 4.5 us sooner), the walk has the CU's path
// to L2 to itself (stores issued during the walk slowed it from 3.8 to 7.4 us), and the
// writes drain during phase 3. Issuing 16 KB of stores takes a wave a while once HBM
// backs up, so the row waves then leave, and the walkers run phase 3 for two tokens
// each: its barriers count only the waves still running. Otherwise (every logit exact,
// or E = 256, where the second tile does not fit in LDS) the row waves store each row
// as soon as it is formed. A store counts in the issuing wave's vmcnt until it
// completes, so only walkers, which store nothing before the end, load anything after
// phase 1: the walk and the exact recomputations.
// The barriers below are lds_barrier() (common.hpp): __syncthreads() would make every
// wave wait for the row waves' stores; nothing here reads global memory another wave of
// the workgroup wrote.

template <int E>
struct SplitShape {
  static constexpr int VPL = 4;
  static constexpr int H = 512 * VPL;
  static constexpr int kRowWaves = 8;                        // two rows each in phase 1
  static constexpr int kWalkers = kWaves - kRowWaves;
  static constexpr int kTiles = E / 16;                      // 16-expert MFMA tiles
  static constexpr int kSlices = 2;                          // halves of H
  static constexpr int kSlice = H / kSlices;
  static constexpr int kSteps = kSlice / 32;                 // MFMA steps per (tile, slice)
  static constexpr int kTilesPerWalker = kTiles * kSlices / kWalkers;
  static constexpr int kBlocks = kTilesPerWalker * kSteps;   // B blocks one walker streams
  static constexpr int kRing = E <= 128 ? 18 : 8;           // blocks in flight per walker
  static constexpr int kRowPitch = H + 8;
  // LDS: the normalized tile, one fp32 logit tile per slice [16][E] (the first reused
  // for the recomputed bits), the row norms, the task count (padded to 16 bytes) and
  // the task list [16 * E] of uint16.
  static constexpr size_t kTileBytes = static_cast<size_t>(kTileTokens) * kRowPitch * 2;
  static constexpr size_t kLogitBytes = static_cast<size_t>(kTileTokens) * E * 4;
  // The selection-only form at E = 128 also keeps the summed rows, to store them after
  // the walk (the tile's pitch).
  static constexpr bool kDeferStores = E == 128;
  static constexpr size_t kLdsCore = kTileBytes + kSlices * kLogitBytes + kTileTokens * 4 + 16 +
                                     static_cast<size_t>(kTileTokens) * E * 2 + E * 4;
  static constexpr size_t kLds = kLdsCore + (kDeferStores ? kTileBytes : 0);
  // Each 32-wide step is one v_mfma_f32_16x16x32_bf16 with a zero accumulator, summing
  // 32 exact products with at most 31 roundings, counted at a full ulp (62 half-ulps of
  // a partial bounded by the step's Cauchy-Schwarz product; those sum to at most A).
  // With two tiles per walker the kSteps step results of a (tile, slice) are summed in
  // groups of kGroup, each in order (kGroup - 1 roundings: the first is a copy), and
  // the four group sums in a tree of depth 2 (at four tiles per walker the tree's
  // registers would spill, and the steps are summed in order: kSteps - 1 roundings);
  // then the two slices. Each fp32 add on an element's path carries one half-ulp
  // rounding of a partial sum bounded by A; 1% covers the rounding of A, delta and
  // L +- delta. One MFMA per step rather than two 16x16x16 halves (30 half-ulps each
  // at the half's own bound) doubles the internal term but halves the fp32 adds, which
  // the walk's VALU time is made of.
  static constexpr int kGroup = 8;
  static constexpr bool kTree = kTilesPerWalker <= 2;
  static constexpr int kChain = kTree ? (kGroup - 1) + 2 : kSteps - 1;
  static constexpr float kDelta = (62.0f + kChain + (kSlices - 1)) * 1.01f / 16777216.0f;
  // When every logit is made exact (logits or keys written), each step is four
  // v_mfma_f32_16x16x16bf16_1k quarters: each takes one 32-bit word (two k's) of every
  // lane's operands and zeros in place of the other two, so it sums eight real products
  // (an exact zero adds no rounding: 7 roundings, 14 half-ulps of the quarter's own
  // bound), and the quarters join in a tree of two fp32 adds: 16 half-ulps of the
  // step's bound where one 16x16x32 MFMA counts 62. At E = 128 the bound drops from 72
  // to 26 half-ulps, and with it the share of unsure logits, which that form recomputes
  // in fp64; the extra MFMAs and adds cost the walk far less.
  static constexpr float kDeltaQuarters = (14.0f + 2.0f + kChain + (kSlices - 1)) * 1.01f / 16777216.0f;
  static_assert(kSteps == 4 * kGroup, "four groups of steps per (tile, slice)");
  static_assert(kTiles * kSlices % kWalkers == 0 && kWalkers % kSlices == 0, "shape");
  static_assert(kTileTokens == 2 * kRowWaves, "two rows per row wave");
  static_assert(kTileTokens * E * 2 >= kWaves * kWave * 4, "64 contender slots per wave in the task list");
};

// Phase 1 of one token row, for a row wave: residual add + RMSNorm (the arithmetic of
// add_rms_norm.hip), the outputs stored, the bf16 normalized row and an upper bound of
// its norm kept. The sum of squares is fp64 (four independent chains; the squares of
// bf16 values are exact, and the fp64 sum rounds to the fp32 of the exact sum, which
// is what the arithmetic defines). The norm of the normalized row only bounds the
// logits' error, so it is summed in fp32 from the products w * bf16(s * inv) before
// their bf16 rounding and inflated: a rounding to bf16 moves a value by at most 2^-9 of
// itself, and the 8 FMAs of a chain, the 2 adds joining the chains and the 6 of the wave
// sum round at most 16 times, so the sum times (1 + 2^-7) bounds the squared norm.
template <int VPL>
__device__ __forceinline__ void router_row(const u32x4 (&xv)[VPL], const u32x4 (&bv)[VPL],
                                           const u32x4 (&wv)[VPL], bool live, int64_t t,
                                           float eps, int lane, const RouterArgs& a,
                                           uint16_t* tile_row, float* norm_slot, bool store,
                                           u32x4 (&sv)[VPL]) {
  constexpr int H = 512 * VPL;
  // sv: s = bf16(x + b), packed as stored (kept for the caller when `store` is false)
  double part[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    float xf[8], bf[8];
    unpack8(xv[i], xf);
    unpack8(bv[i], bf);
    uint32_t words[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      words[j / 2] = pack_bf16(xf[j] + bf[j], xf[j + 1] + bf[j + 1]);
      const double lo = bf16_lo(words[j / 2]), hi = bf16_hi(words[j / 2]);
      part[j / 2] = __builtin_fma(lo, lo, part[j / 2]);
      part[j / 2] = __builtin_fma(hi, hi, part[j / 2]);
    }
    sv[i] = u32x4{words[0], words[1], words[2], words[3]};
  }
  const double sumsq = wave_sum_f64((part[0] + part[1]) + (part[2] + part[3]));
  const float inv = 1.0f / sqrtf(static_cast<float>(sumsq) / static_cast<float>(H) + eps);
  float nparts[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    float s[8], w[8], n[8];
    unpack8(sv[i], s);
    unpack8(wv[i], w);
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      float lo = s[j] * inv, hi = s[j + 1] * inv;
      round_pair(lo, hi);
      n[j] = w[j] * lo;
      n[j + 1] = w[j + 1] * hi;
      nparts[j / 2] = __builtin_fmaf(n[j], n[j], nparts[j / 2]);
      nparts[j / 2] = __builtin_fmaf(n[j + 1], n[j + 1], nparts[j / 2]);
    }
    const u32x4 packed = pack8(n);
    const int v = lane + i * kWave;
    *reinterpret_cast<u32x4*>(tile_row + v * 8) = live ? packed : u32x4{0u, 0u, 0u, 0u};
    if (live && store) {
      store_nt(a.summed + t * (H / 8) + v, sv[i]);
      store_nt(a.normalized + t * (H / 8) + v, packed);
    }
  }
  const float nsq = wave_sum((nparts[0] + nparts[1]) + (nparts[2] + nparts[3]));
  if (lane == 0) *norm_slot = live ? norm_upper(static_cast<double>(nsq) * (1.0 + 0x1p-7)) : 0.0f;
}

template <int VPL>
__device__ __forceinline__ void router_row(const u32x4 (&xv)[VPL], const u32x4 (&bv)[VPL],
                                           const u32x4 (&wv)[VPL], bool live, int64_t t,
                                           float eps, int lane, const RouterArgs& a,
                                           uint16_t* tile_row, float* norm_slot, bool store = true) {
  u32x4 sv[VPL];
  router_row<VPL>(xv, bv, wv, live, t, eps, lane, a, tile_row, norm_slot, store, sv);
}

// kExactAll: the logits or the keys are written, so every logit is made exact (the launch
// picks the instantiation; the selection-only one keeps its registers to itself).
template <int E, bool kExactAll>
__global__ __launch_bounds__(kThreads) void residual_rms_router_split_kernel(RouterArgs a) {
  using S = SplitShape<E>;
  constexpr int VPL = S::VPL, H = S::H, kRowPitch = S::kRowPitch;
  constexpr int kTPW = S::kTilesPerWalker, kSteps = S::kSteps, kBlocks = S::kBlocks;
  constexpr int kRing = S::kRing;
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* tile = reinterpret_cast<uint16_t*>(smem);
  float* logit_tile = reinterpret_cast<float*>(smem + S::kTileBytes);            // slice 0
  float* logit_tile1 = reinterpret_cast<float*>(smem + S::kTileBytes + S::kLogitBytes);
  float* row_norm = reinterpret_cast<float*>(smem + S::kTileBytes + S::kSlices * S::kLogitBytes);
  int* task_count = reinterpret_cast<int*>(row_norm + kTileTokens);
  uint16_t* tasks = reinterpret_cast<uint16_t*>(task_count + 4);
  float* bias_lds = reinterpret_cast<float*>(tasks + kTileTokens * E);   // the sigmoid form's bias
  uint16_t* summed_tile = reinterpret_cast<uint16_t*>(smem + S::kLdsCore);  // deferred form only
  constexpr bool kDefer = S::kDeferStores && !kExactAll;
  if (threadIdx.x == 0) *task_count = 0;  // ordered before phase 3 by the barriers below

  // The wave index through readfirstlane: the compiler then knows the role branches are
  // uniform and keeps the walkers' ring and the row waves' rows in the same registers.
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int lane = threadIdx.x % kWave;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kTileTokens;
  const bool walker = wave >= S::kRowWaves;

  // Walker geometry: slice of H, first tile, and the block stream (step-major, the
  // walker's tiles inside a step). Each workgroup starts its steps at a different
  // offset, so the workgroups of an XCD do not read the same W lines at once (the order
  // of the step adds changes per workgroup; the error bound does not).
  const int wk = wave - S::kRowWaves;
  const int slice = wk / (S::kWalkers / S::kSlices);
  const int tile0 = (wk % (S::kWalkers / S::kSlices)) * kTPW;
  const int start = static_cast<int>(blockIdx.x % kSteps);
  const uint16_t* wbase =
      a.packed + (static_cast<int64_t>(tile0) * (H / 32) + slice * kSteps) * 512 + lane * 8;
  auto block_at = [&](int i) {
    const int step = (start + i / kTPW) % kSteps;
    return wbase + (static_cast<int64_t>(i % kTPW) * (H / 32) + step) * 512;
  };

  constexpr int V = E / kWave;  // experts per lane in phase 3
  float weight_norm[V];         // loaded first: a row wave's later loads would wait for its stores
#pragma unroll
  for (int v = 0; v < V; ++v) weight_norm[v] = a.weight_norms[lane + v * kWave];
  float bias[V];                // the sigmoid form's correction bias, loaded with them
#pragma unroll
  for (int v = 0; v < V; ++v) bias[v] = a.bias ? a.bias[lane + v * kWave] : 0.0f;
  if (wave == 0) {              // an LDS copy for phase 3, which loads nothing from memory
#pragma unroll
    for (int v = 0; v < V; ++v) bias_lds[lane + v * kWave] = bias[v];
  }

  OMNIA_CLOCK(a, wave, lane, 0);  // entry
  u32x4 ring[kRing];

  if (walker) {
#pragma unroll
    for (int i = 0; i < kRing; ++i) ring[i] = *reinterpret_cast<const u32x4*>(block_at(i));
  } else {
    // Phase 1: rows 2 * wave and 2 * wave + 1.
    const int r0 = 2 * wave;
    const int64_t t0 = first + r0, t1 = t0 + 1;
    const bool live0 = t0 < a.rows, live1 = t1 < a.rows;
    // Every load issued before any arithmetic, none inside a branch (a row past the end
    // loads the last row, in bounds, and is discarded): the waits then count loads
    // exactly, so row 0's arithmetic starts as soon as its own data is in, while row 1
    // is still arriving. The order is row 0, the norm weight, row 1.
    const int64_t l0 = live0 ? t0 : a.rows - 1, l1 = live1 ? t1 : a.rows - 1;
    u32x4 x0[VPL], b0[VPL], x1[VPL], b1[VPL], wv[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int v = lane + i * kWave;
      x0[i] = load_nt(a.x + l0 * (H / 8) + v);
      b0[i] = load_nt(a.branch + l0 * (H / 8) + v);
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) wv[i] = a.norm_weight[lane + i * kWave];  // L2-resident
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int v = lane + i * kWave;
      x1[i] = load_nt(a.x + l1 * (H / 8) + v);
      b1[i] = load_nt(a.branch + l1 * (H / 8) + v);
    }
    // Keeps the scheduler from sinking row 1's loads below row 0's arithmetic.
    __builtin_amdgcn_sched_barrier(0);
    // The selection-only form keeps the summed rows in registers and stores both rows'
    // outputs once the tile is complete: the launch's reads then have HBM to themselves,
    // and its writes drain while the walk streams W from L2. The form that writes every
    // exact logit stores at once (its row waves load W rows later, and a load waits for
    // the wave's earlier stores).
    u32x4 held[VPL];
    router_row<VPL>(x0, b0, wv, live0, t0, a.eps, lane, a, tile + r0 * kRowPitch, row_norm + r0,
                    !kDefer, held);
    if constexpr (kDefer) {
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        *reinterpret_cast<u32x4*>(summed_tile + r0 * kRowPitch + (lane + i * kWave) * 8) = held[i];
    }
    OMNIA_CLOCK(a, wave, lane, 1);  // row 0 normalized
    router_row<VPL>(x1, b1, wv, live1, t1, a.eps, lane, a, tile + (r0 + 1) * kRowPitch,
                    row_norm + r0 + 1, !kDefer, held);
    if constexpr (kDefer) {
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        *reinterpret_cast<u32x4*>(summed_tile + (r0 + 1) * kRowPitch + (lane + i * kWave) * 8) = held[i];
    }
  }
  OMNIA_CLOCK(a, wave, lane, 2);  // phase 1 done (walkers: ring issued)
  lds_barrier();
  OMNIA_CLOCK(a, wave, lane, 3);  // tile complete

  // Phase 2 (walkers): logits = tile x W^T over the walker's slice for its tiles. Lane l
  // feeds row (token) l % 16 of A and column (expert) l % 16 of B, both over
  // k = (l / 16) * 8 .. + 8 of each 32-wide step.
  if (walker) {
    const f32x4 zero = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc[kTPW], l1[kTPW], l2[kTPW];  // group sum, tree levels
    const uint16_t* arow = tile + (lane % 16) * kRowPitch + slice * S::kSlice + (lane / 16) * 8;
    u32x4 av;
    // Adds the step result at position n of this walker's order into tile tt's sum:
    // in order inside a group of kGroup steps, then ((g0 + g1) + (g2 + g3)).
    auto add_step = [&](int tt, int n, const f32x4& part) {
      if (n % (S::kTree ? S::kGroup : kSteps) == 0) {
        acc[tt] = part;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[tt][j] = acc[tt][j] + part[j];
      }
      if (S::kTree && n % S::kGroup == S::kGroup - 1) {
        const int g = n / S::kGroup;
        if (g == 0 || g == 2) {
          l1[tt] = acc[tt];
        } else if (g == 1) {
#pragma unroll
          for (int j = 0; j < 4; ++j) l2[tt][j] = l1[tt][j] + acc[tt][j];
        } else {  // g == 3: the tile's total
#pragma unroll
          for (int j = 0; j < 4; ++j) l1[tt][j] = l1[tt][j] + acc[tt][j];
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[tt][j] = l2[tt][j] + l1[tt][j];
        }
      }
    };
    // Fully unrolled: the ring is indexed by constants only (a partly unrolled loop
    // would index it at run time and put it in scratch memory).
#pragma clang loop unroll(full)
    for (int i = 0; i < kBlocks; ++i) {
      const int tt = i % kTPW;
      const int n = i / kTPW;  // position of the step in this walker's order
      if (tt == 0) {
        const int step = (start + n) % kSteps;
        av = *reinterpret_cast<const u32x4*>(arow + step * 32);
      }
      const u32x4 b = ring[i % kRing];
      if (i + kRing < kBlocks) ring[i % kRing] = *reinterpret_cast<const u32x4*>(block_at(i + kRing));
      f32x4 part;
      if constexpr (kExactAll) {
        // Quarter w: word w of each lane's operands (k = 8 (l / 16) + 2w, + 1), zeros for
        // the operand's other two k's. The four-element operands are taken from a cast
        // of a whole vector (this hipcc compiles a bit cast of an ext-vector swizzle as
        // one of its first elements).
        f32x4 q[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const s16x8 a8 = __builtin_bit_cast(s16x8, u32x4{av[w], 0u, 0u, 0u});
          const s16x8 b8 = __builtin_bit_cast(s16x8, u32x4{b[w], 0u, 0u, 0u});
          q[w] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a8.s0123, b8.s0123, zero, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) part[j] = (q[0][j] + q[1][j]) + (q[2][j] + q[3][j]);
      } else {
        part = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, b), zero, 0, 0, 0);
      }
      add_step(tt, n, part);
    }
    // D layout: lane l holds column (expert) l % 16, rows (tokens) (l / 16) * 4 + i.
    float* out = slice == 0 ? logit_tile : logit_tile1;
#pragma unroll
    for (int tt = 0; tt < kTPW; ++tt) {
      const int e = (tile0 + tt) * 16 + lane % 16;
#pragma unroll
      for (int i = 0; i < 4; ++i) out[((lane / 16) * 4 + i) * E + e] = acc[tt][i];
    }
    OMNIA_CLOCK(a, wave, lane, 4);  // walk done
  }
  lds_barrier();
  OMNIA_CLOCK(a, wave, lane, 5);  // logits complete
  if constexpr (kDefer) {
    if (!walker) {
      // The row waves' outputs, stored now that the walk no longer needs the CU's path
      // to L2; the row waves then leave. Issuing 16 KB of stores takes a wave a while
      // once HBM backs up, so the walkers run phase 3 for all 16 tokens, two each, and
      // its barriers wait for them alone (a barrier counts the waves still running).
      const int r0 = 2 * wave;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int64_t tq = first + r0 + q;
        if (tq < a.rows) {
#pragma unroll
          for (int i = 0; i < VPL; ++i) {
            const int v = lane + i * kWave;
            store_nt(a.summed + tq * (H / 8) + v,
                     *reinterpret_cast<const u32x4*>(summed_tile + (r0 + q) * kRowPitch + v * 8));
            store_nt(a.normalized + tq * (H / 8) + v,
                     *reinterpret_cast<const u32x4*>(tile + (r0 + q) * kRowPitch + v * 8));
          }
        }
      }
      return;
    }
  }

  // Phase 3: as in residual_rms_router_kernel, one token per wave (two per walker when
  // the row waves have left); the recomputations go to the walkers.
  constexpr int kTokens = kDefer ? 2 : 1;
  const bool emit = a.logits != nullptr;
  const bool sigmoid = a.bias != nullptr;
  // Every logit exact (no selection on the bounds) when logits or keys are written out.
  constexpr bool exact_all = kExactAll;
  int rr[kTokens];
  bool active[kTokens];
  uint32_t bits[kTokens][V], upper[kTokens][V], keys[kTokens][V];
  bool need[kTokens][V];
  bool refined[kTokens];
  uint32_t chosen[kTokens], threshold[kTokens];
#pragma unroll
  for (int u = 0; u < kTokens; ++u) {
    const int r = kDefer ? wk + S::kWalkers * u : wave;
    rr[u] = r;
    const int64_t t = first + r;
    active[u] = t < a.rows;  // wave-uniform; inactive waves still meet the barriers
    const float n_norm = row_norm[r];
    bool unsure[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e = lane + v * kWave;
      const float logit = logit_tile[r * E + e] + logit_tile1[r * E + e];
      const float w_norm = weight_norm[v];
      const float delta = (kExactAll ? S::kDeltaQuarters : S::kDelta) * (n_norm * w_norm) +
                          kDeltaFloor * (n_norm + w_norm + 1.0f);
      const uint32_t lo = f32_to_bf16(logit - delta);
      const uint32_t hi = f32_to_bf16(logit + delta);
      bits[u][v] = lo;
      unsure[v] = lo != hi;
      if (sigmoid && !exact_all) {
        // The ordinal key falls as the logit rises: the worst key comes from the lower
        // bound, the best from the upper. Inverted, so that select_topk's largest are the
        // best (ties take one round together, which only lowers the threshold).
        float worst, best, unused;
        sigmoid_bounds(bf16_to_f32(static_cast<uint16_t>(lo)), worst, unused);
        sigmoid_bounds(bf16_to_f32(static_cast<uint16_t>(hi)), unused, best);
        keys[u][v] = ~ordinal_of(-(worst + bias[v]));
        upper[u][v] = ~ordinal_of(-(best + bias[v]));
      } else {
        keys[u][v] = route_key(lo, e);
        upper[u][v] = route_key(hi, e);
      }
    }
    chosen[u] = 0;
    threshold[u] = 0xFFFFFFFFu;
    if (active[u] && !exact_all) threshold[u] = select_topk<V>(keys[u], a.k, lane, chosen[u]);
    refined[u] = false;
    if constexpr (exact_all) {
      // Every unsure logit, about a fifth of them at the config: the token's experts go
      // to the shared task list in one stretch (one atomic per wave), so a slice of the
      // list spans few tokens.
      uint64_t masks[V];
      int total = 0;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        need[u][v] = active[u] && unsure[v];
        masks[v] = __ballot(need[u][v]);
        total += __popcll(masks[v]);
      }
      if (total > 0) {  // wave-uniform
        refined[u] = true;
        int base = 0;
        if (lane == 0) base = atomicAdd(task_count, total);
        base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int below = __builtin_amdgcn_mbcnt_hi(
              static_cast<uint32_t>(masks[v] >> 32),
              __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(masks[v]), 0));
          if (need[u][v]) tasks[base + below] = static_cast<uint16_t>(r * E + lane + v * kWave);
          base += __popcll(masks[v]);
        }
      }
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        need[u][v] = active[u] && unsure[v] && upper[u][v] >= threshold[u];
        const uint64_t mask = __ballot(need[u][v]);
        if (mask != 0) {  // wave-uniform
          refined[u] = true;
          int base = 0;
          if (lane == 0) base = atomicAdd(task_count, __popcll(mask));
          base = __builtin_amdgcn_readfirstlane(base);
          const int below = __builtin_amdgcn_mbcnt_hi(
              static_cast<uint32_t>(mask >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
          if (need[u][v]) tasks[base + below] = static_cast<uint16_t>(r * E + lane + v * kWave);
        }
      }
    }
  }
  OMNIA_CLOCK(a, wave, lane, 6);  // bounds, selection on them, tasks posted
  lds_barrier();
  OMNIA_CLOCK(a, wave, lane, 7);  // task list complete
  uint32_t* exact_bits = reinterpret_cast<uint32_t*>(logit_tile);
  const int count = *task_count;
  if constexpr (exact_all) {
    // Hundreds of tasks per workgroup: all 16 waves take equal slices of the list (the
    // row waves' stores, issued in phase 1, have long completed).
    exact_task_run<VPL, E>(tile, kRowPitch, a.weight_rows, tasks, count * wave / kWaves,
                           count * (wave + 1) / kWaves, lane, exact_bits);
  } else if (walker) {
    for (int i = 2 * wk; i < count; i += 2 * S::kWalkers) {  // wave-uniform
      const int task0 = tasks[i];
      const int task1 = i + 1 < count ? tasks[i + 1] : task0;
      uint32_t exact0, exact1;
      exact_logits<VPL>(tile + (task0 / E) * kRowPitch, tile + (task1 / E) * kRowPitch,
                        a.weight_rows + static_cast<int64_t>(task0 % E) * H,
                        a.weight_rows + static_cast<int64_t>(task1 % E) * H, lane, exact0, exact1);
      if (lane == 0) {
        exact_bits[task0] = exact0;
        exact_bits[task1] = exact1;
      }
    }
  }
  lds_barrier();
  OMNIA_CLOCK(a, wave, lane, 8);  // recomputations done
  // No barrier follows.
#pragma unroll
  for (int u = 0; u < kTokens; ++u) {
    if (!active[u]) continue;
    const int r = rr[u];
    const int64_t t = first + r;
    if (refined[u]) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if (need[u][v]) bits[u][v] = exact_bits[r * E + lane + v * kWave];
      }
    }
    if (emit) {
#pragma unroll
      for (int v = 0; v < V; ++v) a.logits[t * E + lane + v * kWave] = static_cast<uint16_t>(bits[u][v]);
    }
    if (sigmoid) {
      if (exact_all) {
        sigmoid_finish<V>(bits[u], bias, E, a.k, lane, a.keys, a.indices, a.weights, t);
      } else {
        sigmoid_select_contenders<V>(bits[u], upper[u], threshold[u], bias, E, a.k, lane,
                                     a.indices, a.weights, t,
                                     reinterpret_cast<uint32_t*>(tasks) + r * kWave, bias_lds);
      }
      continue;
    }
    uint32_t chosen_u = chosen[u];
    if (refined[u] || exact_all) {
#pragma unroll
      for (int v = 0; v < V; ++v) keys[u][v] = route_key(bits[u][v], lane + v * kWave);
      // A refined selection ranks its few contenders; with every logit exact (or more
      // contenders than lanes) the k rounds over the whole row run.
      if (exact_all || !rank_contenders<V>(keys[u], upper[u], threshold[u], a.k, lane,
                                           reinterpret_cast<uint32_t*>(tasks) + r * kWave, chosen_u)) {
        select_topk<V>(keys[u], a.k, lane, chosen_u);
      }
    }
    write_winners(chosen_u, a.k, lane, a.indices + t * a.k, a.weights + t * a.k);
  }
  OMNIA_CLOCK(a, wave, lane, 9);  // tokens written
}

// ---- up to 512 tokens with the logits written: the projection spread over the chip --
//
// At a decode step one workgroup would read all of W through one CU (512 KB at
// H = 2048, about 4 us at the CU's ~120 GB/s; 2 MB at 4096 x 256). Here a workgroup of 4
// waves owns 8 experts and up to 4 tokens (grid: experts / 8 by tokens / 4). Every wave
// first issues the token rows' loads (the first `rows` waves use them) and then its 2
// experts' rows of W's row-major copy; the first `rows` waves run phase 1 of one token
// each (only the workgroups of the first expert group store the summed and normalized
// rows), and each wave then takes its experts' logits of the group's tokens as fp64 dot
// products (each product of two bf16 values exact, each fused add rounded once), rounded
// to bf16 once: the correctly rounded logits, the fused kernel's own. They go to the
// caller's logits output, and softmax_topk_kernel or sigmoid_topk_kernel selects from
// there, with the same functions as the fused kernel's phase 3.
// The path's limit when the logits are written: every logit an fp64 dot product spread
// over the chip costs less than the fused kernel's exact recomputation of the unsure
// logits up to about 512 tokens at 2048 x 128 (measured on MI355X against the fused
// kernel with its pooled recomputation and MFMA quarters: 9.6 against 31.0 us at 17
// tokens, 21.1 against 32.6 at 256, 32.3 against 33.5 at 512).
constexpr int kDecodeRows = 512;
constexpr int kDecodeGroupRows = 4;  // tokens per workgroup
constexpr int kDecodeWaves = 4;
constexpr int kDecodeExperts = 2;    // per wave

template <int VPL>
__global__ __launch_bounds__(kDecodeWaves * kWave) void router_decode_logits_kernel(RouterArgs a, int experts) {
  constexpr int H = 512 * VPL;
  __shared__ __align__(16) uint16_t tile[kDecodeGroupRows][H];
  __shared__ float norm_bound[kDecodeGroupRows];   // phase 1 writes it; unused here
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int row0 = static_cast<int>(blockIdx.y) * kDecodeGroupRows;
  const int rows = min(kDecodeGroupRows, static_cast<int>(a.rows) - row0);   // 1 .. 4
  const int e0 = (static_cast<int>(blockIdx.x) * kDecodeWaves + wave) * kDecodeExperts;
  // Loads in the order they are used (results are counted in issue order), with no
  // branch among them: a wave past the group's last token reads that token's rows.
  const int64_t row = row0 + (wave < rows ? wave : rows - 1);
  u32x4 xv[VPL], bv[VPL], nw[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int v = lane + i * kWave;
    xv[i] = load_nt(a.x + row * (H / 8) + v);
    bv[i] = load_nt(a.branch + row * (H / 8) + v);
    nw[i] = a.norm_weight[v];
  }
  u32x4 w[kDecodeExperts][VPL];
#pragma unroll
  for (int j = 0; j < kDecodeExperts; ++j) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      w[j][i] = *reinterpret_cast<const u32x4*>(a.weight_rows + static_cast<int64_t>(e0 + j) * H +
                                                (lane + i * kWave) * 8);
    }
  }
  if (wave < rows) {
    router_row<VPL>(xv, bv, nw, true, row, a.eps, lane, a, tile[wave], &norm_bound[wave], blockIdx.x == 0);
  }
  __syncthreads();
  double acc[kDecodeGroupRows][kDecodeExperts];
#pragma unroll
  for (int t = 0; t < kDecodeGroupRows; ++t) {
#pragma unroll
    for (int j = 0; j < kDecodeExperts; ++j) acc[t][j] = 0.0;
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int h0 = (lane + i * kWave) * 8;
    double wd[kDecodeExperts][8];
#pragma unroll
    for (int j = 0; j < kDecodeExperts; ++j) {
      float wf[8];
      unpack8(w[j][i], wf);
#pragma unroll
      for (int q = 0; q < 8; ++q) wd[j][q] = wf[q];
    }
#pragma unroll
    for (int t = 0; t < kDecodeGroupRows; ++t) {
      if (t < rows) {   // uniform
        float n[8];
        unpack8(*reinterpret_cast<const u32x4*>(&tile[t][h0]), n);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const double nq = n[q];
#pragma unroll
          for (int j = 0; j < kDecodeExperts; ++j) acc[t][j] = __builtin_fma(nq, wd[j][q], acc[t][j]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kDecodeGroupRows; ++t) {
    if (t < rows) {
#pragma unroll
      for (int j = 0; j < kDecodeExperts; ++j) {
        const uint32_t bits = f64_to_bf16(wave_sum_f64(acc[t][j]));
        if (lane == 0) a.logits[static_cast<int64_t>(row0 + t) * experts + e0 + j] = static_cast<uint16_t>(bits);
      }
    }
  }
}

// The decode path: rows <= kDecodeRows with the logits written out.
template <int VPL, int E>
int32_t launch_decode(const RouterArgs& a, hipStream_t stream) {
  const dim3 groups(E / (kDecodeWaves * kDecodeExperts),
                    static_cast<unsigned>((a.rows + kDecodeGroupRows - 1) / kDecodeGroupRows));
  router_decode_logits_kernel<VPL><<<groups, kDecodeWaves * kWave, 0, stream>>>(a, E);
  const dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
  constexpr int V = E / kWave;
  if (a.bias != nullptr) {
    if (a.keys != nullptr || a.indices != nullptr) {
      sigmoid_topk_kernel<V, false><<<grid, 256, 0, stream>>>(a.logits, E, a.bias, a.rows, E, a.k, a.keys,
                                                               a.indices, a.weights);
    }
  } else {
    softmax_topk_kernel<V, true, false><<<grid, 256, 0, stream>>>(a.logits, E, a.rows, E, a.k, a.indices,
                                                                  a.weights);
  }
  return launched("residual_rms_router");
}

template <int E, bool kExactAll>
int32_t launch_split_form(const RouterArgs& a, hipStream_t stream) {
  constexpr size_t lds = SplitShape<E>::kLds;
  const hipError_t status = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&residual_rms_router_split_kernel<E, kExactAll>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (status != hipSuccess) {
    return fail(-1, std::string("residual_rms_router: LDS attribute: ") + hipGetErrorString(status));
  }
  const dim3 grid(static_cast<unsigned>((a.rows + kTileTokens - 1) / kTileTokens));
  residual_rms_router_split_kernel<E, kExactAll><<<grid, kThreads, lds, stream>>>(a);
  return launched("residual_rms_router");
}

template <int E>
int32_t launch_split(const RouterArgs& a, hipStream_t stream) {
  const bool exact_all = a.logits != nullptr || (a.bias != nullptr && a.keys != nullptr);
  return exact_all ? launch_split_form<E, true>(a, stream) : launch_split_form<E, false>(a, stream);
}

bool fused_shape(int64_t hidden, int64_t experts) {
  return (hidden == 2048 && (experts == 128 || experts == 256)) ||
         (hidden == 4096 && (experts == 128 || experts == 256));
}

}  // namespace
}  // namespace omnia

namespace omnia {
namespace {

template <bool kNormalize, bool kShared>
void launch_softmax_topk(const uint16_t* logits, int64_t stride, int64_t rows, int64_t experts,
                         int64_t k, int32_t* indices, float* weights, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  const int e = static_cast<int>(experts), top = static_cast<int>(k);
  switch ((experts + kWave - 1) / kWave) {
    case 1: softmax_topk_kernel<1, kNormalize, kShared><<<grid, 256, 0, stream>>>(logits, stride, rows, e, top, indices, weights); break;
    case 2: softmax_topk_kernel<2, kNormalize, kShared><<<grid, 256, 0, stream>>>(logits, stride, rows, e, top, indices, weights); break;
    case 3: softmax_topk_kernel<3, kNormalize, kShared><<<grid, 256, 0, stream>>>(logits, stride, rows, e, top, indices, weights); break;
    default: softmax_topk_kernel<4, kNormalize, kShared><<<grid, 256, 0, stream>>>(logits, stride, rows, e, top, indices, weights); break;
  }
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_softmax_topk_slots(const uint16_t* logits, int64_t stride, int64_t rows,
                                            int64_t experts, int64_t k, int32_t normalize,
                                            int32_t shared, int32_t* indices, float* weights,
                                            hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), "softmax_topk: bad row count");
  OMNIA_REQUIRE(experts > 0 && experts <= 4 * kWave, "softmax_topk: experts must be in [1, 256]");
  OMNIA_REQUIRE(k > 0 && k <= experts && k < kMaxTopK + (shared ? 0 : 1),
                "softmax_topk: k must be in [1, min(experts, 64)] (63 with a shared slot)");
  OMNIA_REQUIRE(normalize == 0 || normalize == 1, "softmax_topk: normalize must be 0 or 1");
  OMNIA_REQUIRE(shared == 0 || shared == 1, "softmax_topk: shared must be 0 or 1");
  OMNIA_REQUIRE(stride >= experts + shared, "softmax_topk: row stride smaller than the row's logits");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(logits && indices && weights, "softmax_topk: null pointer");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  if (normalize) {
    if (shared) launch_softmax_topk<true, true>(logits, stride, rows, experts, k, indices, weights, stream);
    else launch_softmax_topk<true, false>(logits, stride, rows, experts, k, indices, weights, stream);
  } else {
    if (shared) launch_softmax_topk<false, true>(logits, stride, rows, experts, k, indices, weights, stream);
    else launch_softmax_topk<false, false>(logits, stride, rows, experts, k, indices, weights, stream);
  }
  return launched("softmax_topk");
}

extern "C" int32_t omnia_softmax_topk(const uint16_t* logits, int64_t stride, int64_t rows,
                                      int64_t experts, int64_t k, int32_t* indices,
                                      float* weights, hipStream_t stream) {
  return omnia_softmax_topk_slots(logits, stride, rows, experts, k, 1, 0, indices, weights, stream);
}

extern "C" int64_t omnia_router_pack_bytes(int64_t experts, int64_t hidden) {
  using namespace omnia;
  OMNIA_REQUIRE(experts > 0 && experts % 16 == 0 && experts <= 4096 && hidden > 0 &&
                    hidden % 32 == 0 && hidden <= 65536,
                "router_pack_bytes: experts must be a multiple of 16, hidden of 32");
  return packed_bytes(experts, hidden);
}

extern "C" int32_t omnia_pack_router_weight(const uint16_t* router_weight, int64_t experts,
                                            int64_t hidden, void* packed,
                                            hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(experts > 0 && experts % 16 == 0 && experts <= 4096 && hidden > 0 &&
                    hidden % 32 == 0 && hidden <= 65536,
                "pack_router_weight: experts must be a multiple of 16, hidden of 32");
  OMNIA_REQUIRE(router_weight && packed, "pack_router_weight: null pointer");
  OMNIA_REQUIRE(aligned16(router_weight) && aligned16(packed),
                "pack_router_weight: pointers must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const int chunks = static_cast<int>(experts * hidden / 8);
  const int chunk_blocks = (chunks + kPackBlock - 1) / kPackBlock;
  const int norm_blocks = static_cast<int>((experts + kPackBlock / kWave - 1) / (kPackBlock / kWave));
  uint16_t* base = static_cast<uint16_t*>(packed);
  pack_router_kernel<<<chunk_blocks + norm_blocks, kPackBlock, 0, stream>>>(
      reinterpret_cast<const u32x4*>(router_weight), reinterpret_cast<u32x4*>(base),
      reinterpret_cast<float*>(base + packed_weight_elements(experts, hidden)),
      reinterpret_cast<u32x4*>(base + packed_rows_offset(experts, hidden)),
      static_cast<int>(experts), static_cast<int>(hidden), chunk_blocks);
  return launched("pack_router_weight");
}

namespace omnia {
namespace {

#ifdef OMNIA_PHASE_CLOCKS
uint64_t* phase_clocks = nullptr;  // set by omnia_router_phase_clocks_set
#endif

int32_t launch_router(RouterArgs a, int64_t hidden, int64_t experts, hipStream_t stream) {
#ifdef OMNIA_PHASE_CLOCKS
  a.clocks = hidden == 2048 ? phase_clocks : nullptr;
#endif
  if (a.rows <= kDecodeRows && a.logits != nullptr) {
    if (hidden == 2048) return experts == 128 ? launch_decode<4, 128>(a, stream) : launch_decode<4, 256>(a, stream);
    return experts == 128 ? launch_decode<8, 128>(a, stream) : launch_decode<8, 256>(a, stream);
  }
  if (hidden == 2048) {
    return experts == 128 ? launch_split<128>(a, stream) : launch_split<256>(a, stream);
  }
  return experts == 128 ? launch_fused<8, 128>(a, stream) : launch_fused<8, 256>(a, stream);
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_residual_rms_router(
    const uint16_t* x, const uint16_t* branch, const uint16_t* norm_weight,
    const void* packed_router, int64_t rows, int64_t hidden, int64_t experts, int64_t k,
    float eps, uint16_t* summed, uint16_t* normalized, uint16_t* logits, int32_t* indices,
    float* weights, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), "residual_rms_router: bad row count");
  OMNIA_REQUIRE(fused_shape(hidden, experts),
                "residual_rms_router: hidden must be 2048 or 4096 and experts 128 or 256");
  OMNIA_REQUIRE(k > 0 && k <= experts && k <= kMaxTopK,
                "residual_rms_router: k must be in [1, min(experts, 64)]");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(x && branch && norm_weight && packed_router && summed && normalized &&
                    indices && weights,
                "residual_rms_router: null pointer");
  OMNIA_REQUIRE(aligned16(x) && aligned16(branch) && aligned16(norm_weight) &&
                    aligned16(packed_router) && aligned16(summed) && aligned16(normalized),
                "residual_rms_router: pointers must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const uint16_t* packed = static_cast<const uint16_t*>(packed_router);
  RouterArgs a{reinterpret_cast<const u32x4*>(x), reinterpret_cast<const u32x4*>(branch),
               reinterpret_cast<const u32x4*>(norm_weight), packed,
               reinterpret_cast<const float*>(packed + packed_weight_elements(experts, hidden)),
               packed + packed_rows_offset(experts, hidden),
               reinterpret_cast<u32x4*>(summed), reinterpret_cast<u32x4*>(normalized),
               logits, indices, weights, nullptr, nullptr, rows, static_cast<int>(k), eps};
  return launch_router(a, hidden, experts, stream);
}

extern "C" int32_t omnia_residual_rms_router_sigmoid(
    const uint16_t* x, const uint16_t* branch, const uint16_t* norm_weight,
    const void* packed_router, const float* bias, int64_t rows, int64_t hidden, int64_t experts,
    int64_t k, float eps, uint16_t* summed, uint16_t* normalized, uint16_t* logits,
    uint32_t* keys, int32_t* indices, float* weights, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), "residual_rms_router_sigmoid: bad row count");
  OMNIA_REQUIRE(fused_shape(hidden, experts),
                "residual_rms_router_sigmoid: hidden must be 2048 or 4096 and experts 128 or 256");
  OMNIA_REQUIRE((indices == nullptr) == (weights == nullptr),
                "residual_rms_router_sigmoid: indices and weights come together");
  OMNIA_REQUIRE(indices == nullptr || (k > 0 && k <= experts && k <= kMaxTopK),
                "residual_rms_router_sigmoid: k must be in [1, min(experts, 64)]");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(x && branch && norm_weight && packed_router && bias && summed && normalized,
                "residual_rms_router_sigmoid: null pointer");
  OMNIA_REQUIRE(aligned16(x) && aligned16(branch) && aligned16(norm_weight) &&
                    aligned16(packed_router) && aligned16(summed) && aligned16(normalized),
                "residual_rms_router_sigmoid: pointers must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const uint16_t* packed = static_cast<const uint16_t*>(packed_router);
  RouterArgs a{reinterpret_cast<const u32x4*>(x), reinterpret_cast<const u32x4*>(branch),
               reinterpret_cast<const u32x4*>(norm_weight), packed,
               reinterpret_cast<const float*>(packed + packed_weight_elements(experts, hidden)),
               packed + packed_rows_offset(experts, hidden),
               reinterpret_cast<u32x4*>(summed), reinterpret_cast<u32x4*>(normalized),
               logits, indices, weights, bias, keys, rows,
               indices ? static_cast<int>(k) : 0, eps};
  return launch_router(a, hidden, experts, stream);
}

extern "C" int32_t omnia_sigmoid_topk(const void* logits, int64_t stride, int32_t logits_fp32,
                                      const float* bias, int64_t rows, int64_t experts, int64_t k,
                                      uint32_t* keys, int32_t* indices, float* weights,
                                      hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), "sigmoid_topk: bad row count");
  OMNIA_REQUIRE(experts > 0 && experts <= 16 * kWave, "sigmoid_topk: experts must be in [1, 1024]");
  OMNIA_REQUIRE(stride >= experts, "sigmoid_topk: row stride smaller than experts");
  OMNIA_REQUIRE(logits_fp32 == 0 || logits_fp32 == 1, "sigmoid_topk: logits_fp32 must be 0 or 1");
  OMNIA_REQUIRE((indices == nullptr) == (weights == nullptr),
                "sigmoid_topk: indices and weights come together");
  OMNIA_REQUIRE(indices == nullptr || (k > 0 && k <= experts && k <= kMaxTopK),
                "sigmoid_topk: k must be in [1, min(experts, 64)]");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(logits && bias && (keys || indices), "sigmoid_topk: null pointer");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  const int kk = indices ? static_cast<int>(k) : 0;
  const int e = static_cast<int>(experts);
  const int v = (e + kWave - 1) / kWave;
#define OMNIA_SIGMOID_TOPK(V)                                                                  \
  (logits_fp32 ? sigmoid_topk_kernel<V, true><<<grid, 256, 0, stream>>>(logits, stride, bias, rows, e, kk, keys, indices, weights) \
               : sigmoid_topk_kernel<V, false><<<grid, 256, 0, stream>>>(logits, stride, bias, rows, e, kk, keys, indices, weights))
  if (v <= 1) OMNIA_SIGMOID_TOPK(1);
  else if (v <= 2) OMNIA_SIGMOID_TOPK(2);
  else if (v <= 4) OMNIA_SIGMOID_TOPK(4);
  else if (v <= 8) OMNIA_SIGMOID_TOPK(8);
  else OMNIA_SIGMOID_TOPK(16);
#undef OMNIA_SIGMOID_TOPK
  return launched("sigmoid_topk");
}

#ifdef OMNIA_PHASE_CLOCKS
// Diagnostic build only: the buffer the H = 2048 router kernels record their phase
// clocks into ([workgroups, 16, 10] uint64, 100 MHz ticks), or null to stop recording.
extern "C" void omnia_router_phase_clocks_set(void* buffer) {
  omnia::phase_clocks = static_cast<uint64_t*>(buffer);
}
#endif
