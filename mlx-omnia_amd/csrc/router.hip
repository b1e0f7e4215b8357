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
// (sign flip for positives, all bits for negatives, -0 folded onto +0, NaN above
// everything) in the high half and 0xFFFF - expert in the low half. Unsigned key order
// is then descending logit with the lower index first on ties; k rounds of a wave-wide
// max extract the winners.
//
// Fused kernel (core/kernels/route/residual.py:117-299 is the one-token precedent;
// config: x, residual [4096, 2048], router [128, 2048], k = 8): a workgroup of 8 waves
// owns 16 tokens; a workgroup is 16 waves.
//   1. residual add + RMSNorm, one row per wave (arithmetic of add_rms_norm.hip),
//      writing summed and normalized and keeping the bf16 normalized tile in LDS;
//   2. logits[16, E] = tile [16, H] x W^T on v_mfma_f32_16x16x32_bf16 (fp32
//      accumulation), each wave owning one 16-expert tile over a slice of H (E = 128:
//      two halves), W streamed from L2 (every workgroup reads all of it; 512 KB at the
//      config). A second MFMA accumulates A = |tile| x |W|^T, the sum of the products'
//      magnitudes. The slices' partial sums meet in LDS;
//   3. per token: the bf16 rounding of each logit, made exact. Each MFMA forms the
//      sum of its 32 products (at most 31 roundings, any order) and adds it to the
//      accumulator (one more); adding the slices' partials costs one more, so the fp32
//      logit L is within delta = 97 * 2^-23 * A (1% slack for the rounding of A itself)
//      of the exact dot product, each rounding counted at a full ulp. When [L - delta, L + delta]
//      rounds to one bf16 value, that value is the correctly rounded logit; otherwise
//      the logit is recomputed as an fp64 dot product from the LDS tile and W (the
//      products of two bf16 values are exact in fp32) and rounded once. Recomputed
//      are the unsure logits whose upper bound could reach the top k (all of them when
//      the logits are written out), so the selection, the weights and any emitted
//      logit equal those of the correctly rounded logits. Then the selection and the
//      weights above.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kTileTokens = 16;   // MFMA M
constexpr int kWaves = 16;        // one row per wave in phases 1 and 3
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxTopK = 64;

__device__ __forceinline__ uint32_t order16(uint32_t bits) {
  if ((bits & 0x7FFFu) > 0x7F80u) return 0xFFFFu;  // NaN above everything
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

// Maximum over the wave, returned as a wave-uniform value: DPP steps inside each
// 16-lane row (quad swaps, half-row and row mirrors), then the four row results read
// into scalar registers. No LDS round trips on the dependency chain.
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
  constexpr int kQuadSwap1 = 0xB1;        // quad_perm [1, 0, 3, 2]
  constexpr int kQuadSwap2 = 0x4E;        // quad_perm [2, 3, 0, 1]
  constexpr int kRowHalfMirror = 0x141;
  constexpr int kRowMirror = 0x140;
  v = umax(v, dpp<kQuadSwap1>(v));
  v = umax(v, dpp<kQuadSwap2>(v));
  v = umax(v, dpp<kRowHalfMirror>(v));
  v = umax(v, dpp<kRowMirror>(v));
  const uint32_t r0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0));
  const uint32_t r1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16));
  const uint32_t r2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
  const uint32_t r3 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 48));
  return umax(umax(r0, r1), umax(r2, r3));
}

// Sum over the wave (same DPP pattern), wave-uniform result.
__device__ __forceinline__ float wave_sum(float v) {
  constexpr int kQuadSwap1 = 0xB1, kQuadSwap2 = 0x4E, kRowHalfMirror = 0x141, kRowMirror = 0x140;
  v += __uint_as_float(dpp<kQuadSwap1>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kQuadSwap2>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowMirror>(__float_as_uint(v)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
}

// Extracts the top k of the wave's keys (V per lane; a taken key becomes 0, below
// every real key). Lane j < k ends with the j-th winner; returns the k-th (uniform).
template <int V>
__device__ __forceinline__ uint32_t select_topk(uint32_t (&keys)[V], int k, int lane,
                                                uint32_t& chosen) {
  chosen = 0;
  uint32_t best = 0;
  for (int j = 0; j < k; ++j) {
    uint32_t local = 0;
#pragma unroll
    for (int v = 0; v < V; ++v) local = umax(local, keys[v]);
    best = wave_max(local);
#pragma unroll
    for (int v = 0; v < V; ++v) keys[v] = keys[v] == best ? 0u : keys[v];
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

// ---- softmax -> top-k over given bf16 logits: one wave per row --------------------

template <int V>
__global__ __launch_bounds__(256) void softmax_topk_kernel(const uint16_t* __restrict__ logits,
                                                           int64_t stride, int64_t rows,
                                                           int experts, int k,
                                                           int32_t* __restrict__ indices,
                                                           float* __restrict__ weights) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (row >= rows) return;
  uint32_t keys[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int e = lane + v * kWave;
    keys[v] = e < experts ? route_key(logits[row * stride + e], e) : 0u;
  }
  uint32_t chosen;
  select_topk<V>(keys, k, lane, chosen);
  write_winners(chosen, k, lane, indices + row * k, weights + row * k);
}

// ---- fused residual add + RMSNorm + router projection + top-k ---------------------

// Bound on |fp32 MFMA logit - exact dot product| per unit of sum |n_k * W_ek|.
constexpr float kDeltaPerMagnitude = 97.0f * 1.01f / 8388608.0f;

// Correctly rounded bf16 bits of sum_k n_k * W_k over one row pair, by one wave: the
// products of two bf16 values are exact in fp32 and are summed in fp64.
template <int VPL>
__device__ __forceinline__ uint32_t exact_logit(const uint16_t* n_row, const uint16_t* w_row,
                                                int lane) {
  double acc = 0.0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int v = lane + i * kWave;
    float n[8], w[8];
    unpack8(*reinterpret_cast<const u32x4*>(n_row + v * 8), n);
    unpack8(*reinterpret_cast<const u32x4*>(w_row + v * 8), w);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += static_cast<double>(n[j] * w[j]);
  }
  acc = group_sum<kWave>(acc);
  return f64_to_bf16(acc);
}

struct RouterArgs {
  const u32x4* x;
  const u32x4* branch;
  const u32x4* norm_weight;
  const uint16_t* router_weight;  // [E, H]
  u32x4* summed;
  u32x4* normalized;
  uint16_t* logits;               // [T, E] bf16, optional
  int32_t* indices;               // [T, k]
  float* weights;                 // [T, k]
  int64_t rows;
  int k;
  float eps;
};

// VPL: 16-byte vectors per lane per row (H = 512 * VPL). E: experts, a multiple of 16
// with E / 16 dividing the 16 waves; the waves split H into 16 / (E / 16) slices.
template <int VPL, int E>
__global__ __launch_bounds__(kThreads) void residual_rms_router_kernel(RouterArgs a) {
  constexpr int H = 512 * VPL;
  constexpr int kTiles = E / 16;
  constexpr int kSlices = kWaves / kTiles;
  constexpr int kSlice = H / kSlices;
  constexpr int kRowPitch = H + 8;  // bf16 elements; the pad staggers LDS banks per row
  constexpr int kRowsPerWave = kTileTokens / kWaves;
  constexpr int TPW = 1;
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* tile = reinterpret_cast<uint16_t*>(smem);
  // Logits and magnitudes [token][expert]; the slices' partials are added in turn.
  float* logit_tile = reinterpret_cast<float*>(smem + kTileTokens * kRowPitch * 2);
  float* magnitude_tile = logit_tile + kTileTokens * E;

  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kTileTokens;

  // Phase 1: residual add + RMSNorm, rows wave and wave + 8.
  {
    u32x4 xv[kRowsPerWave][VPL], bv[kRowsPerWave][VPL], wv[VPL];
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const int64_t t = first + wave + rr * kWaves;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        xv[rr][i] = u32x4{0u, 0u, 0u, 0u};
        bv[rr][i] = u32x4{0u, 0u, 0u, 0u};
        if (t < a.rows) {
          xv[rr][i] = load_nt(a.x + t * (H / 8) + lane + i * kWave);
          bv[rr][i] = load_nt(a.branch + t * (H / 8) + lane + i * kWave);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) wv[i] = a.norm_weight[lane + i * kWave];
#pragma unroll
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const int r = wave + rr * kWaves;
      const int64_t t = first + r;
      float s[VPL][8];
      double sumsq = 0.0;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float xf[8], bf[8];
        unpack8(xv[rr][i], xf);
        unpack8(bv[rr][i], bf);
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          s[i][j] = xf[j] + bf[j];
          s[i][j + 1] = xf[j + 1] + bf[j + 1];
          round_pair(s[i][j], s[i][j + 1]);
          sumsq += static_cast<double>(s[i][j] * s[i][j]);
          sumsq += static_cast<double>(s[i][j + 1] * s[i][j + 1]);
        }
      }
      sumsq = group_sum<kWave>(sumsq);
      const float inv = 1.0f / sqrtf(static_cast<float>(sumsq) / static_cast<float>(H) + a.eps);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float w[8], n[8];
        unpack8(wv[i], w);
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          float lo = s[i][j] * inv, hi = s[i][j + 1] * inv;
          round_pair(lo, hi);
          n[j] = w[j] * lo;
          n[j + 1] = w[j + 1] * hi;
        }
        const u32x4 packed = pack8(n);
        const int v = lane + i * kWave;
        *reinterpret_cast<u32x4*>(tile + r * kRowPitch + v * 8) =
            t < a.rows ? packed : u32x4{0u, 0u, 0u, 0u};
        if (t < a.rows) {
          store_nt(a.summed + t * (H / 8) + v, pack8(s[i]));
          store_nt(a.normalized + t * (H / 8) + v, packed);
        }
      }
    }
  }
  __syncthreads();

  // Phase 2: logits = tile x W^T and magnitudes = |tile| x |W|^T. Lane l feeds row
  // (token) l % 16 of A and column (expert) l % 16 of B, both over
  // k = (l / 16) * 8 .. + 8 of each 32-wide step.
  f32x4 acc[TPW], mag[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    mag[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  {
    constexpr uint32_t kAbs = 0x7FFF7FFFu;
    const int quad = lane / 16;
    const int expert_tile = wave % kTiles;
    const int slice = wave / kTiles;
    const uint16_t* arow = tile + (lane % 16) * kRowPitch + slice * kSlice + quad * 8;
    const uint16_t* brow[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      brow[j] = a.router_weight + static_cast<int64_t>(expert_tile * 16 + lane % 16) * H +
                slice * kSlice + quad * 8;
    }
    // Each workgroup starts its walk over k at a different 256-wide block, so the
    // workgroups of an XCD do not all read the same W lines (the same L2 channels) at
    // once. The accumulation order changes per workgroup; the error bound does not.
    constexpr int kUnroll = 8;
    constexpr int kSteps = kSlice / (32 * kUnroll);
    const int start = static_cast<int>(blockIdx.x % kSteps);
    u32x4 next[kUnroll][TPW];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        next[u][j] = *reinterpret_cast<const u32x4*>(brow[j] + start * 32 * kUnroll + u * 32);
      }
    }
    for (int step = 0; step < kSteps; ++step) {
      const int k0 = ((start + step) % kSteps) * 32 * kUnroll;
      const int k1 = ((start + step + 1) % kSteps) * 32 * kUnroll;
      u32x4 b[kUnroll][TPW];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
          b[u][j] = next[u][j];
          if (step + 1 < kSteps) {
            next[u][j] = *reinterpret_cast<const u32x4*>(brow[j] + k1 + u * 32);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const u32x4 av = *reinterpret_cast<const u32x4*>(arow + k0 + u * 32);
        const u32x4 aabs = av & kAbs;
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, b[u][j]), acc[j], 0, 0, 0);
          mag[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, aabs), __builtin_bit_cast(bf16x8, b[u][j] & kAbs),
              mag[j], 0, 0, 0);
        }
      }
    }
  }
  // D layout: lane l holds column (expert) l % 16, rows (tokens) (l / 16) * 4 + i.
  {
    const int e = (wave % kTiles) * 16 + lane % 16;
    const int slice = wave / kTiles;
#pragma unroll 1
    for (int turn = 0; turn < kSlices; ++turn) {
      if (slice == turn) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int at = ((lane / 16) * 4 + i) * E + e;
          logit_tile[at] = turn == 0 ? acc[0][i] : logit_tile[at] + acc[0][i];
          magnitude_tile[at] = turn == 0 ? mag[0][i] : magnitude_tile[at] + mag[0][i];
        }
      }
      __syncthreads();
    }
  }

  // Phase 3: exact bf16 logits where they decide anything, then the selection; two
  // tokens per wave.
  const bool emit = a.logits != nullptr;
#pragma unroll 1
  for (int rr = 0; rr < kRowsPerWave; ++rr) {
    const int r = wave * kRowsPerWave + rr;
    const int64_t t = first + r;
    if (t >= a.rows) break;  // wave-uniform
    constexpr int V = E / kWave;
    uint32_t bits[V], lower[V], upper[V];
    bool unsure[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int e = lane + v * kWave;
      const float logit = logit_tile[r * E + e];
      const float delta = kDeltaPerMagnitude * magnitude_tile[r * E + e];
      const uint32_t lo = f32_to_bf16(logit - delta);
      const uint32_t hi = f32_to_bf16(logit + delta);
      bits[v] = lo;
      unsure[v] = lo != hi;
      lower[v] = route_key(lo, e);
      upper[v] = route_key(hi, e);
    }
    // Select on the lower bounds. A certain logit's lower bound is its value; an
    // unsure logit whose upper bound stays below the k-th selected key cannot be
    // selected. If every selected logit is certain and no unsure one can reach the
    // k-th, this selection is final.
    uint32_t chosen;
    uint32_t keys[V];
#pragma unroll
    for (int v = 0; v < V; ++v) keys[v] = lower[v];
    const uint32_t threshold = select_topk<V>(keys, a.k, lane, chosen);
    const uint16_t* n_row = tile + r * kRowPitch;
    bool refined = false;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const bool need = unsure[v] && (emit || upper[v] >= threshold);
      uint64_t pending = __ballot(need);
      refined = refined || pending != 0;
      while (pending != 0) {  // wave-uniform loop
        const int src = __ffsll(static_cast<unsigned long long>(pending)) - 1;
        pending &= pending - 1;
        const int e = src + v * kWave;
        const uint32_t exact =
            exact_logit<VPL>(n_row, a.router_weight + static_cast<int64_t>(e) * H, lane);
        if (lane == src) bits[v] = exact;
      }
    }
    if (refined) {
#pragma unroll
      for (int v = 0; v < V; ++v) keys[v] = route_key(bits[v], lane + v * kWave);
      select_topk<V>(keys, a.k, lane, chosen);
    }
    if (emit) {
#pragma unroll
      for (int v = 0; v < V; ++v) a.logits[t * E + lane + v * kWave] = static_cast<uint16_t>(bits[v]);
    }
    write_winners(chosen, a.k, lane, a.indices + t * a.k, a.weights + t * a.k);
  }
}

template <int VPL, int E>
int32_t launch_fused(const RouterArgs& a, hipStream_t stream) {
  constexpr int H = 512 * VPL;
  const size_t lds = static_cast<size_t>(kTileTokens) * (H + 8) * 2 +
                     static_cast<size_t>(kTileTokens) * E * 4 * 2;
  static bool configured = false;  // the attribute is per kernel, set once per process
  if (!configured) {
    const hipError_t status = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&residual_rms_router_kernel<VPL, E>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (status != hipSuccess) {
      return fail(-1, std::string("residual_rms_router: LDS attribute: ") +
                          hipGetErrorString(status));
    }
    configured = true;
  }
  const dim3 grid(static_cast<unsigned>((a.rows + kTileTokens - 1) / kTileTokens));
  residual_rms_router_kernel<VPL, E><<<grid, kThreads, lds, stream>>>(a);
  return launched("residual_rms_router");
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_softmax_topk(const uint16_t* logits, int64_t stride, int64_t rows,
                                      int64_t experts, int64_t k, int32_t* indices,
                                      float* weights, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), "softmax_topk: bad row count");
  OMNIA_REQUIRE(experts > 0 && experts <= 4 * kWave, "softmax_topk: experts must be in [1, 256]");
  OMNIA_REQUIRE(k > 0 && k <= experts && k <= kMaxTopK, "softmax_topk: k must be in [1, min(experts, 64)]");
  OMNIA_REQUIRE(stride >= experts, "softmax_topk: row stride smaller than experts");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(logits && indices && weights, "softmax_topk: null pointer");
  int32_t rc = check_device();
  if (rc != 0) return rc;
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  const int v = static_cast<int>((experts + kWave - 1) / kWave);
  switch (v) {
    case 1: softmax_topk_kernel<1><<<grid, 256, 0, stream>>>(logits, stride, rows, experts, k, indices, weights); break;
    case 2: softmax_topk_kernel<2><<<grid, 256, 0, stream>>>(logits, stride, rows, experts, k, indices, weights); break;
    case 3: softmax_topk_kernel<3><<<grid, 256, 0, stream>>>(logits, stride, rows, experts, k, indices, weights); break;
    default: softmax_topk_kernel<4><<<grid, 256, 0, stream>>>(logits, stride, rows, experts, k, indices, weights); break;
  }
  return launched("softmax_topk");
}

extern "C" int32_t omnia_residual_rms_router(
    const uint16_t* x, const uint16_t* branch, const uint16_t* norm_weight,
    const uint16_t* router_weight, int64_t rows, int64_t hidden, int64_t experts, int64_t k,
    float eps, uint16_t* summed, uint16_t* normalized, uint16_t* logits, int32_t* indices,
    float* weights, hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), "residual_rms_router: bad row count");
  OMNIA_REQUIRE((hidden == 2048 && (experts == 128 || experts == 256)) ||
                    (hidden == 4096 && experts == 128),
                "residual_rms_router: (hidden, experts) must be (2048, 128), (2048, 256) "
                "or (4096, 128)");
  OMNIA_REQUIRE(k > 0 && k <= experts && k <= kMaxTopK,
                "residual_rms_router: k must be in [1, min(experts, 64)]");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(x && branch && norm_weight && router_weight && summed && normalized &&
                    indices && weights,
                "residual_rms_router: null pointer");
  OMNIA_REQUIRE(aligned16(x) && aligned16(branch) && aligned16(norm_weight) &&
                    aligned16(router_weight) && aligned16(summed) && aligned16(normalized),
                "residual_rms_router: pointers must be 16-byte aligned");
  int32_t rc = check_device();
  if (rc != 0) return rc;
  RouterArgs a{reinterpret_cast<const u32x4*>(x), reinterpret_cast<const u32x4*>(branch),
               reinterpret_cast<const u32x4*>(norm_weight), router_weight,
               reinterpret_cast<u32x4*>(summed), reinterpret_cast<u32x4*>(normalized),
               logits, indices, weights, rows, static_cast<int>(k), eps};
  if (hidden == 2048) {
    return experts == 128 ? launch_fused<4, 128>(a, stream) : launch_fused<4, 256>(a, stream);
  }
  return launch_fused<8, 128>(a, stream);
}
