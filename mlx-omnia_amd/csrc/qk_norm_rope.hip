// Per-head q/k RMSNorm + half-split rotary, one dispatch for every head of a segment.
//
// Arithmetic (core/kernels/qkv_rope/qk_norm_rope.py:21-24,120-140,295-308; the norm
// rounds as mx.fast.rms_norm does):
//   inv  = 1 / sqrt(sum_d x_d^2 / D + eps)
//   n_d  = bf16(w_d * bf16(x_d * inv))
//   for p < P:  a = bf16(n_p * bf16(mscale)),  b = bf16(n_{p+P} * bf16(mscale))
//               out_p     = bf16(a * cos_p - b * sin_p)
//               out_{p+P} = bf16(a * sin_p + b * cos_p)
//   for 2P <= d < D:  out_d = n_d                     (partial-rotary tail)
// (cos_p, sin_p) come either from a caller's fp32 table row `offset + t`
// (`omnia_qk_norm_rope`), or are derived in-kernel exactly as
// core/kernels/qkv_rope/epilogue.py:57-63 derives them (`omnia_rope_epilogue`):
//   angle_p = f32(pos) * exp2(-(p / P) * log2(base)),  with cos/sin of that fp32 angle.
// In-kernel, exp2, cos and sin are evaluated in fp64 and rounded once to fp32, i.e.
// correctly rounded for all practical purposes (the reference's Metal code uses
// fast::cos/sin, which no other machine reproduces bit for bit).
//
// Layout (wave64): a head of D bf16 is D/8 lanes x one 16-byte vector, so a wave holds
// 64/(D/8) heads (4 at D=128). The rotary partner of element p is element p+P, which
// sits on lane `lane ^ (P/8)` of the same head group: one cross-lane exchange of four
// packed dwords. One workgroup is one token: the token's cos/sin row (2P floats) is
// staged once in LDS and read by all its heads. Input is token-major with a row stride
// (so q and k can be read straight out of a fused qkv projection); output is head-major
// [heads, T, D], the layout attention consumes (qk_norm_rope.py:163-175).
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kMaxPairs = 128;  // P <= D/2 <= 128

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
  float eps;
  float mscale;
  float log2_base;
};

template <int D, bool TABLE>
__global__ __launch_bounds__(1024) void qk_norm_rope_kernel(RopeArgs a) {
  constexpr int G = D / 8;            // lanes per head
  __shared__ float cos_row[kMaxPairs];
  __shared__ float sin_row[kMaxPairs];

  const int64_t t = blockIdx.x;
  const int64_t position = a.offset + t;
  const int lane_in_head = threadIdx.x % G;
  const int group = threadIdx.x / G;
  const int groups = blockDim.x / G;
  const int heads = a.query_heads + a.kv_heads;
  const int pair_lanes = a.pairs / 8;  // lanes holding the first rotary half

  // Stage this token's cos/sin row.
  if constexpr (TABLE) {
    const int chunks = a.pairs / 4;  // 16-byte chunks per half-row
    if (threadIdx.x < 2 * chunks) {
      const bool is_sin = threadIdx.x >= chunks;
      const int c = is_sin ? threadIdx.x - chunks : threadIdx.x;
      const float* src = (is_sin ? a.sin_table : a.cos_table) + position * a.table_stride;
      const f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * c);
      *reinterpret_cast<f32x4*>((is_sin ? sin_row : cos_row) + 4 * c) = v;
    }
  } else {
    if (threadIdx.x < a.pairs) {
      const float d = static_cast<float>(threadIdx.x) / static_cast<float>(a.pairs);
      const float exponent = -d * a.log2_base;
      const float frequency = static_cast<float>(exp2(static_cast<double>(exponent)));
      const float angle = static_cast<float>(position) * frequency;
      double s, c;
      sincos(static_cast<double>(angle), &s, &c);
      cos_row[threadIdx.x] = static_cast<float>(c);
      sin_row[threadIdx.x] = static_cast<float>(s);
    }
  }
  __syncthreads();

  const float rounded_mscale = round_bf16(a.mscale);
  for (int head = group; head < heads; head += groups) {
    const bool is_query = head < a.query_heads;
    const int kv = head - a.query_heads;
    const uint16_t* in = is_query ? a.queries_in + t * a.query_stride + head * D
                                  : a.keys_in + t * a.key_stride + kv * D;
    const uint16_t* weight = is_query ? a.query_weight : a.key_weight;
    uint16_t* out = is_query ? a.queries_out + (head * a.length + t) * D
                             : a.keys_out + (kv * a.length + t) * D;

    float x[8], w[8];
    unpack8(load_nt(reinterpret_cast<const u32x4*>(in) + lane_in_head), x);
    unpack8(*(reinterpret_cast<const u32x4*>(weight) + lane_in_head), w);

    float sumsq = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) sumsq += x[j] * x[j];
    sumsq = group_sum<G>(sumsq);
    const float inv = 1.0f / sqrtf(sumsq / static_cast<float>(D) + a.eps);

    float n[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) n[j] = round_bf16(w[j] * round_bf16(x[j] * inv));

    // Partner lane holds the other half of each pair.
    const u32x4 mine = pack8(n);
    u32x4 theirs;
    theirs.x = __shfl_xor(mine.x, pair_lanes, kWave);
    theirs.y = __shfl_xor(mine.y, pair_lanes, kWave);
    theirs.z = __shfl_xor(mine.z, pair_lanes, kWave);
    theirs.w = __shfl_xor(mine.w, pair_lanes, kWave);
    float other[8];
    unpack8(theirs, other);

    float o[8];
    if (lane_in_head < 2 * pair_lanes) {
      const bool first_half = lane_in_head < pair_lanes;
      const int base = (first_half ? lane_in_head : lane_in_head - pair_lanes) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float first = round_bf16((first_half ? n[j] : other[j]) * rounded_mscale);
        const float second = round_bf16((first_half ? other[j] : n[j]) * rounded_mscale);
        const float c = cos_row[base + j];
        const float s = sin_row[base + j];
        o[j] = first_half ? first * c - second * s : first * s + second * c;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = n[j];
    }
    store_nt(reinterpret_cast<u32x4*>(out) + lane_in_head, pack8(o));
  }
}

// One workgroup per token: enough lanes for every head (looping beyond 1024) and at
// least kMaxPairs, so the in-kernel angle derivation has a lane per pair.
int block_threads(int heads, int lanes_per_head) {
  int threads = heads * lanes_per_head;
  threads = (threads + kWave - 1) / kWave * kWave;
  if (threads < kMaxPairs) threads = kMaxPairs;
  return threads > 1024 ? 1024 : threads;
}

template <bool TABLE>
int32_t launch(const RopeArgs& a, int head_dim, hipStream_t stream, const char* name) {
  const int heads = a.query_heads + a.kv_heads;
  const dim3 grid(static_cast<unsigned>(a.length));
  switch (head_dim) {
    case 64:
      qk_norm_rope_kernel<64, TABLE><<<grid, block_threads(heads, 8), 0, stream>>>(a);
      break;
    case 128:
      qk_norm_rope_kernel<128, TABLE><<<grid, block_threads(heads, 16), 0, stream>>>(a);
      break;
    case 256:
      qk_norm_rope_kernel<256, TABLE><<<grid, block_threads(heads, 32), 0, stream>>>(a);
      break;
    default:
      return fail(-EINVAL, std::string(name) + ": head_dim must be 64, 128 or 256");
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
  rc = check_device();
  if (rc != 0) return rc;
  RopeArgs a{raw_queries, raw_keys, query_weight, key_weight, cos_table, sin_table,
             queries, keys, length, query_stride, key_stride, table_stride, offset,
             static_cast<int>(query_heads), static_cast<int>(kv_heads),
             static_cast<int>(rotary_pairs), eps, mscale, 0.0f};
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
  rc = check_device();
  if (rc != 0) return rc;
  RopeArgs a{fused, fused + query_heads * head_dim, query_weight, key_weight, nullptr,
             nullptr, queries, keys, length, fused_stride, fused_stride, 0, offset,
             static_cast<int>(query_heads), static_cast<int>(kv_heads),
             static_cast<int>(head_dim / 2), eps, 1.0f, log2_base};
  return launch<false>(a, static_cast<int>(head_dim), stream, "rope_epilogue");
}
