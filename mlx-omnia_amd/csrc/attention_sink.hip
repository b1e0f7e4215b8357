// The one-token attention of a layer with learned sink logits, over a growing KV buffer:
// core/kernels/attention/sink.py:60-166 (`sink_attention`, the split-K flash-decode the
// reference's SinkAttentionStep dispatches), head_dim 64.
//
// Arithmetic (fp32, as the reference keeps the score, the softmax and the accumulation):
//   s_j   = (q . k_j) * scale + mask_j        keys whose mask is +-inf are skipped
//   out   = sum_j exp(s_j - M) v_j / (exp(sink - M) + sum_j exp(s_j - M)),
//           M = max(sink, max_j s_j), rounded once to bf16.
// The sink takes part in the denominator only. The split into key chunks changes only how
// the fp32 sums are grouped. Exponents run in log2 units (v_exp_f32).
//
// Layout. A workgroup (4 waves) owns one kv head and one chunk of keys, and serves every
// query head of that kv head, so grouped queries share each key and value load. A wave
// takes 64 keys at a time:
// - scores on v_mfma_f32_16x16x32_bf16: the G query heads (padded to 16) are the A
//   operand, held in registers for the whole chunk; 16 keys are the B operand, loaded
//   straight from their rows (16 bytes per lane); four tiles of 16 keys, two steps each;
// - lane l then holds heads 4 (l / 16) .. + 3 against key l % 16 of each tile, so a
//   head's block maximum is a reduction inside one DPP row and its running maximum is
//   uniform over that row;
// - values: the weights (and each head's rescale factor) go through LDS to a second
//   layout, lane (key group kg, slice g): keys 8 kg .. 8 kg + 7, elements 8 g .. 8 g + 7,
//   so a value load instruction reads 1 KiB of contiguous cache and each lane
//   accumulates G x 8 outputs in fp32.
// Measured at gpt-oss-120b's geometry (32,768 / 4,096 rows, one call): scores on
// v_dot2_f32_bf16 with the queries read from LDS 25.3 / 11.5 us, on MFMA 22.3 / 10.9 us;
// the next block's loads issued ahead into a second register set (occupancy 1) 32.8 /
// 12.1 us.
// At the chunk's end the eight key groups add up across lanes (DPP, permlane swaps), the
// four waves merge through LDS, and the chunk's (max, sum, context) state goes to the
// workspace, or, with one chunk, straight to the output with the sink folded in. A chunk
// whose mask hides every key does no loads. A second kernel merges the chunks of each
// query head and folds in the sink.
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kD = 64;                 // head_dim
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kBlock = kWave;          // keys per wave per step
constexpr int kPartial = kD + 2;       // context, max, sum
constexpr int kTargetGroups = 512;     // split workgroups aimed for
constexpr int kMinChunk = kWaves * kBlock;
constexpr int kMaxChunks = kTargetGroups;   // chunks per kv head, at most
constexpr float kLog2e = 1.4426950408889634f;

struct SinkArgs {
  const uint16_t* q;        // [heads, 64] bf16
  const uint16_t* keys;     // head h, row j at h * key_head_stride + j * 64
  const uint16_t* values;   // the same with value_head_stride
  int64_t key_head_stride;
  int64_t value_head_stride;
  const float* mask;        // [key_length] additive fp32, or null
  const uint16_t* sinks;    // [heads] bf16
  float* partial;           // [kv_heads, chunks, G, kPartial]
  uint16_t* out;            // [heads, 64] bf16
  int key_length;
  int chunk;
  int chunks;
  float scale;
};

// (m, l, o) <- the merge of two softmax states in log2 units (m the running maximum, l the
// sum of exp2(s - m), o the weighted values at the same scale).
template <int N>
__device__ __forceinline__ void merge_state(float& m, float& l, float (&o)[N], float m2, float l2,
                                            const float (&o2)[N]) {
  const float mx = fmaxf(m, m2);
  const float f1 = m == mx ? 1.0f : __builtin_amdgcn_exp2f(m - mx);
  const float f2 = m2 == mx ? 1.0f : __builtin_amdgcn_exp2f(m2 - mx);
  m = mx;
  l = l * f1 + l2 * f2;
#pragma unroll
  for (int e = 0; e < N; ++e) o[e] = o[e] * f1 + o2[e] * f2;
}

// The final value of one output element: the state (m, l, o) with the sink (log2 units).
__device__ __forceinline__ float with_sink(float m, float l, float o, float sink) {
  const float top = fmaxf(m, sink);
  const float f = m == top ? 1.0f : __builtin_amdgcn_exp2f(m - top);
  const float total = l * f + __builtin_amdgcn_exp2f(sink - top);
  return o * f / total;
}

template <int G>
__global__ __launch_bounds__(kThreads) void sink_split_kernel(SinkArgs a) {
  __shared__ __align__(16) float p_lds[kWaves][G][kBlock];     // a block's weights
  __shared__ __align__(16) float corr_lds[kWaves][G];          // a block's rescale factors
  __shared__ float merge_lds[kWaves][G][kPartial];
  __shared__ int live;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int chunk = blockIdx.x;
  const int kvh = blockIdx.y;
  const int j0 = chunk * a.chunk;
  const int j1 = min(j0 + a.chunk, a.key_length);
  const int n = lane % 16;    // score layout: key within a 16-key tile / query row
  const int r = lane / 16;    // score layout: DPP row, heads 4 r .. 4 r + 3
  const int kg = lane / 8;    // value layout: key group
  const int g = lane % 8;     // value layout: element slice

  // The queries as the MFMA A operand: lane l holds head l % 16's elements
  // 8 (l / 16) + 32 kk .. + 8 (rows past the group's G heads are zero).
  bf16x8 qa[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const u32x4 q = n < G ? reinterpret_cast<const u32x4*>(a.q + static_cast<int64_t>(kvh * G + n) * kD)[r + 4 * kk]
                          : u32x4{0u, 0u, 0u, 0u};
    qa[kk] = __builtin_bit_cast(bf16x8, q);
  }
  if (threadIdx.x == 0) live = 0;
  __syncthreads();
  bool any = false;
  for (int j = j0 + static_cast<int>(threadIdx.x); j < j1; j += kThreads) {
    any |= a.mask == nullptr || !__builtin_isinf(a.mask[j]);
  }
  if (any) live = 1;   // every writer stores the same value
  __syncthreads();

  // Score-layout state of heads 4 r + i: the running maximum m (uniform over the DPP row)
  // and the lane's part of the sum l. Value-layout state: o[h][d], element 8 g + d of
  // head h over the lane's key group.
  float m[4], l[4], o[G][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
  }
  if (live) {
    const uint16_t* khead = a.keys + static_cast<int64_t>(kvh) * a.key_head_stride;
    const uint16_t* vhead = a.values + static_cast<int64_t>(kvh) * a.value_head_stride;
    for (int base = j0 + wave * kBlock; base < j1; base += kWaves * kBlock) {   // uniform over the wave
      // Every load of the block goes out first, with no branch among them: a key past the
      // chunk re-reads the chunk's last row and is dropped below. Keys as the MFMA B
      // operand: tile t, lane l: key 16 t + l % 16, elements 8 (l / 16) + 32 kk .. + 8.
      u32x4 k[4][2];
      float mk[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int jk = min(base + 16 * t + n, j1 - 1);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          k[t][kk] = reinterpret_cast<const u32x4*>(khead + static_cast<int64_t>(jk) * kD)[r + 4 * kk];
        }
        mk[t] = a.mask != nullptr ? a.mask[jk] : 0.0f;
      }
      u32x4 v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int jv = min(base + 8 * kg + e, j1 - 1);
        v[e] = reinterpret_cast<const u32x4*>(vhead + static_cast<int64_t>(jv) * kD)[g];
      }
      __builtin_amdgcn_sched_barrier(0);
      // s[t][i]: head 4 r + i against key 16 t + n, in log2 units.
      float s[4][4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[kk], __builtin_bit_cast(bf16x8, k[t][kk]), acc, 0, 0, 0);
        }
        const bool valid = base + 16 * t + n < j1 && !__builtin_isinf(mk[t]);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[t][i] = valid ? (acc[i] * a.scale + mk[t]) * kLog2e : -INFINITY;
      }
      // The block's maximum per head: over the four tiles in the lane, then over the
      // sixteen keys of the DPP row.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float top = fmaxf(fmaxf(s[0][i], s[1][i]), fmaxf(s[2][i], s[3][i]));
        top = fmaxf(top, __uint_as_float(dpp<kRowRor8>(__float_as_uint(top))));
        top = fmaxf(top, __uint_as_float(dpp<kRowRor4>(__float_as_uint(top))));
        top = fmaxf(top, __uint_as_float(dpp<kRowRor2>(__float_as_uint(top))));
        top = fmaxf(top, __uint_as_float(dpp<kRowRor1>(__float_as_uint(top))));
        const float mx = fmaxf(m[i], top);
        const float corr = m[i] == mx ? 1.0f : __builtin_amdgcn_exp2f(m[i] - mx);
        m[i] = mx;
        float sum = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float p = s[t][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[t][i] - mx);
          sum += p;
          if (4 * r + i < G) p_lds[wave][4 * r + i][16 * t + n] = p;
        }
        l[i] = l[i] * corr + sum;
        if (4 * r + i < G && n == 0) corr_lds[wave][4 * r + i] = corr;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float corr = corr_lds[wave][h];
        if (corr != 1.0f) {   // uniform over the wave
#pragma unroll
          for (int d = 0; d < 8; ++d) o[h][d] *= corr;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float vf[8];
        unpack8(v[e], vf);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float p = p_lds[wave][h][8 * kg + e];
#pragma unroll
          for (int d = 0; d < 8; ++d) o[h][d] = __builtin_fmaf(p, vf[d], o[h][d]);
        }
      }
      // The next block overwrites p_lds and corr_lds only after every lane has read them.
      __builtin_amdgcn_wave_barrier();
    }
  }

  // The wave's state. l: over the sixteen lanes of each DPP row; o: over the eight key
  // groups (lanes g, g + 8, ...).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x = l[i];
    x += __uint_as_float(dpp<kRowRor8>(__float_as_uint(x)));
    x += __uint_as_float(dpp<kRowRor4>(__float_as_uint(x)));
    x += __uint_as_float(dpp<kRowRor2>(__float_as_uint(x)));
    x += __uint_as_float(dpp<kRowRor1>(__float_as_uint(x)));
    if (n == 0 && 4 * r + i < G) {
      merge_lds[wave][4 * r + i][kD] = m[i];
      merge_lds[wave][4 * r + i][kD + 1] = x;
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      float x = o[h][d];
      x += __uint_as_float(dpp<kRowRor8>(__float_as_uint(x)));
      uint32_t lo, hi;
      row_pair(__float_as_uint(x), lo, hi);
      x = __uint_as_float(lo) + __uint_as_float(hi);
      half_pair(__float_as_uint(x), lo, hi);
      o[h][d] = __uint_as_float(lo) + __uint_as_float(hi);
    }
    if (lane < 8) {
#pragma unroll
      for (int d = 0; d < 8; ++d) merge_lds[wave][h][8 * lane + d] = o[h][d];
    }
  }
  __syncthreads();

  // Merge the four waves in wave order: thread t serves element t % 64 of head t / 64.
  for (int idx = threadIdx.x; idx < G * kD; idx += kThreads) {
    const int h = idx / kD;
    const int e = idx % kD;
    float mm = merge_lds[0][h][kD], ll = merge_lds[0][h][kD + 1];
    float oo[1] = {merge_lds[0][h][e]};
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      const float o2[1] = {merge_lds[w][h][e]};
      merge_state(mm, ll, oo, merge_lds[w][h][kD], merge_lds[w][h][kD + 1], o2);
    }
    const int head = kvh * G + h;
    if (a.chunks == 1) {
      const float sink = bf16_to_f32(a.sinks[head]) * kLog2e;
      a.out[static_cast<int64_t>(head) * kD + e] = f32_to_bf16(with_sink(mm, ll, oo[0], sink));
    } else {
      float* slot = a.partial + ((static_cast<int64_t>(kvh) * a.chunks + chunk) * G + h) * kPartial;
      slot[e] = oo[0];
      if (e == 0) {
        slot[kD] = mm;
        slot[kD + 1] = ll;
      }
    }
  }
}

// One workgroup per query head. Wave 0 takes the chunks' maxima and sums lane by lane
// and leaves each chunk's factor exp2(m_c - top) in LDS; then wave w sums element `lane`
// of chunks w, w + 4, ... with their loads issued together, and wave 0 adds the four
// partial sums in wave order and folds in the sink.
template <int G>
__global__ __launch_bounds__(kThreads) void sink_combine_kernel(SinkArgs a) {
  __shared__ float factor[kMaxChunks];
  __shared__ float partial[kWaves][kD];
  __shared__ float shared_total;
  const int head = blockIdx.x;
  const int kvh = head / G;
  const int h = head % G;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const float* base = a.partial + (static_cast<int64_t>(kvh) * a.chunks * G + h) * kPartial;
  const int64_t stride = static_cast<int64_t>(G) * kPartial;   // between chunks
  if (wave == 0) {
    const float sink = bf16_to_f32(a.sinks[head]) * kLog2e;
    float top = sink;
    for (int c = lane; c < a.chunks; c += kWave) top = fmaxf(top, base[c * stride + kD]);
    top = wave_max_f32(top);
    float total = 0.0f;
    for (int c = lane; c < a.chunks; c += kWave) {
      const float mc = base[c * stride + kD];
      const float f = mc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc - top);
      factor[c] = f;
      total = __builtin_fmaf(base[c * stride + kD + 1], f, total);
    }
    total = wave_sum_f32(total) + __builtin_amdgcn_exp2f(sink - top);
    if (lane == 0) shared_total = total;
  }
  __syncthreads();
  constexpr int kBatch = 8;
  float acc = 0.0f;
  for (int c0 = wave; c0 < a.chunks; c0 += kWaves * kBatch) {   // uniform over the wave
    float values[kBatch], factors[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int c = min(c0 + kWaves * i, a.chunks - 1);
      values[i] = base[c * stride + lane];
      factors[i] = c0 + kWaves * i < a.chunks ? factor[c] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) acc = __builtin_fmaf(values[i], factors[i], acc);
  }
  partial[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    const float sum = ((partial[0][lane] + partial[1][lane]) + partial[2][lane]) + partial[3][lane];
    a.out[static_cast<int64_t>(head) * kD + lane] = f32_to_bf16(sum / shared_total);
  }
}

int chunk_keys(int key_length, int kv_heads) {
  const int per_head = (kTargetGroups + kv_heads - 1) / kv_heads;
  int chunk = (key_length + per_head - 1) / per_head;
  chunk = (chunk + kMinChunk - 1) / kMinChunk * kMinChunk;
  return chunk < kMinChunk ? kMinChunk : chunk;
}

int chunk_count(int key_length, int kv_heads) {
  const int chunk = chunk_keys(key_length, kv_heads);
  const int chunks = (key_length + chunk - 1) / chunk;
  return chunks < 1 ? 1 : chunks;
}

template <int G>
void launch(const SinkArgs& a, int kv_heads, hipStream_t stream) {
  sink_split_kernel<G><<<dim3(static_cast<unsigned>(a.chunks), static_cast<unsigned>(kv_heads)), kThreads, 0,
                         stream>>>(a);
  if (a.chunks > 1) {
    sink_combine_kernel<G><<<dim3(static_cast<unsigned>(kv_heads * G)), kThreads, 0, stream>>>(a);
  }
}

}  // namespace
}  // namespace omnia

extern "C" int64_t omnia_attention_sink_workspace_bytes(int64_t heads, int64_t kv_heads, int64_t key_length) {
  if (heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || key_length < 0 || key_length >= (int64_t{1} << 30)) {
    return -EINVAL;
  }
  const int chunks = omnia::chunk_count(static_cast<int>(key_length), static_cast<int>(kv_heads));
  return chunks == 1 ? 0 : static_cast<int64_t>(chunks) * heads * omnia::kPartial * sizeof(float);
}

extern "C" int32_t omnia_attention_sink_decode(const uint16_t* queries, const uint16_t* keys, const uint16_t* values,
                                               int64_t key_head_stride, int64_t value_head_stride, int64_t heads,
                                               int64_t kv_heads, int64_t head_dim, int64_t key_length,
                                               const float* mask, const uint16_t* sinks, float scale,
                                               void* workspace, int64_t workspace_bytes, uint16_t* out,
                                               hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(head_dim == kD, "attention_sink_decode: head_dim must be 64");
  OMNIA_REQUIRE(kv_heads > 0 && heads > 0 && heads % kv_heads == 0 && heads <= 4096,
                "attention_sink_decode: heads must be a multiple of kv_heads");
  const int64_t gqa = heads / kv_heads;
  OMNIA_REQUIRE(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8,
                "attention_sink_decode: 1, 2, 4 or 8 query heads per kv head");
  OMNIA_REQUIRE(key_length >= 0 && key_length < (int64_t{1} << 30), "attention_sink_decode: bad key length");
  OMNIA_REQUIRE(queries && sinks && out && (key_length == 0 || (keys && values)),
                "attention_sink_decode: null pointer");
  OMNIA_REQUIRE(aligned16(queries) && aligned16(keys) && aligned16(values),
                "attention_sink_decode: q, keys and values must be 16-byte aligned");
  OMNIA_REQUIRE(key_head_stride % 8 == 0 && value_head_stride % 8 == 0 && key_head_stride >= key_length * kD &&
                    value_head_stride >= key_length * kD,
                "attention_sink_decode: head strides must be multiples of 8 covering key_length rows");
  const int64_t need = omnia_attention_sink_workspace_bytes(heads, kv_heads, key_length);
  OMNIA_REQUIRE(need >= 0 && workspace_bytes >= need && (need == 0 || workspace != nullptr),
                "attention_sink_decode: workspace too small (omnia_attention_sink_workspace_bytes)");
  OMNIA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "attention_sink_decode: workspace alignment");
  OMNIA_REQUIRE(chunk_count(static_cast<int>(key_length), static_cast<int>(kv_heads)) <= kMaxChunks,
                "attention_sink_decode: too many chunks");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  SinkArgs a{queries, keys, values, key_head_stride, value_head_stride, mask, sinks,
             static_cast<float*>(workspace), out, static_cast<int>(key_length),
             chunk_keys(static_cast<int>(key_length), static_cast<int>(kv_heads)),
             chunk_count(static_cast<int>(key_length), static_cast<int>(kv_heads)), scale};
  switch (gqa) {
    case 1: launch<1>(a, static_cast<int>(kv_heads), stream); break;
    case 2: launch<2>(a, static_cast<int>(kv_heads), stream); break;
    case 4: launch<4>(a, static_cast<int>(kv_heads), stream); break;
    default: launch<8>(a, static_cast<int>(kv_heads), stream); break;
  }
  return launched("attention_sink_decode");
}
