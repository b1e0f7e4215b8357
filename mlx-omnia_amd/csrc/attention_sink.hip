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
// takes 64 keys at a time, both products on v_mfma_f32_16x16x32_bf16:
// - scores: the G query heads (padded to 16) are the A operand, held in registers for the
//   whole chunk; 16 keys are the B operand, loaded straight from their rows (16 bytes per
//   lane); four tiles of 16 keys, two steps each. Lane l then holds heads
//   4 (l / 16) .. + 3 against key l % 16 of each tile, so a head's block maximum is a
//   reduction inside one DPP row and its running maximum is uniform over that row;
// - values: the fp32 weights, through LDS, become the A operand split into bf16 high and
//   low parts (p = hi + lo to about 2^-17 of p); the block's values, loaded 1 KiB of
//   contiguous cache per instruction and transposed through LDS, are the B operand. The
//   context accumulates in fp32 in the MFMA's output layout, the same rows (heads) as
//   the scores', so the online rescale needs no exchange.
// At the chunk's end the sums add up inside each DPP row, the four waves merge through
// LDS, and the chunk's (max, sum, context) state goes to the workspace, or, with one
// chunk, straight to the output with the sink folded in. A chunk whose mask hides every
// key does no loads. A second kernel merges the chunks of each query head and folds in
// the sink.
// Measured at gpt-oss-120b's geometry (32,768 / 4,096 rows, one call each): scores on
// v_dot2_f32_bf16 and the value sum on VALU fp32 FMAs 25.3 / 11.5 us; scores on MFMA
// 22.3 / 10.9 us; the value sum on MFMA as well 20.1 / 9.7 us, and with the LDS cut to
// 45.5 KB (three workgroups per CU) 20.3 / 9.2 us. The next block's loads issued ahead
// into a second register set were slower every time (32.8 / 12.1 over the first form,
// 21.4 / 9.4 over the last), as were twice as many chunks (24.8 / 9.4).
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

// The arguments the first loads need come first, as scalars (copies of SinkArgs fields,
// which replace the struct's own; 14 dwords): gfx950 preloads a kernel's leading scalar
// and pointer arguments into SGPRs at wave launch, so the queries' and the first block's
// loads go out with no scalar round trip ahead of them.
template <int G>
__global__ __launch_bounds__(kThreads) void sink_split_kernel(
    const uint16_t* q, const uint16_t* keys, const uint16_t* values, int64_t key_head_stride,
    int64_t value_head_stride, const float* mask, int chunk_rows, int key_length, SinkArgs a) {
  a.q = q;
  a.keys = keys;
  a.values = values;
  a.key_head_stride = key_head_stride;
  a.value_head_stride = value_head_stride;
  a.mask = mask;
  a.chunk = chunk_rows;
  a.key_length = key_length;
  constexpr int kPPitch = kBlock + 4;         // weight rows padded against bank conflicts
  constexpr int kVPitch = kBlock + 8;         // transposed value rows (bf16), padded
  // LDS: per wave a block's weights (G rows) and its values transposed; the waves'
  // final states reuse the same memory.
  constexpr int kWaveBytes = G * kPPitch * 4 + kD * kVPitch * 2;
  static_assert(kWaves * G * kPartial * 4 <= kWaves * kWaveBytes, "merge fits");
  __shared__ __align__(16) unsigned char lds[kWaves * kWaveBytes];
  __shared__ int live;
  float (*p_lds)[kPPitch] = reinterpret_cast<float (*)[kPPitch]>(lds + (threadIdx.x / kWave) * kWaveBytes);
  uint16_t (*vt_lds)[kVPitch] =
      reinterpret_cast<uint16_t (*)[kVPitch]>(lds + (threadIdx.x / kWave) * kWaveBytes + G * kPPitch * 4);
  float (*merge_lds)[G][kPartial] = reinterpret_cast<float (*)[G][kPartial]>(lds);
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int chunk = blockIdx.x;
  const int kvh = blockIdx.y;
  const int j0 = chunk * a.chunk;
  const int j1 = min(j0 + a.chunk, a.key_length);
  const int n = lane % 16;    // MFMA layouts: key (scores) / query row (operands) / element
  const int r = lane / 16;    // DPP row: heads 4 r .. 4 r + 3 of the outputs
  const int kg = lane / 8;    // value loads: key group
  const int g = lane % 8;     // value loads: element slice

  // The queries as the MFMA A operand: lane l holds head l % 16's elements
  // 8 (l / 16) + 32 kk .. + 8 (rows past the group's G heads are zero).
  bf16x8 qa[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const u32x4 q = n < G ? reinterpret_cast<const u32x4*>(a.q + static_cast<int64_t>(kvh * G + n) * kD)[r + 4 * kk]
                          : u32x4{0u, 0u, 0u, 0u};
    qa[kk] = __builtin_bit_cast(bf16x8, q);
  }
  // Whether any row of the chunk is unmasked: always without a mask (no check, so the
  // queries' loads stay in flight into the first block's); with one, through LDS behind
  // barriers that order LDS only.
  bool attends = true;
  if (a.mask != nullptr) {   // uniform
    if (threadIdx.x == 0) live = 0;
    lds_barrier();
    bool any = false;
    for (int j = j0 + static_cast<int>(threadIdx.x); j < j1; j += kThreads) any |= !__builtin_isinf(a.mask[j]);
    if (any) live = 1;   // every writer stores the same value
    lds_barrier();
    attends = live != 0;
  }

  // State of heads 4 r + i (the MFMA output rows of the lane): the running maximum m
  // (uniform over the DPP row), the lane's part of the sum l, and the context o[dt][i],
  // element 16 dt + n.
  float m[4], l[4];
  f32x4 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
    o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  if (attends) {
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
      // SinkArgs' remaining fields taken here, behind the block's loads, one wait for all
      // (loop-invariant: their loads go out ahead of the loop); each was otherwise loaded
      // at its first use, the outputs' at the end, a scalar round trip there.
      asm volatile("" ::"s"(a.scale), "s"(a.sinks), "s"(a.partial), "s"(a.out));
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
      // The values, transposed through LDS: element d of key j at vt_lds[d][j - base].
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const uint32_t a0 = (d & 1) ? (v[e][d / 2] >> 16) : (v[e][d / 2] & 0xFFFFu);
          const uint32_t a1 = (d & 1) ? (v[e + 1][d / 2] >> 16) : (v[e + 1][d / 2] & 0xFFFFu);
          w[e / 2] = a0 | (a1 << 16);
        }
        *reinterpret_cast<u32x4*>(&vt_lds[8 * g + d][8 * kg]) = u32x4{w[0], w[1], w[2], w[3]};
      }
      // The block's maximum per head: over the four tiles in the lane, then over the
      // sixteen keys of the DPP row; then the weights and the rescale of the context.
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
          if (4 * r + i < G) p_lds[4 * r + i][16 * t + n] = p;
        }
        l[i] = l[i] * corr + sum;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt][i] *= corr;
      }
      __builtin_amdgcn_wave_barrier();
      // o += P V on the MFMA: P (head l % 16, keys 8 (l / 16) + 32 ks .. + 8) split into
      // bf16 high and low parts as the A operand (rows past the G heads zero), the
      // transposed values as the B operand.
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int row = n < G ? n : 0;
        const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4 p0 = n < G ? *reinterpret_cast<const f32x4*>(&p_lds[row][32 * ks + 8 * r]) : zero;
        const f32x4 p1 = n < G ? *reinterpret_cast<const f32x4*>(&p_lds[row][32 * ks + 8 * r + 4]) : zero;
        const float pf[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          hi[e / 2] = pack_bf16(pf[e], pf[e + 1]);
          lo[e / 2] = pack_bf16(pf[e] - bf16_lo(hi[e / 2]), pf[e + 1] - bf16_hi(hi[e / 2]));
        }
        const bf16x8 pa_hi = __builtin_bit_cast(bf16x8, u32x4{hi[0], hi[1], hi[2], hi[3]});
        const bf16x8 pa_lo = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], lo[2], lo[3]});
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const u32x4 vb = *reinterpret_cast<const u32x4*>(&vt_lds[16 * dt + n][32 * ks + 8 * r]);
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa_hi, __builtin_bit_cast(bf16x8, vb), o[dt], 0, 0, 0);
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa_lo, __builtin_bit_cast(bf16x8, vb), o[dt], 0, 0, 0);
        }
      }
      // The next block overwrites the weights and values only after every lane has read them.
      __builtin_amdgcn_wave_barrier();
    }
  }

  // The wave's state: l over the sixteen lanes of each DPP row; o is whole per lane. The
  // states go to LDS the blocks used, once every wave is done with its blocks.
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x = l[i];
    x += __uint_as_float(dpp<kRowRor8>(__float_as_uint(x)));
    x += __uint_as_float(dpp<kRowRor4>(__float_as_uint(x)));
    x += __uint_as_float(dpp<kRowRor2>(__float_as_uint(x)));
    x += __uint_as_float(dpp<kRowRor1>(__float_as_uint(x)));
    const int h = 4 * r + i;
    if (h < G) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) merge_lds[wave][h][16 * dt + n] = o[dt][i];
      if (n == 0) {
        merge_lds[wave][h][kD] = m[i];
        merge_lds[wave][h][kD + 1] = x;
      }
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
// The arguments the first loads need come first, as scalars (copies of SinkArgs fields,
// which replace the struct's own), preloaded into SGPRs at wave launch.
template <int G>
__global__ __launch_bounds__(kThreads) void sink_combine_kernel(float* states, const uint16_t* sinks,
                                                                 int chunks, SinkArgs a) {
  a.partial = states;
  a.sinks = sinks;
  a.chunks = chunks;
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
  // Every load goes out before anything waits, in the order they are used: each lane's
  // first chunk (max, sum) pair and the sink, then the wave's first batch of context
  // values (wave w sums chunks w, w + kWaves, ... in that order, kBatch a pass). Every
  // wave computes the factors (so no load is used on one wave's path alone, where the
  // compiler would sink it); wave 0 stores them.
  const float2 first_ms = *reinterpret_cast<const float2*>(base + min(lane, a.chunks - 1) * stride + kD);
  const uint16_t sink_bits = a.sinks[head];
  constexpr int kBatch = 8;
  float values[kBatch];
  auto load_values = [&](int c0) {
#pragma unroll
    for (int i = 0; i < kBatch; ++i) values[i] = base[min(c0 + kWaves * i, a.chunks - 1) * stride + lane];
  };
  load_values(wave);
  // The running maximum over the sink and the chunks, lane by lane in chunk order.
  const float sink = bf16_to_f32(sink_bits) * kLog2e;
  float top = sink;
  if (lane < a.chunks) top = fmaxf(top, first_ms.x);
  for (int c = lane + kWave; c < a.chunks; c += kWave) top = fmaxf(top, base[c * stride + kD]);
  top = wave_max_f32(top);
  const float first_f =
      lane < a.chunks && first_ms.x != -INFINITY ? __builtin_amdgcn_exp2f(first_ms.x - top) : 0.0f;
  float total = lane < a.chunks ? __builtin_fmaf(first_ms.y, first_f, 0.0f) : 0.0f;
  if (wave == 0 && lane < a.chunks) factor[lane] = first_f;
  for (int c = lane + kWave; c < a.chunks; c += kWave) {   // past 64 chunks
    const float mc = base[c * stride + kD];
    const float f = mc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc - top);
    if (wave == 0) factor[c] = f;
    total = __builtin_fmaf(base[c * stride + kD + 1], f, total);
  }
  total = wave_sum_f32(total) + __builtin_amdgcn_exp2f(sink - top);
  if (wave == 0 && lane == 0) shared_total = total;
  __syncthreads();
  float acc = 0.0f;
  for (int c0 = wave; c0 < a.chunks; c0 += kWaves * kBatch) {   // uniform over the wave
    if (c0 != wave) load_values(c0);
    float factors[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int c = min(c0 + kWaves * i, a.chunks - 1);
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
                         stream>>>(a.q, a.keys, a.values, a.key_head_stride, a.value_head_stride, a.mask,
                                   a.chunk, a.key_length, a);
  if (a.chunks > 1) {
    sink_combine_kernel<G><<<dim3(static_cast<unsigned>(kv_heads * G)), kThreads, 0, stream>>>(
        a.partial, a.sinks, a.chunks, a);
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
