// One decode step of an attention layer over a KV cache: per-head RMSNorm of the new
// query and key rows, the half-split rotation, the write of the new key/value row into
// the cache, and the attention of every query head over the cache rows written so far.
//
// Arithmetic (core/kernels/attention/full.py:133-471, sliding.py:136-430 for the ring;
// the Core chain core/kernels/attention/default.py:114-156):
//   n      = bf16(w * bf16(x * inv)), inv = 1 / sqrt(sum x^2 / 128 + eps)   per head
//   a, b   = bf16(n_p * bf16(mscale)), bf16(n_{p+P} * bf16(mscale))         p < P
//   q_p    = bf16(a cos - b sin), q_{p+P} = bf16(a sin + b cos), the tail n_d (d >= 2P)
//   the same for the new key row; the value row is stored as given;
//   s_r    = scale * (q . k_r),  o = sum_r softmax(s)_r v_r  over the attended rows,
//   scores, softmax and accumulators in fp32; the context rounds to bf16 once.
//
// Cache geometry. key_cache / value_cache are [kv_heads, capacity, 128] bf16. The step's
// position p is read on the device (so a captured graph replays it), and decides:
//   fixed cache (window 0):  write row p, attend rows [0, p]
//   ring (window = capacity): write row p % window, attend rows [0, min(p + 1, window))
// `max_rows` bounds the attended rows; it sizes the grid.
//
// Layout. A workgroup (4 waves) owns one kv head and one chunk of cache rows, a multiple
// of 128; all `gqa` query heads of that kv head attend through it, so every key and value
// byte is read once per step. A wave walks blocks of 32 rows. Scores come from
// v_mfma_f32_16x16x32_bf16 (the query heads as M, 16 cache rows as N, four steps over the
// 128 dimensions); the running max is uniform over the wave, and the weights pass
// through LDS to the value layout, where lane c of each 16-lane DPP row holds elements
// [8c, 8c + 8) of a row and the wave's four DPP rows take rows 4j + 0..3 (one load
// instruction reads 1 KiB of contiguous values). The four DPP rows' context slices add
// through permlane swaps, the four waves merge through LDS. With one chunk the
// workgroup writes the context; with several it writes (max, sum, context) to the
// workspace and a second kernel merges the chunks of each query head.
//
// The chunk holding the write row computes the new key row itself and reads that row
// from LDS, never from the cache line it has just written.
#include <mutex>
#include <string>

#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kD = 128;
constexpr int kWaves = 4;
constexpr int kBlockRows = 32;                        // rows per wave iteration
constexpr int kChunkUnit = kWaves * kBlockRows;       // a chunk is a multiple of 128 rows
constexpr int kPartial = kD + 2;                      // context slice, max, sum
constexpr int kTargetGroups = 512;                    // workgroups a long cache is split into
constexpr int kMaxSplits = 1024;                      // chunks per kv head at most
constexpr int kCombineWaves = 16;                     // waves merging one query head
constexpr int kKeyPitch = kD + 8;                     // bf16; a key tile row in LDS, padded
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* raw_q;      // [heads, 128]
  const uint16_t* raw_k;      // [kv_heads, 128]
  const uint16_t* raw_v;      // [kv_heads, 128]
  const uint16_t* q_weight;   // [128]
  const uint16_t* k_weight;   // [128]
  const float* angles;        // [angle_rows, 2 * pairs]: cos || sin per position
  uint16_t* k_cache;          // [kv_heads, capacity, 128]
  uint16_t* v_cache;
  const int32_t* position;
  float* partial;             // [kv_heads, splits, gqa, kPartial]
  uint16_t* out;              // [heads, 128]
  int angle_rows;
  int pairs;
  float mscale;
  int capacity;
  int window;                 // 0: fixed cache
  int max_rows;
  int kv_heads;
  float scale_log2;           // scale * log2(e)
  float eps;
  int chunk;                  // rows per workgroup
  int splits;                 // chunks per kv head
};

struct StepRows {
  int position;
  int write;                  // the row the new key/value land in, or -1
  int count;                  // rows [0, count) are attended
};

__device__ __forceinline__ StepRows step_rows(const AttnArgs& a, int position) {
  StepRows r;
  r.position = position;
  if (r.position < 0) {
    r.write = -1;
    r.count = 0;
  } else if (a.window > 0) {
    r.write = r.position % a.window;
    r.count = min(r.position + 1, a.window);
  } else {
    r.write = r.position < a.capacity ? r.position : -1;
    r.count = min(r.position + 1, a.capacity);
  }
  r.count = min(r.count, a.max_rows);
  if (r.write >= r.count) r.write = -1;
  return r;
}
__device__ __forceinline__ StepRows step_rows(const AttnArgs& a) { return step_rows(a, *a.position); }

__device__ __forceinline__ float row16_fsum(float v) {
  v += __uint_as_float(dpp<kRowRor8>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor4>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp<kRowRor1>(__float_as_uint(v)));
  return v;
}

__device__ __forceinline__ float row16_fmax(float v) {
  v = fmaxf(v, __uint_as_float(dpp<kRowRor8>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp<kRowRor4>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp<kRowRor2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp<kRowRor1>(__float_as_uint(v))));
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_fmax(v);
  uint32_t lo, hi;
  row_pair(__float_as_uint(v), lo, hi);
  v = fmaxf(__uint_as_float(lo), __uint_as_float(hi));
  half_pair(__float_as_uint(v), lo, hi);
  return fmaxf(__uint_as_float(lo), __uint_as_float(hi));
}

__device__ __forceinline__ float wave_total(float v) {
  v = row16_fsum(v);
  uint32_t lo, hi;
  row_pair(__float_as_uint(v), lo, hi);
  v = __uint_as_float(lo) + __uint_as_float(hi);
  half_pair(__float_as_uint(v), lo, hi);
  return __uint_as_float(lo) + __uint_as_float(hi);
}

// Merge two online-softmax states (running max m, sum l, context slice o). Both lanes of
// a swap pair call it with the same (lower, upper) order, so they end bit-identical.
template <int N>
__device__ __forceinline__ void merge_state(float& m, float& l, float (&o)[N], float m2,
                                            float l2, const float (&o2)[N]) {
  const float mx = fmaxf(m, m2);
  const float f1 = m == mx ? 1.0f : __builtin_amdgcn_exp2f(m - mx);
  const float f2 = m2 == mx ? 1.0f : __builtin_amdgcn_exp2f(m2 - mx);
  m = mx;
  l = l * f1 + l2 * f2;
#pragma unroll
  for (int e = 0; e < N; ++e) o[e] = o[e] * f1 + o2[e] * f2;
}

// RMSNorm + rotation of one 128-wide head row by a 16-lane DPP row: lane c holds elements
// [8c, 8c + 8) (raw, weight: 16-byte slices already loaded; cs, sn: the cosines and sines
// of the lane's pairs, for rotated lanes). Returns the bf16 result (already rounded) in
// `out`. Every lane of the row must call it (the rotation partner comes by a lane shuffle).
__device__ __forceinline__ void norm_rope_row(const u32x4& raw, const u32x4& weight,
                                              const float (&cs)[8], const float (&sn)[8],
                                              int pairs, bool scaled, float mscale_bf,
                                              float eps, int c, float out[8]) {
  float x[8], w[8];
  unpack8(raw, x);
  unpack8(weight, w);
  double sumsq = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) sumsq += static_cast<double>(x[j] * x[j]);
  sumsq = row16_sum(sumsq);
  const float inv = 1.0f / sqrtf(static_cast<float>(sumsq) / static_cast<float>(kD) + eps);
  float n[8];
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    float a0 = x[j] * inv, a1 = x[j + 1] * inv;
    round_pair(a0, a1);
    n[j] = w[j] * a0;
    n[j + 1] = w[j + 1] * a1;
    round_pair(n[j], n[j + 1]);
  }
  const int lanes = pairs / 8;        // lanes per rotated half (a power of two <= 8)
  const bool rotated = c < 2 * lanes;
  if (scaled && rotated) {
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      n[j] *= mscale_bf;
      n[j + 1] *= mscale_bf;
      round_pair(n[j], n[j + 1]);
    }
  }
  float partner[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) partner[j] = __shfl_xor(n[j], lanes, kWave);
  if (!rotated) {
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = n[j];
    return;
  }
  const bool first_half = c < lanes;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // a: the first-half value of the pair, b: the second-half one.
    const float av = first_half ? n[j] : partner[j];
    const float bv = first_half ? partner[j] : n[j];
    out[j] = first_half ? av * cs[j] - bv * sn[j] : av * sn[j] + bv * cs[j];
  }
#pragma unroll
  for (int j = 0; j < 8; j += 2) round_pair(out[j], out[j + 1]);
}

// A block of 32 cache rows: lane (drow, c) loads row b0 + 4j + drow, dimensions
// 8c .. + 8, of the keys (k[j]) and of the values (v[j]), so one load instruction reads
// 1 KiB of contiguous cache. The keys are turned into the score MFMAs' operand layout
// through LDS (consume_block). Rows at or past `bound` (1 <= bound <= max_rows <=
// capacity) re-read row bound - 1: such rows are past the attended count, so the masked
// consume drops their scores and zeroes their values, or they are never consumed. No
// branch: with one per row, the compiler copied a loaded row to another register inside
// its branch, which waited for that row's data before the next rows' loads went out.
__device__ __forceinline__ void load_block(const AttnArgs& a, int64_t head_base, int b0, int bound,
                                           int drow, int c, u32x4 (&k)[8], u32x4 (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = min(b0 + 4 * j + drow, bound - 1);
    k[j] = load_nt(reinterpret_cast<const u32x4*>(a.k_cache + (head_base + r) * kD + 8 * c));
    v[j] = load_nt(reinterpret_cast<const u32x4*>(a.v_cache + (head_base + r) * kD + 8 * c));
  }
}

// The uniform running max of head h, picked per lane for the heads 4 drow + i it scores.
template <int GQA>
__device__ __forceinline__ float head_value(const float (&x)[GQA], int drow, int i) {
  float out = x[i < GQA ? i : 0];
#pragma unroll
  for (int h = 4; h < GQA; h += 4) {
    if (drow == h / 4) out = x[h + i];
  }
  return out;
}

// One block of 32 rows into the wave's online softmax. Scores: q (A operand: head c,
// dimensions 32 kk + 8 drow) times the key tile (B operand) on v_mfma_f32_16x16x32_bf16,
// four steps over the 128 dimensions; the result gives lane (drow, c) the scores of heads
// 4 drow + i for row c of the tile. The running max is uniform over the wave; the
// weights p pass through LDS to the value layout, where each lane accumulates its slice.
// MASKED: rows at or past c1 drop out (score -inf, value zero).
template <int GQA, bool MASKED>
__device__ __forceinline__ void consume_block(const u32x4 (&kb)[8], u32x4 (&vb)[8],
                                              const bf16x8 (&qa)[4], float (&m)[GQA],
                                              float (&lsum)[4], float (&o)[GQA][8],
                                              float (*p_lds)[4 * ((GQA + 3) / 4)], uint16_t* kt_lds,
                                              float scale_log2, int b0, int drow, int c, int c1) {
  constexpr int kPitch = 4 * ((GQA + 3) / 4);
  // The key block into the wave's LDS tile (rows padded to 272 bytes, so the 16 rows an
  // operand read touches fall on different banks), read back as the B operand: lane
  // (drow, c) takes row 16t + c, dimensions 32 kk + 8 drow .. + 8. Loading the operand
  // layout straight from HBM (16 rows per instruction) measured 32.8 us at 32k rows,
  // against 32.0 us this way.
#pragma unroll
  for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4*>(kt_lds + (4 * j + drow) * kKeyPitch + 8 * c) = kb[j];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float s[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 kt = *reinterpret_cast<const u32x4*>(kt_lds + (16 * t + c) * kKeyPitch + 32 * kk + 8 * drow);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[kk], __builtin_bit_cast(bf16x8, kt), acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[t][i] = acc[i] * scale_log2;
      if constexpr (MASKED) s[t][i] = b0 + 16 * t + c < c1 ? s[t][i] : -INFINITY;
    }
  }
  // Block max per head: over the two tiles in the lane, then over the 16 rows (lanes).
  float bmax[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bmax[i] = row16_fmax(fmaxf(s[0][i], s[1][i]));
  float f[GQA];
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    const float bm = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(bmax[h % 4]), 16 * (h / 4)));
    const float mx = fmaxf(m[h], bm);
    f[h] = m[h] == mx ? 1.0f : __builtin_amdgcn_exp2f(m[h] - mx);
    m[h] = mx;
  }
  // Weights of the lane's heads for its two rows; partial sums stay per lane.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float mh = head_value(m, drow, i);
    const float fh = head_value(f, drow, i);
    float p0, p1;
    if constexpr (MASKED) {
      p0 = s[0][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[0][i] - mh);
      p1 = s[1][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[1][i] - mh);
    } else {
      p0 = __builtin_amdgcn_exp2f(s[0][i] - mh);
      p1 = __builtin_amdgcn_exp2f(s[1][i] - mh);
    }
    lsum[i] = lsum[i] * fh + (p0 + p1);
    s[0][i] = p0;
    s[1][i] = p1;
  }
  if (4 * drow < GQA) {
    *reinterpret_cast<f32x4*>(&p_lds[c][4 * drow]) = f32x4{s[0][0], s[0][1], s[0][2], s[0][3]};
    *reinterpret_cast<f32x4*>(&p_lds[16 + c][4 * drow]) = f32x4{s[1][0], s[1][1], s[1][2], s[1][3]};
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // Values: rescale, then add p * v for the lane's rows 4j + drow.
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] *= f[h];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (MASKED) {
      if (b0 + 4 * j + drow >= c1) vb[j] = u32x4{0u, 0u, 0u, 0u};  // never-written rows
    }
    float vf[8];
    unpack8(vb[j], vf);
    float pw[kPitch];
#pragma unroll
    for (int h4 = 0; h4 < kPitch; h4 += 4) {
      const f32x4 w4 = *reinterpret_cast<const f32x4*>(&p_lds[4 * j + drow][h4]);
      pw[h4] = w4[0];
      pw[h4 + 1] = w4[1];
      pw[h4 + 2] = w4[2];
      pw[h4 + 3] = w4[3];
    }
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = __builtin_fmaf(pw[h], vf[e], o[h][e]);
    }
  }
  // The next block overwrites p_lds only after every lane has read this one.
  __builtin_amdgcn_wave_barrier();
}

// The arguments the first loads need come first, as scalars (copies of AttnArgs fields,
// which replace the struct's own): gfx950 preloads a kernel's leading scalar and pointer
// arguments into SGPRs at wave launch, so the prologue rows' and the first cache block's
// loads go out with no scalar round trip ahead of them. As values they also keep the
// per-lane choice between the key and value rows a select of two registers: on the
// struct it was a vector load of the chosen pointer from the argument segment, waited on
// before the row's own load.
template <int GQA, bool SCALED, bool PREFETCH = (GQA <= 4)>
__global__ __launch_bounds__(kWaves * kWave) void attention_split_kernel(
    const uint16_t* raw_q, const uint16_t* raw_k, const uint16_t* raw_v, uint16_t* k_cache,
    uint16_t* v_cache, int capacity, int chunk, int max_rows, AttnArgs a) {
  a.raw_q = raw_q;
  a.raw_k = raw_k;
  a.raw_v = raw_v;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.capacity = capacity;
  a.chunk = chunk;
  a.max_rows = max_rows;
  constexpr int kPitch = 4 * ((GQA + 3) / 4);
  __shared__ u32x4 q_lds[GQA][16];      // the roped queries, bf16 pairs
  __shared__ u32x4 kv_lds[2][16];       // the new key and value rows
  __shared__ float merge_lds[kWaves][GQA][kPartial];
  __shared__ __align__(16) float p_lds[kWaves][kBlockRows][kPitch];  // a block's weights
  __shared__ __align__(16) uint16_t kt_lds[kWaves][kBlockRows * kKeyPitch];  // a block's keys

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int drow = lane / 16;           // DPP row of the lane
  const int c = lane % 16;              // tile row (scores) / 8-element slice (values)
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int c0 = split * a.chunk;
  const int64_t head_base = static_cast<int64_t>(kvh) * a.capacity;

  // Everything that does not depend on the device-side position goes out before it is
  // known. Prologue inputs: item i = wave * 4 + drow; items [0, GQA) are the query heads,
  // GQA the new key row, GQA + 1 the new value row (used only in the chunk holding the
  // write row, read by every chunk: 512 bytes from L2). Then the wave's first block of
  // cache rows, bounded by max_rows (rows past the attended count are masked when the
  // block is consumed; the write row is read stale and replaced from LDS before use).
  // Measured at 32k and 4k rows: 0.4-0.5 us less than loading after the position.
  // The item's loads carry no branch (in a divergent branch the compiler waits for one
  // branch's load before the other's, a round trip ahead of the cache rows): items past
  // GQA + 1 read the value row as well and leave it unused.
  const int item = wave * 4 + drow;
  const bool is_q = item < GQA;
  const uint16_t* row = is_q ? a.raw_q + static_cast<int64_t>(kvh * GQA + min(item, GQA - 1)) * kD
                             : (item == GQA ? a.raw_k : a.raw_v) + static_cast<int64_t>(kvh) * kD;
  const u32x4 raw = *reinterpret_cast<const u32x4*>(row + 8 * c);
  u32x4 kcur[8], vcur[8];
  int b0 = c0 + wave * kBlockRows;
  load_block(a, head_base, b0, min(c0 + a.chunk, a.max_rows), drow, c, kcur, vcur);
  __builtin_amdgcn_sched_barrier(0);   // the loads above ahead of any wait for AttnArgs
  // The norm weight after the block (it is used only once the position is known). The
  // AttnArgs fields the prologue uses next are taken together, so one wait covers them:
  // the two weight pointers as values (the per-lane choice between the struct's fields
  // was otherwise a vector load of the chosen pointer from the argument segment) and the
  // window (otherwise loaded in a branch after the position arrived). Taking the score
  // scale, eps and split count here as well measured 0.2 us slower at 4k rows.
  const uint16_t* q_weight = a.q_weight;
  const uint16_t* k_weight = a.k_weight;
  int window = a.window;
  asm("" : "+s"(q_weight), "+s"(k_weight), "+s"(window));
  a.window = window;
  // (A global-memory pointer again: through the opaque values it was a flat load, which
  // the scalar-load wait for the position would also have waited on.)
  using GlobalVector = __attribute__((address_space(1))) const u32x4;
  const u32x4 wgt = *(GlobalVector*)((is_q ? q_weight : k_weight) + 8 * c);

  // The angle row at the host's bound (max_rows - 1, the position whenever the host
  // knows it) goes out before the position is read; a different position reloads.
  const int lanes = a.pairs / 8;
  const int aoff = 8 * (c < lanes ? c : (c < 2 * lanes ? c - lanes : 0));
  const int guess = min(a.max_rows - 1, a.angle_rows - 1);
  f32x4 ga[4];
  {
    const float* angle = a.angles + static_cast<int64_t>(guess) * 2 * a.pairs + aoff;
    ga[0] = *reinterpret_cast<const f32x4*>(angle);
    ga[1] = *reinterpret_cast<const f32x4*>(angle + 4);
    ga[2] = *reinterpret_cast<const f32x4*>(angle + a.pairs);
    ga[3] = *reinterpret_cast<const f32x4*>(angle + a.pairs + 4);
  }
  const StepRows rows = step_rows(a);
  if (c0 >= rows.count) return;         // whole workgroup, before any barrier
  const int c1 = min(c0 + a.chunk, rows.count);
  const bool writer = rows.write >= c0 && rows.write < c1;
  const bool norm_item = is_q || (item == GQA && writer);
  const bool value_item = item == GQA + 1 && writer;
  const int arow = min(max(rows.position, 0), a.angle_rows - 1);
  if (arow != guess) {                  // uniform: the position is the same everywhere
    const float* angle = a.angles + static_cast<int64_t>(arow) * 2 * a.pairs + aoff;
    ga[0] = *reinterpret_cast<const f32x4*>(angle);
    ga[1] = *reinterpret_cast<const f32x4*>(angle + 4);
    ga[2] = *reinterpret_cast<const f32x4*>(angle + a.pairs);
    ga[3] = *reinterpret_cast<const f32x4*>(angle + a.pairs + 4);
  }
  float cs[8], sn[8];
  const bool rotates = norm_item && c < 2 * lanes;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    cs[j] = rotates ? ga[0][j] : 0.0f;
    cs[4 + j] = rotates ? ga[1][j] : 0.0f;
    sn[j] = rotates ? ga[2][j] : 0.0f;
    sn[4 + j] = rotates ? ga[3][j] : 0.0f;
  }

  if (norm_item) {
    float r[8];
    norm_rope_row(raw, wgt, cs, sn, a.pairs, SCALED, round_bf16(a.mscale), a.eps, c, r);
    const u32x4 packed = pack8(r);
    if (is_q) {
      q_lds[item][c] = packed;
    } else {
      kv_lds[0][c] = packed;
      *reinterpret_cast<u32x4*>(a.k_cache + (head_base + rows.write) * kD + 8 * c) = packed;
    }
  } else if (value_item) {
    kv_lds[1][c] = raw;
    *reinterpret_cast<u32x4*>(a.v_cache + (head_base + rows.write) * kD + 8 * c) = raw;
  }
  __syncthreads();

  // The A operand: head c (zero past the group), dimensions 32 kk + 8 drow .. + 8.
  bf16x8 qa[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const u32x4 q = c < GQA ? q_lds[c < GQA ? c : 0][4 * kk + drow] : u32x4{0u, 0u, 0u, 0u};
    qa[kk] = __builtin_bit_cast(bf16x8, q);
  }

  float m[GQA], lsum[4], o[GQA][8];
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    m[h] = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) lsum[i] = 0.0f;

  // Blocks of the wave: b0, b0 + 128, ... With PREFETCH (the register budget allows a
  // second buffer) the next block's loads are issued before the current one is consumed,
  // the two buffers taking turns. Only the chunk's last, partial block runs the masked
  // form.
  constexpr int kStride = kWaves * kBlockRows;
  auto run = [&](u32x4 (&kb)[8], u32x4 (&vb)[8]) {
    if (writer && rows.write >= b0 && rows.write < b0 + kBlockRows) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (b0 + 4 * j + drow == rows.write) {
          kb[j] = kv_lds[0][c];
          vb[j] = kv_lds[1][c];
        }
      }
    }
    if (b0 + kBlockRows <= c1) {
      consume_block<GQA, false>(kb, vb, qa, m, lsum, o, p_lds[wave], kt_lds[wave], a.scale_log2, b0, drow, c, c1);
    } else {
      consume_block<GQA, true>(kb, vb, qa, m, lsum, o, p_lds[wave], kt_lds[wave], a.scale_log2, b0, drow, c, c1);
    }
  };
  if constexpr (PREFETCH) {
    u32x4 knext[8], vnext[8];
    while (b0 < c1) {
      load_block(a, head_base, b0 + kStride, c1, drow, c, knext, vnext);
      run(kcur, vcur);
      b0 += kStride;
      if (b0 >= c1) break;
      load_block(a, head_base, b0 + kStride, c1, drow, c, kcur, vcur);
      run(knext, vnext);
      b0 += kStride;
    }
  } else {
    for (; b0 < c1; b0 += kStride) {
      run(kcur, vcur);
      load_block(a, head_base, b0 + kStride, c1, drow, c, kcur, vcur);
    }
  }

  // The wave's state: the max is uniform already; the sums add over the 16 lanes of each
  // DPP row (rows of the tiles), the context slices over the four DPP rows.
  float l[GQA];
#pragma unroll
  for (int i = 0; i < 4; ++i) lsum[i] = row16_fsum(lsum[i]);
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    l[h] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(lsum[h % 4]), 16 * (h / 4)));
  }
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t lo, hi;
      row_pair(__float_as_uint(o[h][e]), lo, hi);
      float v = __uint_as_float(lo) + __uint_as_float(hi);
      half_pair(__float_as_uint(v), lo, hi);
      o[h][e] = __uint_as_float(lo) + __uint_as_float(hi);
    }
    if (drow == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) merge_lds[wave][h][8 * c + e] = o[h][e];
      if (c == 0) {
        merge_lds[wave][h][kD] = m[h];
        merge_lds[wave][h][kD + 1] = l[h];
      }
    }
  }
  __syncthreads();

  // Merge the four waves (in wave order) and emit: thread t serves elements of the heads.
  for (int idx = threadIdx.x; idx < GQA * kD; idx += kWaves * kWave) {
    const int g = idx / kD;
    const int e = idx % kD;
    float mm = merge_lds[0][g][kD], ll = merge_lds[0][g][kD + 1];
    float oo[1] = {merge_lds[0][g][e]};
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      const float o2[1] = {merge_lds[w][g][e]};
      merge_state(mm, ll, oo, merge_lds[w][g][kD], merge_lds[w][g][kD + 1], o2);
    }
    if (a.splits == 1) {
      const float value = ll == 0.0f ? oo[0] : oo[0] / ll;
      a.out[static_cast<int64_t>(kvh * GQA + g) * kD + e] = f32_to_bf16(value);
    } else {
      float* slot = a.partial + ((static_cast<int64_t>(kvh) * a.splits + split) * GQA + g) * kPartial;
      slot[e] = oo[0];
      if (e == 0) {
        slot[kD] = mm;
        slot[kD + 1] = ll;
      }
    }
  }
}

// One workgroup of kCombineWaves waves per query head merges the chunks' states. Wave w
// takes chunks w, w + kCombineWaves, ... and merges them online (at the configured sizes a
// wave has at most four, all loaded at once); wave 0 then merges the waves' states in
// wave order and normalises.
// Every AttnArgs field the kernel uses comes first, as a scalar (copies that replace the
// struct's own; 11 dwords): gfx950 preloads a kernel's leading scalar and pointer
// arguments into SGPRs at wave launch, so the position's and the states' loads go out
// with no scalar round trip ahead of them and the kernel loads nothing else from its
// arguments (from the struct, the row bounds took two dependent scalar round trips, one
// register being shared, and `out` a third at the store).
template <int GQA>
__global__ __launch_bounds__(kCombineWaves * kWave) void attention_combine_kernel(
    const int32_t* position_in, float* partial, uint16_t* out, int splits, int capacity, int window,
    int max_rows, int chunk, AttnArgs a) {
  a.position = position_in;
  a.partial = partial;
  a.out = out;
  a.splits = splits;
  a.capacity = capacity;
  a.window = window;
  a.max_rows = max_rows;
  a.chunk = chunk;
  __shared__ float wave_m[kCombineWaves], wave_l[kCombineWaves];
  __shared__ float2 wave_o[kCombineWaves][kWave];
  const int head = blockIdx.x;
  const int kvh = head / GQA;
  const int g = head % GQA;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const float* base = a.partial + (static_cast<int64_t>(kvh) * a.splits * GQA + g) * kPartial;
  const int64_t stride = static_cast<int64_t>(GQA) * kPartial;  // between chunks

  // A wave merges chunks wave, wave + kCombineWaves, ... in that order. Their states are
  // loaded kAhead at a time over every chunk of the split, not only the `used` ones, so
  // no load waits for the position read on the device; the unused ones (stale, from an
  // earlier step) are loaded and dropped. The position itself is a vector load issued
  // first (vector loads complete in order, so waiting for it leaves the states in flight;
  // a scalar load would be waited on with the kernel arguments, before any state load).
  constexpr int kAhead = 4;
  const int position = __hip_atomic_load(a.position, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float2 v[kAhead], ml[kAhead];
  auto load_states = [&](int s0) {
#pragma unroll
    for (int i = 0; i < kAhead; ++i) {
      const float* slot = base + min(s0 + kCombineWaves * i, a.splits - 1) * stride;
      v[i] = *reinterpret_cast<const float2*>(slot + 2 * lane);
      ml[i] = *reinterpret_cast<const float2*>(slot + kD);
    }
  };
  load_states(wave);
  const StepRows rows = step_rows(a, position);
  const int used = min(a.splits, (rows.count + a.chunk - 1) / a.chunk);
  float m = -INFINITY, l = 0.0f, o[2] = {0.0f, 0.0f};
  for (int s0 = wave; s0 < a.splits; s0 += kCombineWaves * kAhead) {   // uniform
    if (s0 != wave) load_states(s0);
#pragma unroll
    for (int i = 0; i < kAhead; ++i) {
      if (s0 + kCombineWaves * i < used) {   // uniform
        const float o2[2] = {v[i].x, v[i].y};
        merge_state(m, l, o, ml[i].x, ml[i].y, o2);
      }
    }
  }
  wave_o[wave][lane] = float2{o[0], o[1]};
  if (lane == 0) {
    wave_m[wave] = m;
    wave_l[wave] = l;
  }
  __syncthreads();
  if (wave == 0) {
    float mm = wave_m[0], ll = wave_l[0];
    float oo[2] = {wave_o[0][lane].x, wave_o[0][lane].y};
#pragma unroll
    for (int w = 1; w < kCombineWaves; ++w) {
      const float o2[2] = {wave_o[w][lane].x, wave_o[w][lane].y};
      merge_state(mm, ll, oo, wave_m[w], wave_l[w], o2);
    }
    const float v0 = ll == 0.0f ? oo[0] : oo[0] / ll;
    const float v1 = ll == 0.0f ? oo[1] : oo[1] / ll;
    reinterpret_cast<uint32_t*>(a.out + static_cast<int64_t>(head) * kD)[lane] = pack_bf16(v0, v1);
  }
}

int chunk_rows(int max_rows, int kv_heads) {
  const int per_head = (kTargetGroups + kv_heads - 1) / kv_heads;
  int chunk = (max_rows + per_head - 1) / per_head;
  chunk = max(chunk, (max_rows + kMaxSplits - 1) / kMaxSplits);  // bounds the combine loop
  chunk = (chunk + kChunkUnit - 1) / kChunkUnit * kChunkUnit;
  return chunk < kChunkUnit ? kChunkUnit : chunk;
}

template <int GQA>
void launch(const AttnArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.splits), static_cast<unsigned>(a.kv_heads));
  if (a.mscale != 1.0f) {
    attention_split_kernel<GQA, true><<<grid, kWaves * kWave, 0, stream>>>(
        a.raw_q, a.raw_k, a.raw_v, a.k_cache, a.v_cache, a.capacity, a.chunk, a.max_rows, a);
  } else {
    attention_split_kernel<GQA, false><<<grid, kWaves * kWave, 0, stream>>>(
        a.raw_q, a.raw_k, a.raw_v, a.k_cache, a.v_cache, a.capacity, a.chunk, a.max_rows, a);
  }
  if (a.splits > 1) {
    attention_combine_kernel<GQA><<<dim3(static_cast<unsigned>(a.kv_heads * GQA)), kCombineWaves * kWave, 0, stream>>>(
        a.position, a.partial, a.out, a.splits, a.capacity, a.window, a.max_rows, a.chunk, a);
  }
}

}  // namespace
}  // namespace omnia

extern "C" int64_t omnia_attention_workspace_bytes(int64_t heads, int64_t kv_heads, int64_t head_dim,
                                                   int64_t capacity) {
  using namespace omnia;
  if (heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || head_dim != kD || capacity <= 0) {
    return -EINVAL;
  }
  const int64_t splits = (capacity + kChunkUnit - 1) / kChunkUnit;
  return kv_heads * splits * (heads / kv_heads) * kPartial * static_cast<int64_t>(sizeof(float));
}

namespace omnia {
namespace {

// Checks the arguments, sizes the split and launches both kernels; `workspace` holds
// the per-chunk states when the cache is split over several workgroups per kv head.
int32_t attention_decode_checked(
    const uint16_t* raw_queries, const uint16_t* raw_keys, const uint16_t* raw_values,
    const uint16_t* query_weight, const uint16_t* key_weight, const float* angles,
    int64_t angle_rows, int64_t rotary_pairs, float mscale, uint16_t* key_cache,
    uint16_t* value_cache, int64_t capacity, int64_t window, const int32_t* position,
    int64_t max_rows, int64_t heads, int64_t kv_heads, int64_t head_dim, float scale, float eps,
    void* workspace, int64_t workspace_bytes, uint16_t* out, hipStream_t stream) {
  const int64_t gqa = heads / kv_heads;
  const int chunk = chunk_rows(static_cast<int>(max_rows), static_cast<int>(kv_heads));
  const int splits = static_cast<int>((max_rows + chunk - 1) / chunk);
  if (splits > 1) {
    const int64_t need = kv_heads * splits * gqa * kPartial * static_cast<int64_t>(sizeof(float));
    OMNIA_REQUIRE(workspace != nullptr && workspace_bytes >= need,
                  "attention_decode: workspace smaller than omnia_attention_workspace_bytes()");
    OMNIA_REQUIRE(aligned16(workspace), "attention_decode: workspace must be 16-byte aligned");
  }
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  AttnArgs a{raw_queries, raw_keys, raw_values, query_weight, key_weight, angles, key_cache,
             value_cache, position, static_cast<float*>(workspace), out,
             static_cast<int>(angle_rows), static_cast<int>(rotary_pairs), mscale,
             static_cast<int>(capacity), static_cast<int>(window), static_cast<int>(max_rows),
             static_cast<int>(kv_heads), scale * kLog2e, eps, chunk, splits};
  switch (gqa) {
    case 1: launch<1>(a, stream); break;
    case 2: launch<2>(a, stream); break;
    case 4: launch<4>(a, stream); break;
    default: launch<8>(a, stream); break;
  }
  return launched("attention_decode");
}

// The geometry checks both entry points share; 0 when the step can be served.
int32_t check_geometry(const uint16_t* raw_queries, const uint16_t* raw_keys,
                       const uint16_t* raw_values, const uint16_t* query_weight,
                       const uint16_t* key_weight, const float* angles, int64_t angle_rows,
                       int64_t rotary_pairs, const uint16_t* key_cache,
                       const uint16_t* value_cache, int64_t capacity, int64_t window,
                       const int32_t* position, int64_t max_rows, int64_t heads,
                       int64_t kv_heads, int64_t head_dim, const uint16_t* out) {
  OMNIA_REQUIRE(head_dim == kD, "attention_decode: head_dim must be 128");
  OMNIA_REQUIRE(kv_heads > 0 && heads > 0 && heads % kv_heads == 0,
                "attention_decode: heads must be a positive multiple of kv_heads");
  const int64_t gqa = heads / kv_heads;
  OMNIA_REQUIRE(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8,
                "attention_decode: heads / kv_heads must be 1, 2, 4 or 8");
  OMNIA_REQUIRE(kv_heads <= 65535, "attention_decode: too many kv heads");
  OMNIA_REQUIRE(rotary_pairs == 8 || rotary_pairs == 16 || rotary_pairs == 32 || rotary_pairs == 64,
                "attention_decode: rotary_pairs must be 8, 16, 32 or 64");
  OMNIA_REQUIRE(capacity > 0 && capacity < (int64_t{1} << 30), "attention_decode: bad capacity");
  OMNIA_REQUIRE(window == 0 || window == capacity,
                "attention_decode: a ring's window must be its capacity (0: fixed cache)");
  OMNIA_REQUIRE(max_rows > 0 && max_rows <= capacity, "attention_decode: max_rows must be in [1, capacity]");
  OMNIA_REQUIRE(angle_rows > 0 && angle_rows < (int64_t{1} << 30), "attention_decode: bad angle_rows");
  OMNIA_REQUIRE(raw_queries && raw_keys && raw_values && query_weight && key_weight && angles &&
                key_cache && value_cache && position && out, "attention_decode: null pointer");
  OMNIA_REQUIRE(aligned16(raw_queries) && aligned16(raw_keys) && aligned16(raw_values) &&
                aligned16(query_weight) && aligned16(key_weight) && aligned16(key_cache) &&
                aligned16(value_cache) && aligned16(out) && aligned16(angles),
                "attention_decode: bf16 rows and the angle table must be 16-byte aligned");
  return 0;
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_attention_decode(
    const uint16_t* raw_queries, const uint16_t* raw_keys, const uint16_t* raw_values,
    const uint16_t* query_weight, const uint16_t* key_weight, const float* angles,
    int64_t angle_rows, int64_t rotary_pairs, float mscale, uint16_t* key_cache,
    uint16_t* value_cache, int64_t capacity, int64_t window, const int32_t* position,
    int64_t max_rows, int64_t heads, int64_t kv_heads, int64_t head_dim, float scale, float eps,
    void* workspace, int64_t workspace_bytes, uint16_t* out, hipStream_t stream) {
  using namespace omnia;
  int32_t rc = check_geometry(raw_queries, raw_keys, raw_values, query_weight, key_weight, angles,
                              angle_rows, rotary_pairs, key_cache, value_cache, capacity, window,
                              position, max_rows, heads, kv_heads, head_dim, out);
  if (rc != 0) return rc;
  return attention_decode_checked(raw_queries, raw_keys, raw_values, query_weight, key_weight,
                                  angles, angle_rows, rotary_pairs, mscale, key_cache, value_cache,
                                  capacity, window, position, max_rows, heads, kv_heads, head_dim,
                                  scale, eps, workspace, workspace_bytes, out, stream);
}

// ---- the same step with the per-chunk states in a static device array ------------
//
// For callers that cannot allocate device memory (code under graph capture, serving
// loops that forbid hipMalloc). The states live in `scratch`, one array per GPU that
// the library runs on, held until the process ends. Its device address comes from
// hipGetSymbolAddress once per device, at the entry point's first call on that device;
// the host-side name `scratch` is never passed to a kernel. Every call on one GPU
// shares that GPU's array: calls that overlap on one GPU (different streams, or
// different host threads without ordering) race. Nothing in it has to start at zero:
// each chunk that the combine kernel reads is written by the split kernel first.

constexpr int64_t kAttentionScratchBytes = OMNIA_ATTENTION_SCRATCH_BYTES;

static __device__ __align__(256) float scratch[kAttentionScratchBytes / sizeof(float)];

namespace omnia {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex scratch_lock;
void* scratch_address[kMaxScratchDevices] = {};

// The current device's copy of `scratch`, looked up on the first call there.
int32_t device_scratch(void** address) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) {
    return fail(-ENODEV, std::string("hipGetDevice: ") + hipGetErrorString(status));
  }
  if (device < 0 || device >= kMaxScratchDevices) {
    return fail(-ENODEV, "attention_decode_noalloc: device ordinal out of range");
  }
  std::lock_guard<std::mutex> hold(scratch_lock);
  if (scratch_address[device] == nullptr) {
    void* found = nullptr;
    status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
    if (status != hipSuccess || found == nullptr) {
      return fail(-1, std::string("attention_decode_noalloc: hipGetSymbolAddress(scratch): ") +
                          hipGetErrorString(status));
    }
    scratch_address[device] = found;
  }
  *address = scratch_address[device];
  return 0;
}

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_attention_decode_noalloc(
    const uint16_t* raw_queries, const uint16_t* raw_keys, const uint16_t* raw_values,
    const uint16_t* query_weight, const uint16_t* key_weight, const float* angles,
    int64_t angle_rows, int64_t rotary_pairs, float mscale, uint16_t* key_cache,
    uint16_t* value_cache, int64_t capacity, int64_t window, const int32_t* position,
    int64_t max_rows, int64_t heads, int64_t kv_heads, int64_t head_dim, float scale, float eps,
    uint16_t* out, hipStream_t stream) {
  using namespace omnia;
  int32_t rc = check_geometry(raw_queries, raw_keys, raw_values, query_weight, key_weight, angles,
                              angle_rows, rotary_pairs, key_cache, value_cache, capacity, window,
                              position, max_rows, heads, kv_heads, head_dim, out);
  if (rc != 0) return rc;
  const int chunk = chunk_rows(static_cast<int>(max_rows), static_cast<int>(kv_heads));
  const int64_t splits = (max_rows + chunk - 1) / chunk;
  const int64_t need = splits > 1 ? kv_heads * splits * (heads / kv_heads) * kPartial *
                                        static_cast<int64_t>(sizeof(float))
                                  : 0;
  if (need > kAttentionScratchBytes) {
    return fail(-EINVAL, "attention_decode_noalloc: this step needs " + std::to_string(need) +
                             " bytes of chunk states, above the static scratch of " +
                             std::to_string(kAttentionScratchBytes) +
                             " bytes; use omnia_attention_decode with a workspace");
  }
  rc = check_device(stream);
  if (rc != 0) return rc;
  void* address = nullptr;
  rc = device_scratch(&address);
  if (rc != 0) return rc;
  return attention_decode_checked(raw_queries, raw_keys, raw_values, query_weight, key_weight,
                                  angles, angle_rows, rotary_pairs, mscale, key_cache, value_cache,
                                  capacity, window, position, max_rows, heads, kv_heads, head_dim,
                                  scale, eps, address, kAttentionScratchBytes, out, stream);
}
