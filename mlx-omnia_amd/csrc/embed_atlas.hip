// Embedding gather + RoPE angle-atlas rows: pure copies, bit-exact by construction.
//
// Semantics (core/kernels/embed/atlas.py:23-69 and embed/default.py:35-42, generalised
// from one token to a segment):
//   hidden_out[i]  = embedding[tokens[i]]            i < n_tokens   (bf16 rows)
//   full_out[j]    = full_atlas[position + j]        j < n_positions (fp32 rows)
//   sliding_out[j] = sliding_atlas[position + j]     j < n_positions
// A token id outside [0, vocab) yields a zero row (the gather never reads outside the
// table); positions are checked on the host.
//
// Layout: one wave64 per output row. A hidden row of H bf16 is H/8 16-byte vectors,
// lane l copying vectors l, l+64, ...: every load of the row is issued before the
// first store, so a wave keeps the whole 5 KiB row (H = 2560) in flight. Waves past the
// token rows copy one position's atlas rows each. Stores are nontemporal (each output
// byte is written once); the table and atlas loads are ordinary loads, so their lines may
// stay in the 256 MB Infinity Cache between calls (the table is a parameter shared by
// every call; measured on MI355X at the config: 30.7 us with nontemporal loads, 27.2 us
// without).
#include "common.hpp"
#include "host.hpp"

namespace omnia {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kMaxVectorsPerLane = 16;  // hidden <= 8192

struct EmbedArgs {
  const int32_t* tokens;
  const u32x4* embedding;
  const f32x4* full_atlas;
  const f32x4* sliding_atlas;
  u32x4* hidden_out;
  f32x4* full_out;
  f32x4* sliding_out;
  int64_t n_tokens;
  int64_t vocab;
  int64_t position;
  int64_t n_positions;
  int vecs;           // 16-byte vectors per hidden row
  int full_vecs;      // 16-byte vectors per atlas row
  int sliding_vecs;
};

// The arguments the token rows need come first, as scalars (copies of EmbedArgs fields,
// which replace the struct's own; 11 dwords): gfx950 preloads a kernel's leading scalar
// and pointer arguments into SGPRs at wave launch, so a token wave's id load goes out with
// no scalar round trip ahead of it. The atlas rows' waves load the rest of EmbedArgs.
template <int VPL>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void embed_atlas_kernel(
    const int32_t* tokens, const u32x4* embedding, u32x4* hidden_out, int64_t n_tokens, int64_t vocab,
    int vecs, EmbedArgs a) {
  a.tokens = tokens;
  a.embedding = embedding;
  a.hidden_out = hidden_out;
  a.n_tokens = n_tokens;
  a.vocab = vocab;
  a.vecs = vecs;
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (row < a.n_tokens) {
    const int64_t id = a.tokens[row];
    const bool valid = id >= 0 && id < a.vocab;  // wave-uniform
    const u32x4* src = a.embedding + (valid ? id : 0) * a.vecs;
    u32x4* dst = a.hidden_out + row * a.vecs;
    // Every load goes out before the first store, with no branch among them (a load in a
    // branch makes the compiler wait on it): a lane past the row's end re-reads the row's
    // last vector, and an invalid id reads row 0 and writes zeros.
    u32x4 v[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = src[min(lane + i * kWave, a.vecs - 1)];
    __builtin_amdgcn_sched_barrier(0);
    const u32x4 zero{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int k = lane + i * kWave;
      if (k < a.vecs) store_nt(dst + k, valid ? v[i] : zero);
    }
    return;
  }
  const int64_t j = row - a.n_tokens;
  if (j >= a.n_positions) return;
  const int64_t p = a.position + j;
  for (int k = lane; k < a.full_vecs + a.sliding_vecs; k += kWave) {
    if (k < a.full_vecs) {
      store_nt(a.full_out + j * a.full_vecs + k, a.full_atlas[p * a.full_vecs + k]);
    } else {
      const int m = k - a.full_vecs;
      store_nt(a.sliding_out + j * a.sliding_vecs + m, a.sliding_atlas[p * a.sliding_vecs + m]);
    }
  }
}

template <int VPL>
void launch(const EmbedArgs& a, dim3 grid, hipStream_t stream) {
  embed_atlas_kernel<VPL><<<grid, kWavesPerBlock * kWave, 0, stream>>>(a.tokens, a.embedding, a.hidden_out,
                                                                      a.n_tokens, a.vocab, a.vecs, a);
}

using Launcher = void (*)(const EmbedArgs&, dim3, hipStream_t);
constexpr Launcher kLaunchers[kMaxVectorsPerLane] = {
    launch<1>,  launch<2>,  launch<3>,  launch<4>,  launch<5>,  launch<6>,
    launch<7>,  launch<8>,  launch<9>,  launch<10>, launch<11>, launch<12>,
    launch<13>, launch<14>, launch<15>, launch<16>};

}  // namespace
}  // namespace omnia

extern "C" int32_t omnia_embed_atlas(const int32_t* tokens, int64_t n_tokens,
                                     const uint16_t* embedding, int64_t vocab,
                                     int64_t hidden, const float* full_atlas,
                                     int64_t full_rows, int64_t full_width,
                                     const float* sliding_atlas, int64_t sliding_rows,
                                     int64_t sliding_width, int64_t position,
                                     int64_t n_positions, uint16_t* hidden_out,
                                     float* full_out, float* sliding_out,
                                     hipStream_t stream) {
  using namespace omnia;
  OMNIA_REQUIRE(n_tokens >= 0 && n_positions >= 0, "embed_atlas: negative count");
  OMNIA_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= 8 * kWave * kMaxVectorsPerLane,
                "embed_atlas: hidden must be a multiple of 8 in [8, 8192]");
  OMNIA_REQUIRE(vocab > 0, "embed_atlas: empty embedding table");
  OMNIA_REQUIRE(full_width >= 0 && full_width % 4 == 0 && sliding_width >= 0 &&
                    sliding_width % 4 == 0,
                "embed_atlas: atlas widths must be multiples of 4");
  OMNIA_REQUIRE(full_width / 4 + sliding_width / 4 <= (int64_t{1} << 20),
                "embed_atlas: atlas rows too wide");
  OMNIA_REQUIRE(n_positions == 0 || position >= 0, "embed_atlas: negative position");
  OMNIA_REQUIRE(n_positions == 0 || full_width == 0 || position + n_positions <= full_rows,
                "embed_atlas: positions beyond the full atlas");
  OMNIA_REQUIRE(n_positions == 0 || sliding_width == 0 ||
                    position + n_positions <= sliding_rows,
                "embed_atlas: positions beyond the sliding atlas");
  const int64_t rows = n_tokens + n_positions;
  OMNIA_REQUIRE(rows < (int64_t{1} << 31), "embed_atlas: too many rows");
  if (rows == 0) return 0;
  OMNIA_REQUIRE(n_tokens == 0 || (tokens && embedding && hidden_out),
                "embed_atlas: null token pointer");
  OMNIA_REQUIRE(n_positions == 0 || full_width == 0 || (full_atlas && full_out),
                "embed_atlas: null full atlas pointer");
  OMNIA_REQUIRE(n_positions == 0 || sliding_width == 0 || (sliding_atlas && sliding_out),
                "embed_atlas: null sliding atlas pointer");
  OMNIA_REQUIRE(aligned16(embedding) && aligned16(hidden_out) && aligned16(full_atlas) &&
                    aligned16(full_out) && aligned16(sliding_atlas) && aligned16(sliding_out),
                "embed_atlas: pointers must be 16-byte aligned");
  int32_t rc = check_device(stream);
  if (rc != 0) return rc;
  EmbedArgs a{tokens,
              reinterpret_cast<const u32x4*>(embedding),
              reinterpret_cast<const f32x4*>(full_atlas),
              reinterpret_cast<const f32x4*>(sliding_atlas),
              reinterpret_cast<u32x4*>(hidden_out),
              reinterpret_cast<f32x4*>(full_out),
              reinterpret_cast<f32x4*>(sliding_out),
              n_tokens, vocab, position, n_positions,
              static_cast<int>(hidden / 8), static_cast<int>(full_width / 4),
              static_cast<int>(sliding_width / 4)};
  const int vpl = static_cast<int>((hidden / 8 + kWave - 1) / kWave);
  const dim3 grid(static_cast<unsigned>((rows + kWavesPerBlock - 1) / kWavesPerBlock));
  kLaunchers[vpl - 1](a, grid, stream);
  return launched("embed_atlas");
}
