/* omnia_hip.h — C ABI of the MI355X (gfx950) fused per-layer kernels.
 *
 * Every entry point is a drop-in for one kernel binding of mlx-omnia's Layer
 * declaration API (the strategies its facades resolve between); the reference
 * interface each one replaces is cited beside it (paths relative to the
 * mlx-omnia tree, `src/mlx_omnia/engine/` omitted).
 *
 * Conventions shared by all entry points:
 *   - bf16 tensors travel as `uint16_t` bit patterns; fp32 as `float`.
 *   - Pointers are device pointers, caller-allocated; the library never
 *     allocates, frees or caches device memory and keeps no per-call state.
 *   - Tensors are row-major. Row strides are in elements. Every bf16 row
 *     pointer and stride must keep 16-byte alignment (checked: -EINVAL).
 *   - Work is enqueued on `stream` and returns without synchronising.
 *   - Return value: 0 on success, -EINVAL (-22) for a shape, pointer or
 *     alignment the kernel does not serve, -ENODEV (-19) when the current
 *     device is not gfx950, -1 when the launch itself failed. The reason is
 *     available from omnia_last_error() on the calling thread.
 *   - A zero row count is valid and launches nothing.
 */
#ifndef OMNIA_HIP_H
#define OMNIA_HIP_H

#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OMNIA_ABI_VERSION 15

/* Version of this ABI (OMNIA_ABI_VERSION). Pure; touches no device. */
int32_t omnia_abi_version(void);

/* Text of the last error raised on the calling thread ("" if none). */
const char* omnia_last_error(void);

/* Builds rows of a rotary angle atlas on the device:
 *   atlas[r][i]         = fp32(cos(theta)),  atlas[r][pairs + i] = fp32(sin(theta)),
 *   theta = (first + r) * frequencies[i] in fp64, cos and sin in fp64, each rounded once,
 * for r < rows, i < pairs. frequencies [pairs] fp64 (device): exp(-ln(base) * i / pairs)
 * for the plain rotary, 1 / freqs for a YaRN table; atlas rows `stride` floats apart.
 * Replaces: models/laguna/layers/attention.py:171-196,235-243 (`LagunaAttention.angles`,
 * `_angle_atlas`, built once and regrown past its last row) with the fp64 build of
 * tests/test_kernel_qk_norm_rope.py:51-66. */
int32_t omnia_rope_angle_atlas(const double* frequencies, int64_t pairs, int64_t first,
                               int64_t rows, float* atlas, int64_t stride, hipStream_t stream);

/* The same atlas in the fp32 order of the reference's builder:
 *   theta[r, i] = fp32(fp32(first + r) / inverse_frequencies[i]),
 *   atlas[r, i] = fp32(cos(theta)), atlas[r, pairs + i] = fp32(sin(theta)),
 * every operation correctly rounded (quotient formed in fp64 and rounded once; cos and
 * sin of the fp32 angle evaluated in fp64 and rounded once). inverse_frequencies [pairs]
 * fp32: base ** (2i / D) as fp32 operations (or a YaRN table). Limits as above.
 * Replaces: models/laguna/layers/attention.py:236-243 (`_angle_atlas`: theta =
 * arange(rows, fp32) / inverse, then cos, sin and a concatenate), one launch. */
int32_t omnia_rope_angle_atlas_fp32(const float* inverse_frequencies, int64_t pairs,
                                    int64_t first, int64_t rows, float* atlas, int64_t stride,
                                    hipStream_t stream);

/* Residual add + RMSNorm over `rows` rows of `hidden` bf16 values.
 *   summed[r]     = bf16(x[r] + branch[r])
 *   normalized[r] = bf16(weight * bf16(summed[r] * rsqrt(mean(summed[r]^2) + eps)))
 * Replaces: core/kernels/add_norm/rows.py:48-128 (`residual_rms_norm_rows`,
 * RowsAddRmsNorm.__call__) and the Core chain it restates,
 * core/kernels/add_norm/default.py:28-29 (DefaultAddRmsNorm.__call__).
 * hidden: multiple of 8, at most 8192. */
int32_t omnia_add_rms_norm(const uint16_t* x, const uint16_t* branch,
                           const uint16_t* weight, uint16_t* summed,
                           uint16_t* normalized, int64_t rows, int64_t hidden,
                           float eps, hipStream_t stream);

/* Per-head q/k RMSNorm + table-driven half-split rotary for a segment of `length`
 * tokens at positions offset .. offset+length-1.
 *   raw_queries [length, query_heads, head_dim] (row stride `query_stride` elements),
 *   raw_keys    [length, kv_heads, head_dim]    (row stride `key_stride`),
 *   query_weight, key_weight [head_dim] bf16,
 *   cos_table, sin_table: fp32 rows of `rotary_pairs` values, `table_stride` floats
 *     apart, `table_rows` rows; row offset+t is used for token t. (The reference's
 *     `[positions, 2P]` cos||sin atlas is cos_table = atlas, sin_table = atlas + P,
 *     table_stride = 2P.)
 *   queries [query_heads, length, head_dim], keys [kv_heads, length, head_dim] out.
 * Elements [2*rotary_pairs, head_dim) are the normed values verbatim; the rotary inputs
 * are pre-scaled through bf16(x * bf16(mscale)) (pass 1.0 for a plain rotary).
 * Replaces: core/kernels/qkv_rope/qk_norm_rope.py:64-327 (`qk_norm_rope_decode`,
 * `qk_norm_rope_prefill`, `qk_norm_rope_prefill_scaled`, QkNormRope.__call__ at
 * :653-708); Core chain core/kernels/qkv_rope/default.py:75-84.
 * head_dim in {64, 128, 256}; rotary_pairs = 8 * 2^k with 2*rotary_pairs <= head_dim;
 * strides multiples of 8. */
int32_t omnia_qk_norm_rope(const uint16_t* raw_queries, int64_t query_stride,
                           const uint16_t* raw_keys, int64_t key_stride,
                           const uint16_t* query_weight, const uint16_t* key_weight,
                           const float* cos_table, const float* sin_table,
                           int64_t table_stride, int64_t table_rows, int64_t offset,
                           uint16_t* queries, uint16_t* keys, int64_t length,
                           int64_t query_heads, int64_t kv_heads, int64_t head_dim,
                           int64_t rotary_pairs, float eps, float mscale,
                           hipStream_t stream);

/* The rope epilogue of a fused qkv projection: rows of `fused` are
 * [q (query_heads*head_dim) | k (kv_heads*head_dim) | v (kv_heads*head_dim)], row
 * stride `fused_stride`. q and k are normed per head and fully rotated with the angle
 * derived in-kernel, angle_i = f32(offset + t) * exp2(-(i / (head_dim/2)) * log2_base);
 * v is not touched. Outputs are head-major like omnia_qk_norm_rope's.
 * Replaces: core/kernels/qkv_rope/epilogue.py:34-115 (`rope_epilogue`,
 * RopeEpilogue.__call__ at :202-217), generalised from one token to `length` tokens.
 * Positions must stay below 2^24. */
int32_t omnia_rope_epilogue(const uint16_t* fused, int64_t fused_stride,
                            const uint16_t* query_weight, const uint16_t* key_weight,
                            int64_t offset, uint16_t* queries, uint16_t* keys,
                            int64_t length, int64_t query_heads, int64_t kv_heads,
                            int64_t head_dim, float log2_base, float eps,
                            hipStream_t stream);

/* Embedding gather + RoPE angle-atlas rows, pure copies:
 *   hidden_out [n_tokens, hidden] bf16:  row i = embedding[tokens[i]]
 *     (embedding [vocab, hidden]; an id outside [0, vocab) gives a zero row);
 *   full_out [n_positions, full_width] fp32:  row j = full_atlas[position + j]
 *   sliding_out [n_positions, sliding_width] fp32: row j = sliding_atlas[position + j]
 * A zero width skips that atlas (its pointers may be NULL).
 * Replaces: core/kernels/embed/atlas.py:23-69,111-135
 * (`decode_embedding_rope_atlas_bf16`, AtlasEmbed.__call__), generalised from one token
 * to a segment sharing positions position .. position+n_positions-1; Core chain
 * core/kernels/embed/default.py:35-42.
 * hidden: multiple of 8, at most 8192; atlas widths multiples of 4. */
int32_t omnia_embed_atlas(const int32_t* tokens, int64_t n_tokens,
                          const uint16_t* embedding, int64_t vocab, int64_t hidden,
                          const float* full_atlas, int64_t full_rows, int64_t full_width,
                          const float* sliding_atlas, int64_t sliding_rows,
                          int64_t sliding_width, int64_t position, int64_t n_positions,
                          uint16_t* hidden_out, float* full_out, float* sliding_out,
                          hipStream_t stream);

/* SwiGLU activation of blocked gate/up rows:
 *   out[r, i] = bf16(bf16(g * bf16(sigmoid(g))) * u),  g = gate[r, i], u = up[r, i]
 * gate, up [rows, inner] bf16 with row strides (elements) gate_stride, up_stride, e.g.
 * two tensors, or the halves of a fused [rows, 2*inner] projection; out contiguous
 * [rows, inner]. The sigmoid is the correctly rounded bf16 value.
 * Replaces the Core chain core/layers.py:249-250,284-287 (`swish`, `SwiGLU`,
 * SwitchGLU.activate) and core/kernels/gate_up/default.py:71-81 (the routed epilogue).
 * inner and both strides: multiples of 8. */
int32_t omnia_swiglu(const uint16_t* gate, int64_t gate_stride, const uint16_t* up,
                     int64_t up_stride, uint16_t* out, int64_t rows, int64_t inner,
                     hipStream_t stream);

/* DeltaNet gate: out[r, h] = -exp(A_log[h]) * softplus(f32(a[r, h]) + dt_bias[h]), fp32,
 * softplus(x) = mx.logaddexp(x, 0) = max(x,0) + log1p(exp(-|x|)) with its inf/NaN arms,
 * each fp32 step correctly rounded. a [rows, heads] bf16 (row stride a_stride),
 * A_log and dt_bias [heads] fp32, out contiguous [rows, heads] fp32.
 * Replaces: models/qwen3_5/layers/deltanet.py:222-224 (also models/qwen3_next/layers/
 * deltanet.py:122-123); softplus lowering as core/kernels/qmv/softplus.py:64-76. */
int32_t omnia_gate_softplus(const uint16_t* a, int64_t a_stride, const float* a_log,
                            const float* dt_bias, float* out, int64_t rows, int64_t heads,
                            hipStream_t stream);

/* Both gated activations in one dispatch: omnia_swiglu over gate/up -> y [rows, inner]
 * and omnia_gate_softplus over a -> g [a_rows, heads], with the same arithmetic and
 * results as the two entries. heads must be even, a's row stride even, a 4-byte and
 * A_log, dt_bias, g 8-byte aligned; either part may be empty (rows or a_rows 0).
 * Replaces: the pair of Core chains core/layers.py:249-250,284-287 (SwiGLU) and
 * models/qwen3_5/layers/deltanet.py:222-224 (gate-softplus), issued as one launch; the
 * reference has no fused form, so this is the one-dispatch answer to the gate-softplus's
 * launch cost at small sizes. */
int32_t omnia_gated_activations(const uint16_t* gate, int64_t gate_stride, const uint16_t* up,
                                int64_t up_stride, uint16_t* y, int64_t rows, int64_t inner,
                                const uint16_t* a, int64_t a_stride, const float* a_log,
                                const float* dt_bias, float* g, int64_t a_rows, int64_t heads,
                                hipStream_t stream);

/* Softmax -> top-k -> renormalise over given router logits, one row per token:
 *   indices[r, :k] = the k largest bf16 logits of row r in descending order, an exact
 *                    tie going to the lower expert index (int32);
 *   weights[r, :k] = softmax(logits[r])[indices] / sum of the same (fp32).
 * logits [rows, experts] bf16 with row stride `stride`; experts <= 256, k <= 64.
 * Replaces: core/kernels/route/softmax_topk.py:20-75,215-230 (`moe_softmax_topk`,
 * SoftmaxTopkRoute.__call__) and the Core chain core/kernels/route/default.py:44-69 /
 * models/qwen3/layers/moe.py:34-42, served for many rows at once, with the
 * lowest-index tie rule of core/kernels/route/ordinal.py:1-27 (the reference's softmax
 * path breaks ties toward the higher index). */
int32_t omnia_softmax_topk(const uint16_t* logits, int64_t stride, int64_t rows,
                           int64_t experts, int64_t k, int32_t* indices, float* weights,
                           hipStream_t stream);

/* The same selection with the two other softmax declarations of the reference's Route:
 *   normalize = 1: weights as omnia_softmax_topk (renormalised over the kept experts);
 *   normalize = 0: weights[r, j] = softmax(logits[r, :experts])[indices[r, j]], the
 *                  probability over the whole row (Route(..., normalize=False));
 *   shared = 1:    the row holds experts + 1 logits, the last the shared expert's gate;
 *                  slot k of each output row is the shared expert: index `experts`,
 *                  weight sigmoid(logit) in fp32 (correctly rounded), after the k routed
 *                  slots (Route(..., shared=True)).
 * indices, weights [rows, k + shared]; stride >= experts + shared; k <= 63 with a shared
 * slot, 64 without; the other limits as omnia_softmax_topk.
 * Replaces: core/kernels/route/softmax_topk.py:20-75 (`moe_softmax_topk` with SHARED)
 * and 295-336 (the declarations SoftmaxTopkRoute.build serves), and the Core chain
 * core/kernels/route/default.py:44-69 for `normalize=False` (its `if routing.normalize`
 * and `if routing.shared` arms), as models/qwen3_5/layers/moe.py:157-162 (shared) and
 * models/qwen3/layers/moe.py:50-52 (normalize=norm_topk) declare them. */
int32_t omnia_softmax_topk_slots(const uint16_t* logits, int64_t stride, int64_t rows,
                                 int64_t experts, int64_t k, int32_t normalize, int32_t shared,
                                 int32_t* indices, float* weights, hipStream_t stream);

/* Bytes of the packed router weight for [experts, hidden] (experts a multiple of 16,
 * hidden of 32), or -EINVAL. Pure; touches no device. */
int64_t omnia_router_pack_bytes(int64_t experts, int64_t hidden);

/* Repacks a router weight [experts, hidden] bf16 for omnia_residual_rms_router, into a
 * caller-allocated buffer of omnia_router_pack_bytes(experts, hidden) bytes: the weight
 * in 1 KiB blocks of 16 experts x 32 columns in the matrix-core operand order, then
 * experts fp32 row norms (rounded up), then the weight row-major (read to recompute
 * single logits exactly). Run once per weight, when the strategy is
 * built, as the reference's strategies take their weights at build
 * (core/kernels/route/residual.py:206-299 holds the gate for the dispatch); no
 * reference function is replaced. */
int32_t omnia_pack_router_weight(const uint16_t* router_weight, int64_t experts,
                                 int64_t hidden, void* packed, hipStream_t stream);

/* Residual add + RMSNorm + router projection + softmax top-k, fused:
 *   summed, normalized [rows, hidden] bf16 exactly as omnia_add_rms_norm;
 *   logits [rows, experts] = bf16(normalized x router_weight^T), the correctly rounded
 *     dot products (matrix-core accumulation, with an fp64 recomputation wherever the
 *     fp32 accumulation error could change the rounding), written only when `logits`
 *     is not NULL;
 *   indices [rows, k] int32, weights [rows, k] fp32 exactly as omnia_softmax_topk
 *     applied to those logits.
 * x, branch [rows, hidden] bf16; norm_weight [hidden] bf16; packed_router: the router
 * weight [experts, hidden] bf16 as omnia_pack_router_weight wrote it.
 * hidden in {2048, 4096}, experts in {128, 256}; k <= 64.
 * With rows <= 512 and `logits` given (decode steps and short prefills) the launch is
 * two dispatches: the projection spread over many workgroups, every logit an fp64 dot
 * product rounded once, then the selection of omnia_softmax_topk over the written
 * logits. The outputs are the same bits either way.
 * Replaces: core/kernels/route/residual.py:117-299 (`residual_rms_router`, the
 * one-token residual join with the router gemv fused), generalised to many tokens and
 * to softmax routing; the Core chain is add_norm/default.py:28-29 followed by
 * route/default.py:44-69. */
int32_t omnia_residual_rms_router(const uint16_t* x, const uint16_t* branch,
                                  const uint16_t* norm_weight, const void* packed_router,
                                  int64_t rows, int64_t hidden, int64_t experts, int64_t k,
                                  float eps, uint16_t* summed, uint16_t* normalized,
                                  uint16_t* logits, int32_t* indices, float* weights,
                                  hipStream_t stream);

/* Sigmoid routing with a correction bias over given router logits, one row per wave:
 *   score_e = sigmoid(x_e), correctly rounded to fp32 (x_e the fp32 logit, or the bf16
 *             logit widened)
 *   key_e   = ordinal(-(score_e + bias_e)), the sum in fp32; ordinal maps fp32 bits to a
 *             uint32 whose ascending order is the float order (+-0 one value, NaN above all)
 *   indices = the k smallest keys, the lower expert first on equal keys (NaN last)
 *   weights_j = score_{i_j} / (sum of the k winners' scores, in fp32, in winner order)
 * logits [rows, stride] bf16 (logits_fp32 = 0) or fp32 (logits_fp32 = 1); bias [experts]
 * fp32; keys [rows, experts] uint32 or null; indices [rows, k] int32 and weights [rows, k]
 * fp32, both or neither (then k is ignored); keys or indices must be given.
 * Replaces: core/kernels/route/ordinal.py:200-286 (`router_tournament`,
 * OrdinalRoute.__call__) and `ordinal_keys` at :253-262, which the Core chain restates.
 * experts <= 1024; k in [1, min(experts, 64)]. */
int32_t omnia_sigmoid_topk(const void* logits, int64_t stride, int32_t logits_fp32,
                           const float* bias, int64_t rows, int64_t experts, int64_t k,
                           uint32_t* keys, int32_t* indices, float* weights,
                           hipStream_t stream);

/* The fused residual router's sigmoid form: the join, the norm and the exact logits of
 * omnia_residual_rms_router, then the keys and optional selection of
 * omnia_sigmoid_topk from those bf16 logits and bias [experts] fp32.
 *   logits [rows, experts] bf16 or null; keys [rows, experts] uint32 or null;
 *   indices [rows, k] int32 and weights [rows, k] fp32, both or neither.
 * Every logit is the correctly rounded bf16 of the exact dot product, so the keys and
 * the selection equal those computed from the exact logits. With rows <= 512 and `logits`
 * given the launch is the two dispatches of omnia_residual_rms_router's decode path,
 * the second omnia_sigmoid_topk over the written logits.
 * Replaces: core/kernels/route/residual.py:117-299 (`residual_rms_router` with its
 * `correction_bias`, emitting logits and ordinal keys; its T = 1 only).
 * hidden 2048 or 4096, experts 128 or 256. */
int32_t omnia_residual_rms_router_sigmoid(const uint16_t* x, const uint16_t* branch,
                                          const uint16_t* norm_weight, const void* packed_router,
                                          const float* bias, int64_t rows, int64_t hidden,
                                          int64_t experts, int64_t k, float eps,
                                          uint16_t* summed, uint16_t* normalized,
                                          uint16_t* logits, uint32_t* keys, int32_t* indices,
                                          float* weights, hipStream_t stream);

/* Routed expert gate/up projection of one token, dense bf16 weights, "blocked" layout
 * (gate and up block-concatenated on the output axis and left un-activated):
 *   out[j, n] = bf16(sum_h x[h] * weight[chosen[j], n, h])   j < k, n < rows (= 2 * inner)
 * with fp32 accumulation. x [hidden] bf16; weight [experts, rows, hidden] bf16; chosen
 * [k] int32 (an id outside [0, experts) gives a zero row); out [k, rows] bf16.
 * Replaces: core/kernels/gate_up/dense.py:30-119 (`moe_dense_gate_up`,
 * DenseGateUp.__call__ at :104-119); Core chain core/kernels/gate_up/default.py:59-66.
 * hidden: multiple of 8, at most 8192. */
int32_t omnia_moe_gate_up(const uint16_t* x, const uint16_t* weight, int64_t experts,
                          int64_t rows, int64_t hidden, const int32_t* chosen, int64_t k,
                          uint16_t* out, hipStream_t stream);

/* Routed expert down projection of one token with the SwiGLU and the combine fused:
 *   a[j, i] = g / (1 + exp(-g)) * u          fp32; g = act[j, i], u = act[j, inner + i]
 *   d[j, n] = bf16(fp32(sum_i a[j, i] * weight[chosen[j], n, i]) * weights[j])
 *   out[n]  = bf16(bf16(sum_j d[j, n]) + residual[n])     (residual NULL: no add)
 * act [k, 2 * inner] bf16 (omnia_moe_gate_up's output); weight [experts, hidden, inner]
 * bf16; chosen [k] int32 (an id outside [0, experts) contributes zero); weights [k] fp32;
 * out [hidden] bf16.
 * Replaces: core/kernels/down_combine/dense.py:21-109 (`moe_dense_down` and the
 * `routed.sum(axis=0) + residual` of DenseDownCombine.__call__ at :91-109); Core chain
 * core/kernels/down_combine/default.py:43-58.
 * inner: multiple of 8, at most 2048; 1 <= k <= 16. */
int32_t omnia_moe_down_combine(const uint16_t* act, const uint16_t* weight, int64_t experts,
                               int64_t hidden, int64_t inner, const int32_t* chosen,
                               const float* weights, int64_t k, const uint16_t* residual,
                               uint16_t* out, hipStream_t stream);

/* Routed expert gate/up of one token over an affine-quantized stack (MLX's
 * QuantizedSwitchLinear, mode "affine"), the interleaved layout, silu fused:
 *   r = sum over groups of scale * sum_j x[j] q[j] + bias * sum_j x[j]     fp32
 *   g = bf16(r[2n]), u = bf16(r[2n + 1]); with limit < +inf, g = min(g, limit) and
 *   u = clip(u, -limit, limit); out[s, n] = bf16(bf16(g * bf16(1 / (1 + exp(-g)))) * u)
 * x [hidden] bf16; weight [experts, 2 * inner, hidden * bits / 32] uint32 (each row a
 * little-endian bit stream of bits-wide values); scales, biases [experts, 2 * inner,
 * hidden / group_size] bf16; chosen [slots] int32; out [slots, inner] bf16. A non-null
 * shared_weight ([2 * inner, ...], with its own scales, biases, width and group) serves the
 * last slot, whose index is then ignored. An index outside [0, experts) gives zeros.
 * bits in {2, 3, 4, 5, 6, 8}, groups in {32, 64, 128} dividing hidden; hidden a multiple
 * of 32, at most 16384; limit >= 0 or +inf (none).
 * Replaces: core/kernels/gate_up/affine.py:24-191 (`AffineGateUp`, `moe_gateup_act`); Core
 * chain core/kernels/gate_up/default.py:60-81 over QuantizedSwitchLinear.__call__
 * (core/layers.py:183-197). */
int32_t omnia_moe_gate_up_affine(const uint16_t* x, const uint32_t* weight, const uint16_t* scales,
                                 const uint16_t* biases, int64_t experts, int64_t hidden,
                                 int64_t inner, int64_t bits, int64_t group_size,
                                 const int32_t* chosen, int64_t slots, float limit,
                                 const uint32_t* shared_weight, const uint16_t* shared_scales,
                                 const uint16_t* shared_biases, int64_t shared_bits,
                                 int64_t shared_group_size, uint16_t* out, hipStream_t stream);

/* Routed expert down/combine of one token over an affine-quantized stack:
 *   t[s, n] = sum over groups of scale * sum_i act[s, i] q[i] + bias * sum_i act[s, i]   fp32
 *   acc[n] = sum over s in order of bf16(bf16(t[s, n]) * weights[s])                      fp32
 *   out[n] = bf16(bf16(acc[n]) + residual[n])   (no add when residual is null)
 * act [slots, inner] bf16; weight [experts, hidden, inner * bits / 32] uint32; scales,
 * biases [experts, hidden, inner / group_size] bf16; chosen [slots] int32; weights [slots]
 * fp32; residual, out [hidden] bf16. The shared leaf serves the last slot as in
 * omnia_moe_gate_up_affine.
 * inner a multiple of 32, at most 1536, divisible by the groups; 1 <= slots <= 16.
 * Replaces: core/kernels/down_combine/affine.py:17-178 (`AffineDownCombine`,
 * `moe_down_combine`); Core chain core/kernels/down_combine/default.py:43-58. */
int32_t omnia_moe_down_combine_affine(const uint16_t* act, const uint32_t* weight,
                                      const uint16_t* scales, const uint16_t* biases,
                                      int64_t experts, int64_t hidden, int64_t inner, int64_t bits,
                                      int64_t group_size, const int32_t* chosen,
                                      const float* weights, int64_t slots, const uint16_t* residual,
                                      const uint32_t* shared_weight, const uint16_t* shared_scales,
                                      const uint16_t* shared_biases, int64_t shared_bits,
                                      int64_t shared_group_size, uint16_t* out, hipStream_t stream);

/* Routed expert gate/up of one token over an MXFP4 stack (MLX's QuantizedSwitchLinear,
 * mode "mxfp4", the gpt-oss format), the interleaved layout, the clamped swiglu_oai fused:
 *   r = sum over groups of 32 of s * sum_j x[j] v[j]       v e2m1, s = fp32(scale << 23)
 *   g = bf16(r[2n] + bias[2n]), u = bf16(r[2n + 1] + bias[2n + 1]); with limit < +inf,
 *   g = bf16(min(g, limit)), u = bf16(clamp(u, -limit, limit));
 *   out[s, n] = bf16(bf16(g * bf16(1 / (1 + exp(-1.702 g)))) * bf16(u + 1))
 * x [hidden] bf16; weight [experts, 2 * inner, hidden / 8] uint32 (two e2m1 codes per byte,
 * low nibble first); scales [experts, 2 * inner, hidden / 32] uint8 (e8m0); bias
 * [experts, 2 * inner] bf16 or NULL (zero); chosen [slots] int32; out [slots, inner] bf16.
 * An index outside [0, experts) gives zeros. hidden a multiple of 32, at most 16384.
 * Replaces: core/kernels/gate_up/mxfp4.py:24-138 (`Mxfp4GateUp`, `mxfp4_gateup_act`); Core
 * chain core/kernels/gate_up/default.py:60-78. */
int32_t omnia_moe_gate_up_mxfp4(const uint16_t* x, const uint32_t* weight, const uint8_t* scales,
                                const uint16_t* bias, int64_t experts, int64_t hidden, int64_t inner,
                                const int32_t* chosen, int64_t slots, float limit, uint16_t* out,
                                hipStream_t stream);

/* Routed expert down/combine of one token over an MXFP4 stack:
 *   t[s, n] = sum over groups of 32 of s * sum_i act[s, i] v[i]                   fp32
 *   acc[n] = sum over s in order of bf16(bf16(t[s, n] + bias[n]) * weights[s])    fp32
 *   out[n] = bf16(bf16(acc[n]) + residual[n])   (no add when residual is null)
 * act [slots, inner] bf16; weight [experts, hidden, inner / 8] uint32; scales [experts,
 * hidden, inner / 32] uint8; bias [experts, hidden] bf16 or NULL; chosen [slots] int32;
 * weights [slots] fp32; residual, out [hidden] bf16.
 * inner a multiple of 32, at most 4096; 1 <= slots <= 16.
 * Replaces: core/kernels/down_combine/mxfp4.py:16-120 (`Mxfp4DownCombine`,
 * `mxfp4_down_combine`); Core chain core/kernels/down_combine/default.py:43-58. */
int32_t omnia_moe_down_combine_mxfp4(const uint16_t* act, const uint32_t* weight, const uint8_t* scales,
                                     const uint16_t* bias, int64_t experts, int64_t hidden,
                                     int64_t inner, const int32_t* chosen, const float* weights,
                                     int64_t slots, const uint16_t* residual, uint16_t* out,
                                     hipStream_t stream);

/* Routed expert gate/up of one token over an NVFP4 stack (MLX's QuantizedSwitchLinear,
 * mode "nvfp4"), the interleaved layout, the plain SwiGLU chain fused:
 *   r = sum over groups of 16 of s * sum_j x[j] v[j]      v e2m1, s the group's e4m3 byte
 *   decoded as mlx does (0x7F and 0xFF are +-480)
 *   g = bf16(r[2n]), u = bf16(r[2n + 1]); out[s, n] = bf16(bf16(g * bf16(1 / (1 + exp(-g)))) * u)
 * x [hidden] bf16; weight [experts, 2 * inner, hidden / 8] uint32 (two e2m1 codes per byte,
 * low nibble first); scales [experts, 2 * inner, hidden / 16] uint8, 2-byte aligned;
 * chosen [slots] int32; out [slots, inner] bf16. An index outside [0, experts) gives
 * zeros. hidden a multiple of 32 (the reference's 16), at most 16384.
 * Replaces: core/kernels/gate_up/nvfp4.py:24-128 (`Nvfp4GateUp`, `nvfp4_gateup_act`); Core
 * chain core/kernels/gate_up/default.py:60-81. */
int32_t omnia_moe_gate_up_nvfp4(const uint16_t* x, const uint32_t* weight, const uint8_t* scales,
                                int64_t experts, int64_t hidden, int64_t inner, const int32_t* chosen,
                                int64_t slots, uint16_t* out, hipStream_t stream);

/* The same NVFP4 gate/up with the routing decided in the kernel: slot s (s < top_k) runs
 * the expert of rank s in the ordinal keys (ascending = better, equal keys to the lower
 * index), as the reference's OrdinalRouting declaration defines it. keys [experts] uint32;
 * experts <= 1024, top_k <= experts; out [top_k, inner] bf16. Other arguments as
 * omnia_moe_gate_up_nvfp4.
 * Replaces: core/kernels/gate_up/nvfp4_packed.py:1-346 (`Nvfp4PackedGateUp`, routing
 * inside the kernel; its repacked weight layout is not used); ordinal routing
 * core/kernels/gate_up/kernel.py:23-36. */
int32_t omnia_moe_gate_up_nvfp4_ordinal(const uint16_t* x, const uint32_t* weight, const uint8_t* scales,
                                        int64_t experts, int64_t hidden, int64_t inner, const uint32_t* keys,
                                        int64_t top_k, uint16_t* out, hipStream_t stream);

/* Routed expert down/combine of one token over an NVFP4 stack:
 *   t[s, n] = sum over groups of 16 of s * sum_i act[s, i] v[i]       fp32
 *   acc[n] = sum over s in order of bf16(bf16(t[s, n]) * weights[s])  fp32
 *   out[n] = bf16(bf16(acc[n]) + residual[n])   (no add when residual is null)
 * act [slots, inner] bf16; weight [experts, hidden, inner / 8] uint32; scales [experts,
 * hidden, inner / 16] uint8, 2-byte aligned; chosen [slots] int32; weights [slots] fp32;
 * residual, out [hidden] bf16. inner a multiple of 32, at most 4096; 1 <= slots <= 16.
 * Replaces: core/kernels/down_combine/nvfp4.py:16-117 (`Nvfp4DownCombine`,
 * `nvfp4_down_combine`); Core chain core/kernels/down_combine/default.py:43-58. */
int32_t omnia_moe_down_combine_nvfp4(const uint16_t* act, const uint32_t* weight, const uint8_t* scales,
                                     int64_t experts, int64_t hidden, int64_t inner, const int32_t* chosen,
                                     const float* weights, int64_t slots, const uint16_t* residual,
                                     uint16_t* out, hipStream_t stream);

/* The packed NVFP4 down/combine: for each of `tokens` tokens, the routed down projections,
 * the unrouted (shared) stack's and the residual add in one dispatch, with a bf16 epilogue:
 *   d[t, s, n] = bf16(sum over groups of 16 of s * sum_i act[t, s, i] v[i])   fp32 sum
 *                (slot s < top_k: expert chosen[t, s]; slot top_k: the shared stack)
 *   total = bf16(bf16(d[t, s, n] * bf16(weights[t, s])) + total) over s < top_k in order
 *   out[t, n] = bf16(residual[t, n] + bf16(total + d[t, top_k, n]))
 * each operation in fp32. act [tokens, top_k + 1, inner] bf16; weight [experts, hidden,
 * inner / 8] and shared_weight [hidden, inner / 8] uint32; scales and shared_scales the
 * group-16 e4m3 planes [.., hidden, inner / 16] uint8, 2-byte aligned; chosen [tokens,
 * top_k] int32 (an id outside [0, experts) gives zero rows); weights [tokens, top_k] fp32;
 * residual, out [tokens, hidden] bf16. inner a multiple of 32, at most 2048; 0 <= top_k
 * <= 31; tokens <= 65535.
 * Replaces: core/kernels/down_combine/nvfp4_packed.py:38-138,224-270
 * (`nvfp4_fused_down_residual`, Nvfp4PackedDownCombine.__call__). The reference reads a
 * halved scale plane (shared/nvfp4/packed.py:126-164) that equals this group-16 plane
 * wherever its build accepts the checkpoint; the caller checks that certificate. */
int32_t omnia_moe_down_combine_nvfp4_shared(const uint16_t* act, const uint32_t* weight,
                                            const uint8_t* scales, int64_t experts,
                                            const uint32_t* shared_weight, const uint8_t* shared_scales,
                                            int64_t hidden, int64_t inner, const int32_t* chosen,
                                            const float* weights, int64_t tokens, int64_t top_k,
                                            const uint16_t* residual, uint16_t* out, hipStream_t stream);

/* Dense SwiGLU MLP of one token, first half: the fused gate||up projection with the
 * SwiGLU applied in bf16 steps,
 *   g = bf16(sum_h x[h] * fused[n, h]),  u = bf16(sum_h x[h] * fused[inner + n, h])   fp32 sums
 *   e = bf16(exp(|g|)), den = bf16(1 + e), y = bf16(1 / den), sig = g < 0 ? y : bf16(1 - y)
 *   activated[n] = bf16(bf16(g * sig) * u)
 * x [hidden] bf16; fused_weight [2 * inner, hidden] bf16 (gate rows first); activated
 * [inner] bf16.
 * Replaces: core/kernels/mlp/dense.py:34-97,185-199 (`dense_gate_up_swiglu`, the first
 * dispatch of DenseMlp.__call__ at :244-246); Core chain core/kernels/mlp/default.py:28-29
 * through SwiGLU.__call__ at core/layers.py:270-272.
 * hidden: multiple of 8, at most 8192. */
int32_t omnia_dense_gate_up_swiglu(const uint16_t* x, const uint16_t* fused_weight,
                                   int64_t hidden, int64_t inner, uint16_t* activated,
                                   hipStream_t stream);

/* Dense SwiGLU MLP of one token, second half: the down projection with the residual,
 *   out[n] = bf16(residual[n] + bf16(sum_i activated[i] * down[n, i]))   fp32 sum
 * activated [inner] bf16; down_weight [hidden, inner] bf16; residual, out [hidden] bf16.
 * Replaces: core/kernels/mlp/dense.py:100-147,202-218 (`dense_down_residual`, the second
 * dispatch of DenseMlp.__call__ at :246); Core chain core/kernels/mlp/default.py:28-29.
 * inner: multiple of 8. */
int32_t omnia_dense_down_residual(const uint16_t* activated, const uint16_t* down_weight,
                                  const uint16_t* residual, int64_t hidden, int64_t inner,
                                  uint16_t* out, hipStream_t stream);

/* Workspace bytes omnia_attention_decode needs for a cache of `capacity` rows (the
 * per-chunk softmax states of a long cache). Pure; touches no device. -EINVAL for a
 * geometry the kernel does not serve. */
int64_t omnia_attention_workspace_bytes(int64_t heads, int64_t kv_heads, int64_t head_dim,
                                        int64_t capacity);

/* One decode step of an attention layer over a KV cache, fused:
 *   per head: n = bf16(w * bf16(x * inv)), inv = 1 / sqrt(sum x^2 / 128 + eps)
 *   a, b = bf16(n_p * bf16(mscale)), bf16(n_{p+P} * bf16(mscale))       p < P = rotary_pairs
 *   q_p = bf16(a cos - b sin), q_{p+P} = bf16(a sin + b cos), q_d = n_d for d >= 2P
 *   (the same for the key row; cos || sin from row `position` of `angles` [angle_rows, 2P]
 *   fp32, 16-byte aligned)
 *   the new key and value rows written into the caches, then for every query head h
 *   out[h] = bf16(sum_r softmax_r(scale * q_h . k_r) v_r) over the attended rows of kv
 *   head h / (heads / kv_heads), softmax and sums in fp32.
 * raw_queries [heads, 128], raw_keys / raw_values [kv_heads, 128], query_weight /
 * key_weight [128] bf16; key_cache / value_cache [kv_heads, capacity, 128] bf16, written
 * in place; position: one device int32, read and not advanced. window 0 (fixed cache):
 * write row p, attend rows [0, p]; window == capacity (ring): write row p % window, attend
 * rows [0, min(p + 1, window)). max_rows: an upper bound on the attended rows (sizes the
 * grid; the host's position + 1, or capacity under graph capture). workspace: at least
 * omnia_attention_workspace_bytes(heads, kv_heads, 128, capacity) bytes, 16-byte
 * aligned (unused when max_rows <= 128). out [heads, 128] bf16.
 * Replaces: core/kernels/attention/full.py:133-471,557-629 (`full_fused_attention`,
 * FullAttentionStep at :632-740) and sliding.py:136-430,504-580 (`sliding_fused_attention`
 * over a RingKVCache, SlidingAttentionStep at :583-691); Core chain
 * core/kernels/attention/default.py:114-156.
 * head_dim 128; heads / kv_heads in {1, 2, 4, 8}; rotary_pairs in {8, 16, 32, 64}. */
int32_t omnia_attention_decode(const uint16_t* raw_queries, const uint16_t* raw_keys,
                               const uint16_t* raw_values, const uint16_t* query_weight,
                               const uint16_t* key_weight, const float* angles,
                               int64_t angle_rows, int64_t rotary_pairs, float mscale,
                               uint16_t* key_cache, uint16_t* value_cache, int64_t capacity,
                               int64_t window, const int32_t* position, int64_t max_rows,
                               int64_t heads, int64_t kv_heads, int64_t head_dim, float scale,
                               float eps, void* workspace, int64_t workspace_bytes,
                               uint16_t* out, hipStream_t stream);

/* Bytes of the static device array omnia_attention_decode_noalloc keeps its per-chunk
 * softmax states in (one array per GPU, held until the process ends). */
#define OMNIA_ATTENTION_SCRATCH_BYTES (4 * 1024 * 1024)

/* Workspace bytes omnia_attention_sink_decode needs for `heads` query heads over
 * `key_length` keys: the per-chunk softmax states; 0 when one chunk covers the keys.
 * -EINVAL for a bad geometry. Pure; touches no device. */
int64_t omnia_attention_sink_workspace_bytes(int64_t heads, int64_t kv_heads, int64_t key_length);

/* One query per head against `key_length` cached rows, the learned sink logit in the
 * softmax's denominator (head_dim 64):
 *   s[h, j] = (q[h] . keys[h / gqa, j]) * scale + mask[j]   (keys with mask +-inf skipped)
 *   out[h]  = sum_j exp(s[h, j] - M) values[h / gqa, j] / (exp(sink[h] - M) + sum_j exp(s[h, j] - M))
 * in fp32, M the maximum of the sink and the scores, rounded once to bf16. queries [heads,
 * 64] bf16 (normed and rotated); keys, values: head h, row j at h * head_stride + j * 64
 * bf16 elements (rows packed, 16-byte aligned); mask [key_length] fp32 additive or null;
 * sinks [heads] bf16; out [heads, 64] bf16; gqa = heads / kv_heads in {1, 2, 4, 8}.
 * Replaces: core/kernels/attention/sink.py:60-166,227-244 (`sink_attention`, its partial
 * and combine kernels), called by SinkAttentionStep.__call__ (:330-352). */
int32_t omnia_attention_sink_decode(const uint16_t* queries, const uint16_t* keys, const uint16_t* values,
                                    int64_t key_head_stride, int64_t value_head_stride, int64_t heads,
                                    int64_t kv_heads, int64_t head_dim, int64_t key_length, const float* mask,
                                    const uint16_t* sinks, float scale, void* workspace, int64_t workspace_bytes,
                                    uint16_t* out, hipStream_t stream);

/* omnia_attention_decode without a workspace argument: the same step, the same kernels
 * and the same results, with the per-chunk states in a static device array of
 * OMNIA_ATTENTION_SCRATCH_BYTES per GPU instead of caller memory. It calls no
 * hipMalloc, hipFree or allocating library routine.
 * No counterpart in the reference. It is for callers that cannot allocate device
 * memory: code under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc. The array's device address is looked up once per device, on the first
 * call there.
 * Limits: -EINVAL when the step needs more than OMNIA_ATTENTION_SCRATCH_BYTES of
 * states: 520 bytes per query head and chunk, at most
 * (511 + kv_heads) * (heads / kv_heads) * 520 bytes at any cache length (1.1 MB for 32
 * query heads over 8 kv heads; none when max_rows <= 128). Every call on one GPU shares
 * that GPU's array and it keeps the last call's contents: calls that overlap on one
 * GPU (other streams, or other threads without ordering) race. */
int32_t omnia_attention_decode_noalloc(const uint16_t* raw_queries, const uint16_t* raw_keys,
                                       const uint16_t* raw_values, const uint16_t* query_weight,
                                       const uint16_t* key_weight, const float* angles,
                                       int64_t angle_rows, int64_t rotary_pairs, float mscale,
                                       uint16_t* key_cache, uint16_t* value_cache,
                                       int64_t capacity, int64_t window, const int32_t* position,
                                       int64_t max_rows, int64_t heads, int64_t kv_heads,
                                       int64_t head_dim, float scale, float eps, uint16_t* out,
                                       hipStream_t stream);

/* Calibration copy: dst[0 .. bytes) = src[0 .. bytes), 16-byte nontemporal loads and
 * stores, `vectors_per_thread` (1, 2 or 4) vectors per thread issued before the first
 * store. bytes a multiple of 16; both pointers 16-byte aligned; the ranges must not
 * overlap.
 * No counterpart in the reference: measurement infrastructure, the copy of known size
 * that the bench times as each workload's ceiling (a kernel moving B bytes against this
 * copy of B / 2 bytes) and that scales the HBM byte counters. */
int32_t omnia_stream_copy(const void* src, void* dst, int64_t bytes, int32_t vectors_per_thread,
                          hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OMNIA_HIP_H */
