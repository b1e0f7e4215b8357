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

#define OMNIA_ABI_VERSION 1

/* Version of this ABI (OMNIA_ABI_VERSION). Pure; touches no device. */
int32_t omnia_abi_version(void);

/* Text of the last error raised on the calling thread ("" if none). */
const char* omnia_last_error(void);

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

#ifdef __cplusplus
}
#endif

#endif /* OMNIA_HIP_H */
