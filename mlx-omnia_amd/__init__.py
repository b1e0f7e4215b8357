"""mlx_omnia_amd — MI355X (gfx950) HIP bindings for mlx-omnia's fused per-layer
elementwise and normalisation primitives.

The package mirrors the reference's Layer declaration API (one facade per primitive, an
ordered strategy tuple, first `build` that returns an instance wins) over torch tensors,
and registers hand-written HIP kernels ahead of the stock-op Core chains:

- `kernels.add_norm.AddRmsNorm`          residual add + RMSNorm
- `kernels.qkv_rope.QkvRope`             per-head q/k RMSNorm + RoPE (table and epilogue)
- `kernels.embed.Embed`                  embedding gather + RoPE atlas rows
- `kernels.gate_up.GateUpActivation`     SwiGLU activation
- `kernels.gate_softplus.GateSoftplus`   -exp(A_log) * softplus(a + dt_bias)
- `kernels.route.Route`                  softmax -> top-k -> renormalise
- `kernels.route.ResidualRouter`         residual add + RMSNorm + router projection + top-k

The kernels live in `libomnia_hip.so` (sources under `csrc/`, C ABI in
`include/omnia_hip.h`), loaded by `runtime.library`.
"""

__all__ = ["kernels", "runtime"]
