"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference (mlx-omnia) holds no golden tensors for these kernels and cannot run here
(no MLX, Python 3.10, Metal-only kernels), so the vectors are produced by this repo's
own oracle on seeded inputs and serve as regression pins: `tests/test_golden.py`
recomputes them on the CPU and the GPU tests compare the HIP kernels with them.
Run: `python tests/golden/make_golden.py`.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import activations, add_norm, affine, attention, embed, mlp, moe, mxfp4, nvfp4, rope, route  # noqa: E402
from oracle.bf16 import from_float  # noqa: E402


def make_add_norm() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(1)
    rows, hidden, eps = 4, 2560, 1e-6
    x = from_float(rng.standard_normal((rows, hidden)))
    branch = from_float(rng.standard_normal((rows, hidden)))
    weight = from_float(1.0 + 0.1 * rng.standard_normal(hidden))
    summed, normalized = add_norm.add_rms_norm(x, branch, weight, eps)
    return dict(x=x, branch=branch, weight=weight, eps=np.float32(eps),
                summed=summed, normalized=normalized)


def make_qk_norm_rope() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(2)
    length, hq, hkv, d, pairs, offset, eps, mscale = 5, 4, 2, 128, 32, 3, 1e-6, 1.3465735912322998
    raw_q = from_float(rng.standard_normal((length, hq, d)))
    raw_k = from_float(rng.standard_normal((length, hkv, d)))
    q_weight = from_float(1.0 + 0.1 * rng.standard_normal(d))
    k_weight = from_float(1.0 + 0.1 * rng.standard_normal(d))
    cos, sin = rope.angle_table(offset + length, pairs, 1e6)
    q, k = rope.qk_norm_rope(raw_q, raw_k, q_weight, k_weight, cos, sin, offset, eps, pairs, mscale)
    fused = from_float(rng.standard_normal((3, (hq + 2 * hkv) * d)))
    epilogue_offset = 32_000
    eq, ek = rope.rope_epilogue(fused, hq, hkv, d, q_weight, k_weight, epilogue_offset, 1e6, eps)
    return dict(raw_q=raw_q, raw_k=raw_k, q_weight=q_weight, k_weight=k_weight, cos=cos, sin=sin,
                offset=np.int64(offset), eps=np.float32(eps), pairs=np.int64(pairs),
                mscale=np.float64(mscale), q=q, k=k, fused=fused, hq=np.int64(hq),
                hkv=np.int64(hkv), epilogue_offset=np.int64(epilogue_offset),
                epilogue_q=eq, epilogue_k=ek)


def make_embed() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(3)
    vocab, hidden, length, position = 300, 256, 12, 7
    embedding = from_float(0.02 * rng.standard_normal((vocab, hidden)))
    tokens = rng.integers(0, vocab, size=(2, length), dtype=np.int32)
    full, sliding = rope.angle_table(40, 8, 1e6)
    out, full_out, sliding_out = embed.embed_atlas(tokens, embedding, full, sliding, position, length)
    return dict(embedding=embedding, tokens=tokens, full=full, sliding=sliding,
                position=np.int64(position), hidden=out, full_out=full_out,
                sliding_out=sliding_out)


def make_activations() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(4)
    gate = from_float(3 * rng.standard_normal((16, 256)))
    up = from_float(rng.standard_normal((16, 256)))
    a = from_float(rng.standard_normal((16, 32)))
    a_log = rng.uniform(0, 2.7, 32).astype(np.float32)
    dt_bias = (0.5 * rng.standard_normal(32)).astype(np.float32)
    return dict(gate=gate, up=up, swiglu=activations.swiglu(gate, up), a=a, a_log=a_log,
                dt_bias=dt_bias, gate_softplus=activations.gate_softplus(a, a_log, dt_bias))


def make_route() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(5)
    logits = from_float(rng.standard_normal((24, 128)))
    values = np.arange(128, dtype=np.float64) * -0.5
    values[[3, 11, 35, 67, 99, 120]] = values[3]
    logits[0] = from_float(values)
    indices, weights = route.softmax_topk(logits, 8)
    return dict(logits=logits, k=np.int64(8), indices=indices, weights=weights)


def make_moe() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(6)
    experts, hidden, inner, k = 4, 128, 32, 3
    x = from_float(rng.standard_normal(hidden))
    gate_up_weight = from_float(0.05 * rng.standard_normal((experts, 2 * inner, hidden)))
    down_weight = from_float(0.05 * rng.standard_normal((experts, hidden, inner)))
    chosen = np.array([3, 0, 2], dtype=np.int32)
    weights = np.array([0.5, 0.3, 0.2], dtype=np.float32)
    residual = from_float(rng.standard_normal(hidden))
    act = moe.gate_up(x, gate_up_weight, chosen)
    out = moe.down_combine(act, down_weight, chosen, weights, residual)
    return dict(x=x, gate_up_weight=gate_up_weight, down_weight=down_weight, chosen=chosen,
                weights=weights, residual=residual, act=act, out=out)


def make_moe_affine() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(9)
    experts, hidden, inner = 4, 128, 64
    gate_up = affine.quantize(rng.standard_normal((experts, 2 * inner, hidden)) / np.sqrt(hidden), 32, 4)
    down = affine.quantize(rng.standard_normal((experts, hidden, inner)) / np.sqrt(inner), 64, 4)
    shared_gate_up = affine.quantize(rng.standard_normal((2 * inner, hidden)) / np.sqrt(hidden), 64, 3)
    shared_down = affine.quantize(rng.standard_normal((hidden, inner)) / np.sqrt(inner), 32, 3)
    x = from_float(rng.standard_normal(hidden))
    chosen = np.array([3, 0, 2, 0], dtype=np.int32)           # the last slot is the shared expert's
    weights = np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float32)
    residual = from_float(rng.standard_normal(hidden))
    act = affine.gate_up(x, gate_up, chosen, shared=shared_gate_up)
    out = affine.down_combine(act, down, chosen, weights, residual, shared=shared_down)
    arrays = dict(x=x, chosen=chosen, weights=weights, residual=residual, act=act, out=out)
    for name, stack in (("gate_up", gate_up), ("down", down), ("shared_gate_up", shared_gate_up),
                        ("shared_down", shared_down)):
        arrays.update({f"{name}_weight": stack.weight, f"{name}_scales": stack.scales,
                       f"{name}_biases": stack.biases,
                       f"{name}_format": np.array([stack.bits, stack.group], dtype=np.int32)})
    return arrays


def make_moe_mxfp4() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(10)
    experts, hidden, inner = 4, 128, 64

    def stack(rows, features):
        codes = rng.integers(0, 16, size=(experts, rows, features))
        scales = rng.integers(119, 123, size=(experts, rows, features // 32)).astype(np.uint8)
        return mxfp4.Stack(mxfp4.pack(codes), scales, from_float(0.25 * rng.standard_normal((experts, rows))))

    gate_up, down = stack(2 * inner, hidden), stack(hidden, inner)
    x = from_float(2 * rng.standard_normal(hidden))
    chosen = np.array([3, 0, 2], dtype=np.int32)
    weights = np.array([0.5, 0.3, 0.2], dtype=np.float32)
    residual = from_float(rng.standard_normal(hidden))
    limit = np.float32(7.0)
    act = mxfp4.gate_up(x, gate_up, chosen, float(limit))
    out = mxfp4.down_combine(act, down, chosen, weights, residual)
    arrays = dict(x=x, chosen=chosen, weights=weights, residual=residual, limit=limit, act=act, out=out)
    for name, s in (("gate_up", gate_up), ("down", down)):
        arrays.update({f"{name}_weight": s.weight, f"{name}_scales": s.scales, f"{name}_bias": s.bias})
    return arrays


def make_moe_nvfp4() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(11)
    experts, hidden, inner = 4, 128, 64

    def stack(rows, features):
        codes = rng.integers(0, 16, size=(experts, rows, features))
        scales = rng.integers(0x18, 0x28, size=(experts, rows, features // 16)).astype(np.uint8)
        return nvfp4.Stack(nvfp4.pack(codes), scales)

    gate_up, down = stack(2 * inner, hidden), stack(hidden, inner)
    x = from_float(2 * rng.standard_normal(hidden))
    chosen = np.array([3, 0, 2], dtype=np.int32)
    weights = np.array([0.5, 0.3, 0.2], dtype=np.float32)
    residual = from_float(rng.standard_normal(hidden))
    act = nvfp4.gate_up(x, gate_up, chosen)
    out = nvfp4.down_combine(act, down, chosen, weights, residual)
    arrays = dict(x=x, chosen=chosen, weights=weights, residual=residual, act=act, out=out)
    for name, s in (("gate_up", gate_up), ("down", down)):
        arrays.update({f"{name}_weight": s.weight, f"{name}_scales": s.scales})
    return arrays


def make_moe_nvfp4_shared() -> dict[str, np.ndarray]:
    """The packed NVFP4 down/combine: the reference test's shape (hidden 64, inner 512,
    top-4 of 8 plus the shared expert), two tokens, paired scale planes."""
    rng = np.random.default_rng(12)
    experts, hidden, inner, k, tokens = 8, 64, 512, 4, 2

    def stack(lead):
        codes = rng.integers(0, 16, size=(*lead, hidden, inner))
        scales = np.repeat(rng.integers(0x18, 0x28, size=(*lead, hidden, inner // 32)).astype(np.uint8), 2, axis=-1)
        return nvfp4.Stack(nvfp4.pack(codes), scales)

    down, shared = stack((experts,)), stack(())
    act = from_float(rng.standard_normal((tokens, k + 1, inner)))
    chosen = np.array([[0, 2, 5, 7], [3, 0, 5, 1]], dtype=np.int32)
    weights = (rng.random((tokens, k)) * 2.5).astype(np.float32)
    residual = from_float(rng.standard_normal((tokens, hidden)))
    out = nvfp4.down_combine_shared(act, down, shared, chosen, weights, residual)
    return dict(act=act, chosen=chosen, weights=weights, residual=residual, out=out,
                down_weight=down.weight, down_scales=down.scales, shared_weight=shared.weight,
                shared_scales=shared.scales)


def make_mlp() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(7)
    hidden, inner = 128, 192
    x = from_float(rng.standard_normal(hidden))
    fused_weight = from_float(0.1 * rng.standard_normal((2 * inner, hidden)))
    down_weight = from_float(0.05 * rng.standard_normal((hidden, inner)))
    residual = from_float(rng.standard_normal(hidden))
    act = mlp.gate_up_swiglu(x, fused_weight)
    out = mlp.down_residual(act, down_weight, residual)
    return dict(x=x, fused_weight=fused_weight, down_weight=down_weight, residual=residual,
                act=act, out=out)


def make_attention() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(8)
    heads, kv_heads, capacity, pairs, position = 4, 2, 40, 32, 23
    cos, sin = rope.angle_table(capacity, pairs, 10000.0)
    angles = np.concatenate([cos, sin], axis=1).astype(np.float32)
    raw_q = from_float(rng.standard_normal(heads * 128))
    raw_k = from_float(rng.standard_normal(kv_heads * 128))
    raw_v = from_float(rng.standard_normal(kv_heads * 128))
    q_weight = from_float(1 + 0.1 * rng.standard_normal(128))
    k_weight = from_float(1 + 0.1 * rng.standard_normal(128))
    k_cache = from_float(rng.standard_normal((kv_heads, capacity, 128)))
    v_cache = from_float(rng.standard_normal((kv_heads, capacity, 128)))
    out, new_keys, new_values = attention.decode_step(
        raw_q, raw_k, raw_v, q_weight, k_weight, angles[position], k_cache, v_cache, position,
        window=0, scale=128 ** -0.5, eps=1e-6, pairs=pairs)
    return dict(raw_q=raw_q, raw_k=raw_k, raw_v=raw_v, q_weight=q_weight, k_weight=k_weight,
                angles=angles, k_cache=k_cache, v_cache=v_cache,
                position=np.array([position], dtype=np.int32), out=out,
                key_row=new_keys[:, position], value_row=new_values[:, position])


MAKERS = {"attention": make_attention, "add_norm": make_add_norm, "qk_norm_rope": make_qk_norm_rope, "embed": make_embed,
          "activations": make_activations, "route": make_route, "moe": make_moe, "mlp": make_mlp,
          "moe_affine": make_moe_affine, "moe_mxfp4": make_moe_mxfp4,
          "moe_nvfp4": make_moe_nvfp4, "moe_nvfp4_shared": make_moe_nvfp4_shared}


def main(names: list[str]) -> None:
    for name in names or list(MAKERS):
        arrays = MAKERS[name]()
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(f"wrote tests/golden/{name}.npz", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
