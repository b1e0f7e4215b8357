#!/usr/bin/env python3
"""Benchmark of the fused per-layer kernels on one MI355X.

Metric: achieved HBM GB/s (% of the 8 TB/s peak) and µs per fused
kernel, on one GPU. A "step" is one launch of a fused kernel over one batch of its
config's synthetic input; the headline line is configs[1], the per-head QK-norm + RoPE
at the T=4096 prefill shape, and every other config's kernel is measured in the same run
and reported under "kernels".

Method, per kernel:
- inputs are seeded numpy draws rounded to bf16 (RNE), placed in HBM before timing;
- the launch cycles through enough copies of inputs and outputs that one cycle touches
  >= 512 MB (twice the 256 MB Infinity Cache), so no launch is served from cache;
- `--warmup` launches, then exactly `--steps` launches between two HIP events recorded
  on the stream the kernels run on, with a device synchronise on both sides; a ~100 us
  spin is queued ahead of the start event, so the host's latency in issuing the first
  launch falls outside the timed region. Each launch
  is a direct call of the C-ABI entry point with its arguments bound in advance (about a
  microsecond of host time), so back-to-back launches keep the GPU queue fed without
  the per-node gap a HIP graph replay adds; `--graph` times a captured graph instead;
- achieved = algorithmic bytes per launch (each input read once, each output written
  once) / average launch duration.
The CPU baseline is the repo's numpy oracle (a port of the reference's Core chains;
MLX does not exist on these machines), timed on this host for every workload on a
bounded sample of that workload's own shapes (about 0.8 s each, 3 s for the headline).

Output: one compact JSON line on stdout (the headline's figures, roofline and CPU
baseline, and `kernels`: name -> [us, fraction of peak, CPU oracle GB/s] for every
workload), and the full record (each workload's description, rotation copies, launch
mode, CPU sample, threads used and thread environment) in the `--results` file.

The headline also carries `roofline.copy_us`: the calibration copy (`omnia_stream_copy`,
16-byte nontemporal loads and stores, the best of 1, 2 and 4 vectors per thread) of the
same bytes, timed in the same run, the practical ceiling at that size. `--ceiling` adds
that copy and torch's `copy_` beside every workload.

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--only NAME[,NAME]]
                       [--results bench_results.json] [--ceiling]
       python bench.py --copy-sweep     (the calibration copy from 32 MB to 1.2 GB moved)
       python bench.py --phase-clocks [--phase-clocks-rows 4096,512]
                                        (the fused router's per-phase wall clocks)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

PEAK_GBS = 8000.0
ROTATE_BYTES = 512 * 2**20
WARM_SECONDS = float(os.environ.get("OMNIA_BENCH_WARM", "1.0"))  # per workload, before timing
MAX_COPIES = 64
METRIC = "achieved HBM GB/s (% of MI355X peak) and µs per fused kernel, 1 GPU"
HEADLINE = "qk_norm_rope_prefill"


@dataclass
class Workload:
    name: str
    kernel: str                      # kernel symbol substring, as rocprof names it
    description: str
    bytes_per_launch: int
    setup: Callable[[object, int], list]   # (device, copies) -> per-copy argument sets
    launch: Callable[[object], None]
    details: dict = field(default_factory=dict)
    default: bool = True             # False: run only when named by --only


def _normal(rng: np.random.Generator, shape, scale=1.0, shift=0.0) -> np.ndarray:
    return (shift + scale * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)


def _to_bf16_device(values: np.ndarray, device):
    """fp32 numpy -> bf16 (RNE, torch's conversion) on the device."""
    import torch

    return torch.from_numpy(values).to(device).to(torch.bfloat16)


def _copies(first: dict, copies: int) -> list[dict]:
    """`copies` argument sets: the first as given, the rest fresh device buffers."""
    sets = [first]
    for _ in range(copies - 1):
        sets.append({k: (v.clone() if hasattr(v, "clone") else v) for k, v in first.items()})
    return sets


def workloads() -> list[Workload]:
    import torch

    from mlx_omnia_amd.runtime import ops

    out: list[Workload] = []

    # residual add + RMSNorm, Qwen3-4B shape.
    for rows, tag in ((512, "prefill"), (1, "decode")):
        hidden = 2560

        def setup(device, copies, rows=rows, hidden=hidden):
            rng = np.random.default_rng(1)
            first = dict(
                x=_to_bf16_device(_normal(rng, (rows, hidden)), device),
                r=_to_bf16_device(_normal(rng, (rows, hidden)), device),
                w=_to_bf16_device(_normal(rng, (hidden,), 0.1, 1.0), device),
                s=torch.empty((rows, hidden), dtype=torch.bfloat16, device=device),
                n=torch.empty((rows, hidden), dtype=torch.bfloat16, device=device),
            )
            return _copies(first, copies)

        out.append(Workload(
            name=f"add_rms_norm_{tag}",
            kernel="add_rms_norm_row_kernel",
            description=f"x, residual bf16 [{rows}, {hidden}] -> summed, normed; eps 1e-6",
            bytes_per_launch=rows * 4 * 2 * hidden + 2 * hidden,
            setup=setup,
            launch=lambda a: ops.add_rms_norm(a["x"], a["r"], a["w"], 1e-6,
                                              summed=a["s"], normalized=a["n"]),
        ))

    # per-head QK-norm + RoPE from a cos/sin table.
    table_rows, pairs = 40960, 64

    def make_tables(device):
        inverse = np.exp(-np.log(1e6) * np.arange(pairs) / pairs)
        theta = np.arange(table_rows)[:, None] * inverse[None, :]
        return (torch.from_numpy(np.cos(theta).astype(np.float32)).to(device),
                torch.from_numpy(np.sin(theta).astype(np.float32)).to(device))

    for length, tag in ((4096, "prefill"), (64, "decode")):
        hq, hkv, d = 32, 8, 128

        def setup(device, copies, length=length, hq=hq, hkv=hkv, d=d):
            rng = np.random.default_rng(2)
            cos, sin = make_tables(device)
            sets = []
            base = dict(
                q=_to_bf16_device(_normal(rng, (length, hq, d)), device),
                k=_to_bf16_device(_normal(rng, (length, hkv, d)), device),
                qw=_to_bf16_device(_normal(rng, (d,), 0.1, 1.0), device),
                kw=_to_bf16_device(_normal(rng, (d,), 0.1, 1.0), device),
                cos=cos, sin=sin,
            )
            for i in range(copies):
                entry = dict(base) if i == 0 else {
                    **base, "q": base["q"].clone(), "k": base["k"].clone()}
                entry["offset"] = int(rng.integers(0, 32768))
                entry["oq"] = torch.empty((hq, length, d), dtype=torch.bfloat16, device=device)
                entry["ok"] = torch.empty((hkv, length, d), dtype=torch.bfloat16, device=device)
                sets.append(entry)
            return sets

        out.append(Workload(
            name=f"qk_norm_rope_{tag}",
            kernel="qk_norm_rope_pairs_kernel",
            description=(f"q [{length},{hq},{d}], k [{length},{hkv},{d}] bf16, cos/sin "
                         f"[{table_rows},{pairs}] fp32 theta=1e6, offset ~U[0,32768)"),
            bytes_per_launch=length * (2 * (hq + hkv) * d * 2 + 2 * pairs * 4) + 2 * d * 2,
            setup=setup,
            launch=lambda a: ops.qk_norm_rope(
                a["q"], a["k"], a["qw"], a["kw"], a["cos"], a["sin"], offset=a["offset"],
                eps=1e-6, rotary_pairs=pairs, queries=a["oq"], keys=a["ok"]),
        ))

    # configs[1], epilogue form: angles derived in-kernel from a fused qkv projection.
    def setup_epilogue(device, copies, length=4096, hq=32, hkv=8, d=128):
        rng = np.random.default_rng(3)
        first = dict(
            fused=_to_bf16_device(_normal(rng, (length, (hq + 2 * hkv) * d)), device),
            qw=_to_bf16_device(_normal(rng, (d,), 0.1, 1.0), device),
            kw=_to_bf16_device(_normal(rng, (d,), 0.1, 1.0), device),
        )
        sets = []
        for i in range(copies):
            entry = dict(first) if i == 0 else {**first, "fused": first["fused"].clone()}
            entry["offset"] = int(rng.integers(0, 32768))
            entry["oq"] = torch.empty((hq, length, d), dtype=torch.bfloat16, device=device)
            entry["ok"] = torch.empty((hkv, length, d), dtype=torch.bfloat16, device=device)
            sets.append(entry)
        return sets

    out.append(Workload(
        name="rope_epilogue_prefill",
        kernel="qk_norm_rope_pairs_kernel",
        description="fused qkv [4096, 48*128] bf16 -> q [32,4096,128], k [8,4096,128]; "
                    "angles in-kernel, theta=1e6",
        bytes_per_launch=4096 * (2 * 40 * 128 * 2) + 2 * 128 * 2,
        setup=setup_epilogue,
        launch=lambda a: ops.rope_epilogue(
            a["fused"], a["qw"], a["kw"], query_heads=32, kv_heads=8, head_dim=128,
            offset=a["offset"], log2_base=math.log2(1e6), eps=1e-6,
            queries=a["oq"], keys=a["ok"]),
    ))
    # SwiGLU over [8192, 9728] and the DeltaNet gate-softplus over [8192, 32].
    def setup_swiglu(device, copies, rows=8192, inner=9728):
        rng = np.random.default_rng(5)
        first = dict(
            g=_to_bf16_device(_normal(rng, (rows, inner)), device),
            u=_to_bf16_device(_normal(rng, (rows, inner)), device),
            y=torch.empty((rows, inner), dtype=torch.bfloat16, device=device),
        )
        return _copies(first, copies)

    out.append(Workload(
        name="swiglu",
        kernel="swiglu_flat_kernel",
        description="gate, up bf16 [8192, 9728] ~N(0,1) -> silu(gate) * up bf16",
        bytes_per_launch=3 * 8192 * 9728 * 2,
        setup=setup_swiglu,
        launch=lambda a: ops.swiglu(a["g"], a["u"], out=a["y"]),
    ))

    def setup_softplus(device, copies, rows=8192, heads=32):
        rng = np.random.default_rng(6)
        first = dict(
            a=_to_bf16_device(_normal(rng, (rows, heads)), device),
            a_log=torch.from_numpy(rng.uniform(0, 2.7, heads).astype(np.float32)).to(device),
            dt_bias=torch.from_numpy((0.5 * rng.standard_normal(heads)).astype(np.float32)).to(device),
            g=torch.empty((rows, heads), dtype=torch.float32, device=device),
        )
        return _copies(first, copies)

    out.append(Workload(
        name="gate_softplus",
        kernel="gate_softplus_kernel",
        description="a bf16 [8192, 32] ~N(0,1), A_log ~U(0,2.7), dt_bias ~N(0,0.5) fp32 [32] "
                    "-> -exp(A_log) * softplus(a + dt_bias) fp32",
        bytes_per_launch=8192 * 32 * 2 + 2 * 32 * 4 + 8192 * 32 * 4,
        setup=setup_softplus,
        launch=lambda a: ops.gate_softplus(a["a"], a["a_log"], a["dt_bias"], out=a["g"]),
    ))

    # configs[3] as one dispatch: both gated activations in one grid.
    def setup_gated(device, copies):
        sets = setup_swiglu(device, copies)
        softplus = setup_softplus(device, copies)
        for entry, extra in zip(sets, softplus):
            entry.update(a=extra["a"], a_log=extra["a_log"], dt_bias=extra["dt_bias"],
                         g_out=extra["g"])
        return sets

    out.append(Workload(
        name="gated_activations",
        kernel="gated_activations_kernel",
        description="SwiGLU gate, up bf16 [8192, 9728] and gate-softplus a bf16 [8192, 32] "
                    "(A_log, dt_bias fp32 [32]) in one dispatch",
        bytes_per_launch=3 * 8192 * 9728 * 2 + 8192 * 32 * 2 + 2 * 32 * 4 + 8192 * 32 * 4,
        setup=setup_gated,
        launch=lambda a: ops.gated_activations(a["g"], a["u"], a["a"], a["a_log"], a["dt_bias"],
                                               y=a["y"], g=a["g_out"]),
    ))

    # residual add + RMSNorm + router projection + softmax top-8 (Qwen3-30B-A3B).
    def setup_router(device, copies, rows=4096, hidden=2048, experts=128, k=8):
        rng = np.random.default_rng(7)
        first = dict(
            x=_to_bf16_device(_normal(rng, (rows, hidden)), device),
            r=_to_bf16_device(_normal(rng, (rows, hidden)), device),
            w=_to_bf16_device(_normal(rng, (hidden,), 0.1, 1.0), device),
            gate=_to_bf16_device(_normal(rng, (experts, hidden), 0.02), device),
            s=torch.empty((rows, hidden), dtype=torch.bfloat16, device=device),
            n=torch.empty((rows, hidden), dtype=torch.bfloat16, device=device),
            idx=torch.empty((rows, k), dtype=torch.int32, device=device),
            wts=torch.empty((rows, k), dtype=torch.float32, device=device),
        )
        # The strategy packs the gate once when it is built; the launch reads the pack.
        first["gate"] = ops.pack_router_weight(first["gate"])
        sets = _copies(first, copies)
        for entry in sets:
            entry["gate"], entry["w"] = first["gate"], first["w"]
        return sets

    out.append(Workload(
        name="residual_rms_router",
        kernel="residual_rms_router_split_kernel",
        description="x, residual bf16 [4096, 2048] ~N(0,1), norm weight 1+N(0,0.1), router "
                    "[128, 2048] ~N(0,0.02) (packed once) -> summed, normed, top-8 indices + "
                    "fp32 weights",
        bytes_per_launch=4 * 4096 * 2048 * 2 + 2048 * 2 + 128 * 2048 * 2 + 128 * 4 + 2 * 4096 * 8 * 4,
        setup=setup_router,
        launch=lambda a: ops.residual_rms_router(
            a["x"], a["r"], a["w"], a["gate"], k=8, eps=1e-6, summed=a["s"],
            normalized=a["n"], indices=a["idx"], weights=a["wts"]),
    ))

    # configs[4] with the bf16 logits written as well (BASELINE.md prices them at +1 MiB):
    # every logit made exact, the unsure ones recomputed in fp64 by their token's wave.
    def setup_router_logits(device, copies):
        sets = setup_router(device, copies)
        for entry in sets:
            entry["l"] = torch.empty((4096, 128), dtype=torch.bfloat16, device=device)
        return sets

    out.append(Workload(
        name="residual_rms_router_logits",
        kernel="residual_rms_router_split_kernel",
        description="configs[4]'s fused router writing its bf16 logits [4096, 128] too (every "
                    "logit the correctly rounded dot product)",
        bytes_per_launch=4 * 4096 * 2048 * 2 + 2048 * 2 + 128 * 2048 * 2 + 128 * 4
        + 2 * 4096 * 8 * 4 + 4096 * 128 * 2,
        setup=setup_router_logits,
        launch=lambda a: ops.residual_rms_router(
            a["x"], a["r"], a["w"], a["gate"], k=8, eps=1e-6, summed=a["s"],
            normalized=a["n"], logits=a["l"], indices=a["idx"], weights=a["wts"]),
    ))

    # configs[4]'s step at Qwen3-235B-A22B's width (hidden 4096, 128 experts, top-8): the
    # fused router's other kernel (phases one after another). Run when named by --only.
    out.append(Workload(
        name="residual_rms_router_h4096",
        kernel="residual_rms_router_kernel",
        description="x, residual bf16 [4096, 4096] ~N(0,1), norm weight 1+N(0,0.1), router [128, 4096] "
                    "~N(0,0.02) (packed once) -> summed, normed, top-8 indices + fp32 weights",
        bytes_per_launch=4 * 4096 * 4096 * 2 + 4096 * 2 + 128 * 4096 * 2 + 128 * 4 + 2 * 4096 * 8 * 4,
        setup=lambda device, copies: setup_router(device, copies, hidden=4096),
        launch=lambda a: ops.residual_rms_router(
            a["x"], a["r"], a["w"], a["gate"], k=8, eps=1e-6, summed=a["s"],
            normalized=a["n"], indices=a["idx"], weights=a["wts"]),
        default=False,
    ))

    # The routing of configs[4] on its own, in the softmax form and in the reference's
    # sigmoid-with-bias form (route/softmax_topk.py, route/ordinal.py), and the fused
    # router in that sigmoid form (route/residual.py): 4096 tokens, 128 experts, top-8.
    def setup_route(device, copies, rows=4096, experts=128, k=8):
        rng = np.random.default_rng(9)
        bias = torch.from_numpy(_normal(rng, (experts,), 0.5)).to(device)
        first = dict(logits=_to_bf16_device(_normal(rng, (rows, experts)), device), bias=bias,
                     idx=torch.empty((rows, k), dtype=torch.int32, device=device),
                     wts=torch.empty((rows, k), dtype=torch.float32, device=device))
        sets = _copies(first, copies)
        for entry in sets:
            entry["bias"] = bias
        return sets

    out.append(Workload(
        name="softmax_topk",
        kernel="softmax_topk_kernel",
        description="router logits bf16 [4096, 128] ~N(0,1) -> top-8 indices + renormalised fp32 "
                    "softmax weights",
        bytes_per_launch=4096 * 128 * 2 + 2 * 4096 * 8 * 4,
        setup=setup_route,
        launch=lambda a: ops.softmax_topk(a["logits"], 8, indices=a["idx"], weights=a["wts"]),
    ))

    def setup_route_shared(device, copies, rows=4096, experts=128, k=8):
        rng = np.random.default_rng(19)
        first = dict(logits=_to_bf16_device(_normal(rng, (rows, experts + 1)), device),
                     idx=torch.empty((rows, k + 1), dtype=torch.int32, device=device),
                     wts=torch.empty((rows, k + 1), dtype=torch.float32, device=device))
        return _copies(first, copies)

    out.append(Workload(
        name="softmax_topk_shared",
        kernel="softmax_topk_kernel",
        description="router logits bf16 [4096, 128 + 1 shared gate] -> top-8 indices + fp32 softmax "
                    "probabilities (normalize=False) + the shared slot's sigmoid (Qwen3.5 / Qwen3 forms)",
        bytes_per_launch=4096 * 129 * 2 + 2 * 4096 * 9 * 4,
        setup=setup_route_shared,
        launch=lambda a: ops.softmax_topk(a["logits"], 8, normalize=False, shared=True,
                                          indices=a["idx"], weights=a["wts"]),
    ))
    out.append(Workload(
        name="sigmoid_topk",
        kernel="sigmoid_topk_kernel",
        description="router logits bf16 [4096, 128] ~N(0,1), correction bias fp32 [128] -> ordinal "
                    "top-8 indices + fp32 weights from the unbiased scores",
        bytes_per_launch=4096 * 128 * 2 + 128 * 4 + 2 * 4096 * 8 * 4,
        setup=setup_route,
        launch=lambda a: ops.sigmoid_topk(a["logits"], a["bias"], 8, indices=a["idx"], weights=a["wts"]),
    ))

    def setup_router_sigmoid(device, copies, rows=4096):
        sets = setup_router(device, copies, rows=rows)
        bias = torch.from_numpy(_normal(np.random.default_rng(10), (128,), 0.5)).to(device)
        for entry in sets:
            entry["bias"] = bias
        return sets

    out.append(Workload(
        name="residual_rms_router_sigmoid",
        kernel="residual_rms_router_split_kernel",
        description="configs[4]'s fused router in the sigmoid form: the same inputs and a correction "
                    "bias fp32 [128] -> summed, normed, ordinal top-8 indices + fp32 weights",
        bytes_per_launch=4 * 4096 * 2048 * 2 + 2048 * 2 + 128 * 2048 * 2 + 128 * 4 + 128 * 4
        + 2 * 4096 * 8 * 4,
        setup=setup_router_sigmoid,
        launch=lambda a: ops.residual_rms_router_sigmoid(
            a["x"], a["r"], a["w"], a["gate"], a["bias"], k=8, eps=1e-6, emit_logits=False,
            emit_keys=False, select=True, summed=a["s"], normalized=a["n"], indices=a["idx"],
            weights=a["wts"]),
    ))

    def setup_router_sigmoid_keys(device, copies):
        sets = setup_router_sigmoid(device, copies)
        for entry in sets:
            entry["l"] = torch.empty((4096, 128), dtype=torch.bfloat16, device=device)
            entry["k"] = torch.empty((4096, 128), dtype=torch.uint32, device=device)
        return sets

    out.append(Workload(
        name="residual_rms_router_sigmoid_keys",
        kernel="residual_rms_router_split_kernel",
        description="the sigmoid form writing the reference's outputs too: bf16 logits and uint32 "
                    "ordinal keys [4096, 128], with the top-8 selection",
        bytes_per_launch=4 * 4096 * 2048 * 2 + 2048 * 2 + 128 * 2048 * 2 + 128 * 4 + 128 * 4
        + 2 * 4096 * 8 * 4 + 4096 * 128 * (2 + 4),
        setup=setup_router_sigmoid_keys,
        launch=lambda a: ops.residual_rms_router_sigmoid(
            a["x"], a["r"], a["w"], a["gate"], a["bias"], k=8, eps=1e-6, select=True,
            summed=a["s"], normalized=a["n"], logits=a["l"], keys=a["k"], indices=a["idx"],
            weights=a["wts"]),
    ))

    # One token (a decode step), the reference's own case for the fused router
    # (route/residual.py:117-299, T = 1): the softmax form with its selection, and the
    # sigmoid form writing the bf16 logits and the ordinal keys as the reference does.
    def setup_router_one(device, copies):
        sets = setup_router_sigmoid(device, copies, rows=1)
        for entry in sets:
            entry["logits"] = torch.empty((1, 128), dtype=torch.bfloat16, device=device)
            entry["keys"] = torch.empty((1, 128), dtype=torch.uint32, device=device)
        return sets

    out.append(Workload(
        name="residual_rms_router_decode",
        kernel="router_decode_logits_kernel",
        description="one token: x, residual bf16 [1, 2048], router [128, 2048] (packed once) -> summed, "
                    "normed, bf16 logits (the facade asks for them at a decode step), top-8 indices + "
                    "fp32 weights",
        bytes_per_launch=4 * 2048 * 2 + 2048 * 2 + 128 * 2048 * 2 + 128 * 4 + 128 * 2 + 2 * 8 * 4,
        setup=setup_router_one,
        launch=lambda a: ops.residual_rms_router(
            a["x"], a["r"], a["w"], a["gate"], k=8, eps=1e-6, summed=a["s"],
            normalized=a["n"], logits=a["logits"], indices=a["idx"], weights=a["wts"]),
    ))
    out.append(Workload(
        name="residual_rms_router_sigmoid_decode",
        kernel="router_decode_logits_kernel",
        description="one token, sigmoid form with a correction bias fp32 [128]: summed, normed, bf16 "
                    "logits and uint32 ordinal keys (the reference's outputs)",
        bytes_per_launch=4 * 2048 * 2 + 2048 * 2 + 128 * 2048 * 2 + 128 * 4 + 128 * 4 + 128 * 2 + 128 * 4,
        setup=setup_router_one,
        launch=lambda a: ops.residual_rms_router_sigmoid(
            a["x"], a["r"], a["w"], a["gate"], a["bias"], k=8, eps=1e-6, summed=a["s"],
            normalized=a["n"], logits=a["logits"], keys=a["keys"]),
    ))

    # The angle atlas the table-driven rotation reads (laguna/layers/attention.py:171-196):
    # 40,960 positions x 64 pairs, cos || sin fp32, built on the device.
    def setup_atlas(device, copies, rows=40960):
        freqs = torch.from_numpy(np.exp(-np.log(1e6) * np.arange(pairs) / pairs)).to(device)
        return [dict(f=freqs, out=torch.empty((rows, 2 * pairs), dtype=torch.float32, device=device))
                for _ in range(copies)]

    out.append(Workload(
        name="rope_angle_atlas",
        kernel="rope_atlas_kernel",
        description="cos || sin atlas [40960, 2 x 64] fp32 from fp64 frequencies of theta=1e6",
        bytes_per_launch=40960 * 2 * pairs * 4 + pairs * 8,
        setup=setup_atlas,
        launch=lambda a: ops.rope_angle_atlas(a["f"], 0, 40960, out=a["out"]),
    ))

    # embedding gather + cos/sin atlas rows.
    def setup_embed(device, copies, vocab=151936, hidden=2560, batch=8, length=2048):
        rng = np.random.default_rng(4)
        table = _to_bf16_device(_normal(rng, (vocab, hidden), 0.02), device)
        cos, sin = make_tables(device)
        sets = []
        for _ in range(copies):
            sets.append(dict(
                table=table, cos=cos, sin=sin,
                ids=torch.from_numpy(rng.integers(0, vocab, (batch, length), dtype=np.int32)).to(device),
                out=torch.empty((batch, length, hidden), dtype=torch.bfloat16, device=device),
                fo=torch.empty((length, pairs), dtype=torch.float32, device=device),
                so=torch.empty((length, pairs), dtype=torch.float32, device=device),
            ))
        return sets

    out.append(Workload(
        name="embed_atlas",
        kernel="embed_atlas_kernel",
        description="table [151936,2560] bf16 ~N(0,0.02), ids [8,2048] int32 uniform, "
                    "cos/sin atlases [40960,64] fp32 theta=1e6, positions 0..2047",
        bytes_per_launch=8 * 2048 * 4 + 2 * 8 * 2048 * 2560 * 2 + 2 * 2048 * 2 * pairs * 4,
        setup=setup_embed,
        launch=lambda a: ops.embed_atlas(
            a["ids"], a["table"], a["cos"], a["sin"], position=0, n_positions=2048,
            hidden_out=a["out"], full_out=a["fo"], sliding_out=a["so"]),
    ))
    # Next after the path: the routed expert MLP of a one-token step at Qwen3-30B-A3B's
    # shape (hidden 2048, moe inner 768, 128 experts, top-8), dense bf16 weights, the
    # "blocked" gate||up layout. The weight stacks are shared parameters (805 MB and
    # 403 MB); each argument set routes to its own random experts.
    moe_e, moe_h, moe_i, moe_k = 128, 2048, 768, 8
    moe_stacks = {}

    def moe_weights(device):
        if not moe_stacks:
            gen = torch.Generator(device=device).manual_seed(8)
            for name, shape in (("gate_up", (moe_e, 2 * moe_i, moe_h)), ("down", (moe_e, moe_h, moe_i))):
                stack = torch.empty(shape, dtype=torch.bfloat16, device=device)
                for e in range(moe_e):  # one expert at a time: bounded fp32 scratch
                    stack[e] = (0.02 * torch.randn(shape[1:], generator=gen, device=device)).to(torch.bfloat16)
                moe_stacks[name] = stack
        return moe_stacks

    def setup_moe(device, copies, down=False):
        rng = np.random.default_rng(9)
        stacks = moe_weights(device)
        sets = []
        for _ in range(copies):
            chosen = torch.from_numpy(rng.choice(moe_e, size=moe_k, replace=False).astype(np.int32)).to(device)
            entry = dict(gu=stacks["gate_up"], dn=stacks["down"], ids=chosen,
                         x=_to_bf16_device(_normal(rng, (moe_h,)), device),
                         act=_to_bf16_device(_normal(rng, (moe_k, 2 * moe_i)), device),
                         w=torch.from_numpy(rng.dirichlet(np.ones(moe_k)).astype(np.float32)).to(device),
                         r=_to_bf16_device(_normal(rng, (moe_h,)), device))
            entry["y"] = torch.empty((moe_k, 2 * moe_i), dtype=torch.bfloat16, device=device)
            entry["o"] = torch.empty((moe_h,), dtype=torch.bfloat16, device=device)
            sets.append(entry)
        return sets

    out.append(Workload(
        name="moe_gate_up_decode",
        kernel="moe_gate_up_kernel",
        description="x [2048] bf16 x 8 of 128 experts' [1536, 2048] bf16 gate||up stacks "
                    "(Qwen3-30B-A3B, T=1) -> [8, 1536] bf16",
        bytes_per_launch=moe_k * 2 * moe_i * moe_h * 2 + moe_h * 2 + moe_k * 4 + moe_k * 2 * moe_i * 2,
        setup=setup_moe,
        launch=lambda a: ops.moe_gate_up(a["x"], a["gu"], a["ids"], out=a["y"]),
    ))
    out.append(Workload(
        name="moe_down_combine_decode",
        kernel="moe_down_kernel",
        description="silu(gate)*up of [8, 1536] x 8 of 128 experts' [2048, 768] bf16 down "
                    "stacks, routing weights, expert sum, residual (Qwen3-30B-A3B, T=1)",
        bytes_per_launch=moe_k * moe_h * moe_i * 2 + moe_k * 2 * moe_i * 2 + moe_k * 8 + 2 * moe_h * 2,
        setup=lambda device, copies: setup_moe(device, copies, down=True),
        launch=lambda a: ops.moe_down_combine(a["act"], a["dn"], a["ids"], a["w"], a["r"], out=a["o"]),
    ))

    # The same routed MLP over 4-bit affine stacks, groups of 64 (the common MLX
    # quantization of Qwen3-30B-A3B): random words, scales of a checkpoint's size and
    # centring biases, gate/up rows interleaved. A 4-bit layer's stacks (226 MB + 113 MB)
    # fit in the 256 MB Infinity Cache, so the copies cycle over four layers' stacks.
    aff_bits, aff_group, aff_layers = 4, 64, 4
    affine_stacks: list = []

    def affine_weights(device):
        if not affine_stacks:
            gen = torch.Generator(device=device).manual_seed(10)
            for _ in range(aff_layers):
                layer = {}
                for name, rows, features in (("gate_up", 2 * moe_i, moe_h), ("down", moe_h, moe_i)):
                    words = torch.randint(-2**31, 2**31, (moe_e, rows, features * aff_bits // 32),
                                          generator=gen, device=device, dtype=torch.int32)
                    scale = 4.0 / ((1 << aff_bits) * features ** 0.5)
                    groups = (moe_e, rows, features // aff_group)
                    scales = (scale * (0.5 + torch.rand(groups, generator=gen, device=device))).to(torch.bfloat16)
                    biases = (-scales.float() * ((1 << aff_bits) - 1) / 2).to(torch.bfloat16)
                    layer[name] = ops.AffineLeaf(words, scales, biases, aff_bits, aff_group)
                affine_stacks.append(layer)
        return affine_stacks

    def setup_moe_affine(device, copies):
        rng = np.random.default_rng(11)
        layers = affine_weights(device)
        sets = []
        for i in range(copies):
            stacks = layers[i % aff_layers]
            chosen = torch.from_numpy(rng.choice(moe_e, size=moe_k, replace=False).astype(np.int32)).to(device)
            sets.append(dict(gu=stacks["gate_up"], dn=stacks["down"], ids=chosen,
                             x=_to_bf16_device(_normal(rng, (moe_h,)), device),
                             act=_to_bf16_device(_normal(rng, (moe_k, moe_i)), device),
                             w=torch.from_numpy(rng.dirichlet(np.ones(moe_k)).astype(np.float32)).to(device),
                             r=_to_bf16_device(_normal(rng, (moe_h,)), device),
                             y=torch.empty((moe_k, moe_i), dtype=torch.bfloat16, device=device),
                             o=torch.empty((moe_h,), dtype=torch.bfloat16, device=device)))
        return sets

    def affine_row_bytes(features):
        return features * aff_bits // 8 + 2 * 2 * (features // aff_group)

    out.append(Workload(
        name="moe_affine_gate_up_decode",
        kernel="moe_gate_up_affine_kernel",
        description="x [2048] bf16 x 8 of 128 experts' 4-bit affine (group 64) interleaved "
                    "gate||up stacks [1536, 2048] -> silu(gate)*up [8, 768] bf16 (Qwen3-30B-A3B, T=1)",
        bytes_per_launch=moe_k * 2 * moe_i * affine_row_bytes(moe_h) + moe_h * 2 + moe_k * 4 + moe_k * moe_i * 2,
        setup=setup_moe_affine,
        launch=lambda a: ops.moe_gate_up_affine(a["x"], a["gu"], a["ids"], out=a["y"]),
    ))
    out.append(Workload(
        name="moe_affine_down_combine_decode",
        kernel="moe_down_affine_kernel",
        description="activation [8, 768] x 8 of 128 experts' 4-bit affine (group 64) down "
                    "stacks [2048, 768], routing weights, slot sum, residual (Qwen3-30B-A3B, T=1)",
        bytes_per_launch=moe_k * moe_h * affine_row_bytes(moe_i) + moe_k * moe_i * 2 + moe_k * 8 + 2 * moe_h * 2,
        setup=setup_moe_affine,
        launch=lambda a: ops.moe_down_combine_affine(a["act"], a["dn"], a["ids"], a["w"], a["r"], out=a["o"]),
    ))

    # The routed MLP of gpt-oss-120b (hidden 2880, inner 2880, 128 experts, top-4) over its
    # MXFP4 stacks: random e2m1 words, e8m0 scales near 2^-6, a bf16 projection bias,
    # gate/up rows interleaved, the clamp at 7. One layer's stacks (1.13 GB + 0.56 GB)
    # dwarf the Infinity Cache; each argument set routes to its own random experts.
    mx_e, mx_h, mx_i, mx_k, mx_limit = 128, 2880, 2880, 4, 7.0
    mxfp4_stacks: dict = {}

    def mxfp4_weights(device):
        if not mxfp4_stacks:
            gen = torch.Generator(device=device).manual_seed(12)
            for name, rows, features in (("gate_up", 2 * mx_i, mx_h), ("down", mx_h, mx_i)):
                words = torch.randint(-2**31, 2**31, (mx_e, rows, features // 8), generator=gen,
                                      device=device, dtype=torch.int32)
                scales = torch.randint(119, 123, (mx_e, rows, features // 32), generator=gen,
                                       device=device, dtype=torch.int32).to(torch.uint8)
                bias = (0.25 * torch.randn((mx_e, rows), generator=gen, device=device)).to(torch.bfloat16)
                mxfp4_stacks[name] = ops.Mxfp4Leaf(words, scales, bias)
        return mxfp4_stacks

    def setup_moe_mxfp4(device, copies):
        rng = np.random.default_rng(13)
        stacks = mxfp4_weights(device)
        sets = []
        for _ in range(copies):
            chosen = torch.from_numpy(rng.choice(mx_e, size=mx_k, replace=False).astype(np.int32)).to(device)
            sets.append(dict(gu=stacks["gate_up"], dn=stacks["down"], ids=chosen,
                             x=_to_bf16_device(_normal(rng, (mx_h,)), device),
                             act=_to_bf16_device(_normal(rng, (mx_k, mx_i)), device),
                             w=torch.from_numpy(rng.dirichlet(np.ones(mx_k)).astype(np.float32)).to(device),
                             r=_to_bf16_device(_normal(rng, (mx_h,)), device),
                             y=torch.empty((mx_k, mx_i), dtype=torch.bfloat16, device=device),
                             o=torch.empty((mx_h,), dtype=torch.bfloat16, device=device)))
        return sets

    def mxfp4_row_bytes(features):
        return features // 2 + features // 32 + 2       # codes, e8m0 scales, the row's bias

    out.append(Workload(
        name="moe_mxfp4_gate_up_decode",
        kernel="moe_gate_up_mxfp4_kernel",
        description="x [2880] bf16 x 4 of 128 experts' MXFP4 interleaved gate||up stacks "
                    "[5760, 2880] + bias -> clamped swiglu_oai [4, 2880] bf16 (gpt-oss-120b, T=1)",
        bytes_per_launch=mx_k * 2 * mx_i * mxfp4_row_bytes(mx_h) + mx_h * 2 + mx_k * 4 + mx_k * mx_i * 2,
        setup=setup_moe_mxfp4,
        launch=lambda a: ops.moe_gate_up_mxfp4(a["x"], a["gu"], a["ids"], limit=mx_limit, out=a["y"]),
    ))
    out.append(Workload(
        name="moe_mxfp4_down_combine_decode",
        kernel="moe_down_mxfp4_kernel",
        description="activation [4, 2880] x 4 of 128 experts' MXFP4 down stacks [2880, 2880] + "
                    "bias, routing weights, slot sum, residual (gpt-oss-120b, T=1)",
        bytes_per_launch=mx_k * mx_h * mxfp4_row_bytes(mx_i) + mx_k * mx_i * 2 + mx_k * 8 + 2 * mx_h * 2,
        setup=setup_moe_mxfp4,
        launch=lambda a: ops.moe_down_combine_mxfp4(a["act"], a["dn"], a["ids"], a["w"], a["r"], out=a["o"]),
    ))

    # Qwen3-30B-A3B's routed MLP over NVFP4 stacks (e2m1 codes, an e4m3 scale per 16
    # values, the interleaved layout, the plain SwiGLU): random words and scales near
    # 2^-4. A layer's stacks (226 MB + 113 MB) fit the Infinity Cache, so the copies cycle
    # over four layers' stacks, as for the affine stacks.
    nv_layers = 4
    nvfp4_stacks: list = []

    def nvfp4_weights(device):
        if not nvfp4_stacks:
            gen = torch.Generator(device=device).manual_seed(14)
            for _ in range(nv_layers):
                layer = {}
                for name, rows, features in (("gate_up", 2 * moe_i, moe_h), ("down", moe_h, moe_i)):
                    words = torch.randint(-2**31, 2**31, (moe_e, rows, features // 8), generator=gen,
                                          device=device, dtype=torch.int32)
                    scales = torch.randint(0x18, 0x28, (moe_e, rows, features // 16), generator=gen,
                                           device=device, dtype=torch.int32).to(torch.uint8)
                    layer[name] = ops.Nvfp4Leaf(words, scales, None)
                nvfp4_stacks.append(layer)
        return nvfp4_stacks

    def setup_moe_nvfp4(device, copies):
        rng = np.random.default_rng(15)
        layers = nvfp4_weights(device)
        sets = []
        for i in range(copies):
            stacks = layers[i % nv_layers]
            chosen = torch.from_numpy(rng.choice(moe_e, size=moe_k, replace=False).astype(np.int32)).to(device)
            sets.append(dict(gu=stacks["gate_up"], dn=stacks["down"], ids=chosen,
                             x=_to_bf16_device(_normal(rng, (moe_h,)), device),
                             act=_to_bf16_device(_normal(rng, (moe_k, moe_i)), device),
                             w=torch.from_numpy(rng.dirichlet(np.ones(moe_k)).astype(np.float32)).to(device),
                             r=_to_bf16_device(_normal(rng, (moe_h,)), device),
                             y=torch.empty((moe_k, moe_i), dtype=torch.bfloat16, device=device),
                             o=torch.empty((moe_h,), dtype=torch.bfloat16, device=device)))
        return sets

    def nvfp4_row_bytes(features):
        return features // 2 + features // 16          # codes and e4m3 scales

    out.append(Workload(
        name="moe_nvfp4_gate_up_decode",
        kernel="moe_gate_up_nvfp4_kernel",
        description="x [2048] bf16 x 8 of 128 experts' NVFP4 interleaved gate||up stacks [1536, 2048] "
                    "-> silu(gate)*up [8, 768] bf16 (Qwen3-30B-A3B, T=1)",
        bytes_per_launch=moe_k * 2 * moe_i * nvfp4_row_bytes(moe_h) + moe_h * 2 + moe_k * 4 + moe_k * moe_i * 2,
        setup=setup_moe_nvfp4,
        launch=lambda a: ops.moe_gate_up_nvfp4(a["x"], a["gu"], a["ids"], out=a["y"]),
    ))
    def setup_moe_nvfp4_ordinal(device, copies):
        sets = setup_moe_nvfp4(device, copies)
        rng = np.random.default_rng(16)
        for entry in sets:   # the router's ordinal keys over all experts
            entry["keys"] = torch.from_numpy(rng.permutation(moe_e).astype(np.uint32)).to(device)
        return sets

    out.append(Workload(
        name="moe_nvfp4_gate_up_ordinal_decode",
        kernel="moe_gate_up_nvfp4_kernel",
        description="the same NVFP4 gate/up with the top-8 of 128 ordinal keys ranked in the kernel "
                    "(Qwen3-30B-A3B, T=1)",
        bytes_per_launch=moe_k * 2 * moe_i * nvfp4_row_bytes(moe_h) + moe_h * 2 + moe_e * 4 + moe_k * moe_i * 2,
        setup=setup_moe_nvfp4_ordinal,
        launch=lambda a: ops.moe_gate_up_nvfp4_ordinal(a["x"], a["gu"], a["keys"], moe_k, out=a["y"]),
    ))
    out.append(Workload(
        name="moe_nvfp4_down_combine_decode",
        kernel="moe_down_nvfp4_kernel",
        description="activation [8, 768] x 8 of 128 experts' NVFP4 down stacks [2048, 768], routing "
                    "weights, slot sum, residual (Qwen3-30B-A3B, T=1)",
        bytes_per_launch=moe_k * moe_h * nvfp4_row_bytes(moe_i) + moe_k * moe_i * 2 + moe_k * 8 + 2 * moe_h * 2,
        setup=setup_moe_nvfp4,
        launch=lambda a: ops.moe_down_combine_nvfp4(a["act"], a["dn"], a["ids"], a["w"], a["r"], out=a["o"]),
    ))

    # The packed NVFP4 down/combine (core/kernels/down_combine/nvfp4_packed.py) at
    # Qwen3-Next-80B-A3B's sparse block: hidden 2048, inner 512, 512 experts, top-10 plus
    # the shared expert on the last slot, one token. Two layers' routed stacks (302 MB
    # each) alternate, and every argument set holds its own shared stack, so nothing the
    # timed loop reads stays in the 256 MB Infinity Cache between its visits.
    nx_h, nx_i, nx_e, nx_k, nx_layers = 2048, 512, 512, 10, 2
    nx_stacks: list = []

    def setup_moe_nvfp4_shared(device, copies):
        gen = torch.Generator(device=device).manual_seed(17)

        def stack(*lead):
            words = torch.randint(-2**31, 2**31, (*lead, nx_h, nx_i // 8), generator=gen, device=device,
                                  dtype=torch.int32)
            scales = torch.randint(0x18, 0x28, (*lead, nx_h, nx_i // 32), generator=gen, device=device,
                                   dtype=torch.int32).to(torch.uint8).repeat_interleave(2, dim=-1)
            return ops.Nvfp4Leaf(words, scales, None)

        if not nx_stacks:
            nx_stacks.extend(stack(nx_e) for _ in range(nx_layers))
        rng = np.random.default_rng(18)
        sets = []
        for i in range(copies):
            chosen = rng.choice(nx_e, size=nx_k, replace=False).astype(np.int32)[None]
            sets.append(dict(dn=nx_stacks[i % nx_layers], sh=stack(1),
                             ids=torch.from_numpy(chosen).to(device),
                             act=_to_bf16_device(_normal(rng, (1, nx_k + 1, nx_i)), device),
                             w=torch.from_numpy(rng.dirichlet(np.ones(nx_k)).astype(np.float32)[None]).to(device),
                             r=_to_bf16_device(_normal(rng, (1, nx_h)), device),
                             o=torch.empty((1, nx_h), dtype=torch.bfloat16, device=device)))
        return sets

    out.append(Workload(
        name="moe_nvfp4_shared_down_combine_decode",
        kernel="moe_down_nvfp4_shared_kernel",
        description="activation [11, 512] x 10 of 512 experts' NVFP4 down stacks [2048, 512] and the "
                    "shared expert's, bf16 routing sum, residual (Qwen3-Next-80B-A3B, T=1)",
        bytes_per_launch=(nx_k + 1) * nx_h * nvfp4_row_bytes(nx_i) + (nx_k + 1) * nx_i * 2 + nx_k * 8
        + 2 * nx_h * 2,
        setup=setup_moe_nvfp4_shared,
        launch=lambda a: ops.moe_down_combine_nvfp4_shared(a["act"], a["dn"], a["sh"], a["ids"], a["w"], a["r"],
                                                           out=a["o"]),
    ))

    # Next after the routed MLP: the dense SwiGLU MLP of a one-token step at Qwen3-4B's
    # shape (hidden 2560, inner 9728: config 4's inner dimension), bf16 weights, gate rows
    # first. Each argument set holds its own weights, as each layer of a model does.
    mlp_h, mlp_i = 2560, 9728

    def setup_mlp(device, copies, down=False):
        rng = np.random.default_rng(10)
        gen = torch.Generator(device=device).manual_seed(11)
        sets = []
        for _ in range(copies):
            shape = (mlp_h, mlp_i) if down else (2 * mlp_i, mlp_h)
            weight = (torch.randn(shape, generator=gen, device=device) / np.sqrt(shape[1])).to(torch.bfloat16)
            entry = dict(w=weight, x=_to_bf16_device(_normal(rng, (mlp_h,)), device),
                         act=_to_bf16_device(_normal(rng, (mlp_i,)), device),
                         r=_to_bf16_device(_normal(rng, (mlp_h,)), device))
            entry["y"] = torch.empty((mlp_i,), dtype=torch.bfloat16, device=device)
            entry["o"] = torch.empty((mlp_h,), dtype=torch.bfloat16, device=device)
            sets.append(entry)
        return sets

    out.append(Workload(
        name="dense_mlp_gate_up_decode",
        kernel="dense_gate_up_swiglu_kernel",
        description="x [2560] bf16 x fused gate||up [19456, 2560] bf16 -> bf16 SwiGLU [9728] "
                    "(Qwen3-4B MLP, T=1)",
        bytes_per_launch=2 * mlp_i * mlp_h * 2 + mlp_h * 2 + mlp_i * 2,
        setup=setup_mlp,
        launch=lambda a: ops.dense_gate_up_swiglu(a["x"], a["w"], out=a["y"]),
    ))
    out.append(Workload(
        name="dense_mlp_down_decode",
        kernel="dense_down_residual_kernel",
        description="act [9728] bf16 x down [2560, 9728] bf16 + residual [2560] -> [2560] bf16 "
                    "(Qwen3-4B MLP, T=1)",
        bytes_per_launch=mlp_h * mlp_i * 2 + mlp_i * 2 + 2 * mlp_h * 2,
        setup=lambda device, copies: setup_mlp(device, copies, down=True),
        launch=lambda a: ops.dense_down_residual(a["act"], a["w"], a["r"], out=a["o"]),
    ))

    # Decode attention over a KV cache at Qwen3-4B's geometry (32 query heads over 8 kv
    # heads, head_dim 128, full rotary): the step at position 32767 of a 32768-row fixed
    # cache (134 MB of keys and values read) and at position 4095 of a 4096-row one.
    att_h, att_kv, att_d, att_p = 32, 8, 128, 64

    def setup_attention(device, copies, rows):
        rng = np.random.default_rng(12)
        gen = torch.Generator(device=device).manual_seed(13)
        inv = np.exp(-np.log(1e6) * np.arange(att_p) / att_p)
        theta = np.arange(rows)[:, None] * inv[None, :]
        atlas = torch.from_numpy(np.concatenate([np.cos(theta), np.sin(theta)], axis=1).astype(np.float32)).to(device)
        position = torch.tensor([rows - 1], dtype=torch.int32, device=device)
        workspace = torch.empty(ops.attention_workspace_bytes(att_h, att_kv, att_d, rows),
                                dtype=torch.uint8, device=device)
        sets = []
        for _ in range(copies):
            shape = (att_kv, rows, att_d)
            entry = dict(kc=torch.randn(shape, generator=gen, device=device).to(torch.bfloat16),
                         vc=torch.randn(shape, generator=gen, device=device).to(torch.bfloat16),
                         q=_to_bf16_device(_normal(rng, (att_h * att_d,)), device),
                         k=_to_bf16_device(_normal(rng, (att_kv * att_d,)), device),
                         v=_to_bf16_device(_normal(rng, (att_kv * att_d,)), device),
                         qw=_to_bf16_device(_normal(rng, (att_d,), 0.1, 1.0), device),
                         kw=_to_bf16_device(_normal(rng, (att_d,), 0.1, 1.0), device),
                         atlas=atlas, pos=position, ws=workspace, rows=rows)
            entry["o"] = torch.empty((att_h, att_d), dtype=torch.bfloat16, device=device)
            sets.append(entry)
        return sets

    def attention_bytes(rows):
        # K and V rows attended (the written row included), q/k/v in, context out, the new
        # K/V row written, norm weights and the angle row.
        return (2 * att_kv * rows * att_d * 2 + (att_h + 2 * att_kv) * att_d * 2
                + att_h * att_d * 2 + 2 * att_kv * att_d * 2 + 2 * att_d * 2 + 2 * att_p * 4)

    for rows, tag in ((32768, "32k"), (4096, "4k")):
        out.append(Workload(
            name=f"attention_decode_{tag}",
            kernel="attention_split_kernel",
            description=f"decode step: q [32x128], k, v [8x128] bf16, norm + rope + cache write, "
                        f"attention over {rows} cached rows [8, {rows}, 128] bf16 (Qwen3-4B geometry)",
            bytes_per_launch=attention_bytes(rows),
            setup=lambda device, copies, rows=rows: setup_attention(device, copies, rows),
            launch=lambda a: ops.attention_decode(
                a["q"], a["k"], a["v"], a["qw"], a["kw"], a["atlas"], a["kc"], a["vc"], a["pos"],
                heads=att_h, kv_heads=att_kv, max_rows=a["rows"], scale=att_d ** -0.5, eps=1e-6,
                workspace=a["ws"], out=a["o"]),
        ))

    # The attention of a layer with learned sinks (core/kernels/attention/sink.py) at
    # gpt-oss-120b's geometry: 64 query heads over 8 kv heads, head_dim 64, the full
    # layer over 32,768 and 4,096 cached rows (the roped query in, the context out).
    sk_h, sk_kv, sk_d = 64, 8, 64

    def setup_attention_sink(device, copies, rows):
        rng = np.random.default_rng(19)
        gen = torch.Generator(device=device).manual_seed(20)
        sinks = _to_bf16_device(_normal(rng, (sk_h,), 2.0), device)
        workspace = torch.empty(max(ops.attention_sink_workspace_bytes(sk_h, sk_kv, rows) // 4, 1),
                                dtype=torch.float32, device=device)
        sets = []
        for _ in range(copies):
            shape = (1, sk_kv, rows, sk_d)
            sets.append(dict(kc=torch.randn(shape, generator=gen, device=device).to(torch.bfloat16),
                             vc=torch.randn(shape, generator=gen, device=device).to(torch.bfloat16),
                             q=_to_bf16_device(_normal(rng, (sk_h, sk_d)), device), sinks=sinks, ws=workspace,
                             o=torch.empty((sk_h, sk_d), dtype=torch.bfloat16, device=device)))
        return sets

    for rows, tag in ((32768, "32k"), (4096, "4k")):
        out.append(Workload(
            name=f"attention_sink_decode_{tag}",
            kernel="sink_split_kernel",
            description=f"one query per head, 64 heads over 8 kv heads, head_dim 64, learned sinks, attention "
                        f"over {rows} cached rows [8, {rows}, 64] bf16 (gpt-oss-120b geometry)",
            bytes_per_launch=2 * sk_kv * rows * sk_d * 2 + 2 * sk_h * sk_d * 2 + sk_h * 2,
            setup=lambda device, copies, rows=rows: setup_attention_sink(device, copies, rows),
            launch=lambda a: ops.attention_sink_decode(a["q"], a["kc"], a["vc"], a["sinks"], None, sk_d ** -0.5,
                                                       workspace=a["ws"], out=a["o"]),
        ))

    # Not a product kernel: a plain device-to-device copy of known size, the scale for
    # the FETCH_SIZE / WRITE_SIZE counters (run with --only copy_calibration).
    def setup_copy(device, copies, elements=64 * 2**20):
        first = dict(src=torch.ones(elements, dtype=torch.bfloat16, device=device),
                     dst=torch.empty(elements, dtype=torch.bfloat16, device=device))
        return _copies(first, copies)

    out.append(Workload(
        name="copy_calibration",
        kernel="stream_copy_kernel",
        description="omnia_stream_copy of 128 MiB (one 16-byte vector per thread): 128 MiB read "
                    "+ 128 MiB written",
        bytes_per_launch=2 * 64 * 2**20 * 2,
        setup=setup_copy,
        launch=lambda a: ops.stream_copy(a["src"], a["dst"]),
        default=False,
    ))
    out.append(Workload(
        name="copy_calibration_torch",
        kernel="copy",
        description="torch copy_ of 128 MiB bf16 (64 Mi elements): 128 MiB read + 128 MiB written",
        bytes_per_launch=2 * 64 * 2**20 * 2,
        setup=setup_copy,
        launch=lambda a: a["dst"].copy_(a["src"]),
        default=False,
    ))
    return out


def copy_ceiling(moved: int, kind: str = "stream", vectors: int = 1) -> Workload:
    """A plain device-to-device copy that reads and writes `moved` / 2 bytes: what the same
    HBM traffic costs with no arithmetic, the practical ceiling at that size. `kind`
    "stream" is the calibration copy `omnia_stream_copy` (`vectors` 16-byte vectors per
    thread), "torch" is torch's `copy_`."""
    import torch

    from mlx_omnia_amd.runtime import ops

    elements = max(8, (moved // 2) // 2 // 8 * 8)

    def setup(device, copies):
        first = dict(src=torch.ones(elements, dtype=torch.bfloat16, device=device),
                     dst=torch.empty(elements, dtype=torch.bfloat16, device=device))
        return _copies(first, copies)

    if kind == "torch":
        return Workload(
            name="copy_ceiling_torch", kernel="copy",
            description=f"torch copy_ of {elements * 2} bytes ({elements * 4} bytes moved)",
            bytes_per_launch=elements * 4, setup=setup,
            launch=lambda a: a["dst"].copy_(a["src"]), default=False)
    return Workload(
        name=f"copy_ceiling_stream{vectors}", kernel="stream_copy_kernel",
        description=f"omnia_stream_copy of {elements * 2} bytes ({elements * 4} bytes moved), "
                    f"{vectors} vector(s) per thread",
        bytes_per_launch=elements * 4, setup=setup,
        launch=lambda a: ops.stream_copy(a["src"], a["dst"], vectors_per_thread=vectors),
        default=False)


def best_copy(moved: int, steps: int, warmup: int, device) -> dict:
    """The calibration copy of `moved` bytes at 1, 2 and 4 vectors per thread; the fastest."""
    runs = [time_workload(copy_ceiling(moved, "stream", v), steps, warmup, device, False)
            for v in (1, 2, 4)]
    best = min(runs, key=lambda r: r["us"])
    return dict(best, vectors=(1, 2, 4)[runs.index(best)], all_us=[r["us"] for r in runs])


COPY_SWEEP_BYTES = (32 * 10**6, 85_983_744, 169_934_848, 320 * 10**6, 640 * 10**6, 1_200 * 10**6)


def _bound_launch(w: Workload, argset):
    """The workload's single C-ABI call for one argument set, arguments bound once.

    The ops wrapper is run with `ops.call` swapped for a recorder, which yields the entry
    point's name and its converted arguments; the returned closure calls the ctypes
    function directly."""
    from mlx_omnia_amd.runtime import loader, ops

    recorded = []
    original = ops.call
    ops.call = lambda name, *args: recorded.append((name, args))
    try:
        w.launch(argset)
    finally:
        ops.call = original
    if not recorded:  # not a C-ABI workload (the copy calibration)
        return lambda: (w.launch(argset), 0)[1]
    (name, args), = recorded
    fn = getattr(loader.library(), name)

    def run() -> int:
        return fn(*args)

    return run


_PREROLL_CYCLES: list[int] = []


def _preroll(stream) -> None:
    """Queue about 100 us of spin on `stream` ahead of the start event, so the timed
    launches find the queue already running: the host's latency in issuing the first
    launch is not inside the timed region (it would add several us to a 20-launch
    region). The spin's length in clock cycles is calibrated once with events."""
    import torch

    if not _PREROLL_CYCLES:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(1000)
            start.record(stream)
            torch.cuda._sleep(1_000_000)
            end.record(stream)
        torch.cuda.synchronize()
        us = max(start.elapsed_time(end) * 1000.0, 1.0)
        _PREROLL_CYCLES.append(max(1000, min(int(1_000_000 * 100.0 / us), 50_000_000)))
    with torch.cuda.stream(stream):
        torch.cuda._sleep(_PREROLL_CYCLES[0])


def time_workload(w: Workload, steps: int, warmup: int, device, graph_mode: bool) -> dict:
    import torch

    copies = max(1, min(MAX_COPIES, math.ceil(ROTATE_BYTES / max(1, w.bytes_per_launch))))
    sets = w.setup(device, copies)
    stream = torch.cuda.Stream(device)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        # Warm up for `warmup` launches, two passes over the rotation buffers and at
        # least WARM_SECONDS, so clocks have ramped and every buffer has been touched
        # (measured: 25 ms left the rope epilogue ~7% and the headline ~3% slow).
        began, i = time.perf_counter(), 0
        while i < max(warmup, 2 * copies) or time.perf_counter() - began < WARM_SECONDS:
            w.launch(sets[i % copies])
            i += 1
            if i % 64 == 0:
                torch.cuda.synchronize(device)
        torch.cuda.synchronize(device)
        if graph_mode:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(steps):
                    w.launch(sets[i % copies])
            graph.replay()  # untimed: first replay uploads the graph
            torch.cuda.synchronize(device)
            _preroll(stream)
            start.record(stream)
            graph.replay()
            end.record(stream)
            torch.cuda.synchronize(device)
            del graph
        else:
            runs = [_bound_launch(w, argset) for argset in sets]
            for i in range(min(warmup, copies)):
                runs[i % copies]()
            torch.cuda.synchronize(device)
            codes = 0
            _preroll(stream)
            start.record(stream)
            for i in range(steps):
                codes |= runs[i % copies]()
            end.record(stream)
            torch.cuda.synchronize(device)
            if codes:
                raise RuntimeError(f"{w.name}: a launch returned an error code")
    elapsed_ms = start.elapsed_time(end)
    us = elapsed_ms * 1000.0 / steps
    gbs = w.bytes_per_launch / (us * 1e-6) / 1e9
    del sets
    torch.cuda.empty_cache()
    return dict(us=round(us, 3), GBps=round(gbs, 1), frac=round(gbs / PEAK_GBS, 4),
                bytes=w.bytes_per_launch, copies=copies, kernel=w.kernel,
                workload=w.description, ms_total=round(elapsed_ms, 4),
                launch="hip graph" if graph_mode else "direct")


def _bits(rng: np.random.Generator, shape, low: int = 0x3A00, high: int = 0x3D00,
          signed: bool = True) -> np.ndarray:
    """Random finite bf16 bit patterns (magnitudes 2^-11 .. 2^-5 by default), for large
    CPU-leg operands whose values do not change the oracle's work."""
    bits = rng.integers(low, high, size=shape, dtype=np.uint16)
    if not signed:
        return bits
    return bits | (rng.integers(0, 2, size=shape, dtype=np.uint16) << np.uint16(15))


def _cpu_legs() -> dict:
    """Per workload: a factory returning (run, algorithmic bytes one run stands for,
    sample description, uses BLAS). Each run is the numpy oracle (a port of the
    reference's Core chain) on a bounded sample of the workload's own shapes."""
    from oracle import activations, add_norm, attention, embed, mlp, moe, route, rope
    from oracle import affine, mxfp4, nvfp4
    from oracle.bf16 import from_float, to_f32

    rng = np.random.default_rng(42)

    def bf(shape, scale=1.0, shift=0.0):
        return from_float(shift + scale * rng.standard_normal(shape, dtype=np.float32))

    def add_norm_leg(rows):
        x, r, w = bf((rows, 2560)), bf((rows, 2560)), bf((2560,), 0.1, 1.0)
        return (lambda: add_norm.add_rms_norm(x, r, w, 1e-6),
                rows * 4 * 2 * 2560 + 2 * 2560, f"[{rows}, 2560], whole", False)

    tables = {}

    def angle_table():
        if "t" not in tables:
            tables["t"] = rope.angle_table(40960, 64, 1e6)
        return tables["t"]

    def qk_leg(tokens, total):
        q, k = bf((tokens, 32, 128)), bf((tokens, 8, 128))
        qw, kw = bf((128,), 0.1, 1.0), bf((128,), 0.1, 1.0)
        cos, sin = angle_table()
        return (lambda: rope.qk_norm_rope(q, k, qw, kw, cos, sin, int(rng.integers(0, 32768)),
                                          1e-6, 64),
                tokens * (2 * 40 * 128 * 2 + 2 * 64 * 4) + 2 * 128 * 2,
                f"{tokens} of {total} tokens", False)

    def epilogue_leg():
        fused, qw, kw = bf((256, 48 * 128)), bf((128,), 0.1, 1.0), bf((128,), 0.1, 1.0)
        return (lambda: rope.rope_epilogue(fused, 32, 8, 128, qw, kw, int(rng.integers(0, 32768)),
                                           1e6, 1e-6),
                256 * 2 * 40 * 128 * 2 + 2 * 128 * 2, "256 of 4096 tokens", False)

    def swiglu_leg():
        g, u = bf((64, 9728)), bf((64, 9728))
        return (lambda: activations.swiglu(g, u), 3 * 64 * 9728 * 2, "64 of 8192 rows", False)

    def softplus_leg():
        a = bf((8192, 32))
        a_log = rng.uniform(0, 2.7, 32).astype(np.float32)
        dt_bias = (0.5 * rng.standard_normal(32)).astype(np.float32)
        return (lambda: activations.gate_softplus(a, a_log, dt_bias),
                8192 * 32 * 2 + 2 * 32 * 4 + 8192 * 32 * 4, "[8192, 32], whole", False)

    def gated_leg():
        run_swiglu, swiglu_bytes, _, _ = swiglu_leg()
        run_softplus, softplus_bytes, _, _ = softplus_leg()
        return (lambda: (run_swiglu(), run_softplus()), swiglu_bytes + softplus_bytes,
                "64 of 8192 SwiGLU rows and the whole [8192, 32] gate", False)

    def router_leg(logits=False):
        # The oracle's chain forms every logit exactly either way; written, they add bytes.
        x, r, w = bf((256, 2048)), bf((256, 2048)), bf((2048,), 0.1, 1.0)
        gate = bf((128, 2048), 0.02)
        return (lambda: route.residual_rms_router(x, r, w, gate, 1e-6, 8),
                256 * (4 * 2048 * 2 + 2 * 8 * 4 + (128 * 2 if logits else 0)) + 2048 * 2
                + 128 * 2048 * 2, "256 of 4096 tokens", True)

    def route_leg(sigmoid):
        logits = bf((4096, 128))
        if sigmoid:
            bias = (0.5 * rng.standard_normal(128)).astype(np.float32)
            scores = to_f32(logits)
            return (lambda: route.sigmoid_topk(scores, bias, 8),
                    4096 * 128 * 2 + 128 * 4 + 2 * 4096 * 8 * 4, "[4096, 128], whole", False)
        return (lambda: route.softmax_topk(logits, 8), 4096 * 128 * 2 + 2 * 4096 * 8 * 4,
                "[4096, 128], whole", False)

    def route_shared_leg():
        logits = bf((4096, 129))
        return (lambda: route.softmax_topk_slots(logits, 8, normalize=False, shared=True),
                4096 * 129 * 2 + 2 * 4096 * 9 * 4, "[4096, 129], whole", False)

    def router_sigmoid_leg(keys=False):
        x, r, w = bf((256, 2048)), bf((256, 2048)), bf((2048,), 0.1, 1.0)
        gate = bf((128, 2048), 0.02)
        bias = (0.5 * rng.standard_normal(128)).astype(np.float32)
        return (lambda: route.residual_rms_router_sigmoid(x, r, w, gate, bias, 1e-6, 8),
                256 * (4 * 2048 * 2 + 2 * 8 * 4 + (128 * 6 if keys else 0)) + 2048 * 2
                + 128 * 2048 * 2 + 2 * 128 * 4, "256 of 4096 tokens", True)

    def router_one_leg(sigmoid):
        x, r, w = bf((1, 2048)), bf((1, 2048)), bf((2048,), 0.1, 1.0)
        gate = bf((128, 2048), 0.02)
        if sigmoid:
            bias = (0.5 * rng.standard_normal(128)).astype(np.float32)
            return (lambda: route.residual_rms_router_sigmoid(x, r, w, gate, bias, 1e-6, 8),
                    4 * 2048 * 2 + 2048 * 2 + 128 * 2048 * 2 + 128 * 4 + 128 * 4 + 128 * 2 + 128 * 4,
                    "[1, 2048], whole", True)
        return (lambda: route.residual_rms_router(x, r, w, gate, 1e-6, 8),
                4 * 2048 * 2 + 2048 * 2 + 128 * 2048 * 2 + 128 * 4 + 128 * 2 + 2 * 8 * 4, "[1, 2048], whole",
                True)

    def atlas_leg():
        return (lambda: rope.angle_table(40960, 64, 1e6), 40960 * 2 * 64 * 4 + 64 * 8,
                "[40960, 2 x 64], whole", False)

    def embed_leg():
        table = np.full((151936, 2560), 0x3C00, dtype=np.uint16)  # a gather: values do not matter
        ids = rng.integers(0, 151936, 2048, dtype=np.int32)
        cos, sin = angle_table()
        return (lambda: embed.embed_atlas(ids, table, cos, sin, 0, 2048),
                2048 * 4 + 2 * 2048 * 2560 * 2 + 2 * 2048 * 2 * 64 * 4,
                "1 of 8 sequences (2048 tokens), full table", False)

    # Routed experts: a stack of just the routed experts (the oracle only touches those).
    def moe_leg(down):
        chosen = np.arange(8, dtype=np.int32)
        weights = rng.dirichlet(np.ones(8)).astype(np.float32)
        if down:
            stack, act, res = _bits(rng, (8, 2048, 768)), bf((8, 1536)), bf((2048,))
            return (lambda: moe.down_combine(act, stack, chosen, weights, res),
                    8 * 2048 * 768 * 2 + 8 * 1536 * 2 + 8 * 8 + 2 * 2048 * 2, "the 8 routed experts", True)
        stack, x = _bits(rng, (8, 1536, 2048)), bf((2048,))
        return (lambda: moe.gate_up(x, stack, chosen),
                8 * 1536 * 2048 * 2 + 2048 * 2 + 8 * 4 + 8 * 1536 * 2, "the 8 routed experts", True)

    def affine_stack(slots, rows, features):
        words = rng.integers(0, 2**32, (slots, rows, features // 8), dtype=np.uint32)
        scale = 4.0 / (16 * features ** 0.5)
        scales = from_float(scale * (0.5 + rng.random((slots, rows, features // 64), dtype=np.float32)))
        biases = from_float(-scale * 7.5 * np.ones((slots, rows, features // 64), dtype=np.float32))
        return affine.Stack(words, scales, biases, 64, 4)

    def affine_leg(down):
        slots = 2  # of the workload's 8: the oracle's bit unpacking is slow
        chosen = np.arange(slots)
        weights = rng.dirichlet(np.ones(slots)).astype(np.float32)
        if down:
            stack, act, res = affine_stack(slots, 2048, 768), bf((slots, 768)), bf((2048,))
            return (lambda: affine.down_combine(act, stack, chosen, weights, res),
                    slots * 2048 * (768 // 2 + 4 * 12) + slots * (768 * 2 + 8) + 2 * 2048 * 2,
                    f"{slots} of the 8 routed experts", True)
        stack, x = affine_stack(slots, 1536, 2048), bf((2048,))
        return (lambda: affine.gate_up(x, stack, chosen),
                slots * 1536 * (2048 // 2 + 4 * 32) + 2048 * 2 + slots * (4 + 768 * 2),
                f"{slots} of the 8 routed experts", True)

    def mxfp4_leg(down):
        slots = 1  # of the workload's 4
        rows, features = (2880, 2880) if down else (5760, 2880)
        stack = mxfp4.Stack(rng.integers(0, 2**32, (slots, rows, features // 8), dtype=np.uint32),
                            rng.integers(119, 123, (slots, rows, features // 32), dtype=np.uint8),
                            bf((slots, rows), 0.25))
        row_bytes = features // 2 + features // 32 + 2
        chosen = np.arange(slots)
        if down:
            act, weights, res = bf((slots, 2880)), np.ones(slots, dtype=np.float32), bf((2880,))
            return (lambda: mxfp4.down_combine(act, stack, chosen, weights, res),
                    slots * (2880 * row_bytes + 2880 * 2 + 8) + 2 * 2880 * 2,
                    f"{slots} of the 4 routed experts", True)
        x = bf((2880,))
        return (lambda: mxfp4.gate_up(x, stack, chosen, 7.0),
                slots * (5760 * row_bytes + 4 + 2880 * 2) + 2880 * 2,
                f"{slots} of the 4 routed experts", True)

    def nvfp4_leg(down, ordinal=False):
        rows, features = (2048, 768) if down else (1536, 2048)
        stack = nvfp4.Stack(rng.integers(0, 2**32, (8, rows, features // 8), dtype=np.uint32),
                            rng.integers(0x18, 0x28, (8, rows, features // 16), dtype=np.uint8))
        row_bytes = features // 2 + features // 16
        if down:
            act, weights, res = bf((8, 768)), rng.dirichlet(np.ones(8)).astype(np.float32), bf((2048,))
            return (lambda: nvfp4.down_combine(act, stack, np.arange(8), weights, res),
                    8 * 2048 * row_bytes + 8 * 768 * 2 + 8 * 8 + 2 * 2048 * 2, "the 8 routed experts", True)
        x = bf((2048,))
        if ordinal:  # the 8 lowest of 128 keys name experts 0..7, the stack's slots
            keys = np.concatenate([rng.permutation(8), 8 + rng.permutation(120)]).astype(np.uint32)
            return (lambda: nvfp4.gate_up(x, stack, np.argsort(keys, kind="stable")[:8]),
                    8 * 1536 * row_bytes + 2048 * 2 + 128 * 4 + 8 * 768 * 2,
                    "the 8 routed experts, ranked from 128 keys", True)
        return (lambda: nvfp4.gate_up(x, stack, np.arange(8)),
                8 * 1536 * row_bytes + 2048 * 2 + 8 * 4 + 8 * 768 * 2, "the 8 routed experts", True)

    def nvfp4_shared_leg():
        stack = nvfp4.Stack(rng.integers(0, 2**32, (10, 2048, 64), dtype=np.uint32),
                            rng.integers(0x18, 0x28, (10, 2048, 32), dtype=np.uint8))
        shared = nvfp4.Stack(stack.weight[0], stack.scales[0])
        act, res = bf((1, 11, 512)), bf((1, 2048))
        weights = rng.dirichlet(np.ones(10)).astype(np.float32)[None]
        return (lambda: nvfp4.down_combine_shared(act, stack, shared, np.arange(10)[None], weights, res),
                11 * 2048 * 288 + 11 * 512 * 2 + 10 * 8 + 2 * 2048 * 2, "the 10 routed experts and the shared one",
                True)

    def sink_leg(rows):
        q, sinks = bf((64, 64)), bf((64,), 2.0)
        k, v = bf((8, rows, 64)), bf((8, rows, 64))
        return (lambda: attention.sink_attend(q, k, v, sinks, None, 0.125),
                2 * 8 * rows * 64 * 2 + 2 * 64 * 64 * 2 + 64 * 2, f"[8, {rows}, 64], whole", True)

    def mlp_leg(down):
        if down:
            w, act, res = _bits(rng, (2560, 9728)), bf((9728,)), bf((2560,))
            return (lambda: mlp.down_residual(act, w, res),
                    2560 * 9728 * 2 + 9728 * 2 + 2 * 2560 * 2, "[2560, 9728], whole", True)
        inner = 9728 // 8  # an eighth of the gate rows with their up rows: a smaller GEMV
        w, x = _bits(rng, (2 * inner, 2560)), bf((2560,))
        return (lambda: mlp.gate_up_swiglu(x, w),
                2 * inner * 2560 * 2 + 2560 * 2 + inner * 2, "1/8 of the gate and up rows", True)

    def attention_leg(rows):
        kc, vc = _bits(rng, (8, rows, 128)), _bits(rng, (8, rows, 128))
        q, k, v = bf((32 * 128,)), bf((8 * 128,)), bf((8 * 128,))
        qw, kw = bf((128,), 0.1, 1.0), bf((128,), 0.1, 1.0)
        cos, sin = angle_table()
        row = np.concatenate([cos[rows - 1], sin[rows - 1]]).astype(np.float32)
        byte_count = (2 * 8 * rows * 128 * 2 + 48 * 128 * 2 + 32 * 128 * 2 + 2 * 8 * 128 * 2
                      + 2 * 128 * 2 + 2 * 64 * 4)
        return (lambda: attention.decode_step(q, k, v, qw, kw, row, kc, vc, rows - 1, window=0,
                                              scale=128 ** -0.5, eps=1e-6, pairs=64),
                byte_count, f"position {rows - 1} of a {rows}-row cache, whole", True)

    return {
        "add_rms_norm_prefill": lambda: add_norm_leg(512),
        "add_rms_norm_decode": lambda: add_norm_leg(1),
        "qk_norm_rope_prefill": lambda: qk_leg(256, 4096),
        "qk_norm_rope_decode": lambda: qk_leg(64, 64),
        "rope_epilogue_prefill": epilogue_leg,
        "swiglu": swiglu_leg,
        "gate_softplus": softplus_leg,
        "gated_activations": gated_leg,
        "residual_rms_router": router_leg,
        "residual_rms_router_logits": lambda: router_leg(logits=True),
        "softmax_topk": lambda: route_leg(False),
        "softmax_topk_shared": route_shared_leg,
        "sigmoid_topk": lambda: route_leg(True),
        "residual_rms_router_sigmoid": router_sigmoid_leg,
        "residual_rms_router_sigmoid_keys": lambda: router_sigmoid_leg(keys=True),
        "residual_rms_router_decode": lambda: router_one_leg(False),
        "residual_rms_router_sigmoid_decode": lambda: router_one_leg(True),
        "rope_angle_atlas": atlas_leg,
        "embed_atlas": embed_leg,
        "moe_gate_up_decode": lambda: moe_leg(False),
        "moe_down_combine_decode": lambda: moe_leg(True),
        "moe_affine_gate_up_decode": lambda: affine_leg(False),
        "moe_affine_down_combine_decode": lambda: affine_leg(True),
        "moe_mxfp4_gate_up_decode": lambda: mxfp4_leg(False),
        "moe_mxfp4_down_combine_decode": lambda: mxfp4_leg(True),
        "moe_nvfp4_gate_up_decode": lambda: nvfp4_leg(False),
        "moe_nvfp4_gate_up_ordinal_decode": lambda: nvfp4_leg(False, ordinal=True),
        "moe_nvfp4_down_combine_decode": lambda: nvfp4_leg(True),
        "moe_nvfp4_shared_down_combine_decode": nvfp4_shared_leg,
        "dense_mlp_gate_up_decode": lambda: mlp_leg(False),
        "dense_mlp_down_decode": lambda: mlp_leg(True),
        "attention_decode_32k": lambda: attention_leg(32768),
        "attention_decode_4k": lambda: attention_leg(4096),
        "attention_sink_decode_32k": lambda: sink_leg(32768),
        "attention_sink_decode_4k": lambda: sink_leg(4096),
    }


def _thread_settings() -> tuple[int, dict, int]:
    """(BLAS threads in effect, the thread environment, cores this process may use)."""
    env = {name: os.environ.get(name) for name in
           ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")}
    blas = 1
    try:
        from threadpoolctl import threadpool_info

        pools = [p for p in threadpool_info() if p.get("user_api") == "blas"]
        if pools:
            blas = int(pools[0].get("num_threads") or 1)
    except Exception:  # threadpoolctl absent or unable to inspect: report one thread
        blas = 1
    return blas, env, len(os.sched_getaffinity(0))


def cpu_baseline(name: str, full_bytes: int, seconds: float = 0.8) -> dict | None:
    """The numpy oracle on a bounded sample of one workload, timed on this host: runs
    for at least `seconds` (one run at least); value = algorithmic bytes per second.
    `cores` is the threads the leg used: one for elementwise numpy, the BLAS pool's size
    for legs whose oracle multiplies matrices (numpy's `@` runs in BLAS)."""
    legs = _cpu_legs()
    if name not in legs:
        return None
    run, sample_bytes, sample, uses_blas = legs[name]()
    run()  # untimed: first touch of the sample's pages
    done, start = 0, time.perf_counter()
    while done == 0 or time.perf_counter() - start < seconds:
        run()
        done += 1
    elapsed = time.perf_counter() - start
    blas, env, affinity = _thread_settings()
    rate = done * sample_bytes / elapsed
    return dict(value=round(rate / 1e9, 4), unit="GB/s",
                us_per_launch=round(full_bytes / rate * 1e6, 1),
                cores=blas if uses_blas else 1, kind="port",
                sample=f"numpy oracle, {sample}: {done} run(s) in {elapsed:.2f} s",
                affinity_cores=affinity, threads_env=env)


PHASES = ("entry", "row 0 done", "phase 1 done", "tile complete", "walk done",
          "logits complete", "selection + tasks", "task list complete", "recomputed", "written")


def router_phase_clocks(device, rows: int = 4096, stamped: int = 8, timed: int = 200,
                        logits: bool = False) -> dict:
    """Per-phase wall clocks of the fused residual router at configs[4] ([4096, 2048],
    128 experts, k = 8), or the same at fewer `rows` (a multiple of 16: one workgroup per
    16 tokens, so fewer workgroups share the chip), from `libomnia_router_clocks.so` (the
    same source compiled with its phase marks on): each of `stamped` launches, taken in the
    rotation's steady state, records the 100 MHz wall clock of every wave at ten phase
    boundaries; the summary is each boundary's spread over the workgroups (median over
    launches of each statistic), in µs from the launch's earliest entry. `launch_us` is
    the event-timed mean of `timed` back-to-back launches of the diagnostic build. With
    `logits` the launch also writes the bf16 logits (every logit exact)."""
    import ctypes

    import torch

    path = REPO / "mlx-omnia_amd" / "libomnia_router_clocks.so"
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built (a diagnostic, built on request): run "
                                "`python mlx-omnia_amd/build.py --clocks` or build() with "
                                "OMNIA_BUILD_CLOCKS=1 first")
    lib = ctypes.CDLL(str(path))
    lib.omnia_router_pack_bytes.restype = ctypes.c_int64
    lib.omnia_router_pack_bytes.argtypes = [ctypes.c_int64, ctypes.c_int64]
    lib.omnia_pack_router_weight.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                             ctypes.c_void_p, ctypes.c_void_p]
    lib.omnia_residual_rms_router.argtypes = ([ctypes.c_void_p] * 4 + [ctypes.c_int64] * 4
                                              + [ctypes.c_float] + [ctypes.c_void_p] * 6)
    lib.omnia_router_phase_clocks_set.argtypes = [ctypes.c_void_p]
    lib.omnia_last_error.restype = ctypes.c_char_p
    if rows <= 0 or rows % 16:
        raise ValueError(f"phase clocks: rows must be a positive multiple of 16, not {rows}")
    hidden, experts, k = 2048, 128, 8
    groups, slots = rows // 16, len(PHASES)
    rng = np.random.default_rng(7)
    copies = 8  # 8 x 68 MB: past the 256 MB Infinity Cache
    xs = [_to_bf16_device(_normal(rng, (rows, hidden)), device) for _ in range(copies)]
    rs = [_to_bf16_device(_normal(rng, (rows, hidden)), device) for _ in range(copies)]
    w = _to_bf16_device(_normal(rng, (hidden,), 0.1, 1.0), device)
    gate = _to_bf16_device(_normal(rng, (experts, hidden), 0.02), device)
    outs = [dict(s=torch.empty_like(xs[0]), n=torch.empty_like(xs[0]),
                 i=torch.empty((rows, k), dtype=torch.int32, device=device),
                 w=torch.empty((rows, k), dtype=torch.float32, device=device),
                 l=torch.empty((rows, experts), dtype=torch.bfloat16, device=device) if logits else None)
            for _ in range(copies)]
    stream = torch.cuda.current_stream(device)
    handle = ctypes.c_void_p(stream.cuda_stream)
    packed = torch.empty(lib.omnia_router_pack_bytes(experts, hidden), dtype=torch.uint8,
                         device=device)
    if lib.omnia_pack_router_weight(gate.data_ptr(), experts, hidden, packed.data_ptr(), handle):
        raise RuntimeError(lib.omnia_last_error().decode())

    def launch(c: int) -> None:
        o = outs[c]
        if lib.omnia_residual_rms_router(xs[c].data_ptr(), rs[c].data_ptr(), w.data_ptr(),
                                         packed.data_ptr(), rows, hidden, experts, k,
                                         ctypes.c_float(1e-6), o["s"].data_ptr(), o["n"].data_ptr(),
                                         o["l"].data_ptr() if logits else None, o["i"].data_ptr(),
                                         o["w"].data_ptr(), handle):
            raise RuntimeError(lib.omnia_last_error().decode())

    for i in range(400):
        launch(i % copies)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(timed):
        launch(i % copies)
    end.record(stream)
    torch.cuda.synchronize(device)
    launch_us = start.elapsed_time(end) * 1000.0 / timed
    records = []
    for rep in range(stamped):
        buffer = torch.zeros(groups * 16 * slots, dtype=torch.int64, device=device)
        lib.omnia_router_phase_clocks_set(ctypes.c_void_p(buffer.data_ptr()))
        launch(rep % copies)
        lib.omnia_router_phase_clocks_set(None)
        for i in range(8):  # back to the steady state before the next stamped launch
            launch((rep + 1 + i) % copies)
        records.append(buffer)
    torch.cuda.synchronize(device)
    walkers = np.arange(16) >= 8
    per_launch = []
    for buffer in records:
        ticks = buffer.view(groups, 16, slots).cpu().numpy().astype(np.int64)
        rel = (ticks - ticks[:, :, 0].min()) * 0.01  # 100 MHz ticks -> µs
        stats = {}
        for j, name in enumerate(PHASES):
            if j in (1, 2):
                col = rel[:, ~walkers, j]  # row waves only
            elif j == 4:
                col = rel[:, walkers, j]   # walkers only
            elif j == 9:
                col = rel[:, :, j].max(axis=1)  # a workgroup's last wave
            elif j >= 6:
                col = rel[:, 8, j]         # phase 3: a walker (row waves may have left)
            else:
                col = rel[:, 0, j]         # barrier exits: every wave alike
            stats[name] = [float(np.percentile(col, q)) for q in (10, 50, 90)] + [float(col.max())]
        per_launch.append(stats)
    summary = {name: [round(float(np.median([s[name][q] for s in per_launch])), 2) for q in range(4)]
               for name in PHASES}
    return dict(kernel="residual_rms_router_split_kernel<128>",
                workload=f"x, residual bf16 [{rows}, 2048], router [128, 2048], k = 8"
                         + (", logits written" if logits else ""),
                workgroups=groups,
                launch_us=round(launch_us, 3), stamped_launches=stamped,
                columns=["p10", "median", "p90", "max"], unit="us from the launch's first entry",
                phases=summary)


def _traffic(kernel_name: str) -> int | None:
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if present."""
    table = REPO / "profiles" / "hbm_traffic.md"
    if not table.exists():
        return None
    for line in table.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == kernel_name and re.fullmatch(r"\d+", cells[4]):
            return int(cells[4])
    return None


def bench_line(results: dict, head_name: str, steps: int, warmup: int) -> dict:
    """The one stdout JSON line: the headline's figures, its roofline and CPU baseline, and
    a compact map of every workload -> [us, fraction of peak, CPU oracle GB/s]. The full
    per-workload record (descriptions, copies, CPU samples) goes to the results file; the
    line stays a few KB whatever the number of workloads."""
    head = results[head_name]
    cpu = head.get("cpu_baseline")
    baseline = None if not cpu else {
        "value": cpu["value"], "unit": cpu["unit"], "cores": cpu["cores"],
        "kind": cpu["kind"], "sample": cpu["sample"],
        "us_per_launch": cpu["us_per_launch"], "affinity_cores": cpu["affinity_cores"]}
    kernels = {}
    for name, r in results.items():
        leg = r.get("cpu_baseline")
        kernels[name] = [r["us"], r["frac"], leg["value"] if leg else None]
    return {
        "metric": METRIC,
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(head["us"] / 1000.0, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded numpy normal draws rounded to bf16 (RNE), resident in HBM",
        "config": {"workload": f"{head_name}: {head['workload']}",
                   "us_per_launch": head["us"], "frac_of_peak": head["frac"],
                   "bytes_per_launch": head["bytes"], "launch": head["launch"]},
        "roofline": {
            "bound": "hbm",
            "achieved": head["GBps"],
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": head["frac"],
            "traffic": _traffic(head_name),
            "copy_us": head.get("copy_ceiling", {}).get("us"),
        },
        "cpu_baseline": baseline,
        "kernels_fields": ["us", "frac_of_peak", "cpu_oracle_GBps"],
        "kernels": kernels,
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--only", default="", help="comma-separated workload names")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--graph", action="store_true", help="also time a captured HIP graph")
    parser.add_argument("--ceiling", action="store_true",
                        help="also time the calibration copy and torch's copy_ moving each "
                             "workload's bytes")
    parser.add_argument("--phase-clocks", action="store_true",
                        help="print the fused router's per-phase wall clocks (diagnostic "
                             "build) as one JSON line instead of the bench line")
    parser.add_argument("--copy-sweep", action="store_true",
                        help="time the calibration copy over a range of sizes (one JSON line "
                             "each) instead of the bench line")
    parser.add_argument("--results", default="bench_results.json",
                        help="file for the full per-workload record ('' for none)")
    parser.add_argument("--phase-clocks-logits", action="store_true",
                        help="--phase-clocks with the logits written (every logit exact)")
    parser.add_argument("--phase-clocks-rows", default="4096",
                        help="comma-separated token counts for --phase-clocks (multiples of 16)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not run "
              "(the fused kernels shard by tokens with no exchange; see DESIGN.md)",
              file=sys.stderr)
        return 2

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    if args.phase_clocks:
        for rows in (int(n) for n in args.phase_clocks_rows.split(",") if n):
            print(json.dumps(router_phase_clocks(device, rows, logits=args.phase_clocks_logits)),
                  flush=True)
        return 0
    if args.copy_sweep:
        for moved in COPY_SWEEP_BYTES:
            r = best_copy(moved, args.steps, args.warmup, device)
            print(json.dumps({"copy_bytes_moved": r["bytes"], "us": r["us"],
                              "TBps": round(r["GBps"] / 1000.0, 3), "frac": r["frac"],
                              "vectors": r["vectors"], "us_by_vectors": r["all_us"]}), flush=True)
        return 0
    only = [n for n in args.only.split(",") if n]
    selected = [w for w in workloads() if ((w.name in only) if only else w.default)]
    results = {}
    for index, w in enumerate(selected, 1):
        window = [time.monotonic_ns(), time.time_ns()]   # host clocks around the workload
        direct = time_workload(w, args.steps, args.warmup, device, False)
        # Small kernels outrun a Python launch loop; a graph replay then gives the
        # tighter figure. Either way the number is events over `steps` launches.
        graphed = time_workload(w, args.steps, args.warmup, device, True) if (
            args.graph or direct["us"] < 12.0) else None
        results[w.name] = min((r for r in (direct, graphed) if r), key=lambda r: r["us"])
        r = results[w.name]
        note = ""
        if args.ceiling or w.name == HEADLINE:
            # The calibration copy of the same bytes, always beside the headline.
            ceiling = best_copy(w.bytes_per_launch, args.steps, args.warmup, device)
            r["copy_ceiling"] = {k: ceiling[k] for k in ("us", "GBps", "frac", "vectors", "all_us")}
            note = f" copy {ceiling['us']}"
        if args.ceiling:
            torch_copy = time_workload(copy_ceiling(w.bytes_per_launch, "torch"), args.steps,
                                       args.warmup, device, False)
            r["torch_copy"] = {k: torch_copy[k] for k in ("us", "GBps", "frac")}
            note += f" torch copy {torch_copy['us']}"
        torch.cuda.synchronize(device)
        r["host_window_ns"] = dict(monotonic=[window[0], time.monotonic_ns()],
                                   realtime=[window[1], time.time_ns()])
        print(f"[bench] {index}/{len(selected)} {w.name} {r['us']} us{note}",
              file=sys.stderr, flush=True)

    head_name = HEADLINE if HEADLINE in results else next(iter(results))
    if not args.no_cpu:
        # The numpy oracle on each workload's own shapes (bounded samples), after the GPU
        # timing; the headline's sample runs longest.
        for name, r in results.items():
            seconds = 3.0 if name == head_name else 0.8
            r["cpu_baseline"] = cpu_baseline(name, r["bytes"], seconds)
        print(f"[bench] CPU oracle legs done ({len(results)})", file=sys.stderr, flush=True)
    line = bench_line(results, head_name, args.steps, args.warmup)
    if args.results:
        record = dict(line, kernels=results)
        Path(args.results).parent.mkdir(parents=True, exist_ok=True)
        Path(args.results).write_text(json.dumps(record, indent=1) + "\n")
    print(json.dumps(line, separators=(",", ":")), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
