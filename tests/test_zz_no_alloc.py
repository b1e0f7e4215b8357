"""`omnia_attention_decode_noalloc` against `omnia_attention_decode`, through the C-ABI.

The no-allocation entry point runs the same kernels with the per-chunk softmax states
in the library's static device array instead of a caller workspace, so its results must
equal the workspace entry point's bit for bit: the context, and both caches after the
step writes its new key/value row. Two GPU calls in a row, the second with a smaller
geometry (fewer heads, a shorter cache, a ring), show that what the first call left in
the shared array does not leak into the second. A request for more chunk states than the
array holds is refused on the host before any device call.
"""

import ctypes
import errno

import numpy as np
import pytest
import torch

from mlx_omnia_amd.runtime import loader, ops
from oracle.bf16 import from_float
from oracle.rope import angle_table
from util import to_device

D = 128


def _step_inputs(heads, kv_heads, capacity, pairs, seed):
    rng = np.random.default_rng(seed)

    def bf16(values):
        return to_device(from_float(values))

    cos, sin = angle_table(max(capacity, 1024), pairs, 10000.0)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    return dict(
        raw_q=bf16(rng.standard_normal(heads * D)),
        raw_k=bf16(rng.standard_normal(kv_heads * D)),
        raw_v=bf16(rng.standard_normal(kv_heads * D)),
        qw=bf16(1 + 0.1 * rng.standard_normal(D)),
        kw=bf16(1 + 0.1 * rng.standard_normal(D)),
        atlas=torch.from_numpy(np.concatenate([cos, sin], axis=1).astype(np.float32)).cuda(),
        kc=torch.randn((kv_heads, capacity, D), generator=gen, device="cuda").to(torch.bfloat16),
        vc=torch.randn((kv_heads, capacity, D), generator=gen, device="cuda").to(torch.bfloat16),
    )


def _both(heads, kv_heads, capacity, pairs, position, *, window=0, mscale=1.0, seed=0):
    """(workspace entry's out, caches), (no-allocation entry's out, caches) on equal inputs."""
    x = _step_inputs(heads, kv_heads, capacity, pairs, seed)
    pos = torch.tensor([position], dtype=torch.int32, device="cuda")
    count = min(position + 1, capacity)
    kw = dict(heads=heads, kv_heads=kv_heads, max_rows=count, scale=D ** -0.5, eps=1e-6,
              mscale=mscale, window=window)
    workspace = torch.empty(ops.attention_workspace_bytes(heads, kv_heads, D, capacity),
                            dtype=torch.uint8, device="cuda")
    kc1, vc1 = x["kc"].clone(), x["vc"].clone()
    kc2, vc2 = x["kc"].clone(), x["vc"].clone()
    args = (x["raw_q"], x["raw_k"], x["raw_v"], x["qw"], x["kw"], x["atlas"])
    out1 = ops.attention_decode(*args, kc1, vc1, pos, workspace=workspace, **kw)
    out2 = torch.full((heads, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.attention_decode_noalloc(*args, kc2, vc2, pos, out=out2, **kw)
    torch.cuda.synchronize()
    return (out1, kc1, vc1), (out2, kc2, vc2)


def _assert_same(first, second):
    for a, b in zip(first, second):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_twice_in_a_row():
    # 32 query heads over 8 kv heads, 8192 rows, the step at row 6000: split over
    # several chunks per kv head, so the chunk states go through the static array.
    print("noalloc call 1: heads 32/8, capacity 8192, position 6000", flush=True)
    first = _both(32, 8, 8192, 64, 6000, seed=1)
    _assert_same(*first)
    assert torch.isfinite(first[1][0].float()).all()
    # Smaller: 8 query heads over 2 kv heads, a ring of 2048 rows past its wrap,
    # partial rotation and the YaRN factor.
    print("noalloc call 2: heads 8/2, ring 2048, position 5000", flush=True)
    second = _both(8, 2, 2048, 32, 5000, window=2048, mscale=1.3465735912322998, seed=2)
    _assert_same(*second)
    assert torch.isfinite(second[1][0].float()).all()
    # One chunk (no states at all): the array is not touched.
    print("noalloc call 3: heads 4/4, capacity 128, position 90", flush=True)
    third = _both(4, 4, 128, 64, 90, seed=3)
    _assert_same(*third)


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="passes placeholder pointers: checked where no GPU can see them")
def test_noalloc_refuses_more_states_than_the_array_holds():
    """505 kv heads of 8 query heads split in two: 505 * 2 * 8 * 520 bytes > 4 MiB.
    The refusal comes before any device call (no GPU needed)."""
    lib = loader.library()
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: the call returns first
    kv_heads, heads, rows = 505, 505 * 8, 256
    assert 505 * 2 * 8 * 520 > ops.ATTENTION_SCRATCH_BYTES
    rc = lib.omnia_attention_decode_noalloc(
        fake, fake, fake, fake, fake, fake, 1024, 64, 1.0, fake, fake, rows, 0, fake, rows,
        heads, kv_heads, D, D ** -0.5, 1e-6, fake, None)
    assert rc == -errno.EINVAL
    assert "static scratch" in loader.last_error()


def test_scratch_size_matches_the_header():
    import re
    from pathlib import Path

    header = (Path(__file__).resolve().parent.parent / "include" / "omnia_hip.h").read_text()
    match = re.search(r"#define OMNIA_ATTENTION_SCRATCH_BYTES \((\d+) \* 1024 \* 1024\)", header)
    assert match and int(match.group(1)) * 1024 * 1024 == ops.ATTENTION_SCRATCH_BYTES
