"""HIP embedding gather + atlas rows against the oracle: bit-exact (pure copies).

Cases: the config (table [151936, 2560] bf16 ~N(0, 0.02), ids [8, 2048] uniform, cos and
sin atlases [40960, 64] fp32 for theta=1e6, positions 0..2047), the reference test's
small fixture (128 x 256 table, 32/64-wide atlases, single tokens), out-of-range ids,
a skipped atlas, an empty segment, and the facade's resolution.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.embed import Embed, HipEmbed
from mlx_omnia_amd.runtime import ops
from oracle import rope
from oracle.bf16 import from_float
from oracle.embed import embed_atlas
from util import bits_of, f32_to_device, to_device

pytestmark = pytest.mark.gpu


def test_config_shape_bit_exact():
    print("embed_atlas config shape", flush=True)
    rng = np.random.default_rng(3)
    vocab, hidden = 151936, 2560
    table = from_float(0.02 * rng.standard_normal((vocab, hidden), dtype=np.float32))
    tokens = rng.integers(0, vocab, size=(8, 2048), dtype=np.int32)
    cos, sin = rope.angle_table(40960, 64, 1e6)
    dev_table = to_device(table)
    out, full, sliding = ops.embed_atlas(
        torch.from_numpy(tokens).cuda(), dev_table, f32_to_device(cos), f32_to_device(sin),
        position=0, n_positions=2048,
    )
    torch.cuda.synchronize()
    want, want_full, want_sliding = embed_atlas(tokens, table, cos, sin, 0, 2048)
    assert out.shape == (8, 2048, hidden)
    assert np.array_equal(bits_of(out), want)
    assert np.array_equal(full.cpu().numpy(), want_full)
    assert np.array_equal(sliding.cpu().numpy(), want_sliding)


def test_reference_fixture_through_facade():
    rng = np.random.default_rng(0)
    embedding = from_float(rng.standard_normal((128, 256)))
    full = rng.standard_normal((1, 1, 16, 32)).astype(np.float32)
    sliding = rng.standard_normal((1, 1, 16, 64)).astype(np.float32)
    embed = Embed(to_device(embedding), full_atlas=f32_to_device(full), sliding_atlas=f32_to_device(sliding))
    assert isinstance(embed.strategy, HipEmbed)
    for token, position in ((0, 0), (7, 5), (127, 15), (11, 9)):
        h, f, s = embed(torch.tensor([[token]], dtype=torch.int32, device="cuda"), position)
        assert h.shape == (256,) and f.shape == (32,) and s.shape == (64,)
        assert np.array_equal(bits_of(h), embedding[token])
        assert np.array_equal(f.cpu().numpy(), full[0, 0, position])
        assert np.array_equal(s.cpu().numpy(), sliding[0, 0, position])
    # A segment: tokens [2, 5] at positions 3..7.
    tokens = rng.integers(0, 128, size=(2, 5), dtype=np.int32)
    h, f, s = embed(torch.from_numpy(tokens).cuda(), 3)
    want_h, want_f, want_s = embed_atlas(tokens, embedding, full, sliding, 3, 5)
    assert np.array_equal(bits_of(h), want_h)
    assert np.array_equal(f.cpu().numpy(), want_f) and np.array_equal(s.cpu().numpy(), want_s)


def test_out_of_range_ids_skipped_atlas_and_empty():
    rng = np.random.default_rng(2)
    embedding = from_float(rng.standard_normal((50, 2048)))
    tokens = np.array([3, -1, 50, 49, 1 << 30], dtype=np.int32)
    atlas = rng.standard_normal((10, 12)).astype(np.float32)
    h, f, s = ops.embed_atlas(torch.from_numpy(tokens).cuda(), to_device(embedding),
                              f32_to_device(atlas), None, position=4, n_positions=6)
    want_h, want_f, _ = embed_atlas(tokens, embedding, atlas, None, 4, 6)
    assert np.array_equal(bits_of(h), want_h) and s is None
    assert np.array_equal(f.cpu().numpy(), want_f)
    h, f, s = ops.embed_atlas(torch.empty(0, dtype=torch.int32, device="cuda"), to_device(embedding),
                              f32_to_device(atlas), None, position=0, n_positions=0)
    assert h.shape == (0, 2048) and f.shape == (0, 12)
    with pytest.raises(ValueError):
        ops.embed_atlas(torch.zeros(2, dtype=torch.int32, device="cuda"), to_device(embedding),
                        f32_to_device(atlas), None, position=8, n_positions=3)


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "embed.npz")
    h, f, s = ops.embed_atlas(
        torch.from_numpy(golden["tokens"]).cuda(), to_device(golden["embedding"]),
        f32_to_device(golden["full"]), f32_to_device(golden["sliding"]),
        position=int(golden["position"]), n_positions=golden["tokens"].shape[-1],
    )
    assert np.array_equal(bits_of(h), golden["hidden"])
    assert np.array_equal(f.cpu().numpy(), golden["full_out"])
    assert np.array_equal(s.cpu().numpy(), golden["sliding_out"])
