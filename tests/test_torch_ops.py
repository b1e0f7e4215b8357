"""The `torch.library` registration (runtime/torch_ops.py) on the CPU: every operator is
registered under `torch.ops.omnia`, and its fake implementation gives the shapes and
dtypes the entry point writes, without a device (what torch.compile and export trace)."""

import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from mlx_omnia_amd.runtime import loader, torch_ops

BF16 = torch.bfloat16


def test_every_operator_is_registered():
    for name in torch_ops.REGISTERED:
        assert hasattr(torch.ops.omnia, name), name


def test_fake_shapes_and_dtypes():
    with FakeTensorMode():
        x = torch.empty(4, 2560, dtype=BF16)
        summed, normed = torch.ops.omnia.add_rms_norm(x, x, torch.empty(2560, dtype=BF16), 1e-6)
        assert summed.shape == normed.shape == (4, 2560) and normed.dtype == BF16
        q, k = torch.ops.omnia.qk_norm_rope(torch.empty(5, 32, 128, dtype=BF16), torch.empty(5, 8, 128, dtype=BF16),
                                            torch.empty(128, dtype=BF16), torch.empty(128, dtype=BF16),
                                            torch.empty(64, 64), torch.empty(64, 64), 0, 1e-6, 64, 1.0)
        assert q.shape == (32, 5, 128) and k.shape == (8, 5, 128)
        q, k = torch.ops.omnia.rope_epilogue(torch.empty(6, 48 * 128, dtype=BF16), torch.empty(128, dtype=BF16),
                                             torch.empty(128, dtype=BF16), 32, 8, 128, 0, 20.0, 1e-6)
        assert q.shape == (32, 6, 128) and k.shape == (8, 6, 128)
        hidden, full, sliding = torch.ops.omnia.embed_atlas(torch.empty(2, 7, dtype=torch.int32),
                                                            torch.empty(100, 64, dtype=BF16), torch.empty(50, 128),
                                                            None, 3, 7)
        assert hidden.shape == (2, 7, 64) and full.shape == (7, 128) and sliding.shape == (0, 0)
        y = torch.ops.omnia.swiglu(torch.empty(3, 96, dtype=BF16), torch.empty(3, 96, dtype=BF16))
        assert y.shape == (3, 96) and y.dtype == BF16
        g = torch.ops.omnia.gate_softplus(torch.empty(3, 32, dtype=BF16), torch.empty(32), torch.empty(32))
        assert g.shape == (3, 32) and g.dtype == torch.float32
        y, g = torch.ops.omnia.gated_activations(torch.empty(3, 96, dtype=BF16), torch.empty(3, 96, dtype=BF16),
                                                 torch.empty(3, 32, dtype=BF16), torch.empty(32), torch.empty(32))
        assert y.shape == (3, 96) and g.shape == (3, 32)
        for op in (lambda t: torch.ops.omnia.softmax_topk(t, 8),
                   lambda t: torch.ops.omnia.sigmoid_topk(t, torch.empty(128), 8)):
            idx, w = op(torch.empty(2, 5, 128, dtype=BF16))
            assert idx.shape == w.shape == (2, 5, 8) and idx.dtype == torch.int32 and w.dtype == torch.float32
        idx, w = torch.ops.omnia.softmax_topk(torch.empty(3, 129, dtype=BF16), 8, False, True)
        assert idx.shape == w.shape == (3, 9)
        packed = torch.ops.omnia.pack_router_weight(torch.empty(128, 2048, dtype=BF16))
        assert packed.shape == (loader.library().omnia_router_pack_bytes(128, 2048),)
        s2, n2, idx, w = torch.ops.omnia.residual_rms_router(x[:, :2048], x[:, :2048], torch.empty(2048, dtype=BF16),
                                                            packed, 128, 8, 1e-6)
        assert s2.shape == (4, 2048) and idx.shape == (4, 8)
        s3, n3, logits, keys = torch.ops.omnia.residual_rms_router_sigmoid(
            x[:, :2048], x[:, :2048], torch.empty(2048, dtype=BF16), packed, torch.empty(128), 128, 8, 1e-6)
        assert logits.shape == (4, 128) and logits.dtype == BF16 and keys.dtype == torch.uint32
        act = torch.ops.omnia.moe_gate_up(torch.empty(2048, dtype=BF16), torch.empty(16, 1536, 2048, dtype=BF16),
                                          torch.empty(4, dtype=torch.int32))
        assert act.shape == (4, 1536) and act.dtype == BF16
        out = torch.ops.omnia.moe_down_combine(act, torch.empty(16, 2048, 768, dtype=BF16),
                                               torch.empty(4, dtype=torch.int32), torch.empty(4), None)
        assert out.shape == (2048,) and out.dtype == BF16
        y = torch.ops.omnia.dense_gate_up_swiglu(torch.empty(2048, dtype=BF16), torch.empty(1536, 2048, dtype=BF16))
        assert y.shape == (768,)
        z = torch.ops.omnia.dense_down_residual(y, torch.empty(2048, 768, dtype=BF16), torch.empty(2048, dtype=BF16))
        assert z.shape == (2048,)
        ctx = torch.ops.omnia.attention_sink_decode(torch.empty(64, 64, dtype=BF16),
                                                    torch.empty(1, 8, 300, 64, dtype=BF16),
                                                    torch.empty(1, 8, 300, 64, dtype=BF16),
                                                    torch.empty(64, dtype=BF16), None, 0.125)
        assert ctx.shape == (64, 64) and ctx.dtype == BF16


def test_embed_atlas_without_atlases_returns_distinct_empties(monkeypatch):
    """A gather-only call (both atlases None) runs the real operator body: the two empty
    atlas outputs are distinct tensors (custom ops refuse outputs that alias). The C-ABI
    gather is replaced by a torch gather, so no device is needed."""
    def gather_only(tokens, embedding, full, sliding, *, position, n_positions):
        assert full is None and sliding is None
        return embedding[tokens.long()], None, None

    monkeypatch.setattr(torch_ops.ops, "embed_atlas", gather_only)
    tokens = torch.tensor([[3, 1, 4]], dtype=torch.int32)
    table = torch.arange(5 * 8, dtype=torch.float32).reshape(5, 8).to(BF16)
    hidden, full, sliding = torch.ops.omnia.embed_atlas(tokens, table, None, None, 0, 3)
    assert torch.equal(hidden, table[tokens.long()])
    assert full.shape == sliding.shape == (0, 0)
    assert full.data_ptr() != sliding.data_ptr() or full is not sliding
