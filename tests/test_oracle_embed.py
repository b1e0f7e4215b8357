"""Pins the embedding/atlas oracle (oracle/embed.py) against torch's gather and the
reference's own known answers (tests/test_kernel_embedding_rope_atlas.py:15-112: a
128 x 256 bf16 table, 32- and 64-wide fp32 atlases over 16 positions, tokens
(0, 0), (7, 5), (127, 15), and the two atlases read independently at position 9)."""

import numpy as np
import torch
import torch.nn.functional as F

from oracle.bf16 import from_float
from oracle.embed import embed_atlas


def _reference_fixture(seed=0):
    rng = np.random.default_rng(seed)
    embedding = from_float(rng.standard_normal((128, 256)))
    full = rng.standard_normal((1, 1, 16, 32)).astype(np.float32)
    sliding = rng.standard_normal((1, 1, 16, 64)).astype(np.float32)
    return embedding, full, sliding


def test_single_token_copies_match_the_reference_cases():
    embedding, full, sliding = _reference_fixture()
    for token, position in ((0, 0), (7, 5), (127, 15)):
        hidden, f, s = embed_atlas(np.array([[token]], np.int32), embedding, full, sliding, position, 1)
        assert np.array_equal(hidden.reshape(-1), embedding[token])
        assert np.array_equal(f.reshape(-1), full[0, 0, position])
        assert np.array_equal(s.reshape(-1), sliding[0, 0, position])


def test_atlases_read_independently():
    embedding, full, sliding = _reference_fixture(seed=3)
    _, f, s = embed_atlas(np.array([11], np.int32), embedding, full, sliding, 9, 1)
    assert np.array_equal(f[0], full[0, 0, 9]) and np.array_equal(s[0], sliding[0, 0, 9])
    assert not np.array_equal(f[0], full[0, 0, 0])


def test_segment_matches_torch_embedding():
    rng = np.random.default_rng(1)
    embedding = from_float(0.02 * rng.standard_normal((1000, 64)))
    tokens = rng.integers(0, 1000, size=(3, 17), dtype=np.int32)
    hidden, f, s = embed_atlas(tokens, embedding, np.zeros((40, 8), np.float32), None, 5, 17)
    want = F.embedding(torch.from_numpy(tokens.astype(np.int64)), torch.from_numpy(embedding.view(np.int16)))
    assert np.array_equal(hidden, want.numpy().view(np.uint16))
    assert f.shape == (17, 8) and s is None


def test_out_of_range_ids_give_zero_rows():
    embedding, full, sliding = _reference_fixture()
    hidden, _, _ = embed_atlas(np.array([-1, 128, 5], np.int32), embedding, full, sliding, 0, 3)
    assert not hidden[:2].any() and np.array_equal(hidden[2], embedding[5])
