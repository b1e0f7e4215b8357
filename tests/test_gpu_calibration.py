"""The calibration copy (`omnia_stream_copy`, csrc/calibration.hip): a bit-for-bit copy at
every vectors-per-thread setting, for sizes that fill whole workgroups, leave the last
one short, and are a single vector; bytes past the end of the destination untouched;
bad arguments refused."""

import pytest
import torch

from mlx_omnia_amd.runtime import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("vectors", [1, 2, 4])
@pytest.mark.parametrize("nbytes", [16, 4096, 16 * 256 * 4 * 3, 16 * 1000 + 16, 85_983_744])
def test_copy_is_exact(vectors, nbytes):
    print(f"stream_copy bytes={nbytes} vectors={vectors}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(nbytes + vectors)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=gen)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device="cuda")
    ops.stream_copy(src, dst[:nbytes], vectors_per_thread=vectors)
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert int(dst[nbytes:].count_nonzero()) == 0


def test_bad_arguments_are_refused():
    src = torch.zeros(64, dtype=torch.uint8, device="cuda")
    dst = torch.zeros(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        ops.stream_copy(src, dst, vectors_per_thread=3)
    with pytest.raises(ValueError):
        ops.stream_copy(src[1:17], dst[:16])          # misaligned source
    with pytest.raises(ValueError):
        ops.stream_copy(src[:24], dst[:24])           # not a multiple of 16 bytes
