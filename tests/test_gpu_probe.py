"""The HBM bandwidth probes through the C ABI: hbm_copy reproduces its source exactly (sizes that are and are not a
multiple of the unrolled stride, grids smaller and larger than the data), hbm_read runs over the same sizes."""
import pytest
import torch

from lowbit import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("words,blocks", [(4, 1), (4 * 1000 + 4, 3), (4 * 256 * 4 * 7, 7), (1 << 22, 512),
                                          ((1 << 22) + 12, 8192)])
def test_copy_is_exact_and_read_runs(cuda, words, blocks):
    g = torch.Generator(device="cuda").manual_seed(words)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (words,), generator=g, dtype=torch.int32, device="cuda")
    dst = torch.full_like(src, 7)
    ops.ext().hbm_copy(src, dst, blocks)
    assert torch.equal(src, dst)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.ext().hbm_read(src, sink, blocks)
    torch.cuda.synchronize()
