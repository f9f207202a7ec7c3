"""Dense -> sparse converter on the GPU (spiky_amd/util/torch_utils.py over
spiky_amd/csrc/lut_densify.hip) against the oracle restatement.

The first test is the reference's own check (torch_utils.py:128-193) over all
four of its (erase, buffers) cases; the reference's loop returns after the
first.  The output here is in ascending index order, so it is compared with
the ground truth directly rather than after a sort."""
import numpy as np
import pytest
import torch

from spiky_amd.util.torch_utils import DenseToSparseConverter

pytestmark = pytest.mark.gpu


def _check(oracle, src_before, idx, val):
    want_i, want_v = oracle.dense_to_sparse_32(src_before.cpu().numpy())
    if want_i.size == 0:
        assert idx is None and val is None
        return
    got_i = idx.cpu().numpy()
    assert got_i.dtype == np.int64
    assert np.array_equal(got_i, want_i)
    assert np.array_equal(val.cpu().numpy().view(np.uint32), want_v.view(np.uint32))


@pytest.mark.parametrize("erase", [True, False])
@pytest.mark.parametrize("buffers", [True, False])
def test_reference_converter_check(oracle, cuda_device, erase, buffers):
    dev = cuda_device
    numel = 150000
    print(f"[densify] reference check erase={erase} buffers={buffers}", flush=True)
    g = torch.Generator(device=dev).manual_seed(7)
    t = torch.rand(numel, device=dev, generator=g)
    t[t > 0.5] = 0.0
    before = t.clone()
    bufs = ((torch.empty(numel, dtype=torch.int64, device=dev), torch.empty(numel, device=dev))
            if buffers else None)
    conv = DenseToSparseConverter()
    idx, val = conv.dense_to_sparse_32(t, erase, bufs)
    _check(oracle, before, idx, val)
    if erase:
        assert torch.count_nonzero(t) == 0
    else:
        assert torch.equal(t, before)


def test_bit_patterns_and_int32(oracle, cuda_device):
    """-0.0 is kept (bitwise test); int32 sources keep their dtype."""
    dev = cuda_device
    f = torch.zeros(4096 + 8, device=dev)
    f[3] = -0.0
    f[4100] = 1.5
    f[17] = float("nan")
    conv = DenseToSparseConverter()
    idx, val = conv.dense_to_sparse_32(f.clone())
    _check(oracle, f, idx, val)
    assert idx.tolist() == [3, 17, 4100]
    i = torch.zeros(64, dtype=torch.int32, device=dev)
    i[5], i[63] = -1, 1 << 30
    idx, val = conv.dense_to_sparse_32(i)
    assert val.dtype == torch.int32
    _check(oracle, i, idx, val)


def test_empty_and_tiny(oracle, cuda_device):
    dev = cuda_device
    conv = DenseToSparseConverter()
    assert conv.dense_to_sparse_32(torch.zeros(4096 * 3, device=dev)) == (None, None)
    bufs = (torch.empty(4, dtype=torch.int64, device=dev), torch.empty(4, device=dev))
    assert conv.dense_to_sparse_32(torch.zeros(4, device=dev), True, bufs) == (None, None)
    t = torch.tensor([0.0, 0.0, 0.0, 2.0], device=dev)
    idx, val = conv.dense_to_sparse_32(t.clone(), True, bufs)
    assert idx.tolist() == [3] and val.tolist() == [2.0]


def test_many_tiles_ragged(oracle, cuda_device):
    """Hundreds of 4096-word tiles with a ragged last one; densities from
    empty tiles to full ones, so offsets carry across zero-count tiles."""
    dev = cuda_device
    n = 4096 * 300 + 12
    g = torch.Generator(device=dev).manual_seed(11)
    t = torch.randn(n, device=dev, generator=g)
    keep = torch.rand(n, device=dev, generator=g)
    dens = torch.linspace(0.0, 1.0, 301, device=dev).repeat_interleave(4096)[:n]
    t[keep >= dens] = 0.0
    t[4096 * 5:4096 * 9] = 0.0
    before = t.clone()
    conv = DenseToSparseConverter()
    idx, val = conv.dense_to_sparse_32(t)
    _check(oracle, before, idx, val)
    assert conv.count_nonzero(before) == idx.numel()


def test_buffers_too_small_are_reported(cuda_device):
    """More non-zero words than buffer entries: the kernel writes only what
    fits and decoupling raises."""
    dev = cuda_device
    t = torch.ones(64, device=dev)
    bufs = (torch.empty(16, dtype=torch.int64, device=dev), torch.empty(16, device=dev))
    with pytest.raises(ValueError, match="non-zero words"):
        DenseToSparseConverter().dense_to_sparse_32(t, False, bufs)
    assert bufs[0].tolist() == list(range(16))
