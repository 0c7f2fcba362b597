"""SparseConvTensor.dense() on the GPU against the reference's definition
(tensor.py:72-99: zeros (B, D, H, W, C), dense[b, z, y, x] = features, then
permute to (B, C, D, H, W)), evaluated with torch on the CPU.  Exact equality:
the values are copied bit for bit."""
import numpy as np
import pytest
import torch

import trispconv.pytorch as spconv
from gpu_util import DEV, needs_gpu, say

pytestmark = [pytest.mark.gpu, needs_gpu]


def _reference_dense(feats, idx, B, shape, channels_first):
    D, H, W = shape
    dense = torch.zeros((B, D, H, W, feats.shape[1]), dtype=feats.dtype)
    i = idx.long()
    dense[i[:, 0], i[:, 1], i[:, 2], i[:, 3]] = feats
    return dense.permute(0, 4, 1, 2, 3).contiguous() if channels_first else dense


def _unique_cells(seed, B, shape, n):
    rng = np.random.default_rng(seed)
    total = B * shape[0] * shape[1] * shape[2]
    cells = rng.choice(total, size=n, replace=False)
    b, r = np.divmod(cells, shape[0] * shape[1] * shape[2])
    z, r = np.divmod(r, shape[1] * shape[2])
    y, x = np.divmod(r, shape[2])
    return torch.from_numpy(np.stack([b, z, y, x], 1).astype(np.int32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("channels_first", [True, False])
@pytest.mark.parametrize("B,shape,C,n", [(2, (4, 5, 6), 3, 50), (1, (3, 5, 7), 3, 40),
                                         (4, (2, 20, 18), 128, 700), (3, (9, 1, 11), 5, 0)])
def test_dense_matches_reference(dtype, channels_first, B, shape, C, n):
    say("dense:", dtype, channels_first, B, shape, C, n)
    idx = _unique_cells(n + C, B, shape, n)
    feats = torch.randn(n, C, generator=torch.Generator().manual_seed(n)).to(dtype)
    x = spconv.SparseConvTensor(feats.to(DEV), idx.to(DEV), list(shape), B)
    got = x.dense(channels_first=channels_first).cpu()
    ref = _reference_dense(feats, idx, B, shape, channels_first)
    assert got.dtype == dtype and got.shape == ref.shape
    assert torch.equal(got, ref)


@pytest.mark.parametrize("dtype", [torch.float64, torch.int64, torch.int16, torch.uint8,
                                   torch.bool])
@pytest.mark.parametrize("channels_first", [True, False])
def test_dense_any_element_size(dtype, channels_first):
    """The reference allocates the dense tensor in the features' own dtype,
    whatever it is (tensor.py:84-88): 8-, 2- and 1-byte elements too."""
    B, shape, C, n = 2, (5, 6, 7), 3, 120
    say("dense any dtype:", dtype, channels_first)
    idx = _unique_cells(7, B, shape, n)
    g = torch.Generator().manual_seed(11)
    if dtype.is_floating_point:
        feats = torch.randn(n, C, generator=g, dtype=torch.float64).to(dtype)
    elif dtype == torch.bool:
        feats = torch.randint(0, 2, (n, C), generator=g).bool()
    else:
        feats = torch.randint(0, 100, (n, C), generator=g).to(dtype)
    x = spconv.SparseConvTensor(feats.to(DEV), idx.to(DEV), list(shape), B)
    got = x.dense(channels_first=channels_first).cpu()
    ref = _reference_dense(feats, idx, B, shape, channels_first)
    assert got.dtype == dtype and got.shape == ref.shape
    assert torch.equal(got, ref)


def test_dense_out_of_range_raises():
    idx = torch.tensor([[0, 1, 1, 1], [0, 4, 0, 0]], dtype=torch.int32, device=DEV)
    x = spconv.SparseConvTensor(torch.ones(2, 3, device=DEV), idx, [4, 4, 4], 1)
    with pytest.raises(AssertionError):
        x.dense()
    idx = torch.tensor([[1, 0, 0, 0]], dtype=torch.int32, device=DEV)
    x = spconv.SparseConvTensor(torch.ones(1, 3, device=DEV), idx, [4, 4, 4], 1)
    with pytest.raises(AssertionError):
        x.dense(channels_first=False)
