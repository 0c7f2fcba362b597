"""The layer shapes of the reference's checkpoint test (tests/test_anigen_weights.py:60-91):
an upsample block of SparseInverseConv3d(768, 192, 3), SubMConv3d(192, 192, 3)
and the skip SparseInverseConv3d(768, 192, 1), bias-free, with KRSC weights
copied in through ``weight.data`` as that test does.  The checkpoint itself
is not available, so the weights are seeded; every output is compared with
the fp64 oracle at the convolution tolerances.
"""
import numpy as np
import pytest
import torch

import trispconv.pytorch as spconv
from gpu_util import DEV, needs_gpu, rel_err, rounded, say, to_np
from oracle import conv as OC
from oracle import pairs as OP

pytestmark = [pytest.mark.gpu, needs_gpu]

TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _cloud(seed, shape, n):
    rng = np.random.default_rng(seed)
    cells = rng.choice(shape[0] * shape[1] * shape[2], size=n, replace=False)
    z, r = np.divmod(cells, shape[1] * shape[2])
    y, x = np.divmod(r, shape[2])
    return np.stack([np.zeros(n), z, y, x], 1).astype(np.int32)


def _krsc(seed, c_out, k, c_in):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(c_out, k, k, k, c_in, generator=g) / np.sqrt(k ** 3 * c_in)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_upsample_block_shapes(dtype):
    shape = (24, 24, 24)
    idx = _cloud(1, shape, 3000)
    x0 = spconv.SparseConvTensor(torch.zeros(len(idx), 192, device=DEV, dtype=dtype),
                                 torch.from_numpy(idx).to(DEV), list(shape), 1)
    # forward convolutions that the inverses undo (their keys hold the pairs)
    down3 = spconv.SparseConv3d(192, 768, 3, stride=2, padding=1, bias=False,
                                indice_key="up0").to(DEV).to(dtype)
    down1 = spconv.SparseConv3d(192, 768, 1, stride=2, bias=False,
                                indice_key="up0_skip").to(DEV).to(dtype)
    inv3 = spconv.SparseInverseConv3d(768, 192, 3, bias=False, indice_key="up0")
    subm3 = spconv.SubMConv3d(192, 192, 3, bias=False)
    inv1 = spconv.SparseInverseConv3d(768, 192, 1, bias=False, indice_key="up0_skip")
    inv3.weight.data.copy_(_krsc(2, 192, 3, 768))    # as the reference's test loads them
    subm3.weight.data.copy_(_krsc(3, 192, 3, 192))
    inv1.weight.data.copy_(_krsc(4, 192, 1, 768))
    inv3, subm3, inv1 = (m.to(DEV).to(dtype) for m in (inv3, subm3, inv1))

    y3 = down3(x0)
    rng = np.random.default_rng(5)
    mid3 = rng.standard_normal((len(y3.indices), 768)).astype(np.float32)
    z3 = inv3(y3.replace_feature(torch.from_numpy(mid3).to(DEV).to(dtype)))
    fwd = OP.strided_pairs(idx, shape, 1, 3, 2, 1)
    inv = OP.inverse_pairs(fwd)
    assert np.array_equal(z3.indices.cpu().numpy(), inv.out_indices)
    w = OC.normalize_weight(to_np(inv3.weight).astype(np.float64), (3, 3, 3), 768, 192)
    ref3 = OC.conv_forward(rounded(mid3, dtype), w, None, inv.pairs_in, inv.pairs_out,
                           len(inv.out_indices))
    err = rel_err(to_np(z3.features), ref3)
    say("inverse 768->192:", dtype, err)
    assert err <= TOL[dtype]

    s = subm3(z3)
    pr = OP.subm_pairs(inv.out_indices, shape, 1, 3, 1)
    w = OC.normalize_weight(to_np(subm3.weight).astype(np.float64), (3, 3, 3), 192, 192)
    ref_s = OC.conv_forward(to_np(z3.features).astype(np.float64), w, None, pr.pairs_in,
                            pr.pairs_out, len(inv.out_indices))
    err = rel_err(to_np(s.features), ref_s)
    say("subm 192->192:", dtype, err)
    assert err <= TOL[dtype]

    y1 = down1(x0)
    mid1 = rng.standard_normal((len(y1.indices), 768)).astype(np.float32)
    z1 = inv1(y1.replace_feature(torch.from_numpy(mid1).to(DEV).to(dtype)))
    # 1x1x1 inverse: the dense product at the inverse input's coordinates
    # (modules.py:162-173), with spconv's fold of the flat KRSC storage
    assert z1.indices is y1.indices
    fold = to_np(inv1.weight).astype(np.float64).reshape(-1).reshape(768, 192)
    err = rel_err(to_np(z1.features), rounded(mid1, dtype) @ fold)
    say("inverse 1x1x1 768->192:", dtype, err)
    assert err <= TOL[dtype]
