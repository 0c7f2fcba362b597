"""The reference's own test suite, run through the HIP backend on the GPU.

Same inputs, oracles and tolerances as the reference's tests; tensors live on
the GPU because this backend has no CPU path:
  tests/test_indices_subm.py, tests/test_indices_strided.py (dense conv3d),
  tests/test_vs_dense.py (24 strided + 8 SubM cases, SparseSequential+BN),
  tests/test_vs_spconv.py (the nine spconv golden fixtures),
  tests/test_large_channel_reduction.py (no NaN / Inf at C_in up to 2048).
"""
import numpy as np
import pytest
import torch
import torch.nn as nn

import golden_io
import trispconv.pytorch as spconv
from gpu_util import DEV, needs_gpu, say
from trispconv.testing.sparse_data import generate_sparse_data, sparse_data_to_tensors

pytestmark = [pytest.mark.gpu, needs_gpu]

torch.backends.cuda.matmul.allow_tf32 = False


def _gpu(m):
    return m.to(DEV)


def _sp(features, indices, shape, B, **kw):
    return spconv.SparseConvTensor(features.to(DEV), indices.to(DEV), shape, B, **kw)


def _krsc_to_conv3d(w):
    return w.permute(0, 4, 1, 2, 3).contiguous()


# ------------------------------------------------- tests/test_indices_subm.py
def _dense_subm_reference(features, indices, shape, weight, bias, B):
    C_in = features.shape[1]
    D, H, W = shape
    dense = torch.zeros(B, C_in, D, H, W, dtype=features.dtype)
    i = indices.long()
    dense[i[:, 0], :, i[:, 1], i[:, 2], i[:, 3]] = features
    k = weight.shape[1:4]
    out = torch.nn.functional.conv3d(dense, _krsc_to_conv3d(weight), bias=bias,
                                     padding=(k[0] // 2, k[1] // 2, k[2] // 2))
    return out[i[:, 0], :, i[:, 1], i[:, 2], i[:, 3]]


def test_subm_3x3x3_vs_dense():
    torch.manual_seed(0)
    N, C_in, C_out = 12, 4, 8
    coords = torch.randint(1, 9, (N, 3), dtype=torch.int32)
    idx = torch.cat([torch.zeros(N, 1, dtype=torch.int32), coords], 1)
    feats = torch.randn(N, C_in)
    w = torch.randn(C_out, 3, 3, 3, C_in)
    b = torch.randn(C_out)
    ref = _dense_subm_reference(feats, idx, (10, 10, 10), w, b, 1)
    conv = spconv.SubMConv3d(C_in, C_out, 3, bias=True)
    conv.weight.data.copy_(w)
    conv.bias.data.copy_(b)
    y = _gpu(conv)(_sp(feats, idx, [10, 10, 10], 1))
    assert y.features.shape == (N, C_out)
    assert torch.allclose(y.features.cpu(), ref, atol=1e-4, rtol=1e-4)


def test_subm_1x1x1_vs_dense():
    torch.manual_seed(1)
    N, C = 8, 6
    coords = torch.randint(0, 8, (N, 3), dtype=torch.int32)
    idx = torch.cat([torch.zeros(N, 1, dtype=torch.int32), coords], 1)
    feats = torch.randn(N, C)
    w = torch.randn(C, 1, 1, 1, C)
    ref = feats @ w.reshape(C * C).view(C, C)
    conv = spconv.SubMConv3d(C, C, 1, bias=False)
    conv.weight.data.copy_(w)
    y = _gpu(conv)(_sp(feats, idx, [8, 8, 8], 1))
    # torch.randint can repeat a coordinate; every row of a 1x1x1 layer maps to
    # the last row with its coordinate, exactly as the reference's table does
    i = idx.long()
    keys = (i[:, 1] * 8 + i[:, 2]) * 8 + i[:, 3]
    last = torch.tensor([int((keys == keys[r]).nonzero().max()) for r in range(N)])
    assert torch.allclose(y.features.cpu(), ref[last], atol=1e-4, rtol=1e-4)


def test_subm_preserves_active_set():
    torch.manual_seed(2)
    N = 15
    coords = torch.randint(1, 11, (N, 3), dtype=torch.int32)
    idx = torch.cat([torch.zeros(N, 1, dtype=torch.int32), coords], 1)
    x = _sp(torch.randn(N, 4), idx, [12, 12, 12], 1)
    y = _gpu(spconv.SubMConv3d(4, 8, 3, bias=False))(x)
    assert torch.equal(y.indices, x.indices)
    assert y.spatial_shape == x.spatial_shape


def test_subm_indice_key_caching():
    torch.manual_seed(3)
    coords = torch.randint(1, 7, (10, 3), dtype=torch.int32)
    idx = torch.cat([torch.zeros(10, 1, dtype=torch.int32), coords], 1)
    conv = _gpu(spconv.SubMConv3d(4, 4, 3, bias=False, indice_key="subm0"))
    y = conv(_sp(torch.randn(10, 4), idx, [8, 8, 8], 1))
    assert "subm0" in y.indice_dict
    cached = y.indice_dict["subm0"]
    y2 = conv(y)
    assert y2.indice_dict["subm0"] is cached


def test_subm_batch_size_2():
    torch.manual_seed(4)
    N = 20
    coords = torch.randint(1, 7, (N, 3), dtype=torch.int32)
    batch = torch.cat([torch.zeros(N // 2, 1, dtype=torch.int32),
                       torch.ones(N // 2, 1, dtype=torch.int32)])
    idx = torch.cat([batch, coords], 1)
    conv = spconv.SubMConv3d(4, 6, 3, bias=False)
    conv.weight.data.copy_(torch.randn(6, 3, 3, 3, 4))
    y = _gpu(conv)(_sp(torch.randn(N, 4), idx, [8, 8, 8], 2))
    assert y.features.shape == (N, 6) and y.batch_size == 2


# ---------------------------------------------- tests/test_indices_strided.py
def test_strided_vs_dense_full_grid():
    torch.manual_seed(10)
    zz, yy, xx = torch.meshgrid(torch.arange(10), torch.arange(10), torch.arange(10), indexing="ij")
    idx = torch.stack([torch.zeros(1000, dtype=torch.long), zz.reshape(-1), yy.reshape(-1),
                       xx.reshape(-1)], 1).int()
    feats = torch.randn(1000, 4)
    w = torch.randn(8, 3, 3, 3, 4)
    b = torch.randn(8)
    conv = spconv.SparseConv3d(4, 8, 3, stride=2, padding=1, bias=True)
    conv.weight.data.copy_(w)
    conv.bias.data.copy_(b)
    y = _gpu(conv)(_sp(feats, idx, [10, 10, 10], 1))
    dense = torch.zeros(1, 4, 10, 10, 10)
    i = idx.long()
    dense[i[:, 0], :, i[:, 1], i[:, 2], i[:, 3]] = feats
    out = torch.nn.functional.conv3d(dense, _krsc_to_conv3d(w), bias=b, stride=2, padding=1)
    o = y.indices.cpu().long()
    ref = out[o[:, 0], :, o[:, 1], o[:, 2], o[:, 3]]
    assert torch.allclose(y.features.cpu(), ref, atol=1e-4, rtol=1e-4)


def test_strided_output_shape():
    torch.manual_seed(11)
    coords = torch.randint(0, 8, (30, 3), dtype=torch.int32)
    idx = torch.cat([torch.zeros(30, 1, dtype=torch.int32), coords], 1)
    y = _gpu(spconv.SparseConv3d(4, 8, 3, stride=2, padding=1, bias=False))(
        _sp(torch.randn(30, 4), idx, [8, 8, 8], 1))
    assert y.spatial_shape == [4, 4, 4]
    assert int(y.indices[:, 1:].max()) < 4


def test_strided_indice_key_stored():
    torch.manual_seed(12)
    coords = torch.randint(0, 8, (20, 3), dtype=torch.int32)
    idx = torch.cat([torch.zeros(20, 1, dtype=torch.int32), coords], 1)
    y = _gpu(spconv.SparseConv3d(4, 8, 3, stride=2, padding=1, bias=False, indice_key="down1"))(
        _sp(torch.randn(20, 4), idx, [8, 8, 8], 1))
    assert "down1" in y.indice_dict


def test_inverse_conv_restores_coords():
    torch.manual_seed(13)
    coords = torch.randint(0, 8, (20, 3), dtype=torch.int32)
    idx = torch.cat([torch.zeros(20, 1, dtype=torch.int32), coords], 1)
    down = _gpu(spconv.SparseConv3d(4, 8, 3, stride=2, padding=1, bias=False, indice_key="down1"))
    up = _gpu(spconv.SparseInverseConv3d(8, 4, 3, bias=False, indice_key="down1"))
    x = _sp(torch.randn(20, 4), idx, [8, 8, 8], 1)
    z = up(down(x))
    assert torch.equal(z.indices, x.indices)
    assert z.spatial_shape == [8, 8, 8]
    assert z.features.shape == (20, 4)


def test_inverse_conv_missing_key_raises():
    conv = _gpu(spconv.SparseInverseConv3d(4, 4, 3, indice_key="missing"))
    with pytest.raises(KeyError):
        conv(_sp(torch.randn(5, 4), torch.zeros(5, 4, dtype=torch.int32), [8, 8, 8], 1))


# ---------------------------------------------------- tests/test_vs_dense.py
SHAPE = [19, 18, 17]
STRIDED = [(bs, k, s, p, d) for bs in [1, 2] for k in [2, 3] for s in [1, 2] for p in [0, 1]
           for d in [1, 2] if not (s > 1 and d > 1)]


def _make(bs, C, seed):
    data = generate_sparse_data(SHAPE, [300] * bs, C, seed=seed)
    return sparse_data_to_tensors(data)


@pytest.mark.parametrize("bs,k,s,p,d", STRIDED)
def test_sparseconv3d_vs_dense(bs, k, s, p, d):
    seed = hash((bs, k, s, p, d)) % (2 ** 31)
    feats, dense_in, idx = _make(bs, 16, seed)
    w = torch.from_numpy(np.random.default_rng(seed).uniform(-1, 1, (16, k, k, k, 16))
                         .astype(np.float32))
    conv = spconv.SparseConv3d(16, 16, k, stride=s, padding=p, dilation=d, bias=False)
    conv.weight.data.copy_(w)
    y = _gpu(conv)(_sp(feats, idx, SHAPE, bs))
    sp_dense = y.dense().cpu()
    ref = nn.functional.conv3d(dense_in, _krsc_to_conv3d(w), stride=s, padding=p, dilation=d)
    assert sp_dense.shape == ref.shape
    o = y.indices.cpu().long()
    a = sp_dense[o[:, 0], :, o[:, 1], o[:, 2], o[:, 3]]
    b = ref[o[:, 0], :, o[:, 1], o[:, 2], o[:, 3]]
    assert torch.allclose(a, b, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("bs,k,d", [(bs, k, d) for bs in [1, 2] for k in [1, 3] for d in [1, 2]])
def test_submconv3d_vs_dense(bs, k, d):
    seed = hash((bs, k, d)) % (2 ** 31)
    feats, dense_in, idx = _make(bs, 16, seed)
    w = torch.from_numpy(np.random.default_rng(seed).uniform(-1, 1, (16, k, k, k, 16))
                         .astype(np.float32))
    conv = spconv.SubMConv3d(16, 16, k, dilation=d, bias=False)
    conv.weight.data.copy_(w)
    y = _gpu(conv)(_sp(feats, idx, SHAPE, bs))
    i = idx.long()
    if k == 1:
        ref = feats @ w.reshape(256).view(16, 16)
    else:
        out = nn.functional.conv3d(dense_in, _krsc_to_conv3d(w), padding=d * (k // 2), dilation=d)
        ref = out[i[:, 0], :, i[:, 1], i[:, 2], i[:, 3]]
    assert torch.allclose(y.features.cpu(), ref, atol=1e-4, rtol=1e-4)


def test_sparse_sequential_with_batchnorm():
    torch.manual_seed(99)
    coords = torch.randint(0, 8, (20, 3), dtype=torch.int32)
    idx = torch.cat([torch.zeros(20, 1, dtype=torch.int32), coords], 1)
    seq = _gpu(spconv.SparseSequential(spconv.SubMConv3d(16, 16, 3, bias=False),
                                       nn.BatchNorm1d(16), nn.ReLU()))
    seq.eval()
    x = _sp(torch.randn(20, 16), idx, [8, 8, 8], 1)
    y = seq(x)
    assert isinstance(y, spconv.SparseConvTensor)
    assert y.features.shape == (20, 16)
    assert bool((y.features >= 0).all())
    assert torch.equal(y.indices, x.indices)


# --------------------------------------------------- tests/test_vs_spconv.py
def _enc(idx, shape):
    D, H, W = shape
    i = idx.long()
    return ((i[:, 0] * D + i[:, 1]) * H + i[:, 2]) * W + i[:, 3]


def _sort(f, i, shape):
    o = _enc(i, shape).argsort()
    return f[o], i[o]


@pytest.mark.parametrize("name", golden_io.fixture_names())
def test_vs_spconv_golden(name):
    a, m = golden_io.load(name)
    t = {k: torch.from_numpy(v) for k, v in a.items()}
    k, s, p, d = m["kernel_size"], m["stride"], m["padding"], m["dilation"]
    B = m["batch_size"]
    use_bias = "bias" in t
    say("golden", name)
    with torch.no_grad():
        if m["conv_type"] in ("subm", "strided"):
            if m["conv_type"] == "subm":
                mod = spconv.SubMConv3d(m["C_in"], m["C_out"], k, dilation=d, bias=use_bias)
            else:
                mod = spconv.SparseConv3d(m["C_in"], m["C_out"], k, stride=s, padding=p,
                                          dilation=d, bias=use_bias)
            mod.weight.data.copy_(t["weight"])
            if use_bias:
                mod.bias.data.copy_(t["bias"])
            y = _gpu(mod)(_sp(t["features"], t["indices"], m["spatial_shape"], B))
            f, i = _sort(y.features.cpu(), y.indices.cpu(), y.spatial_shape)
        else:
            down = spconv.SparseConv3d(m["down_C_in"], m["down_C_out"], k, stride=s, padding=p,
                                       bias=False, indice_key="down")
            down.weight.data.copy_(t["down_weight"])
            xd = _gpu(down)(_sp(t["down_in_features"], t["down_in_indices"],
                                m["down_in_spatial_shape"], B))
            ref_sorted = _enc(t["indices"], xd.spatial_shape).argsort()
            ours_sorted = _enc(xd.indices.cpu(), xd.spatial_shape).argsort()
            perm = torch.empty(len(ours_sorted), dtype=torch.long)
            perm[ours_sorted] = torch.arange(len(ours_sorted))
            feats = t["features"][ref_sorted][perm]
            up = spconv.SparseInverseConv3d(m["C_in"], m["C_out"], k, bias=use_bias,
                                            indice_key="down")
            up.weight.data.copy_(t["weight"])
            if use_bias:
                up.bias.data.copy_(t["bias"])
            xi = spconv.SparseConvTensor(feats.to(DEV), xd.indices, xd.spatial_shape, B,
                                         indice_dict=xd.indice_dict)
            y = _gpu(up)(xi)
            f, i = _sort(y.features.cpu(), y.indices.cpu(), y.spatial_shape)
    assert i.shape == t["out_indices"].shape
    assert torch.equal(i, t["out_indices"])
    assert torch.allclose(f, t["out_features"], atol=1e-4, rtol=1e-4)


# ------------------------------------- tests/test_large_channel_reduction.py
def _subm_input(n, C, seed):
    data = generate_sparse_data([32, 32, 32], [n], C, seed=seed)
    feats, _, idx = sparse_data_to_tensors(data)
    return feats.to(DEV), idx.to(DEV)


def _run_subm(C_in, C_out, k, feats, idx, seed, dtype):
    conv = spconv.SubMConv3d(C_in, C_out, k, bias=False)
    w = np.random.default_rng(seed).uniform(-0.1, 0.1, (C_out, k, k, k, C_in)).astype(np.float32)
    conv.weight.data.copy_(torch.from_numpy(w))
    conv = conv.to(DEV).to(dtype)
    return conv(spconv.SparseConvTensor(feats.to(dtype), idx, [32, 32, 32], 1)).features


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_subm_2048_to_128_no_nan(dtype):
    feats, idx = _subm_input(8083, 2048, 42)
    out = _run_subm(2048, 128, 3, feats * 4000.0, idx, 0, dtype)
    assert not out.isnan().any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_subm_2048_to_128_post_norm_no_nan(dtype):
    feats, idx = _subm_input(8083, 2048, 42)
    out = _run_subm(2048, 128, 3, torch.nn.functional.silu(feats), idx, 0, dtype)
    assert not out.isnan().any()


LARGE = [(ci, co, k, n, dt) for ci, co in [(2048, 128), (2048, 256), (1024, 128), (1024, 64)]
         for k in [1, 3] for n in [1000, 8000] for dt in [torch.float32, torch.float16]]


@pytest.mark.parametrize("C_in,C_out,k,n,dtype", LARGE)
def test_subm_large_reduction_no_nan(C_in, C_out, k, n, dtype):
    say("large reduction", C_in, C_out, k, n, dtype)
    feats, idx = _subm_input(n, C_in, hash((C_in, C_out, k, n)) % (2 ** 31))
    out = _run_subm(C_in, C_out, k, feats * 100.0, idx, hash((C_in, C_out, k)) % (2 ** 31), dtype)
    assert not out.isnan().any()
    assert not out.isinf().any()
