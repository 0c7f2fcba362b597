"""Convolution epilogue (eval-mode BatchNorm1d and ReLU folded into the store).

The fused store computes relu((acc + bias - mean) / sqrt(var + eps) * gamma +
beta) in fp32 and rounds once; it is checked against the fp64 oracle of the
same expression, with the tolerances of the convolution tests (max |out - ref|
/ max |ref|: 1e-5 fp32, 1e-2 fp16/bf16).  A SparseSequential chain with fusion
is checked against the same chain run module by module (which rounds the
features between the layers), the cases that must not fuse (a BatchNorm1d in
training mode, modules with hooks) are checked to run unfused, and changes to
running statistics and weights between calls (including writes through
``.data``) are checked to take effect.
"""
import numpy as np
import pytest
import torch
import torch.nn as nn

import trispconv.pytorch as spconv
from gpu_util import DEV, needs_gpu, oracle_rows, rel_err, rounded, say, to_np
from oracle import conv as OC
from oracle import pairs as OP
from trispconv.pytorch import functional as Fn
from trispconv.pytorch.indices import generate_subm_indice_pairs
from trispconv.pytorch.weight import pack_weight
from trispconv_amd.pytorch import modules as M

pytestmark = [pytest.mark.gpu, needs_gpu]

TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _cloud(seed, shape, n):
    rng = np.random.default_rng(seed)
    cells = rng.choice(shape[0] * shape[1] * shape[2], size=n, replace=False)
    z, r = np.divmod(cells, shape[1] * shape[2])
    y, x = np.divmod(r, shape[2])
    return np.stack([np.zeros(n), z, y, x], 1).astype(np.int32)


# MFMA shapes (f16, bf16, f32) and VALU shapes (narrow / ragged channels)
CASES = [(128, 128, torch.float16), (64, 96, torch.bfloat16), (32, 64, torch.float32),
         (16, 16, torch.float32), (4, 16, torch.float16), (24, 40, torch.bfloat16)]


def _bn_tensors(rng, c_out, bn, dtype):
    """mean, var, gamma, beta as fp32 numpy arrays, the device tensors the
    kernel gets (gamma/beta None for a statistics-only norm; "mixed" gives
    fp32 statistics with gamma/beta in the features' dtype) and the values
    those tensors hold, for the oracle."""
    mean = rng.uniform(-0.3, 0.3, c_out).astype(np.float32)
    var = rng.uniform(0.25, 2.0, c_out).astype(np.float32)
    gamma = rng.uniform(0.5, 2.0, c_out).astype(np.float32)
    beta = rng.uniform(-0.5, 0.5, c_out).astype(np.float32)
    stat_dt = torch.float32 if bn == "mixed" else dtype
    aff_dt = dtype
    t = [torch.from_numpy(v).to(DEV).to(d) for v, d in
         ((mean, stat_dt), (var, stat_dt), (gamma, aff_dt), (beta, aff_dt))]
    if bn == "stats":
        t[2] = t[3] = None
    vals = [to_np(x).astype(np.float64) if x is not None else None for x in t]
    return t, vals


@pytest.mark.parametrize("c_in,c_out,dtype", CASES)
@pytest.mark.parametrize("bn,relu", [("affine", True), (None, True), ("affine", False),
                                     ("stats", True), ("mixed", False)])
def test_conv_epilogue_against_oracle(c_in, c_out, dtype, bn, relu):
    shape = (24, 24, 24)
    idx = _cloud(3, shape, 4000)
    rng = np.random.default_rng(7)
    feats = rng.standard_normal((len(idx), c_in)).astype(np.float32)
    w = (rng.standard_normal((c_out, 3, 3, 3, c_in)) / np.sqrt(27 * c_in)).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, c_out).astype(np.float32)
    eps = 1e-3
    say("epilogue:", c_in, "->", c_out, dtype, "bn", bn, "relu", relu)
    x = torch.from_numpy(idx).to(DEV)
    data = generate_subm_indice_pairs(x, shape, 1, 3)
    wt = torch.from_numpy(w).to(DEV).to(dtype)
    packed = pack_weight(wt, (3, 3, 3), c_in, c_out, dtype)
    if bn:
        tens, (mean, var, gamma, beta) = _bn_tensors(rng, c_out, bn, dtype)
        ep = Fn.Epilogue(*tens, eps, relu)
    else:
        ep = Fn.Epilogue(None, None, None, None, 0.0, relu)
    out = Fn.sparse_conv_forward(torch.from_numpy(feats).to(DEV).to(dtype), packed,
                                 torch.from_numpy(bias).to(DEV).to(dtype), data, len(idx), ep)
    pr = OP.subm_pairs(idx, shape, 1, 3, 1)
    w64 = OC.normalize_weight(rounded(w, dtype), (3, 3, 3), c_in, c_out)
    ref = oracle_rows(rounded(feats, dtype), w64, rounded(bias, dtype), pr.pairs_in,
                      pr.pairs_out, np.arange(len(idx)))
    if bn:
        ref = (ref - mean) / np.sqrt(var + np.float64(np.float32(eps)))
        if gamma is not None:
            ref = ref * gamma + beta
    if relu:
        ref = np.maximum(ref, 0.0)
    got = to_np(out)
    err = rel_err(got, ref)
    say("   rel err", err)
    assert out.dtype == dtype and np.isfinite(got).all()
    if relu:
        assert (got >= 0).all()
    assert err <= TOL[dtype]


def test_epilogue_off_is_bitwise_the_plain_convolution():
    """No batch norm and no ReLU: the same bits as the plain entry point."""
    shape = (20, 20, 20)
    idx = _cloud(5, shape, 3000)
    x = torch.from_numpy(idx).to(DEV)
    data = generate_subm_indice_pairs(x, shape, 1, 3)
    torch.manual_seed(0)
    for c_in, c_out, dtype in [(64, 64, torch.float16), (16, 8, torch.float32)]:
        f = torch.randn(len(idx), c_in, device=DEV).to(dtype)
        w = (torch.randn(c_out, 3, 3, 3, c_in, device=DEV) * 0.05).to(dtype)
        b = (torch.randn(c_out, device=DEV) * 0.1).to(dtype)
        packed = pack_weight(w, (3, 3, 3), c_in, c_out, dtype)
        a = Fn.sparse_conv_forward(f, packed, b, data, len(idx))
        # a ReLU-only epilogue equals clamping the plain result (one rounding
        # of a non-negative or zeroed value)
        r = Fn.sparse_conv_forward(f, packed, b, data, len(idx),
                                   Fn.Epilogue(None, None, None, None, 0.0, True))
        assert torch.equal(r, torch.clamp_min(a, 0)), (c_in, c_out, dtype)
        # an identity batch norm (mean 0, var 1, eps 0, gamma 1, beta 0) changes nothing
        one = torch.ones(c_out, device=DEV)
        zero = torch.zeros(c_out, device=DEV)
        i = Fn.sparse_conv_forward(f, packed, b, data, len(idx),
                                   Fn.Epilogue(zero, one, one, zero, 0.0, False))
        assert torch.equal(i, a), (c_in, c_out, dtype)


def test_epilogue_argument_errors():
    shape = (8, 8, 8)
    idx = _cloud(2, shape, 100)
    data = generate_subm_indice_pairs(torch.from_numpy(idx).to(DEV), shape, 1, 3)
    f = torch.randn(len(idx), 16, device=DEV)
    packed = pack_weight(torch.randn(32, 3, 3, 3, 16, device=DEV), (3, 3, 3), 16, 32,
                         torch.float32)
    one = torch.ones(32, device=DEV)
    with pytest.raises(ValueError):  # mean without var
        Fn.sparse_conv_forward(f, packed, None, data, len(idx),
                               Fn.Epilogue(one, None, None, None, 1e-5, False))
    with pytest.raises(ValueError):  # wrong channel count
        Fn.sparse_conv_forward(f, packed, None, data, len(idx),
                               Fn.Epilogue(one[:16], one[:16], None, None, 1e-5, False))
    with pytest.raises(ValueError):  # affine parameters without statistics
        Fn.sparse_conv_forward(f, packed, None, data, len(idx),
                               Fn.Epilogue(None, None, one, one, 1e-5, False))


def _bn(c, seed):
    g = torch.Generator().manual_seed(seed)
    bn = nn.BatchNorm1d(c)
    with torch.no_grad():
        bn.weight.copy_(torch.rand(c, generator=g) * 1.5 + 0.25)
        bn.bias.copy_(torch.randn(c, generator=g) * 0.2)
        bn.running_mean.copy_(torch.randn(c, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(c, generator=g) * 0.5 + 0.5)
    return bn


def _chain(dtype):
    torch.manual_seed(11)
    net = spconv.SparseSequential(
        spconv.SubMConv3d(16, 32, 3, indice_key="s0"), _bn(32, 1), nn.ReLU(),
        spconv.SparseConv3d(32, 64, 3, stride=2, padding=1), _bn(64, 2), nn.ReLU(inplace=True),
        spconv.SubMConv3d(64, 64, 3, indice_key="s1"), nn.ReLU(),
        spconv.SubMConv3d(64, 32, 3, indice_key="s1"), _bn(32, 3),
        spconv.SubMConv3d(32, 32, 3, indice_key="s1"))
    return net.to(DEV).to(dtype).eval()


def _input(dtype, n=6000, shape=(32, 32, 32)):
    idx = _cloud(9, shape, n)
    feats = torch.randn(n, 16, generator=torch.Generator().manual_seed(4))
    return spconv.SparseConvTensor(feats.to(DEV).to(dtype), torch.from_numpy(idx).to(DEV),
                                   list(shape), 1)


def _record(monkeypatch):
    seen = []
    orig = M.SparseConvolution.forward_with_epilogue

    def rec(self, x, ep):
        seen.append(ep)
        return orig(self, x, ep)

    monkeypatch.setattr(M.SparseConvolution, "forward_with_epilogue", rec)
    return seen


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_sequential_fusion_matches_module_by_module(dtype, monkeypatch):
    net = _chain(dtype)
    x = _input(dtype)
    seen = _record(monkeypatch)
    with torch.no_grad():
        fused = net(x)
    kinds = [None if e is None else (e.mean is not None, e.relu) for e in seen]
    say("epilogues:", kinds)
    assert kinds == [(True, True), (True, True), (False, True), (True, False), None]
    net.fuse_epilogues = False
    seen.clear()
    with torch.no_grad():
        plain = net(x)
    assert all(e is None for e in seen)
    assert torch.equal(fused.indices, plain.indices)
    err = rel_err(to_np(fused.features), to_np(plain.features).astype(np.float64))
    say("   fused vs module by module:", err)
    # module by module rounds the features between conv, BatchNorm and ReLU
    assert err <= TOL[dtype] * (1 if dtype == torch.float32 else 2)


def test_training_batchnorm_and_hooks_are_not_fused(monkeypatch):
    dtype = torch.float32
    net = _chain(dtype)
    x = _input(dtype)
    seen = _record(monkeypatch)
    net._modules["1"].train()  # batch statistics: cannot be folded
    calls = []
    net._modules["7"].register_forward_hook(lambda m, i, o: calls.append(1))  # hook on a ReLU
    with torch.no_grad():
        fused = net(x)
    kinds = [None if e is None else (e.mean is not None, e.relu) for e in seen]
    # conv0: BatchNorm in training mode -> unfused; conv2: its ReLU has a hook -> unfused
    assert kinds == [None, (True, True), None, (True, False), None], kinds
    assert calls == [1]
    net.fuse_epilogues = False
    with torch.no_grad():
        plain = net(x)
    assert rel_err(to_np(fused.features), to_np(plain.features).astype(np.float64)) <= 1e-5


def _fresh_plain(net, x):
    """The chain module by module with every packed weight dropped first."""
    for m in net.modules():
        if isinstance(m, M.SparseConvolution):
            m._packed = m._packed_key = None
    net.fuse_epilogues = False
    with torch.no_grad():
        out = net(x)
    net.fuse_epilogues = True
    return out


def test_changes_between_calls_take_effect():
    """Running statistics, BatchNorm parameters and convolution weights changed
    after a first call (in place, through ``.data``, or by assigning a new
    parameter) are what the next call uses."""
    net = _chain(torch.float32)
    x = _input(torch.float32)
    with torch.no_grad():
        first = net(x)
    conv0, bn1, conv3, bn4 = (net._modules[k] for k in ("0", "1", "3", "4"))
    bn1.running_mean.data.add_(0.25)       # writes through .data leave the version as is
    bn1.weight.data.mul_(1.5)
    with torch.no_grad():
        bn4.running_var.mul_(2.0)          # in place: a version bump
    conv0.weight.data.mul_(-1.0)
    with torch.no_grad():
        second = net(x)
    ref = _fresh_plain(net, x)
    assert not torch.equal(first.features, second.features)
    assert rel_err(to_np(second.features), to_np(ref.features).astype(np.float64)) <= 1e-5
    # a plain Parameter assigned in place of the module's own: repacked on every call
    conv3.weight = nn.Parameter(conv3.weight.detach() * 0.5)
    with torch.no_grad():
        third = net(x)
    conv3.weight.data.mul_(2.0)
    with torch.no_grad():
        fourth = net(x)
    ref = _fresh_plain(net, x)
    assert not torch.equal(third.features, fourth.features)
    assert rel_err(to_np(fourth.features), to_np(ref.features).astype(np.float64)) <= 1e-5


def test_voxelnet_encoder_full_size_fused_against_oracle():
    """The VoxelNet-style encoder workload at full size (4 x 60k LiDAR-like
    voxels, fp16) as the SparseSequential a user writes: eleven conv layers,
    each but the last followed by an eval-mode BatchNorm1d (random affine and
    running statistics) and a ReLU, fused into the conv stores.  Layer by
    layer on the GPU's own layer inputs, every output row against the fp64
    oracle (conv, bias, batch norm and ReLU in fp64) at the fp16 tolerance;
    output coordinates, pair_num and every slot's pair lists of every
    indice_key exact; the whole forward equal to the layer-by-layer chain bit
    for bit."""
    from trispconv_amd import workloads

    w = workloads.make_workload("voxelnet_encoder4x60k")
    dtype = torch.float16
    rng = np.random.default_rng(w.seed)
    mods = []
    for i, lay in enumerate(w.layers):
        if lay["kind"] == "subm":
            m = spconv.SubMConv3d(lay["c_in"], lay["c_out"], lay["kernel_size"],
                                  indice_key=lay["indice_key"])
        else:
            m = spconv.SparseConv3d(lay["c_in"], lay["c_out"], lay["kernel_size"],
                                    stride=lay["stride"], padding=lay["padding"],
                                    indice_key=lay["indice_key"])
        wk, bk = workloads.layer_params(rng, lay)
        with torch.no_grad():
            m.weight.copy_(torch.from_numpy(wk))
            m.bias.copy_(torch.from_numpy(bk))
        mods.append(m)
        if i + 1 < len(w.layers):
            bn = nn.BatchNorm1d(lay["c_out"])
            with torch.no_grad():
                bn.weight.copy_(torch.from_numpy(rng.uniform(0.5, 1.5, lay["c_out"])))
                bn.bias.copy_(torch.from_numpy(rng.uniform(-0.2, 0.2, lay["c_out"])))
                bn.running_mean.copy_(torch.from_numpy(rng.uniform(-0.1, 0.1, lay["c_out"])))
                bn.running_var.copy_(torch.from_numpy(rng.uniform(0.5, 1.5, lay["c_out"])))
            mods += [bn, nn.ReLU()]
    net = spconv.SparseSequential(*mods).to(DEV).to(dtype).eval()
    feats = torch.from_numpy(workloads.features(rng, len(w.indices), 4)).to(DEV).to(dtype)
    x0 = spconv.SparseConvTensor(feats, torch.from_numpy(w.indices).to(DEV),
                                 list(w.spatial_shape), w.batch_size)
    with torch.no_grad():
        whole = net(x0)
    # layer by layer through the same fused path, on a fresh tensor
    x = spconv.SparseConvTensor(feats, x0.indices, list(w.spatial_shape), w.batch_size)
    children = list(net.children())
    oracle_pairs = {}
    i = 0
    li = 0
    with torch.no_grad():
        while i < len(children):
            m = children[i]
            i += 1
            ep, used = M._fusable(children, i, m, x)
            y = m.forward_with_epilogue(x, ep)
            idx = x.indices.cpu().numpy()
            shape = tuple(x.spatial_shape)
            key = m.indice_key
            if key not in oracle_pairs:
                oracle_pairs[key] = (OP.subm_pairs(idx, shape, w.batch_size, m.kernel_size)
                                     if m.subm else
                                     OP.strided_pairs(idx, shape, w.batch_size, m.kernel_size,
                                                      m.stride, m.padding, m.dilation))
                # the layer's pair lists, bit for bit, once per key: the
                # submanifold builds of layers 3, 6 and 9 run on the strided
                # output bitmap (tsc_subm_pairs_from_bitmap)
                got = y.indice_dict[key]
                pr = oracle_pairs[key]
                assert got.pair_num.tolist() == pr.pair_num.tolist(), (li, key)
                for k in range(len(pr.pairs_in)):
                    assert np.array_equal(got.pairs_in[k].cpu().numpy(), pr.pairs_in[k]), (li, k)
                    assert np.array_equal(got.pairs_out[k].cpu().numpy(), pr.pairs_out[k]), (li, k)
                say(f"encoder layer {li} key {key}: pair lists equal,",
                    int(pr.pair_num.sum()), "pairs")
            pr = oracle_pairs[key]
            assert np.array_equal(y.indices.cpu().numpy(), pr.out_indices), li
            wt = OC.normalize_weight(to_np(m.weight).astype(np.float64), m.kernel_size,
                                     m.in_channels, m.out_channels)
            ref = OC.conv_forward(to_np(x.features).astype(np.float64), wt,
                                  to_np(m.bias).astype(np.float64), pr.pairs_in, pr.pairs_out,
                                  len(pr.out_indices))
            if used:
                bn = children[i]
                mean, var, g, b = (to_np(t).astype(np.float64) for t in
                                   (bn.running_mean, bn.running_var, bn.weight, bn.bias))
                ref = (ref - mean) / np.sqrt(var + bn.eps) * g + b
                ref = np.maximum(ref, 0.0)
            err = rel_err(to_np(y.features), ref)
            say(f"encoder layer {li} {m.in_channels}->{m.out_channels}",
                "bn+relu" if used else "plain", "rows", len(ref), "rel err", err)
            assert err <= TOL[dtype], li
            x = y
            i += used
            li += 1
    assert torch.equal(whole.indices, x.indices)
    assert torch.equal(whole.features, x.features)
