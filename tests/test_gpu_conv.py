"""Fused convolution on the GPU against the fp64 oracle.

Tolerance (max |out - ref| / max |ref|, oracle in fp64 over the rounded
inputs and weights): 1e-5 for fp32, 1e-2 for fp16 and bf16.  Covers the VALU,
narrow-MFMA, slot-split and 256-row MFMA kernels, every MFMA tile shape,
ragged and wide channels,
1x1x1 layers, the five workloads at full size (every output row), bitwise
determinism and independence from the execution order.
"""
import numpy as np
import pytest
import torch

import trispconv.pytorch as spconv
from gpu_util import DEV, lists_np, needs_gpu, oracle_rows, rel_err, rounded, say, to_np
from oracle import conv as OC
from oracle import pairs as OP
from trispconv.pytorch import functional as Fn
from trispconv.pytorch.indices import generate_strided_indice_pairs, generate_subm_indice_pairs
from trispconv_amd import workloads
from trispconv_amd import _lib as L
from trispconv_amd.pytorch import indices as I

pytestmark = [pytest.mark.gpu, needs_gpu]

TOL = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}


def _module(kind, c_in, c_out, k, s=1, p=0, d=1, key=None, dtype=torch.float32, seed=0, bias=True):
    torch.manual_seed(seed)
    if kind == "subm":
        m = spconv.SubMConv3d(c_in, c_out, k, dilation=d, bias=bias, indice_key=key)
    elif kind == "strided":
        m = spconv.SparseConv3d(c_in, c_out, k, stride=s, padding=p, dilation=d, bias=bias,
                                indice_key=key)
    else:
        m = spconv.SparseInverseConv3d(c_in, c_out, k, bias=bias, indice_key=key)
    if bias:
        with torch.no_grad():
            m.bias.uniform_(-0.1, 0.1)
    return m.to(DEV).to(dtype)


def _with_tile(feats, pw, bias, data, n_out, tile):
    """The layer through tsc_conv_forward_tile: the 256-row 32x32-tile kernel
    with ``tile`` output columns per workgroup."""
    nbr, order, ordered = data.conv_operands(n_out, feats.device, pw.c_in * feats.element_size())
    out = torch.empty((n_out, pw.c_out), dtype=feats.dtype, device=feats.device)
    L.check(L.lib().tsc_conv_forward_tile(
        feats.data_ptr(), L.dtype_code(feats.dtype), feats.shape[0], pw.c_in, pw.data.data_ptr(),
        L.ptr(bias), L.dtype_code(bias.dtype) if bias is not None else 0, L.ptr(nbr),
        L.ptr(order), int(ordered), n_out, pw.k_vol, pw.c_out, tile, out.data_ptr(),
        L.stream_of(feats)), "conv tile")
    return out


def _tiny(seed, shape, B, n):
    rng = np.random.default_rng(seed)
    total = shape[0] * shape[1] * shape[2]
    parts = []
    for b in range(B):
        cells = rng.choice(total, size=min(n, total), replace=False)
        z, r = np.divmod(cells, shape[1] * shape[2])
        y, x = np.divmod(r, shape[2])
        parts.append(np.stack([np.full(len(cells), b), z, y, x], 1))
    idx = np.concatenate(parts).astype(np.int32)
    return idx[rng.permutation(len(idx))]


def _check_layer(m, feats, idx, shape, B, dtype, rows=None, what=""):
    """Run one subm/strided module on the GPU and compare with the oracle."""
    say("conv layer:", what, m.__class__.__name__, m.in_channels, "->", m.out_channels, dtype,
        feats.shape)
    x = spconv.SparseConvTensor(torch.from_numpy(feats).to(DEV).to(dtype),
                                torch.from_numpy(idx).to(DEV), list(shape), B)
    y = m(x)
    f64 = rounded(feats, dtype)
    w = OC.normalize_weight(to_np(m.weight).astype(np.float64), m.kernel_size, m.in_channels,
                            m.out_channels)
    b = to_np(m.bias).astype(np.float64) if m.bias is not None else None
    if m.subm:
        pr = OP.subm_pairs(idx, shape, B, m.kernel_size, m.dilation)
    else:
        pr = OP.strided_pairs(idx, shape, B, m.kernel_size, m.stride, m.padding, m.dilation)
    assert np.array_equal(y.indices.cpu().numpy(), pr.out_indices)
    n_out = len(pr.out_indices)
    if rows is None or rows >= n_out:
        sel = np.arange(n_out)
    else:
        sel = np.sort(np.random.default_rng(1).choice(n_out, size=rows, replace=False))
    ref = oracle_rows(f64, w, b, pr.pairs_in, pr.pairs_out, sel)
    out = to_np(y.features)[sel]
    err = rel_err(out, ref)
    say("   rel err", err)
    assert y.features.dtype == dtype and y.features.shape == (n_out, m.out_channels)
    assert np.isfinite(out).all()
    assert err <= TOL[dtype], f"{what}: rel err {err}"
    return y


# (c_in, c_out, dtype): VALU shapes (narrow / ragged / fp32) and every MFMA tile
LAYER_CASES = [
    (16, 16, torch.float32), (4, 6, torch.float32), (5, 7, torch.float32),
    (16, 32, torch.float16), (4, 16, torch.bfloat16), (3, 8, torch.float16),
    (32, 32, torch.float16), (32, 64, torch.bfloat16), (64, 32, torch.bfloat16),
    (64, 64, torch.float16), (96, 96, torch.float16), (128, 128, torch.float16),
    (128, 128, torch.bfloat16), (256, 128, torch.float16), (64, 256, torch.bfloat16),
    (160, 192, torch.float16), (64, 64, torch.float32),
    # fp32 on the matrix cores (v_mfma_f32_32x32x2_f32): every column tile width
    (32, 32, torch.float32), (128, 128, torch.float32), (64, 96, torch.float32),
    (96, 64, torch.float32),
    # C_in an odd multiple of 16: the last 32-channel chunk is half padding
    (16, 64, torch.float32), (48, 32, torch.bfloat16), (80, 96, torch.float16),
    (16, 128, torch.bfloat16),
    # the narrow kernel (C_in % 4 == 0, C_out % 16 == 0): 8-byte pieces
    # (f16/bf16 with C_in % 8 == 4, a piece never straddles two slots), 16-byte
    # pieces, 16-column tiles that do not pair up, many reduction steps, and
    # f32 on v_mfma_f32_16x16x4_f32
    (4, 16, torch.float16), (12, 48, torch.float16), (4, 32, torch.bfloat16),
    (8, 16, torch.bfloat16), (16, 48, torch.float16), (40, 80, torch.float16),
    (64, 16, torch.bfloat16), (4, 16, torch.float32), (12, 48, torch.float32),
    (64, 16, torch.float32),
]


@pytest.mark.parametrize("c_in,c_out,dtype", LAYER_CASES)
def test_subm_layer(c_in, c_out, dtype):
    idx = _tiny(5, (20, 22, 24), 2, 2500)
    feats = np.random.default_rng(6).standard_normal((len(idx), c_in)).astype(np.float32)
    m = _module("subm", c_in, c_out, 3, dtype=dtype, seed=c_in + c_out)
    _check_layer(m, feats, idx, (20, 22, 24), 2, dtype, what=f"subm {c_in}->{c_out}")


@pytest.mark.parametrize("c_in,c_out,dtype", [(16, 32, torch.float32), (32, 64, torch.bfloat16),
                                              (64, 128, torch.float16), (5, 3, torch.float16),
                                              (64, 64, torch.float32), (4, 16, torch.float16),
                                              (8, 48, torch.bfloat16)])
@pytest.mark.parametrize("k,s,p", [(3, 2, 1), (2, 2, 0), ((3, 1, 1), (2, 1, 1), 0)])
def test_strided_layer(c_in, c_out, dtype, k, s, p):
    idx = _tiny(7, (21, 18, 25), 2, 3000)
    feats = np.random.default_rng(8).standard_normal((len(idx), c_in)).astype(np.float32)
    m = _module("strided", c_in, c_out, k, s, p, dtype=dtype, seed=3)
    _check_layer(m, feats, idx, (21, 18, 25), 2, dtype, what=f"strided {c_in}->{c_out} k{k}")


@pytest.mark.parametrize("c_in,c_out,dtype", [(4, 64, torch.float16), (8, 32, torch.bfloat16),
                                              (12, 64, torch.bfloat16), (4, 64, torch.float32)])
def test_narrow_layers_with_several_column_tiles_per_wave(c_in, c_out, dtype):
    """Layers of 150 000 rows: enough workgroups for the narrow kernel to give
    each wave two or four 16-column tiles.  Checked on 3000 random rows."""
    shape = (64, 64, 64)
    idx = _tiny(23, shape, 1, 150_000)
    feats = np.random.default_rng(24).standard_normal((len(idx), c_in)).astype(np.float32)
    m = _module("subm", c_in, c_out, 3, dtype=dtype, seed=c_in * c_out)
    _check_layer(m, feats, idx, shape, 1, dtype, rows=3000, what=f"narrow {c_in}->{c_out}")


@pytest.mark.parametrize("c_in,c_out,dtype", [(16, 32, torch.float16), (4, 16, torch.bfloat16),
                                              (8, 16, torch.float32)])
def test_layers_of_more_than_64_slots(c_in, c_out, dtype):
    """5x5x5 (125 slots): past the 32x32 tile's slot table, so the narrow
    kernel takes these shapes; its reduction runs over 63, 16 and 63 steps."""
    idx = _tiny(25, (18, 20, 22), 2, 2500)
    feats = np.random.default_rng(26).standard_normal((len(idx), c_in)).astype(np.float32)
    m = _module("subm", c_in, c_out, 5, dtype=dtype, seed=11)
    _check_layer(m, feats, idx, (18, 20, 22), 2, dtype, what=f"subm 5x5x5 {c_in}->{c_out}")


@pytest.mark.parametrize("c_mid,c_out,dtype", [(64, 32, torch.bfloat16), (16, 8, torch.float32),
                                               (128, 64, torch.float16)])
def test_inverse_layer(c_mid, c_out, dtype):
    shape = (16, 20, 18)
    idx = _tiny(9, shape, 2, 2000)
    down = _module("strided", c_out, c_mid, 3, 2, 1, key="k", dtype=dtype, seed=1)
    up = _module("inverse", c_mid, c_out, 3, key="k", dtype=dtype, seed=2)
    x = spconv.SparseConvTensor(torch.zeros(len(idx), c_out, device=DEV, dtype=dtype),
                                torch.from_numpy(idx).to(DEV), list(shape), 2)
    y = down(x)
    mid = np.random.default_rng(10).standard_normal((len(y.indices), c_mid)).astype(np.float32)
    z = up(y.replace_feature(torch.from_numpy(mid).to(DEV).to(dtype)))
    fwd = OP.strided_pairs(idx, shape, 2, 3, 2, 1)
    inv = OP.inverse_pairs(fwd)
    assert np.array_equal(z.indices.cpu().numpy(), inv.out_indices)
    assert z.spatial_shape == list(shape)
    w = OC.normalize_weight(to_np(up.weight).astype(np.float64), (3, 3, 3), c_mid, c_out)
    ref = OC.conv_forward(rounded(mid, dtype), w, to_np(up.bias).astype(np.float64),
                          inv.pairs_in, inv.pairs_out, len(inv.out_indices))
    err = rel_err(to_np(z.features), ref)
    say("inverse rel err", err)
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_one_by_one_layers(dtype):
    """SubM 1x1x1 (fold quirk) and the inverse 1x1x1 shortcut (dense product)."""
    idx = _tiny(11, (12, 12, 12), 2, 700)
    feats = np.random.default_rng(12).standard_normal((len(idx), 32)).astype(np.float32)
    m = _module("subm", 32, 64, 1, dtype=dtype, seed=4)
    y = _check_layer(m, feats, idx, (12, 12, 12), 2, dtype, what="subm 1x1x1")
    fold = to_np(m.weight).astype(np.float64).reshape(-1).reshape(32, 64)
    ref = rounded(feats, dtype) @ fold + to_np(m.bias).astype(np.float64)
    assert rel_err(to_np(y.features), ref) <= TOL[dtype]
    # inverse 1x1x1: coordinates and shape of the inverse input
    down = _module("strided", 32, 64, 1, 2, 0, key="d", dtype=dtype, seed=5)
    up = _module("inverse", 64, 16, 1, key="d", dtype=dtype, seed=6)
    x = spconv.SparseConvTensor(torch.from_numpy(feats).to(DEV).to(dtype),
                                torch.from_numpy(idx).to(DEV), [12, 12, 12], 2)
    yd = down(x)
    z = up(yd)
    assert z.indices is yd.indices and z.spatial_shape == yd.spatial_shape
    w0 = to_np(up.weight).astype(np.float64).reshape(-1).reshape(64, 16)
    ref = to_np(yd.features).astype(np.float64) @ w0 + to_np(up.bias).astype(np.float64)
    assert rel_err(to_np(z.features), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("c_in,c_out", [(32, 96), (64, 192), (32, 256), (96, 64), (64, 64)])
@pytest.mark.parametrize("n", [1500, 6000])
def test_every_bias_dtype_and_column_tile(c_in, c_out, dtype, n, monkeypatch):
    """A bias of any dtype on every MFMA tile shape, with several column tiles
    per row tile, with (n=6000) and without (n=1500) an execution order (the
    size threshold of the order is lowered so that small layers get one)."""
    monkeypatch.setattr(I, "_PLAN_MIN_BYTES", 0)
    shape = (24, 24, 24)
    idx = _tiny(15, shape, 1, n)
    x = torch.from_numpy(idx).to(DEV)
    data = generate_subm_indice_pairs(x, shape, 1, 3)
    rng = np.random.default_rng(16)
    feats = rng.standard_normal((len(idx), c_in)).astype(np.float32)
    W = (rng.standard_normal((27, c_in, c_out)) / np.sqrt(27 * c_in)).astype(np.float32)
    bias = rng.uniform(-1, 1, c_out).astype(np.float32)
    f = torch.from_numpy(feats).to(DEV).to(dtype)
    pw = Fn.pack_weight(torch.from_numpy(W).to(DEV), (3, 3, 3), c_in, c_out, dtype)
    pr = OP.subm_pairs(idx, shape, 1, 3, 1)
    w64 = rounded(W, dtype)
    for bdt in (None, torch.float32, torch.float16, torch.bfloat16):
        b = None if bdt is None else torch.from_numpy(bias).to(DEV).to(bdt)
        say("bias dtype", bdt, "features", dtype, c_in, "->", c_out, "rows", len(idx))
        out = Fn.sparse_conv_forward(f, pw, b, data, len(idx))
        ref = OC.conv_forward(rounded(feats, dtype), w64,
                              None if b is None else to_np(b).astype(np.float64),
                              pr.pairs_in, pr.pairs_out, len(idx))
        got = to_np(out)
        assert np.isfinite(got).all()
        assert rel_err(got, ref) <= TOL[dtype], f"bias {bdt}: rel err {rel_err(got, ref)}"


@pytest.mark.parametrize("c_in,c_out,dtype", [(16, 16, torch.float32), (128, 128, torch.float16),
                                              (64, 32, torch.bfloat16), (4, 16, torch.float16),
                                              (8, 48, torch.bfloat16)])
def test_deterministic_and_order_independent(c_in, c_out, dtype, monkeypatch):
    monkeypatch.setattr(I, "_PLAN_MIN_BYTES", 0)  # an execution order even for this small layer
    idx = _tiny(13, (30, 30, 30), 1, 9000)
    x = torch.from_numpy(idx).to(DEV)
    feats = torch.randn(len(idx), c_in, generator=torch.Generator().manual_seed(0)).to(DEV).to(dtype)
    data = generate_subm_indice_pairs(x, (30, 30, 30), 1, 3)
    m = _module("subm", c_in, c_out, 3, dtype=dtype, seed=7)
    pw = m._packed_weight(dtype)
    a = Fn.sparse_conv_forward(feats, pw, m.bias, data, len(idx))
    b = Fn.sparse_conv_forward(feats, pw, m.bias, data, len(idx))
    assert data._order is not None
    c = Fn._run(feats, pw, m.bias, data.neighbour_map(len(idx), feats.device), None, len(idx))
    rev = torch.flip(data._order, [0]).contiguous()
    d = Fn._run(feats, pw, m.bias, data.neighbour_map(len(idx), feats.device), rev, len(idx))
    assert torch.equal(a, b) and torch.equal(a, c) and torch.equal(a, d)


@pytest.mark.parametrize("c_in,c_out,dtype", [(16, 16, torch.float32), (20, 16, torch.float32),
                                              (32, 16, torch.float16), (32, 48, torch.bfloat16)])
def test_narrow_kernel_on_a_sparse_grid(c_in, c_out, dtype, monkeypatch):
    """The narrow kernel on a sparse grid (4000 voxels in 48^3: about two
    pairs per row, most of a wave's slots empty), with steps of one slot (16
    f32, 32 f16 channels) and steps across two slots (20 f32 channels): the
    oracle's values, and the same bits in map order, in a planned order and
    in the reverse of it."""
    monkeypatch.setattr(I, "_PLAN_MIN_BYTES", 0)
    shape = (48, 48, 48)
    idx = _tiny(41, shape, 1, 4000)
    feats_np = np.random.default_rng(42).standard_normal((len(idx), c_in)).astype(np.float32)
    m = _module("subm", c_in, c_out, 3, dtype=dtype, seed=c_in + c_out)
    _check_layer(m, feats_np, idx, shape, 1, dtype, what=f"sparse narrow {c_in}->{c_out}")
    x = torch.from_numpy(idx).to(DEV)
    feats = torch.from_numpy(feats_np).to(DEV).to(dtype)
    data = generate_subm_indice_pairs(x, shape, 1, 3)
    pw = m._packed_weight(dtype)
    a = Fn.sparse_conv_forward(feats, pw, m.bias, data, len(idx))
    b = Fn.sparse_conv_forward(feats, pw, m.bias, data, len(idx))  # planned on the second use
    assert data._order is not None
    nbr = data.neighbour_map(len(idx), feats.device)
    c = Fn._run(feats, pw, m.bias, nbr, None, len(idx))
    rev = torch.flip(data._order, [0]).contiguous()
    d = Fn._run(feats, pw, m.bias, nbr, rev, len(idx))
    assert torch.equal(a, b) and torch.equal(a, c) and torch.equal(a, d)


@pytest.mark.parametrize("kind,k,s,p", [("subm", (5, 5, 5), 1, 0), ("subm", (1, 3, 3), 1, 0),
                                        ("strided", (2, 2, 2), 2, 0), ("strided", 3, 2, 1)])
def test_plan_permutes_every_slot_count(kind, k, s, p, monkeypatch):
    """The plan's permuted map is the map read through the order, entry for
    entry, for maps of up to 32 slots (gathered from a row-major copy) and of
    more (125 slots: gathered slot by slot), on a submanifold build's columns
    and a strided build's rows; the planned convolution equals the unplanned
    one bit for bit."""
    monkeypatch.setattr(I, "_PLAN_MIN_BYTES", 0)  # an order even for these small layers
    idx = _tiny(41, (28, 28, 28), 2, 3000)
    x = torch.from_numpy(idx).to(DEV)
    if kind == "subm":
        data = generate_subm_indice_pairs(x, (28, 28, 28), 2, k)
    else:
        data = generate_strided_indice_pairs(x, (28, 28, 28), 2, k, s, p)
    n_out = len(data.out_indices)
    feats = torch.randn(len(idx), 16, generator=torch.Generator().manual_seed(6)).to(DEV)
    m = _module(kind, 16, 32, k, s, p, dtype=torch.float32, seed=15)
    pw = m._packed_weight(torch.float32)
    plain = Fn._run(feats, pw, m.bias, data.neighbour_map(n_out, DEV), None, n_out)
    order = data.execution_order(n_out, DEV, 64, eager=True)
    assert order is not None
    o = order.long().cpu()
    assert torch.equal(torch.sort(o).values, torch.arange(n_out))
    nbr = data.neighbour_map(n_out, DEV).cpu()
    perm = data.ordered_map().cpu()
    say("plan permute", kind, k, nbr.shape)
    assert torch.equal(perm, nbr[:, o])
    planned = Fn.sparse_conv_forward(feats, pw, m.bias, data, n_out)
    assert torch.equal(planned, plain)


@pytest.mark.parametrize("c_in,c_out,dtype", [(64, 64, torch.float16), (32, 32, torch.bfloat16),
                                              (64, 96, torch.float32)])
def test_slot_split_kernel_matches_the_256_row_kernel(c_in, c_out, dtype):
    """A layer small enough for the slot-split kernel (64-row tiles, slots
    split by residue mod 4 over the waves) against the same layer forced onto
    the 256-row kernel: both within tolerance of the oracle and of each
    other (their fp32 sums differ only in association)."""
    idx = _tiny(27, (24, 24, 24), 1, 4000)
    x = torch.from_numpy(idx).to(DEV)
    feats = torch.randn(len(idx), c_in, generator=torch.Generator().manual_seed(3)).to(DEV).to(dtype)
    data = generate_subm_indice_pairs(x, (24, 24, 24), 1, 3)
    m = _module("subm", c_in, c_out, 3, dtype=dtype, seed=12)
    pw = m._packed_weight(dtype)
    split = Fn.sparse_conv_forward(feats, pw, m.bias, data, len(idx))
    assert L.lib().tsc_conv_kernel_name(L.dtype_code(dtype), c_in, c_out, 27,
                                        len(idx)) == b"conv_split_kernel"
    whole = _with_tile(feats, pw, m.bias, data, len(idx), 32)
    pr = OP.subm_pairs(idx, (24, 24, 24), 1, 3, 1)
    w = OC.normalize_weight(to_np(m.weight).astype(np.float64), (3, 3, 3), c_in, c_out)
    ref = OC.conv_forward(to_np(feats).astype(np.float64), w,
                          to_np(m.bias).astype(np.float64), pr.pairs_in, pr.pairs_out, len(idx))
    say("split vs 256-row", c_in, c_out, dtype)
    assert rel_err(to_np(split), ref) <= TOL[dtype]
    assert rel_err(to_np(whole), ref) <= TOL[dtype]
    assert rel_err(to_np(split), to_np(whole).astype(np.float64)) <= TOL[dtype]


@pytest.mark.parametrize("c_in,c_out,dtype", [(64, 128, torch.float16), (32, 128, torch.bfloat16),
                                              (64, 128, torch.float32), (48, 64, torch.float16),
                                              (128, 128, torch.bfloat16)])
def test_every_column_tile_width_gives_the_same_bits(c_in, c_out, dtype):
    """The column tile width (32/64/128) only changes the schedule: each output
    is summed in the same slot and chunk order, so every width returns the same
    bits, equal to the oracle within tolerance.  The forced widths run the
    register-gather kernel; the layer's own choice is its direct-to-LDS variant
    when a stage is 128 bytes of each row (f16/bf16 with C_in % 64 == 0, f32
    with C_in % 32 == 0), which must give those bits too."""
    idx = _tiny(21, (40, 40, 40), 1, 12000)
    x = torch.from_numpy(idx).to(DEV)
    feats = torch.randn(len(idx), c_in, generator=torch.Generator().manual_seed(2)).to(DEV).to(dtype)
    data = generate_subm_indice_pairs(x, (40, 40, 40), 1, 3)
    m = _module("subm", c_in, c_out, 3, dtype=dtype, seed=9)
    pw = m._packed_weight(dtype)
    outs = {}
    for tile in [32, 64] + ([128] if c_out % 128 == 0 else []):
        outs[tile] = _with_tile(feats, pw, m.bias, data, len(idx), tile)
    name = L.lib().tsc_conv_kernel_name(L.dtype_code(dtype), c_in, c_out, 27, len(idx))
    if name != b"conv_split_kernel":  # the slot-split kernel sums in another order
        stage_bytes_fit = c_in % (32 if dtype == torch.float32 else 64) == 0
        assert name == (b"conv_dma_kernel" if stage_bytes_fit else b"conv_mfma_kernel")
        # the layer's own choice is one of these widths
        outs[0] = Fn.sparse_conv_forward(feats, pw, m.bias, data, len(idx))
    assert (0 in outs) == ((c_in, c_out) != (48, 64))
    first = outs[32]
    for tile, o in outs.items():
        say("tile", tile, c_in, c_out, dtype)
        assert torch.equal(o, first), tile
    pr = OP.subm_pairs(idx, (40, 40, 40), 1, 3, 1)
    w = OC.normalize_weight(to_np(m.weight).astype(np.float64), (3, 3, 3), c_in, c_out)
    ref = OC.conv_forward(to_np(feats).astype(np.float64), w,
                          to_np(m.bias).astype(np.float64), pr.pairs_in, pr.pairs_out, len(idx))
    assert rel_err(to_np(first), ref) <= TOL[dtype]
    with pytest.raises(ValueError):
        _with_tile(feats, pw, m.bias, data, len(idx), 48)  # not a column tile width


def _conv_raw(feats, pw, bias, nbr, order, ordered, n_out, tile):
    """One layer through the C-ABI with explicit map operands: tsc_conv_forward
    (tile 0: the layer's own kernel choice) or tsc_conv_forward_tile."""
    out = torch.empty((n_out, pw.c_out), dtype=feats.dtype, device=feats.device)
    lib = L.lib()
    args = (feats.data_ptr(), L.dtype_code(feats.dtype), feats.shape[0], pw.c_in, pw.data.data_ptr(),
            L.ptr(bias), L.dtype_code(bias.dtype), L.ptr(nbr), L.ptr(order), int(ordered), n_out,
            pw.k_vol, pw.c_out)
    if tile:
        L.check(lib.tsc_conv_forward_tile(*args, tile, out.data_ptr(), L.stream_of(feats)), "tile")
    else:
        L.check(lib.tsc_conv_forward(*args, out.data_ptr(), L.stream_of(feats)), "conv")
    return out


@pytest.mark.parametrize("rows,grid", [(50000, 64), (150000, 96), (300000, 128)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_dma_kernel_matches_the_register_gather_kernel(dtype, rows, grid, monkeypatch):
    """A 128-column layer: the direct-to-LDS kernel (the layer's own choice)
    against the register-gather kernel forced to the same width, bit for bit,
    with the map permuted into the execution order (with and without the
    plan's row of slot masks, which only the direct-to-LDS kernel reads), with
    the row-major map plus the order, and with the row-major map alone.  150k rows (586 tiles
    of 256 rows) take its 32-rows-per-wave form, 300k rows (1172 tiles) its
    64-rows-per-wave form; 50k rows (196 tiles) narrow the column tile to
    32."""
    monkeypatch.setattr(I, "_PLAN_MIN_BYTES", 0)  # an execution order at every size
    idx = _tiny(31, (grid, grid, grid), 1, rows)
    x = torch.from_numpy(idx).to(DEV)
    feats = torch.randn(len(idx), 128, generator=torch.Generator().manual_seed(5)).to(DEV).to(dtype)
    data = generate_subm_indice_pairs(x, (grid, grid, grid), 1, 3)
    m = _module("subm", 128, 128, 3, dtype=dtype, seed=21)
    pw = m._packed_weight(dtype)
    n = len(idx)
    assert L.lib().tsc_conv_kernel_name(L.dtype_code(dtype), 128, 128, 27, n) == b"conv_dma_kernel"
    order = data.execution_order(n, DEV, 128 * feats.element_size(), eager=True)
    assert order is not None
    permuted, order2, ordered = data.conv_operands(n, DEV, 128 * feats.element_size())
    assert ordered == 2 and order2 is order
    # the plan's row K after the permuted map: each position's slot mask
    mask_row = permuted.as_strided((n,), (1,), permuted.storage_offset() + 27 * n)
    bits = ((permuted >= 0).to(torch.int64)
            << torch.arange(27, device=DEV, dtype=torch.int64).view(27, 1)).sum(0)
    assert torch.equal(mask_row.to(torch.int64), bits)
    rowmajor = data.neighbour_map(n, DEV)
    for label, ops in (("permuted map + slot masks", (permuted, order, 2)),
                       ("permuted map", (permuted, order, 1)),
                       ("row-major map + order", (rowmajor, order, 0)),
                       ("row-major map", (rowmajor, None, 0))):
        say("dma vs register gather", dtype, label)
        dma = _conv_raw(feats, pw, m.bias, *ops, n, 0)
        reg = _conv_raw(feats, pw, m.bias, *ops, n, 128)
        assert torch.equal(dma, reg), label
        assert torch.isfinite(dma.float()).all()


@pytest.mark.parametrize("dtype,c", [(torch.float16, 64), (torch.bfloat16, 64), (torch.float32, 32)])
def test_dma_kernel_short_stage_lists_and_epilogue(dtype, c):
    """conv_dma_kernel at 64 rows per wave (layers of at least 1024 tiles of
    256 rows) on a sparse grid where most tiles use one to three slots, with
    one channel chunk (a stage per slot): tiles of one or two stages, shorter
    than its prefetch, and a partial last tile.  Bit for bit against the
    register-gather kernel (forced column tile) and, with a fused batch norm
    and ReLU, against the fp64 oracle on a sample of rows."""
    n_rows = 1055 * 256 - 77
    idx = _tiny(57, (256, 256, 256), 1, n_rows)
    x = torch.from_numpy(idx).to(DEV)
    n = len(idx)
    feats = torch.randn(n, c, generator=torch.Generator().manual_seed(8)).to(DEV).to(dtype)
    data = generate_subm_indice_pairs(x, (256, 256, 256), 1, 3)
    m = _module("subm", c, 64, 3, dtype=dtype, seed=13)
    pw = m._packed_weight(dtype)
    assert L.lib().tsc_conv_kernel_name(L.dtype_code(dtype), c, 64, 27, n) == b"conv_dma_kernel"
    pn = data.pair_num
    say("dma kernel short lists", dtype, n, "pairs per row", float(pn.sum()) / n)
    assert float(pn.sum()) / n < 2.0  # mostly one or two slots per row
    own = Fn.sparse_conv_forward(feats, pw, m.bias, data, n)
    reg = _with_tile(feats, pw, m.bias, data, n, 64)
    assert torch.equal(own, reg)
    g = torch.Generator().manual_seed(3)
    mean, var = torch.rand(64, generator=g) * 0.2 - 0.1, torch.rand(64, generator=g) + 0.5
    gamma, beta = torch.rand(64, generator=g) + 0.5, torch.rand(64, generator=g) * 0.4 - 0.2
    ep = Fn.Epilogue(mean.to(DEV), var.to(DEV), gamma.to(DEV), beta.to(DEV), 1e-5, True)
    fused = Fn.sparse_conv_forward(feats, pw, m.bias, data, n, epilogue=ep)
    rows = np.random.default_rng(1).choice(n, size=4000, replace=False)
    w = OC.normalize_weight(to_np(m.weight).astype(np.float64), (3, 3, 3), c, 64)
    ref = oracle_rows(to_np(feats).astype(np.float64), w, to_np(m.bias).astype(np.float64),
                      lists_np(data.pairs_in), lists_np(data.pairs_out), rows)
    ref = np.maximum((ref - mean.double().numpy()) / np.sqrt(var.double().numpy() + 1e-5)
                     * gamma.double().numpy() + beta.double().numpy(), 0.0)
    err = rel_err(to_np(fused)[rows], ref)
    say("  fused rel err", err)
    assert err <= TOL[dtype]


def test_raw_internal_weight_and_user_built_indice_data():
    """sparse_conv_forward with a (K, C_in, C_out) tensor and hand-made pair lists."""
    idx = _tiny(14, (10, 10, 10), 1, 300)
    x = torch.from_numpy(idx).to(DEV)
    data = generate_subm_indice_pairs(x, (10, 10, 10), 1, 3)
    feats = torch.randn(len(idx), 8, device=DEV)
    W = torch.randn(27, 8, 12, device=DEV)
    out = Fn.sparse_conv_forward(feats, W, None, data, len(idx))
    from trispconv.pytorch.indices import IndiceData
    hand = IndiceData(data.out_indices, [p.clone() for p in data.pairs_in],
                      [p.clone() for p in data.pairs_out], data.pair_num, data.input_indices,
                      (10, 10, 10), (10, 10, 10), (3, 3, 3), (1, 1, 1), (0, 0, 0), (1, 1, 1), True)
    out2 = Fn.sparse_conv_forward(feats, W, None, hand, len(idx))
    assert torch.equal(out, out2)
    ref = OC.conv_forward(feats.cpu().numpy(), W.cpu().numpy(), None, lists_np(data.pairs_in),
                          lists_np(data.pairs_out), len(idx))
    assert rel_err(out.cpu().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("name", workloads.WORKLOAD_NAMES)
def test_full_size_workloads(name):
    """Each workload at full size, layer by layer on the GPU's own layer inputs,
    every output row against the oracle."""
    w = workloads.make_workload(name)
    dtype = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[w.dtype]
    rng = np.random.default_rng(w.seed)
    idx, shape = w.indices, tuple(w.spatial_shape)
    feats = workloads.features(rng, len(idx), w.layers[0]["c_in"])
    fwd_store = {}
    for li, lay in enumerate(w.layers):
        m = _module(lay["kind"], lay["c_in"], lay["c_out"], lay["kernel_size"], lay["stride"],
                    lay["padding"], lay["dilation"], key=lay["indice_key"], dtype=dtype, seed=li)
        if lay["kind"] == "inverse":
            x_idx, x_shape, prev = fwd_store[lay["indice_key"]]
            xin = spconv.SparseConvTensor(torch.from_numpy(feats).to(DEV).to(dtype),
                                          torch.from_numpy(idx).to(DEV), list(shape), w.batch_size)
            xin.indice_dict[lay["indice_key"]] = prev
            y = m(xin)
            exp_fwd = OP.strided_pairs(x_idx, x_shape, w.batch_size, prev.kernel_size, prev.stride,
                                       prev.padding, prev.dilation)
            inv = OP.inverse_pairs(exp_fwd)
            assert np.array_equal(y.indices.cpu().numpy(), inv.out_indices)
            wt = OC.normalize_weight(to_np(m.weight).astype(np.float64), m.kernel_size,
                                     m.in_channels, m.out_channels)
            ref = OC.conv_forward(rounded(feats, dtype), wt, to_np(m.bias).astype(np.float64),
                                  inv.pairs_in, inv.pairs_out, len(inv.out_indices))
            err = rel_err(to_np(y.features), ref)
            say(name, "inverse rel err", err)
            assert err <= TOL[dtype]
        else:
            y = _check_layer(m, feats, idx, shape, w.batch_size, dtype,
                             what=f"{name} layer {li}")
            if lay["kind"] == "strided" and lay["indice_key"]:
                key = lay["indice_key"]
                fwd_store[key] = (idx, shape, y.indice_dict[key] if key in y.indice_dict else
                                  generate_strided_indice_pairs(
                                      torch.from_numpy(idx).to(DEV), shape, w.batch_size,
                                      lay["kernel_size"], lay["stride"], lay["padding"],
                                      lay["dilation"]))
        # the next layer consumes this layer's output (ReLU keeps magnitudes sane)
        out = torch.relu(y.features.float())
        feats = out.cpu().numpy().astype(np.float32)
        idx = y.indices.cpu().numpy()
        shape = tuple(y.spatial_shape)
        torch.cuda.synchronize()


@pytest.mark.parametrize("row_bytes,per_sample", [(256, 6000), (2048, 6000), (1 << 17, 6000),
                                                  (1 << 17, 12000)])
def test_plan_tiles_mask_sorted_heaviest_first(row_bytes, per_sample, monkeypatch):
    """The execution order is a permutation of the output rows.  Cut into
    256-row tiles (the convolution's workgroup tiles), each full tile is sorted
    by slot mask, and inside each region the full tiles come in non-increasing
    number of slots used by their rows, tiles of equal count in their mask
    order (a stable sort); the partial tile, if any, is last and mask-sorted
    too.  row_bytes = 2^17 makes regions of 2048 rows: six of them sort the
    tiles in one workgroup (keys of 9 bits), twelve in radix passes."""
    monkeypatch.setattr(I, "_PLAN_MIN_BYTES", 0)  # an order even for this small layer
    idx = _tiny(15, (40, 40, 40), 2, per_sample)
    x = torch.from_numpy(idx).to(DEV)
    data = generate_subm_indice_pairs(x, (40, 40, 40), 2, 3)
    n = len(idx)
    order = data.execution_order(n, x.device, row_bytes, eager=True).cpu().numpy().astype(np.int64)
    region = data._order_region
    assert region % 256 == 0
    assert np.array_equal(np.sort(order), np.arange(n))
    nbr = data.neighbour_map(n, x.device).cpu().numpy()
    mask = ((nbr.T >= 0).astype(np.int64) << np.arange(27)).sum(1)[order]
    for t0 in range(0, n, 256):
        m = mask[t0:t0 + 256]
        assert (np.diff(m) >= 0).all(), f"tile at {t0} not sorted by mask"
    n_full = n // 256
    used = np.array([bin(int(np.bitwise_or.reduce(mask[t * 256:(t + 1) * 256]))).count("1")
                     for t in range(n_full)])
    per_region = region // 256
    for r0 in range(0, n_full, per_region):
        u = used[r0:r0 + per_region]
        assert (np.diff(u) <= 0).all(), f"tiles of the region at row {r0 * 256} not heaviest first"
        for t in range(r0 + 1, min(r0 + per_region, n_full)):
            if used[t] == used[t - 1]:
                assert mask[t * 256] >= mask[t * 256 - 1], f"tiles {t - 1}, {t}: not stable"
    # the same tiles as a plain mask sort inside regions: each region's multiset of rows holds
    for r0 in range(0, n_full * 256, region):
        hi = min(r0 + region, n_full * 256)
        assert hi - r0 == len(np.unique(order[r0:hi]))


@pytest.mark.parametrize("c_in,dtype,first", [(128, torch.float16, True), (64, torch.float32, True),
                                               (32, torch.float16, False)])
def test_plan_on_first_use_only_for_wide_spatially_ordered_maps(c_in, dtype, first, monkeypatch):
    """A bitmap build's map (columns in (b,z,y,x) order) is planned at its
    first convolution when the gathered rows are at least 256 bytes wide;
    narrower rows run the first convolution unplanned and plan at the second.
    Either way the outputs are the same bits."""
    monkeypatch.setattr(I, "_PLAN_MIN_BYTES", 0)  # an order even for this small layer
    idx = _tiny(16, (40, 40, 40), 1, 6000)
    x = torch.from_numpy(idx).to(DEV)
    feats = torch.randn(len(idx), c_in, generator=torch.Generator().manual_seed(4)).to(DEV).to(dtype)
    data = generate_subm_indice_pairs(x, (40, 40, 40), 1, 3)
    assert data._raster
    m = _module("subm", c_in, 32, 3, dtype=dtype, seed=6)
    pw = m._packed_weight(dtype)
    n = len(idx)
    one = Fn.sparse_conv_forward(feats, pw, m.bias, data, n)
    assert (data.ordered_map() is not None) == first
    two = Fn.sparse_conv_forward(feats, pw, m.bias, data, n)
    assert data.ordered_map() is not None
    assert torch.equal(one, two)


def test_unkeyed_subm_layers_share_one_build(monkeypatch):
    """Submanifold layers without an indice_key reuse the pairs of their
    coordinate tensor while it is unchanged; an in-place change rebuilds."""
    from trispconv_amd.pytorch import modules as M
    calls = []
    real = M.generate_subm_indice_pairs

    def counting(*args, **kw):
        calls.append(args[3:])
        return real(*args, **kw)

    monkeypatch.setattr(M, "generate_subm_indice_pairs", counting)
    idx = torch.from_numpy(_tiny(31, (20, 20, 20), 1, 2500)).to(DEV)
    x = spconv.SparseConvTensor(torch.randn(len(idx), 16, device=DEV), idx, [20, 20, 20], 1)
    a = _module("subm", 16, 16, 3, seed=1)
    b = _module("subm", 16, 32, 3, seed=2)
    c = _module("subm", 32, 32, 3, d=2, seed=3)
    y = c(b(a(x)))
    assert len(calls) == 2  # 3x3x3 dilation 1 once, dilation 2 once
    y2 = c(b(a(x)))
    assert len(calls) == 2 and torch.equal(y.features, y2.features)
    idx.add_(0)  # an in-place op: the coordinate tensor may have changed
    y3 = c(b(a(x)))
    assert len(calls) == 4 and torch.equal(y.features, y3.features)
    x._pair_cache.clear()
    fresh = c(b(a(x)))
    assert len(calls) == 6
    assert torch.equal(y.features, fresh.features)
