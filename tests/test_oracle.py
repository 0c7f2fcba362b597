"""Pin the CPU oracle: golden fixtures, dense closed forms and brute force.

Nothing here restates the oracle's own formulas: coordinates and features are
checked against spconv's outputs (the reference's golden fixtures), against
torch's dense conv3d / conv_transpose3d, and pair lists against the
brute-force enumeration in tests/brute.py.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import brute
import golden_io
from oracle import conv as OC
from oracle import pairs as OP

torch.backends.cuda.matmul.allow_tf32 = False


# ---------------------------------------------------------------------------
# golden fixtures (reference tests/test_vs_spconv.py:51-145)
# ---------------------------------------------------------------------------

def _oracle_on_fixture(name):
    a, m = golden_io.load(name)
    k, s, p, d = m["kernel_size"], m["stride"], m["padding"], m["dilation"]
    bias = a.get("bias")
    if m["conv_type"] in ("subm", "strided"):
        out, coords, shape, _ = OC.run_layer(m["conv_type"], a["features"], a["indices"],
                                             m["spatial_shape"], m["batch_size"], a["weight"],
                                             bias, k, s, p, d)
        return a, m, out, coords, shape
    # inverse: rebuild the paired strided layer, then re-order the fixture's
    # features (given in spconv's output order) onto the oracle's order
    _, down_coords, down_shape, fwd = OC.run_layer(
        "strided", a["down_in_features"], a["down_in_indices"], m["down_in_spatial_shape"],
        m["batch_size"], a["down_weight"], None, k, s, p, d)
    ref_order = np.argsort(golden_io.encode(a["indices"], down_shape), kind="stable")
    ours_order = np.argsort(golden_io.encode(down_coords, down_shape), kind="stable")
    feats = np.empty_like(a["features"])
    feats[ours_order] = a["features"][ref_order]
    out, coords, shape, _ = OC.run_layer("inverse", feats, down_coords, down_shape,
                                         m["batch_size"], a["weight"], bias, k, fwd=fwd)
    return a, m, out, coords, shape


@pytest.mark.parametrize("name", golden_io.fixture_names())
def test_oracle_matches_spconv_golden(name):
    a, m, out, coords, shape = _oracle_on_fixture(name)
    f_sorted, i_sorted = golden_io.sort_by_coord(out, coords, shape)
    assert i_sorted.shape == a["out_indices"].shape
    assert np.array_equal(i_sorted, a["out_indices"])
    np.testing.assert_allclose(f_sorted, a["out_features"], atol=1e-4, rtol=1e-4)


def test_golden_fold_quirk_distinguishes_conventions():
    """The 1x1x1 fixture rejects the W.T convention, so the fold quirk is pinned."""
    a, m = golden_io.load("subm_1x1x1_c16")
    w = a["weight"].reshape(m["C_out"], m["C_in"])
    wrong = a["features"].astype(np.float64) @ w.T.astype(np.float64)
    f_sorted, _ = golden_io.sort_by_coord(wrong, a["indices"], m["spatial_shape"])
    assert np.abs(f_sorted - a["out_features"]).max() > 1.0


# ---------------------------------------------------------------------------
# dense closed forms (reference tests/test_vs_dense.py:44-150)
# ---------------------------------------------------------------------------

def _random_sparse(rng, shape, batch, n, c):
    total = shape[0] * shape[1] * shape[2]
    rows = []
    for b in range(batch):
        cells = rng.choice(total, size=n, replace=False)
        z, rem = np.divmod(cells, shape[1] * shape[2])
        y, x = np.divmod(rem, shape[2])
        rows.append(np.stack([np.full(n, b), z, y, x], 1))
    idx = np.concatenate(rows).astype(np.int32)
    idx = idx[rng.permutation(len(idx))]
    feats = rng.uniform(-1, 1, size=(len(idx), c))
    return idx, feats


def _dense(idx, feats, shape, batch):
    t = torch.zeros(batch, feats.shape[1], *shape, dtype=torch.float64)
    i = torch.from_numpy(idx.astype(np.int64))
    t[i[:, 0], :, i[:, 1], i[:, 2], i[:, 3]] = torch.from_numpy(feats)
    return t


def _at(dense, coords):
    i = torch.from_numpy(np.asarray(coords).astype(np.int64))
    return dense[i[:, 0], :, i[:, 1], i[:, 2], i[:, 3]].numpy()


STRIDED = [(bs, k, s, p, d) for bs in [1, 2] for k in [2, 3] for s in [1, 2]
           for p in [0, 1] for d in [1, 2] if not (s > 1 and d > 1)]


@pytest.mark.parametrize("bs,k,s,p,d", STRIDED)
def test_oracle_strided_vs_dense(bs, k, s, p, d):
    rng = np.random.default_rng(1000 + 97 * bs + 31 * k + 7 * s + 3 * p + d)
    shape = (9, 8, 7)
    idx, feats = _random_sparse(rng, shape, bs, 60, 5)
    w = rng.uniform(-1, 1, size=(6, k, k, k, 5))
    out, coords, oshape, _ = OC.run_layer("strided", feats, idx, shape, bs, w, None, k, s, p, d)
    dense = F.conv3d(_dense(idx, feats, shape, bs), torch.from_numpy(w).permute(0, 4, 1, 2, 3),
                     stride=s, padding=p, dilation=d)
    assert tuple(dense.shape[2:]) == tuple(oshape)
    np.testing.assert_allclose(out, _at(dense, coords), atol=1e-10)
    # closed-form active set: reachable outputs, sorted by (b, z, y, x)
    occ = _dense(idx, np.ones((len(idx), 1)), shape, bs)
    reach = F.conv3d(occ, torch.ones(1, 1, k, k, k, dtype=torch.float64), stride=s,
                     padding=p, dilation=d)[:, 0] > 0
    expect = torch.nonzero(reach).numpy().astype(np.int32)
    assert np.array_equal(coords, expect)


@pytest.mark.parametrize("bs,k,d", [(bs, k, d) for bs in [1, 2] for k in [1, 3] for d in [1, 2]])
def test_oracle_subm_vs_dense(bs, k, d):
    rng = np.random.default_rng(2000 + 13 * bs + 5 * k + d)
    shape = (9, 8, 7)
    idx, feats = _random_sparse(rng, shape, bs, 80, 5)
    w = rng.uniform(-1, 1, size=(6, k, k, k, 5))
    out, coords, _, _ = OC.run_layer("subm", feats, idx, shape, bs, w, None, k, 1, 0, d)
    assert coords is idx
    if k == 1:
        ref = feats @ w.reshape(-1).reshape(5, 6)     # spconv's 1x1x1 fold
    else:
        dense = F.conv3d(_dense(idx, feats, shape, bs), torch.from_numpy(w).permute(0, 4, 1, 2, 3),
                         padding=d * (k // 2), dilation=d)
        ref = _at(dense, idx)
    np.testing.assert_allclose(out, ref, atol=1e-10)


@pytest.mark.parametrize("k,s,p", [(3, 2, 1), (2, 2, 0), (3, 1, 1), (3, 2, 0)])
def test_oracle_inverse_vs_conv_transpose(k, s, p):
    rng = np.random.default_rng(3000 + 11 * k + 3 * s + p)
    shape = (9, 8, 10)
    bs = 2
    idx, _ = _random_sparse(rng, shape, bs, 70, 3)
    w_down = rng.uniform(-1, 1, size=(4, k, k, k, 3))
    _, dcoords, dshape, fwd = OC.run_layer("strided", np.zeros((len(idx), 3)), idx, shape, bs,
                                           w_down, None, k, s, p)
    x = rng.uniform(-1, 1, size=(len(dcoords), 4))
    w_inv = rng.uniform(-1, 1, size=(5, k, k, k, 4))
    bias = rng.uniform(-0.1, 0.1, size=5)
    out, coords, oshape, _ = OC.run_layer("inverse", x, dcoords, dshape, bs, w_inv, bias, k,
                                          fwd=fwd)
    assert tuple(oshape) == shape
    # output padding that restores the input shape
    op = tuple(shape[t] - ((dshape[t] - 1) * s - 2 * p + (k - 1) + 1) for t in range(3))
    dense = F.conv_transpose3d(_dense(dcoords, x, dshape, bs),
                               torch.from_numpy(w_inv).permute(4, 0, 1, 2, 3), stride=s,
                               padding=p, output_padding=op, bias=torch.from_numpy(bias))
    np.testing.assert_allclose(out, _at(dense, coords), atol=1e-10)
    # output rows: participating inputs, ascending input-row order, all of them
    used = np.zeros(len(idx), bool)
    for pi in fwd.pairs_in:
        used[pi] = True
    assert np.array_equal(coords, idx[used])


# ---------------------------------------------------------------------------
# brute force: pair order and values
# ---------------------------------------------------------------------------

def _tiny(seed, shape, bs, n):
    rng = np.random.default_rng(seed)
    idx, _ = _random_sparse(rng, shape, bs, n, 1)
    return idx


@pytest.mark.parametrize("k,d", [(3, 1), (3, 2), (1, 1), ((3, 1, 3), (1, 2, 1)), ((2, 3, 2), 1)])
def test_oracle_subm_pairs_brute_force(k, d):
    shape = (5, 6, 4)
    idx = _tiny(7, shape, 2, 25)
    pr = OP.subm_pairs(idx, shape, 2, k, d)
    pin, pout = brute.subm(idx, shape, OP.to3(k), OP.to3(d))
    assert [list(p) for p in pr.pairs_in] == pin
    assert [list(p) for p in pr.pairs_out] == pout
    assert list(pr.pair_num) == [len(p) for p in pin]


@pytest.mark.parametrize("k,s,p,d", [(3, 2, 1, 1), (2, 2, 0, 1), (2, 1, 0, 1), (3, 1, 1, 2),
                                     ((3, 1, 1), (2, 1, 1), 0, 1), (3, (2, 1, 2), (1, 0, 1), 1)])
def test_oracle_strided_pairs_brute_force(k, s, p, d):
    shape = (5, 6, 7)
    idx = _tiny(11, shape, 2, 20)
    pr = OP.strided_pairs(idx, shape, 2, k, s, p, d)
    out_idx, pin, pout, oshape = brute.strided(idx, shape, 2, OP.to3(k), OP.to3(s), OP.to3(p),
                                               OP.to3(d))
    assert pr.output_spatial_shape == oshape
    assert np.array_equal(pr.out_indices, out_idx)
    assert [list(x) for x in pr.pairs_in] == pin
    assert [list(x) for x in pr.pairs_out] == pout
    inv = OP.inverse_pairs(pr)
    bi_idx, bi_in, bi_out = brute.inverse(idx, pin, pout)
    assert np.array_equal(inv.out_indices, bi_idx)
    assert [list(x) for x in inv.pairs_in] == bi_in
    assert [list(x) for x in inv.pairs_out] == bi_out


def test_oracle_subm_repeated_coordinates_later_row_wins():
    idx = np.array([[0, 1, 1, 1], [0, 1, 1, 2], [0, 1, 1, 1]], dtype=np.int32)
    pr = OP.subm_pairs(idx, (3, 3, 3), 1, 3)
    pin, pout = brute.subm(idx, (3, 3, 3), (3, 3, 3), (1, 1, 1))
    assert [list(p) for p in pr.pairs_in] == pin
    assert [list(p) for p in pr.pairs_out] == pout


def test_oracle_strided_empty_output():
    # stride 2, no padding, k=1: odd coordinates produce no candidate
    idx = np.array([[0, 1, 1, 1], [0, 3, 1, 1]], dtype=np.int32)
    pr = OP.strided_pairs(idx, (5, 5, 5), 1, 1, 2, 0)
    assert pr.out_indices.shape == (0, 4)
    assert list(pr.pair_num) == [0]


# ---------------------------------------------------------------------------
# weight layout
# ---------------------------------------------------------------------------

def test_oracle_weight_layouts():
    rng = np.random.default_rng(5)
    w = rng.normal(size=(6, 3, 2, 3, 4))
    W = OC.normalize_weight(w, (3, 2, 3), 4, 6)
    assert W.shape == (18, 4, 6)
    for kz in range(3):
        for ky in range(2):
            for kx in range(3):
                kk = (kz * 2 + ky) * 3 + kx
                assert np.array_equal(W[kk], w[:, kz, ky, kx, :].T)
    w1 = rng.normal(size=(6, 1, 1, 1, 4))
    W1 = OC.normalize_weight(w1, 1, 4, 6)
    assert np.array_equal(W1[0], w1.ravel().reshape(4, 6))
    assert np.array_equal(OC.normalize_weight(w1.reshape(6, 4), 1, 4, 6), W1)
    assert OC.normalize_weight(W, (3, 2, 3), 4, 6) is not None
    with pytest.raises(ValueError):
        OC.normalize_weight(rng.normal(size=(5, 5)), 3, 4, 6)


# ---------------------------------------------------------------------------
# the torch restatement of the reference's CPU path (the timed CPU baseline):
# brute force for pair order, golden fixtures for features and coordinates
# ---------------------------------------------------------------------------
from oracle import torch_path as TP  # noqa: E402


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


@pytest.mark.parametrize("k,d", [(3, 1), (3, 2), (1, 1), ((3, 1, 3), (1, 2, 1)), ((2, 3, 2), 1)])
def test_torch_path_subm_pairs_brute_force(k, d):
    shape = (5, 6, 4)
    idx = _tiny(7, shape, 2, 25)
    pr = TP.subm_pairs(_t(idx), shape, 2, k, d)
    pin, pout = brute.subm(idx, shape, OP.to3(k), OP.to3(d))
    assert [p.tolist() for p in pr.pairs_in] == pin
    assert [p.tolist() for p in pr.pairs_out] == pout
    assert pr.pair_num.tolist() == [len(p) for p in pin]


@pytest.mark.parametrize("k,s,p,d", [(3, 2, 1, 1), (2, 2, 0, 1), (2, 1, 0, 1), (3, 1, 1, 2),
                                     ((3, 1, 1), (2, 1, 1), 0, 1), (3, (2, 1, 2), (1, 0, 1), 1)])
def test_torch_path_strided_and_inverse_brute_force(k, s, p, d):
    shape = (5, 6, 7)
    idx = _tiny(11, shape, 2, 20)
    pr = TP.strided_pairs(_t(idx), shape, 2, k, s, p, d)
    out_idx, pin, pout, oshape = brute.strided(idx, shape, 2, OP.to3(k), OP.to3(s), OP.to3(p),
                                               OP.to3(d))
    assert pr.output_spatial_shape == oshape
    assert np.array_equal(pr.out_indices.numpy(), out_idx)
    assert [x.tolist() for x in pr.pairs_in] == pin
    assert [x.tolist() for x in pr.pairs_out] == pout
    inv = TP.inverse_pairs(pr)
    bi_idx, bi_in, bi_out = brute.inverse(idx, pin, pout)
    assert np.array_equal(inv.out_indices.numpy(), bi_idx)
    assert [x.tolist() for x in inv.pairs_in] == bi_in
    assert [x.tolist() for x in inv.pairs_out] == bi_out


@pytest.mark.parametrize("name", golden_io.fixture_names())
def test_torch_path_matches_spconv_golden(name):
    a, m = golden_io.load(name)
    k, s, p, d = m["kernel_size"], m["stride"], m["padding"], m["dilation"]
    bias = None if a.get("bias") is None else _t(a["bias"]).double()
    cache = {}
    if m["conv_type"] in ("subm", "strided"):
        lay = {"kind": m["conv_type"], "kernel_size": OP.to3(k), "stride": OP.to3(s),
               "padding": OP.to3(p), "dilation": OP.to3(d), "indice_key": None}
        out, coords, shape, _, _, _ = TP.run_layer(
            lay, _t(a["features"]).double(), _t(a["indices"]), tuple(m["spatial_shape"]),
            m["batch_size"], _t(a["weight"]).double(), bias, cache)
    else:
        down = {"kind": "strided", "kernel_size": OP.to3(k), "stride": OP.to3(s),
                "padding": OP.to3(p), "dilation": OP.to3(d), "indice_key": "k"}
        _, dcoords, dshape, _, _, _ = TP.run_layer(
            down, _t(a["down_in_features"]).double(), _t(a["down_in_indices"]),
            tuple(m["down_in_spatial_shape"]), m["batch_size"], _t(a["down_weight"]).double(),
            None, cache)
        ref_order = np.argsort(golden_io.encode(a["indices"], dshape), kind="stable")
        ours_order = np.argsort(golden_io.encode(dcoords.numpy(), dshape), kind="stable")
        feats = np.empty_like(a["features"])
        feats[ours_order] = a["features"][ref_order]
        inv = dict(down, kind="inverse")
        out, coords, shape, _, _, _ = TP.run_layer(
            inv, _t(feats).double(), dcoords, dshape, m["batch_size"],
            _t(a["weight"]).double(), bias, cache)
    f_sorted, i_sorted = golden_io.sort_by_coord(out.numpy(), coords.numpy(), shape)
    assert np.array_equal(i_sorted, a["out_indices"])
    np.testing.assert_allclose(f_sorted, a["out_features"], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_torch_path_conv_native_dtype_matches_oracle(dt):
    """The CPU branch keeps the features' dtype (functional.py:46): its result
    is the fp64 oracle's within that dtype's rounding."""
    rng = np.random.default_rng(77)
    shape = (10, 9, 8)
    idx, feats = _random_sparse(rng, shape, 1, 150, 16)
    w = rng.uniform(-0.3, 0.3, size=(24, 3, 3, 3, 16))
    b = rng.uniform(-0.1, 0.1, size=24)
    fr = _t(feats).to(dt)
    wr = _t(w).to(dt)
    br = _t(b).to(dt)
    lay = {"kind": "subm", "kernel_size": (3, 3, 3), "stride": (1, 1, 1), "padding": (0, 0, 0),
           "dilation": (1, 1, 1), "indice_key": None}
    out, _, _, pr, _, _ = TP.run_layer(lay, fr, _t(idx), shape, 1, wr, br, {})
    assert out.dtype == dt
    ref, _, _, _ = OC.run_layer("subm", fr.double().numpy(), idx, shape, 1, wr.double().numpy(),
                                br.double().numpy(), 3)
    tol = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 4e-2}[dt]
    err = np.abs(out.double().numpy() - ref).max() / np.abs(ref).max()
    assert err < tol


def test_oracle_conv_sums_an_output_repeated_within_a_slot():
    """Hand-assigned lists may name an output row more than once within a
    slot; the reference's CPU branch adds every pair with index_add_
    (functional.py:46).  The oracle's accumulation is pinned against torch's
    own index_add_ over the same lists, slot by slot, in float64."""
    rng = np.random.default_rng(41)
    n_in, n_out, c_in, c_out, K = 30, 12, 5, 4, 3
    f = rng.standard_normal((n_in, c_in))
    w = rng.standard_normal((K, c_in, c_out))
    b = rng.standard_normal(c_out)
    pin = [rng.integers(0, n_in, 20), rng.integers(0, n_in, 0), rng.integers(0, n_in, 9)]
    pout = [rng.integers(0, n_out, 20), rng.integers(0, n_out, 0),
            np.array([3, 3, 3, 0, 1, 3, 11, 0, 3])]
    assert np.bincount(pout[0]).max() > 1  # slot 0 repeats outputs too
    got = OC.conv_forward(f, w, b, pin, pout, n_out)
    ref = torch.zeros(n_out, c_out, dtype=torch.float64)
    ft, wt = torch.from_numpy(f), torch.from_numpy(w)
    for k in range(K):
        if len(pin[k]):
            ref.index_add_(0, torch.from_numpy(pout[k]), ft[torch.from_numpy(pin[k])] @ wt[k])
    ref = ref + torch.from_numpy(b)
    assert np.allclose(got, ref.numpy(), rtol=0, atol=1e-12)
    # a plain fancy-index += would keep one contribution per repeated output:
    # the check above tells the two apart
    once = np.zeros((n_out, c_out))
    once[pout[2]] += f[pin[2]] @ w[2]
    assert not np.allclose(once[3], (f[pin[2][pout[2] == 3]] @ w[2]).sum(0))
