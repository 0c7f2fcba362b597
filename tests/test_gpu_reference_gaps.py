"""Reference behaviours at the edges of the path, on the GPU against the oracle.

* user-assigned pair lists: ids out of range raise IndexError before any
  launch (the reference's ``features[in_ids]`` / ``index_add_``,
  functional.py:46); an output named more than once within a slot gets every
  contribution, as ``index_add_`` adds them;
* the inverse built from user-assigned forward lists (modules.py:175-212
  remaps whatever lists it finds);
* float64 features and weights of another dtype than the features run on
  fp32 copies and are cast back (functional.py:32-36, :51);
* grids of 2^32 cells or more (the reference's int64 keys, indices.py:45-51).

Tolerances (max |out - ref| / max |ref|, fp64 oracle over the rounded
inputs): 1e-5 fp32 and fp64, 1e-2 fp16/bf16.
"""
import numpy as np
import pytest
import torch

import trispconv.pytorch as spconv
from gpu_util import DEV, lists_np, needs_gpu, rel_err, rounded, say, to_np
from oracle import conv as OC
from oracle import pairs as OP
from trispconv.pytorch import functional as Fn
from trispconv.pytorch.indices import (IndiceData, generate_strided_indice_pairs,
                                       generate_subm_indice_pairs)

pytestmark = [pytest.mark.gpu, needs_gpu]


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


def _hand_copy(data, pin=None, pout=None):
    return IndiceData(data.out_indices, pin if pin is not None else [p.clone() for p in data.pairs_in],
                      pout if pout is not None else [p.clone() for p in data.pairs_out],
                      data.pair_num, data.input_indices, data.input_spatial_shape,
                      data.output_spatial_shape, data.kernel_size, data.stride, data.padding,
                      data.dilation, data.subm)


# ------------------------------------------------------------ user lists
def test_user_lists_out_of_range_raise_index_error():
    idx = _tiny(3, (12, 12, 12), 1, 500)
    x = torch.from_numpy(idx).to(DEV)
    data = generate_subm_indice_pairs(x, (12, 12, 12), 1, 3)
    feats = torch.randn(len(idx), 16, device=DEV)
    W = torch.randn(27, 16, 16, device=DEV)
    n = len(idx)
    say("user lists: in range")
    ok = Fn.sparse_conv_forward(feats, W, None, _hand_copy(data), n)
    ref = OC.conv_forward(feats.cpu().numpy(), W.cpu().numpy(), None, lists_np(data.pairs_in),
                          lists_np(data.pairs_out), n)
    assert rel_err(ok.cpu().numpy(), ref) <= 1e-5
    for what, k_bad, val in [("in", 13, n), ("in", 0, -1), ("out", 5, n), ("out", 26, -2)]:
        pin = [p.clone() for p in data.pairs_in]
        pout = [p.clone() for p in data.pairs_out]
        lst = pin if what == "in" else pout
        if lst[k_bad].numel() == 0:
            continue
        lst[k_bad][0] = val
        say("user lists: bad", what, k_bad, val)
        with pytest.raises(IndexError):
            Fn.sparse_conv_forward(feats, W, None, _hand_copy(data, pin, pout), n)
    # mismatched list lengths
    k = max(range(27), key=lambda s: data.pairs_out[s].numel())
    pout = [p.clone() for p in data.pairs_out]
    pout[k] = pout[k][:-1]
    with pytest.raises(ValueError):
        Fn.sparse_conv_forward(feats, W, None, _hand_copy(data, None, pout), n)
    # features with fewer rows than the pairs read
    with pytest.raises(IndexError):
        Fn.sparse_conv_forward(feats[: n // 2], W, None, _hand_copy(data), n)
    with pytest.raises(IndexError):
        Fn.sparse_conv_forward(feats[: n // 2], W, None, data, n)


@pytest.mark.parametrize("dtype,c_in,c_out,reps", [
    (torch.float32, 16, 16, 2),   # 54 map rows: narrow MFMA kernel
    (torch.float16, 32, 32, 2),   # 54 map rows: 32x32-tile MFMA kernel
    (torch.bfloat16, 32, 64, 3),  # 81 map rows: past the 64-slot tile kernels
    (torch.float32, 5, 7, 3),     # VALU kernel
])
def test_user_lists_repeated_output_in_a_slot_sums(dtype, c_in, c_out, reps):
    """Hand-built lists that name an output row more than once within a slot
    (and an input row more than once): the reference's index_add_
    (functional.py:46) adds every contribution; so does the fused kernel,
    against the oracle's np.add.at accumulation."""
    idx = _tiny(21, (12, 12, 12), 1, 600)
    n = len(idx)
    data = generate_subm_indice_pairs(torch.from_numpy(idx).to(DEV), (12, 12, 12), 1, 3)
    rng = np.random.default_rng(c_in + reps)
    pin = lists_np(data.pairs_in)
    pout = lists_np(data.pairs_out)
    for k in (0, 4, 13, 26):
        if len(pout[k]) < 4:
            continue
        # duplicate a few pairs' outputs with other inputs, up to reps times
        pick = rng.choice(len(pout[k]), size=min(5, len(pout[k])), replace=False)
        extra_out = np.concatenate([pout[k][pick]] * (reps - 1))
        extra_in = rng.integers(0, n, size=len(extra_out))
        pout[k] = np.concatenate([pout[k], extra_out])
        pin[k] = np.concatenate([pin[k], extra_in])
        perm = rng.permutation(len(pout[k]))
        pout[k], pin[k] = pout[k][perm], pin[k][perm]
    hand = _hand_copy(data, [torch.from_numpy(p).to(DEV) for p in pin],
                      [torch.from_numpy(p).to(DEV) for p in pout])
    g = torch.Generator().manual_seed(2)
    feats = torch.randn(n, c_in, generator=g).to(dtype)
    W = (torch.randn(27, c_in, c_out, generator=g) / (27 * c_in) ** 0.5).to(dtype)
    b = (torch.rand(c_out, generator=g) * 0.2 - 0.1).to(dtype)
    say("repeated outputs:", dtype, c_in, c_out, reps)
    out = Fn.sparse_conv_forward(feats.to(DEV), W.to(DEV), b.to(DEV), hand, n)
    assert hand.slot_repeat == reps
    ref = OC.conv_forward(rounded(to_np(feats), dtype), rounded(to_np(W), dtype),
                          rounded(to_np(b), dtype), pin, pout, n)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    err = rel_err(to_np(out), ref)
    say("  rel err", err)
    assert err <= tol
    # the same lists without the repeats run on the one-row-per-slot map
    assert data.slot_repeat == 1


def test_inverse_from_forward_lists_with_a_repeated_input_row():
    """A forward pairs_in list that names an input row twice within a slot:
    the inverse names that output twice (modules.py:175-212 remaps the lists
    as they are) and adds both contributions."""
    shape = (10, 12, 11)
    idx = _tiny(23, shape, 1, 400)
    fwd = generate_strided_indice_pairs(torch.from_numpy(idx).to(DEV), shape, 1, 3, 2, 1)
    pin = lists_np(fwd.pairs_in)
    pout = lists_np(fwd.pairs_out)
    k = max(range(27), key=lambda s: len(pin[s]))
    # pair the slot's first input row with one more output of this slot
    extra_out = int(pout[k][1])
    pin[k] = np.concatenate([pin[k], pin[k][:1]])
    pout[k] = np.concatenate([pout[k], [extra_out]])
    fwd.pairs_in = [torch.from_numpy(p).to(DEV) for p in pin]
    fwd.pairs_out = [torch.from_numpy(p).to(DEV) for p in pout]
    fwd.pair_num = torch.tensor([len(p) for p in pin], dtype=torch.long)
    n_down = len(fwd.out_indices)
    torch.manual_seed(6)
    up = spconv.SparseInverseConv3d(16, 8, 3, indice_key="d").to(DEV)
    xs = torch.randn(n_down, 16, device=DEV)
    t = spconv.SparseConvTensor(xs, fwd.out_indices, list(fwd.output_spatial_shape), 1)
    t.indice_dict["d"] = fwd
    say("inverse with a repeated forward input row")
    y = up(t)
    exp_fwd = OP.OraclePairs(fwd.out_indices.cpu().numpy(), pin, pout,
                             np.array([len(p) for p in pin]), idx, shape,
                             tuple(fwd.output_spatial_shape), (3, 3, 3), (2, 2, 2), (1, 1, 1),
                             (1, 1, 1), False)
    inv = OP.inverse_pairs(exp_fwd)
    assert np.array_equal(y.indices.cpu().numpy(), inv.out_indices)
    w = OC.normalize_weight(to_np(up.weight).astype(np.float64), (3, 3, 3), 16, 8)
    ref = OC.conv_forward(to_np(xs).astype(np.float64), w, to_np(up.bias).astype(np.float64),
                          inv.pairs_in, inv.pairs_out, len(inv.out_indices))
    assert rel_err(to_np(y.features), ref) <= 1e-5


def test_reassigning_one_list_keeps_the_other():
    """Setting pairs_in alone keeps pairs_out (the tables both came from go)."""
    idx = _tiny(5, (10, 10, 10), 1, 300)
    data = generate_subm_indice_pairs(torch.from_numpy(idx).to(DEV), (10, 10, 10), 1, 3)
    exp_out = lists_np(data.pairs_out)
    data2 = generate_subm_indice_pairs(torch.from_numpy(idx).to(DEV), (10, 10, 10), 1, 3)
    data2.pairs_in = [p.clone() for p in data2.pairs_in]
    assert [a.tolist() for a in lists_np(data2.pairs_out)] == [a.tolist() for a in exp_out]
    feats = torch.randn(len(idx), 8, device=DEV)
    W = torch.randn(27, 8, 8, device=DEV)
    assert torch.equal(Fn.sparse_conv_forward(feats, W, None, data, len(idx)),
                       Fn.sparse_conv_forward(feats, W, None, data2, len(idx)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_inverse_from_user_assigned_forward_lists(dtype):
    """SparseInverseConv3d on a forward IndiceData whose lists the user
    assigned (here: each slot's pairs reversed, and one slot emptied): output
    coordinates exact against the oracle's inverse of those lists, features
    within tolerance."""
    shape = (14, 16, 15)
    idx = _tiny(9, shape, 2, 700)
    x_idx = torch.from_numpy(idx).to(DEV)
    fwd = generate_strided_indice_pairs(x_idx, shape, 2, 3, 2, 1)
    pin = [torch.flip(p, [0]).clone() for p in fwd.pairs_in]
    pout = [torch.flip(p, [0]).clone() for p in fwd.pairs_out]
    pin[13] = pin[13][:0]
    pout[13] = pout[13][:0]
    fwd.pairs_in = pin
    fwd.pairs_out = pout
    n_down = len(fwd.out_indices)
    torch.manual_seed(4)
    up = spconv.SparseInverseConv3d(24, 12, 3, indice_key="d").to(DEV).to(dtype)
    with torch.no_grad():
        up.bias.uniform_(-0.1, 0.1)
    xs = torch.randn(n_down, 24, device=DEV).to(dtype)
    t = spconv.SparseConvTensor(xs, fwd.out_indices, list(fwd.output_spatial_shape), 2)
    t.indice_dict["d"] = fwd
    y = up(t)
    exp_fwd = OP.OraclePairs(fwd.out_indices.cpu().numpy(), lists_np(pin), lists_np(pout),
                             np.array([len(p) for p in pin]), idx, shape,
                             tuple(fwd.output_spatial_shape), (3, 3, 3), (2, 2, 2), (1, 1, 1),
                             (1, 1, 1), False)
    inv = OP.inverse_pairs(exp_fwd)
    assert np.array_equal(y.indices.cpu().numpy(), inv.out_indices)
    w = OC.normalize_weight(to_np(up.weight).astype(np.float64), (3, 3, 3), 24, 12)
    ref = OC.conv_forward(rounded(to_np(xs), dtype), w, to_np(up.bias).astype(np.float64),
                          inv.pairs_in, inv.pairs_out, len(inv.out_indices))
    err = rel_err(to_np(y.features), ref)
    say("inverse from user lists", dtype, err)
    assert err <= (1e-5 if dtype == torch.float32 else 1e-2)


def test_inverse_from_user_lists_checks_ranges():
    shape = (10, 10, 10)
    idx = _tiny(11, shape, 1, 300)
    fwd = generate_strided_indice_pairs(torch.from_numpy(idx).to(DEV), shape, 1, 3, 2, 1)
    pin = [p.clone() for p in fwd.pairs_in]
    k = max(range(27), key=lambda s: pin[s].numel())
    pin[k][0] = len(idx)  # past the forward's input rows
    fwd.pairs_in = pin
    up = spconv.SparseInverseConv3d(8, 8, 3, indice_key="d").to(DEV)
    t = spconv.SparseConvTensor(torch.randn(len(fwd.out_indices), 8, device=DEV), fwd.out_indices,
                                list(fwd.output_spatial_shape), 1)
    t.indice_dict["d"] = fwd
    with pytest.raises(IndexError):
        up(t)


# ------------------------------------------------------------ dtypes
def test_float64_features_compute_in_fp32_and_come_back_float64():
    shape = (16, 16, 16)
    idx = _tiny(13, shape, 1, 1200)
    torch.manual_seed(2)
    m = spconv.SubMConv3d(16, 24, 3, indice_key="s").to(DEV).double()
    with torch.no_grad():
        m.bias.uniform_(-0.1, 0.1)
    feats = torch.randn(len(idx), 16, device=DEV, dtype=torch.float64)
    y = m(spconv.SparseConvTensor(feats, torch.from_numpy(idx).to(DEV), list(shape), 1))
    assert y.features.dtype == torch.float64
    pr = OP.subm_pairs(idx, shape, 1, 3)
    w = OC.normalize_weight(m.weight.detach().cpu().numpy(), (3, 3, 3), 16, 24)
    ref = OC.conv_forward(feats.cpu().numpy(), w, m.bias.detach().cpu().numpy(), pr.pairs_in,
                          pr.pairs_out, len(idx))
    err = rel_err(y.features.detach().cpu().numpy(), ref)
    say("float64 features", err)
    assert err <= 1e-5
    # a strided layer and its inverse in float64 as well, each against the
    # oracle on its own (GPU-computed) float64 input, at the same tolerance
    down = spconv.SparseConv3d(24, 32, 3, stride=2, padding=1, indice_key="d").to(DEV).double()
    up = spconv.SparseInverseConv3d(32, 16, 3, indice_key="d").to(DEV).double()
    with torch.no_grad():
        down.bias.uniform_(-0.1, 0.1)
        up.bias.uniform_(-0.1, 0.1)
    d = down(y)
    z = up(d)
    assert d.features.dtype == torch.float64 and z.features.dtype == torch.float64
    pd = OP.strided_pairs(idx, shape, 1, 3, 2, 1)
    assert np.array_equal(d.indices.cpu().numpy(), pd.out_indices)
    wd = OC.normalize_weight(down.weight.detach().cpu().numpy(), (3, 3, 3), 24, 32)
    ref_d = OC.conv_forward(y.features.detach().cpu().numpy(), wd, down.bias.detach().cpu().numpy(),
                            pd.pairs_in, pd.pairs_out, len(pd.out_indices))
    err_d = rel_err(d.features.detach().cpu().numpy(), ref_d)
    pu = OP.inverse_pairs(pd)
    assert np.array_equal(z.indices.cpu().numpy(), pu.out_indices)
    wu = OC.normalize_weight(up.weight.detach().cpu().numpy(), (3, 3, 3), 32, 16)
    ref_u = OC.conv_forward(d.features.detach().cpu().numpy(), wu, up.bias.detach().cpu().numpy(),
                            pu.pairs_in, pu.pairs_out, len(pu.out_indices))
    err_u = rel_err(z.features.detach().cpu().numpy(), ref_u)
    say("float64 strided", err_d, "inverse", err_u)
    assert err_d <= 1e-5 and err_u <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fp32_module_on_half_features_keeps_fp32_weights(dtype):
    """An fp32 module on fp16/bf16 features: the reference upcasts the
    features and keeps the fp32 weights (functional.py:34-36), sums in fp32
    and rounds once.  So nearly every output equals the fp64 oracle over
    those values rounded to the features' dtype (fp32 summation order can
    flip an output that lies within ~1e-7 of a rounding boundary); weights
    rounded to the features' dtype would move a third or more of them."""
    shape = (20, 20, 20)
    idx = _tiny(17, shape, 1, 3000)
    torch.manual_seed(6)
    m = spconv.SubMConv3d(32, 64, 3).to(DEV)  # fp32 parameters
    with torch.no_grad():
        m.bias.uniform_(-0.1, 0.1)
    feats = torch.randn(len(idx), 32, device=DEV).to(dtype)
    y = m(spconv.SparseConvTensor(feats, torch.from_numpy(idx).to(DEV), list(shape), 1))
    assert y.features.dtype == dtype
    pr = OP.subm_pairs(idx, shape, 1, 3)
    w = OC.normalize_weight(m.weight.detach().cpu().numpy().astype(np.float64), (3, 3, 3), 32, 64)
    b = m.bias.detach().cpu().numpy().astype(np.float64)
    f = feats.float().cpu().numpy().astype(np.float64)
    ref = OC.conv_forward(f, w, b, pr.pairs_in, pr.pairs_out, len(idx))
    out = y.features.cpu()
    exact = float((out == torch.from_numpy(ref).to(dtype)).double().mean())
    w_r = rounded(w, dtype)
    ref_wr = OC.conv_forward(f, w_r, b, pr.pairs_in, pr.pairs_out, len(idx))
    exact_wr = float((torch.from_numpy(ref_wr).to(dtype) == torch.from_numpy(ref).to(dtype))
                     .double().mean())
    say("fp32 module, half features", dtype, "exact", exact, "(rounded weights would give",
        exact_wr, ")")
    assert exact >= 0.99
    assert exact_wr < 0.9  # the check tells the two apart
    assert rel_err(to_np(y.features), ref) <= 1e-2


# ------------------------------------------------------------ big grids
def test_grids_beyond_32_bit_cells():
    """Batch 16 of an 81 x 3200 x 2816 grid (11.7G cells, cell ids past 2^32):
    SubM pairs on the 64-bit-key hash, a stride-1 strided layer whose output
    grid is that large too, and a SubM layer on its output.  The voxels sit in
    a box well inside the grid, so every pair and output equals the oracle's
    on the box alone, shifted."""
    big = (81, 3200, 2816)
    box = (12, 40, 36)
    off = np.array([50, 3000, 2700], dtype=np.int32)
    B = 16
    small = _tiny(19, box, B, 900)
    # keep one free cell around the box, so that no candidate output of the
    # strided layer leaves it
    inner = (small[:, 1:] >= 1).all(1) & (small[:, 1] < box[0] - 1) & (small[:, 2] < box[1] - 1) \
        & (small[:, 3] < box[2] - 1)
    small = small[inner]
    bigc = small.copy()
    bigc[:, 1:] += off
    assert ((B - 1) * big[0] + int(bigc[:, 1].max())) * big[1] * big[2] > 2 ** 32
    xb = torch.from_numpy(bigc).to(DEV)
    say("big grid subm", len(bigc))
    got = generate_subm_indice_pairs(xb, big, B, 3)
    exp = OP.subm_pairs(small, box, B, 3)
    for k in range(27):
        assert np.array_equal(lists_np(got.pairs_in)[k], exp.pairs_in[k]), k
        assert np.array_equal(lists_np(got.pairs_out)[k], exp.pairs_out[k]), k
    say("big grid strided s1")
    st = generate_strided_indice_pairs(xb, big, B, 3, 1, 1)
    exp_st = OP.strided_pairs(small, box, B, 3, 1, 1)
    shifted = exp_st.out_indices.copy()
    shifted[:, 1:] += off
    assert np.array_equal(st.out_indices.cpu().numpy(), shifted)
    for k in range(27):
        assert np.array_equal(lists_np(st.pairs_in)[k], exp_st.pairs_in[k]), k
        assert np.array_equal(lists_np(st.pairs_out)[k], exp_st.pairs_out[k]), k
    # a network on it: SubM, strided s1, SubM on the strided output
    torch.manual_seed(8)
    net = spconv.SparseSequential(
        spconv.SubMConv3d(16, 32, 3, indice_key="a"),
        spconv.SparseConv3d(32, 32, 3, stride=1, padding=1, indice_key="b"),
        spconv.SubMConv3d(32, 32, 3, indice_key="c")).to(DEV).half()
    feats = torch.randn(len(bigc), 16, device=DEV).half()
    y = net(spconv.SparseConvTensor(feats, xb, list(big), B))
    f = rounded(to_np(feats), torch.float16)
    idx_s, shp = small, box
    for mod in net.children():
        o, idx_s, shp, _ = OC.run_layer("subm" if mod.subm else "strided", f, idx_s, shp, B,
                                        to_np(mod.weight).astype(np.float64),
                                        to_np(mod.bias).astype(np.float64), mod.kernel_size,
                                        mod.stride, mod.padding, mod.dilation)
        f = rounded(o.astype(np.float32), torch.float16)
    exp_idx = idx_s.copy()
    exp_idx[:, 1:] += off
    assert np.array_equal(y.indices.cpu().numpy(), exp_idx)
    err = rel_err(to_np(y.features), f)
    say("big grid network rel err", err)
    assert err <= 1e-2
