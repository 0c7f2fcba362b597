"""Indice pairs on the GPU are bit-exact against the oracle.

Checks pair lists (order and values), pair_num, output coordinates and their
row order for submanifold, strided and inverse builds: on the reference's
golden-fixture inputs, on tiny inputs with unusual kernels, on empty and
single-voxel inputs, and on the five workloads at their full sizes.
"""
import numpy as np
import pytest
import torch

import golden_io
from gpu_util import DEV, lists_np, needs_gpu, say
from oracle import pairs as OP
from trispconv.pytorch.indices import (generate_inverse_indice_pairs,
                                       generate_strided_indice_pairs, generate_subm_indice_pairs)
from trispconv_amd import workloads

pytestmark = [pytest.mark.gpu, needs_gpu]


def _check_lists(got, exp, what):
    g_in, g_out = lists_np(got.pairs_in), lists_np(got.pairs_out)
    assert len(g_in) == len(exp.pairs_in), what
    assert got.pair_num.dtype == torch.int64 and got.pair_num.device.type == "cpu"
    assert np.array_equal(got.pair_num.numpy(), exp.pair_num), what
    for k in range(len(exp.pairs_in)):
        assert np.array_equal(g_in[k], exp.pairs_in[k]), f"{what}: pairs_in[{k}]"
        assert np.array_equal(g_out[k], exp.pairs_out[k]), f"{what}: pairs_out[{k}]"


def _subm(idx, shape, B, k, d, what):
    say("subm pairs:", what, idx.shape, shape, k, d)
    got = generate_subm_indice_pairs(torch.from_numpy(idx).to(DEV), shape, B, k, d)
    exp = OP.subm_pairs(idx, shape, B, k, d)
    _check_lists(got, exp, what)
    assert got.subm and got.output_spatial_shape == tuple(shape)
    return got


def _strided(idx, shape, B, k, s, p, d, what):
    say("strided pairs:", what, idx.shape, shape, k, s, p, d)
    x = torch.from_numpy(idx).to(DEV)
    got = generate_strided_indice_pairs(x, shape, B, k, s, p, d)
    exp = OP.strided_pairs(idx, shape, B, k, s, p, d)
    assert got.output_spatial_shape == tuple(exp.output_spatial_shape), what
    assert np.array_equal(got.out_indices.cpu().numpy(), exp.out_indices), f"{what}: out_indices"
    _check_lists(got, exp, what)
    return got, exp


def _inverse(got_fwd, exp_fwd, what):
    say("inverse pairs:", what)
    got = generate_inverse_indice_pairs(got_fwd)
    exp = OP.inverse_pairs(exp_fwd)
    # the forward build counted the inverse's rows (inputs with a pair), so
    # the inverse needs no host read of its own
    assert got_fwd._n_in_paired == len(exp.out_indices), f"{what}: paired input rows"
    assert np.array_equal(got.out_indices.cpu().numpy(), exp.out_indices), f"{what}: out_indices"
    _check_lists(got, exp, what)
    return got


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


@pytest.mark.parametrize("name", golden_io.fixture_names())
def test_pairs_on_fixture_inputs(name):
    a, m = golden_io.load(name)
    k, s, p, d = m["kernel_size"], m["stride"], m["padding"], m["dilation"]
    B = m["batch_size"]
    if m["conv_type"] == "subm":
        _subm(a["indices"], tuple(m["spatial_shape"]), B, k, d, name)
    elif m["conv_type"] == "strided":
        _strided(a["indices"], tuple(m["spatial_shape"]), B, k, s, p, d, name)
    else:
        g, e = _strided(a["down_in_indices"], tuple(m["down_in_spatial_shape"]), B, k, s, p, d,
                        name + "/fwd")
        if e.kernel_size != (1, 1, 1):
            _inverse(g, e, name)


@pytest.mark.parametrize("k,d", [(3, 1), (3, 2), (1, 1), ((3, 1, 3), (1, 2, 1)), ((2, 3, 2), 1),
                                 (5, 1), ((7, 3, 3), 1)])
def test_subm_pairs_unusual_kernels(k, d):
    idx = _tiny(17, (9, 10, 11), 2, 300)
    _subm(idx, (9, 10, 11), 2, k, d, f"k={k} d={d}")


@pytest.mark.parametrize("k,s,p,d", [(3, 2, 1, 1), (2, 2, 0, 1), (2, 1, 0, 1), (3, 1, 1, 2),
                                     ((3, 1, 1), (2, 1, 1), 0, 1), (3, (2, 1, 2), (1, 0, 1), 1),
                                     (1, 2, 0, 1), (5, 3, 2, 1)])
def test_strided_and_inverse_pairs_unusual(k, s, p, d):
    idx = _tiny(23, (9, 10, 11), 3, 250)
    g, e = _strided(idx, (9, 10, 11), 3, k, s, p, d, f"k={k} s={s} p={p} d={d}")
    if e.kernel_size != (1, 1, 1):
        _inverse(g, e, f"inverse k={k} s={s} p={p} d={d}")


@pytest.mark.parametrize("room", ["none", "one short", "exact", "learned"])
def test_strided_outputs_beyond_their_room_are_filled_again(room, monkeypatch):
    """The strided fill is queued before the output count reaches the host,
    with room for a guessed number of rows; a build whose count exceeds it is
    filled again at its exact size.  Either way the outputs are the oracle's;
    the ratio a build gives becomes its geometry's guess."""
    from trispconv_amd.pytorch import indices as IM
    idx = _tiny(29, (9, 10, 11), 2, 300)
    exp_n = len(OP.strided_pairs(idx, (9, 10, 11), 2, 3, 2, 1, 1).out_indices)
    caps = {"none": 0, "one short": exp_n - 1, "exact": exp_n}
    monkeypatch.setattr(IM, "_STRIDED_OUT_RATIO", {})
    if room != "learned":
        monkeypatch.setattr(IM, "_strided_out_cap", lambda key, n, cells: caps[room])
    g, e = _strided(idx, (9, 10, 11), 2, 3, 2, 1, 1, f"room {room}")
    _inverse(g, e, f"inverse, room {room}")
    key = (2, (9, 10, 11), (3, 3, 3), (2, 2, 2), (1, 1, 1), (1, 1, 1))
    assert IM._STRIDED_OUT_RATIO[key] == exp_n / len(idx)
    if room == "learned":
        cap = IM._strided_out_cap(key, len(idx), 10**9)
        assert exp_n <= cap <= exp_n * 1.0625 + 257
        g, e = _strided(idx, (9, 10, 11), 2, 3, 2, 1, 1, "room learned, second build")


def test_strided_fill_with_too_little_room_writes_no_outputs():
    """Through the C ABI: a fill whose out_cap is below n_out leaves
    out_coords and the map untouched and still writes the pair lists and the
    input ids; with room to spare it writes the map [K][n_out] from the
    buffer's start and nothing past it."""
    from trispconv_amd import _lib as L
    from trispconv_amd.pytorch import indices as IM
    lib = L.lib()
    idx = _tiny(31, (9, 10, 11), 2, 300)
    x = torch.from_numpy(idx).to(DEV)
    shape, ks, st, pd, dl = (9, 10, 11), (3, 3, 3), (2, 2, 2), (1, 1, 1), (1, 1, 1)
    out_shape = IM._output_spatial_shape(shape, ks, st, pd, dl)
    K, n = 27, len(idx)
    geo = (L.i3(shape), L.i3(ks), L.i3(st), L.i3(pd), L.i3(dl), L.i3(out_shape))
    wsb = lib.tsc_strided_workspace_bytes(n, K, 2, geo[5], 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    counts = torch.empty(K + 3, dtype=torch.int32, device=DEV)
    s = L.stream_of(x)
    L.check(lib.tsc_strided_count(x.data_ptr(), n, 2, *geo, ws.data_ptr(), wsb, None, 0, 0,
                                  counts.data_ptr(), s), "count")
    n_out = int(counts.cpu()[K])
    exp = OP.strided_pairs(idx, shape, 2, ks, st, pd, dl)
    assert n_out == len(exp.out_indices)
    res = {}
    for out_cap in (n_out - 1, n_out + 100):
        say("strided fill, out_cap", out_cap, "n_out", n_out)
        oc = torch.full((out_cap, 4), -7, dtype=torch.int32, device=DEV)
        nbr = torch.full((K * out_cap,), -7, dtype=torch.int32, device=DEV)
        pin = torch.full((K, n), -7, dtype=torch.int32, device=DEV)
        pout = torch.full((K, n), -7, dtype=torch.int32, device=DEV)
        ids = torch.full((n,), -7, dtype=torch.int32, device=DEV)
        L.check(lib.tsc_strided_fill(x.data_ptr(), n, 2, *geo, ws.data_ptr(), wsb,
                                     counts.data_ptr(), out_cap, oc.data_ptr(), nbr.data_ptr(),
                                     pin.data_ptr(), pout.data_ptr(), ids.data_ptr(), s), "fill")
        res[out_cap] = (oc.cpu(), nbr.cpu(), pin.cpu(), pout.cpu(), ids.cpu())
    oc, nbr, pin, pout, ids = res[n_out - 1]
    assert bool((oc == -7).all()) and bool((nbr == -7).all()), "no outputs without room"
    oc2, nbr2, pin2, pout2, ids2 = res[n_out + 100]
    assert np.array_equal(oc2[:n_out].numpy(), exp.out_indices)
    assert bool((oc2[n_out:] == -7).all()) and bool((nbr2[K * n_out:] == -7).all())
    pn = exp.pair_num
    for k in range(K):
        assert np.array_equal(pin2[k, :pn[k]].numpy(), exp.pairs_in[k]), f"pairs_in[{k}]"
        assert np.array_equal(pout2[k, :pn[k]].numpy(), exp.pairs_out[k]), f"pairs_out[{k}]"
        m = nbr2[k * n_out:(k + 1) * n_out].numpy()
        want = np.full(n_out, -1, np.int32)
        want[exp.pairs_out[k]] = exp.pairs_in[k]
        assert np.array_equal(m, want), f"map row {k}"
    assert torch.equal(pin, pin2) and torch.equal(pout, pout2) and torch.equal(ids, ids2)


def test_empty_and_single_inputs():
    empty = np.zeros((0, 4), np.int32)
    _subm(empty, (4, 4, 4), 1, 3, 1, "empty subm")
    g, e = _strided(empty, (4, 4, 4), 1, 3, 2, 1, 1, "empty strided")
    assert g.out_indices.shape == (0, 4)
    one = np.array([[0, 2, 2, 2]], np.int32)
    _subm(one, (4, 4, 4), 1, 3, 1, "single subm")
    g, e = _strided(one, (4, 4, 4), 1, 3, 2, 1, 1, "single strided")
    _inverse(g, e, "single inverse")
    # no candidate at all: stride 2, k=1, odd coordinates only
    odd = np.array([[0, 1, 1, 1], [0, 3, 1, 3]], np.int32)
    g, e = _strided(odd, (5, 5, 5), 1, 1, 2, 0, 1, "no candidates")
    assert g.out_indices.shape == (0, 4) and int(g.pair_num.sum()) == 0


def test_repeated_coordinates_later_row_wins():
    idx = np.array([[0, 1, 1, 1], [0, 1, 1, 2], [0, 1, 1, 1], [0, 2, 2, 2], [0, 1, 1, 2]], np.int32)
    _subm(idx, (4, 4, 4), 1, 3, 1, "duplicates")


def _clustered_with_duplicates(seed, shape, B, n, box, dups):
    """n voxels per sample inside a box-sized corner of the grid (so they have
    neighbours), plus `dups` repeats of random rows, shuffled."""
    rng = np.random.default_rng(seed)
    parts = []
    for b in range(B):
        cells = rng.choice(box ** 3, size=n, replace=False)
        z, r = np.divmod(cells, box * box)
        y, x = np.divmod(r, box)
        off = rng.integers(0, [shape[0] - box + 1, shape[1] - box + 1, shape[2] - box + 1])
        parts.append(np.stack([np.full(n, b), z + off[0], y + off[1], x + off[2]], 1))
    idx = np.concatenate(parts).astype(np.int32)
    idx = np.concatenate([idx, idx[rng.choice(len(idx), size=dups)]])
    return idx[rng.permutation(len(idx))]


def _stream_marks():
    from trispconv_amd import _lib as L
    from trispconv_amd.pytorch import indices as IM
    probe = torch.zeros(1, device=DEV)
    return IM._MARKS.by_stream.get((probe.device.index, L.stream_of(probe)))


def test_byte_marks_kept_between_builds_never_leak(monkeypatch):
    """SubM and strided builds on one stream share byte marks that no build
    zeroes.  Builds on shrinking coordinate sets of one grid (every cell of a
    later set was marked by an earlier build), a build that raises on a bad
    batch index followed by good ones, the values running out (zeroed, then
    1 again) and a larger grid (new marks) all give the oracle's pairs."""
    from trispconv_amd.pytorch import indices as IM
    monkeypatch.setattr(IM, "_MARKS", IM._ThreadMarks())  # marks sized by this test's grids alone
    shape, B = (20, 22, 24), 2
    big = _tiny(51, shape, B, 1800)
    small = big[: len(big) // 3]
    for what, idx in (("all", big), ("a third", small), ("all again", big), ("a third", small)):
        _subm(idx, shape, B, 3, 1, f"kept marks, subm on {what}")
        g, e = _strided(idx, shape, B, 3, 2, 1, 1, f"kept marks, strided on {what}")
    m = _stream_marks()
    assert m is not None and m.buf is not None and 2 <= m.gen <= 255
    bad = big.copy()
    bad[5, 0] = B  # batch index out of range
    with pytest.raises(IndexError, match="batch index"):
        generate_subm_indice_pairs(torch.from_numpy(bad).to(DEV), shape, B, 3, 1)
    with pytest.raises(IndexError, match="batch index"):
        generate_strided_indice_pairs(torch.from_numpy(bad).to(DEV), shape, B, 3, 2, 1)
    _subm(small, shape, B, 3, 1, "kept marks, subm after a bad build")
    _strided(small, shape, B, 3, 2, 1, 1, "kept marks, strided after a bad build")
    m.gen = 253  # three values left: the fourth build zeroes the marks first
    for i in range(3):
        _subm(big if i % 2 else small, shape, B, 3, 1, f"kept marks, values running out {i}")
        _strided(small if i % 2 else big, shape, B, 3, 2, 1, 1, f"values running out {i}")
    assert m.gen <= 6
    size = m.buf.numel()
    wide = (40, 44, 48)
    _subm(_tiny(53, wide, B, 12000), wide, B, 3, 1, "kept marks, larger grid")
    assert _stream_marks().buf.numel() > size


def test_byte_marks_over_a_random_sequence_of_builds(monkeypatch):
    """Thirty SubM and strided builds in a seeded random order on one stream,
    on grids of random shapes (so the kept marks grow now and then) and
    random densities, with the mark values made to run out halfway: every
    build gives the oracle's pairs and output set."""
    from trispconv_amd.pytorch import indices as IM
    monkeypatch.setattr(IM, "_MARKS", IM._ThreadMarks())
    rng = np.random.default_rng(81)
    for step in range(30):
        shape = tuple(int(v) for v in rng.integers(6, 36, size=3))
        B = int(rng.integers(1, 3))
        n = int(rng.integers(1, max(2, shape[0] * shape[1] * shape[2] // 3)))
        idx = _tiny(int(rng.integers(1 << 30)), shape, B, min(n, 2500))
        if step == 15:
            m = _stream_marks()
            if m is not None:
                m.gen = 254
        if rng.random() < 0.5:
            _subm(idx, shape, B, 3, 1, f"random sequence {step}: subm {shape} x{B}")
        else:
            _strided(idx, shape, B, 3, 2, 1, 1, f"random sequence {step}: strided {shape} x{B}")


def test_byte_marks_of_two_host_threads_on_one_stream():
    """Two host threads building on the same stream at once: their launches
    interleave on the stream, so each thread keeps marks of its own; every
    build gives the oracle's pairs."""
    import threading
    shape, B = (20, 22, 24), 2
    sets = [_tiny(71 + t, shape, B, 900 + 300 * t) for t in range(2)]
    exp = [OP.subm_pairs(idx, shape, B, 3, 1) for idx in sets]
    errors = []

    def work(t):
        try:
            x = torch.from_numpy(sets[t]).to(DEV)
            for i in range(12):
                got = generate_subm_indice_pairs(x, shape, B, 3, 1)
                _check_lists(got, exp[t], f"thread {t} build {i}")
        except BaseException as e:  # reported by the main thread
            errors.append(e)

    say("two host threads building on one stream")
    threads = [threading.Thread(target=work, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads)
    assert not errors, errors[0]


def test_byte_marks_through_the_c_abi():
    """tsc_subm_pairs_checked and tsc_strided_count with caller-kept marks and
    a new value per build, against the same builds with the marks in the
    workspace: the same map, counts, output set and status flags."""
    import ctypes
    from trispconv_amd import _lib as L
    lib = L.lib()
    shape, B, K = (20, 22, 24), 2, 27
    args = (L.i3(shape), L.i3((3, 3, 3)), L.i3((1, 1, 1)))
    mb = lib.tsc_subm_marks_bytes(3000, K, B, args[0])
    assert mb > 0
    marks = torch.zeros(mb, dtype=torch.uint8, device=DEV)
    for gen, seed in ((1, 61), (2, 62), (3, 61)):
        idx = _tiny(seed, shape, B, 1500 if seed == 61 else 700)
        if gen == 3:
            idx[7, 0] = -1  # a bad batch index: the flag comes from the marks' status words
        c = torch.from_numpy(idx).to(DEV)
        n = len(idx)
        out = {}
        for mode in ("workspace", "kept"):
            say("byte marks through the C ABI:", mode, "gen", gen, "n", n)
            kept = mode == "kept"
            wsb = lib.tsc_subm_workspace_bytes(n, K, B, args[0], int(kept))
            ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
            cols = torch.empty(n, dtype=torch.int32, device=DEV)
            nbr = torch.empty((K, n), dtype=torch.int32, device=DEV)
            counts = torch.empty(K + 2, dtype=torch.int32, device=DEV)
            blocks = torch.empty(lib.tsc_subm_slot_blocks_len(n, K), dtype=torch.int32,
                                 device=DEV)
            result = (ctypes.c_int32 * 2)()
            L.check(lib.tsc_subm_pairs_checked(
                c.data_ptr(), n, B, *args, ws.data_ptr(), wsb,
                marks.data_ptr() if kept else None, mb if kept else 0, gen if kept else 0,
                cols.data_ptr(), nbr.data_ptr(), counts.data_ptr(), blocks.data_ptr(), 0, result,
                L.stream_of(c)), "checked")
            torch.cuda.synchronize()
            st = (result[0], result[1])
            if st[0] == 0:
                L.check(lib.tsc_subm_counts(blocks.data_ptr(), n, K, counts.data_ptr(), None,
                                            L.stream_of(c)), "counts")
            out[mode] = (st, cols.cpu(), nbr.cpu(), counts.cpu())
        assert out["workspace"][0] == out["kept"][0], gen
        assert (out["kept"][0][0] != 0) == (gen == 3)
        if gen != 3:
            for a, b in zip(out["workspace"][1:], out["kept"][1:]):
                assert torch.equal(a, b), gen
        # strided, same marks and the next value
        sgen = gen + 3
        sh_out = (10, 11, 12)
        geo = (L.i3(shape), L.i3((3, 3, 3)), L.i3((2, 2, 2)), L.i3((1, 1, 1)), L.i3((1, 1, 1)),
               L.i3(sh_out))
        smb = lib.tsc_strided_marks_bytes(n, K, B, geo[5])
        assert 0 < smb <= mb
        res = {}
        for mode in ("workspace", "kept"):
            kept = mode == "kept"
            wsb = lib.tsc_strided_workspace_bytes(n, K, B, geo[5], int(kept))
            ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
            counts = torch.empty(K + 3, dtype=torch.int32, device=DEV)
            L.check(lib.tsc_strided_count(c.data_ptr(), n, B, *geo, ws.data_ptr(), wsb,
                                          marks.data_ptr() if kept else None, mb if kept else 0,
                                          sgen if kept else 0, counts.data_ptr(),
                                          L.stream_of(c)), "strided count")
            h = counts.cpu()
            n_out = int(h[K])
            oc = torch.empty((max(n_out, 1), 4), dtype=torch.int32, device=DEV)
            nb = torch.empty(K * max(n_out, 1), dtype=torch.int32, device=DEV)
            pin = torch.empty((K, n), dtype=torch.int32, device=DEV)
            pout = torch.empty((K, n), dtype=torch.int32, device=DEV)
            L.check(lib.tsc_strided_fill(c.data_ptr(), n, B, *geo, ws.data_ptr(), wsb,
                                         counts.data_ptr(), n_out, oc.data_ptr(), nb.data_ptr(),
                                         pin.data_ptr(), pout.data_ptr(), None, L.stream_of(c)),
                    "strided fill")
            pn = h[:K].tolist()
            res[mode] = (h, oc[:n_out].cpu(), nb[:K * n_out].cpu(),
                         torch.cat([pin[k, :pn[k]] for k in range(K)]).cpu(),
                         torch.cat([pout[k, :pn[k]] for k in range(K)]).cpu())
        for a, b in zip(res["workspace"], res["kept"]):
            assert torch.equal(a, b), ("strided", gen)
        assert (int(res["kept"][0][K + 1]) != 0) == (gen == 3)


# The submanifold builder looks cells up in an occupancy bitmap when the grid
# has at most about 2048 cells per voxel (64 words per voxel + 2^20 words), and in
# a hash table otherwise; both must give the same lists, repeated coordinates
# included.
@pytest.mark.parametrize("shape,what", [((20, 24, 28), "bitmap"), ((640, 320, 200), "hash")])
def test_subm_lookup_paths_with_duplicates(shape, what):
    B, n = 2, 3000
    idx = _clustered_with_duplicates(31, shape, B, n, 16, 300)
    words = -(-B * shape[0] * shape[1] * shape[2] // 32)
    assert (words <= 64 * len(idx) + (1 << 20)) == (what == "bitmap")
    _subm(idx, shape, B, 3, 1, f"{what} path")
    _subm(idx, shape, B, (3, 1, 3), (1, 2, 1), f"{what} path, 3x1x3 dilated")


def test_subm_bitmap_every_cell_occupied():
    """A fully occupied grid whose x extent (37) is not a multiple of 32: every
    lookup at the x borders, and every row of three cells that straddles two
    bitmap words, is exercised; repeated rows on top take the duplicate path."""
    shape, B = (5, 6, 37), 2
    b, z, y, x = np.meshgrid(np.arange(B), np.arange(shape[0]), np.arange(shape[1]),
                             np.arange(shape[2]), indexing="ij")
    idx = np.stack([b, z, y, x], -1).reshape(-1, 4).astype(np.int32)
    rng = np.random.default_rng(5)
    idx = idx[rng.permutation(len(idx))]
    _subm(idx, shape, B, 3, 1, "every cell occupied")
    _subm(idx, shape, B, 3, (1, 1, 2), "every cell occupied, x dilation 2")
    dup = np.concatenate([idx, idx[rng.choice(len(idx), 40)]])
    _subm(dup[rng.permutation(len(dup))], shape, B, 3, 1, "every cell occupied, repeats")


def test_subm_bitmap_long_scan():
    """A bitmap of more than 2048 scan tiles (1024 words each): the tile sums
    are scanned in a pass of their own before the ranks are applied."""
    shape, B, n = (300, 512, 512), 1, 200_000
    words = -(-B * shape[0] * shape[1] * shape[2] // 32)
    assert -(-words // 1024) > 2048 and words <= 64 * n + (1 << 20)
    idx = _clustered_with_duplicates(41, shape, B, n, 64, 0)
    _subm(idx, shape, B, 3, 1, "long bitmap scan")


def test_out_of_grid_coordinates_raise():
    idx = torch.tensor([[0, 1, 1, 1], [0, 9, 1, 1]], dtype=torch.int32, device=DEV)
    with pytest.raises(IndexError):
        generate_subm_indice_pairs(idx, (4, 4, 4), 1, 3)
    idx = torch.tensor([[0, 1, 1, 1], [3, 1, 1, 1]], dtype=torch.int32, device=DEV)
    with pytest.raises(IndexError):
        generate_subm_indice_pairs(idx, (4, 4, 4), 2, 3)
    with pytest.raises(IndexError):
        generate_strided_indice_pairs(idx, (4, 4, 4), 2, 3, 2, 1)


@pytest.mark.parametrize("name", workloads.WORKLOAD_NAMES)
def test_pairs_full_size_workloads(name):
    w = workloads.make_workload(name)
    idx, shape, B = w.indices, w.spatial_shape, w.batch_size
    lay = w.layers[0]
    if lay["kind"] == "subm":
        _subm(idx, shape, B, lay["kernel_size"], lay["dilation"], name)
    else:
        g, e = _strided(idx, shape, B, lay["kernel_size"], lay["stride"], lay["padding"],
                        lay["dilation"], name)
        if len(w.layers) > 1 and w.layers[1]["kind"] == "inverse":
            _inverse(g, e, name + "/inverse")


@pytest.mark.parametrize("k,d", [(3, 1), (3, 2), ((3, 1, 3), 1), ((1, 3, 3), (2, 1, 1)), (5, 1)])
def test_subm_on_a_strided_output_probes_its_bitmap(k, d, monkeypatch):
    """A submanifold build on a strided build's output coordinates runs on the
    strided build's bitmap (kernels 3 wide in x) and gives the oracle's pairs;
    other kernels, or coordinates changed since, take the ordinary build."""
    from trispconv_amd.pytorch import indices as I
    used = []
    reallib = I.L.lib()
    real = reallib.tsc_subm_pairs_from_bitmap

    class Spy:
        def __getattr__(self, name):
            fn = getattr(reallib, name)
            if name == "tsc_subm_pairs_from_bitmap":
                def wrapped(*a):
                    used.append(1)
                    return real(*a)
                return wrapped
            return fn

    monkeypatch.setattr(I.L, "lib", lambda spy=Spy(): spy)
    idx = _tiny(41, (17, 18, 19), 2, 900)
    fwd = generate_strided_indice_pairs(torch.from_numpy(idx).to(DEV), (17, 18, 19), 2, 3, 2, 1)
    out = fwd.out_indices
    shape = tuple(fwd.output_spatial_shape)
    got = generate_subm_indice_pairs(out, shape, 2, k, d)
    ks = (k, k, k) if isinstance(k, int) else k
    assert bool(used) == (ks[2] == 3), (k, d)
    exp = OP.subm_pairs(out.cpu().numpy(), shape, 2, k, d)
    _check_lists(got, exp, f"subm on strided output k={k} d={d}")
    used.clear()
    out.add_(0)  # in place: no longer known to be the strided build's output
    again = generate_subm_indice_pairs(out, shape, 2, k, d)
    assert not used
    _check_lists(again, exp, f"subm on changed coordinates k={k} d={d}")


def test_bitmap_build_flags_rows_that_are_not_its_cells():
    """Rows that are only part of the bitmap's cells: neighbours ranked past
    the rows are left out of the map (no entry names a row that does not
    exist) and the status flag says so."""
    from trispconv_amd import _lib as L
    from trispconv_amd.pytorch import indices as I
    idx = _tiny(43, (17, 18, 19), 1, 900)
    fwd = generate_strided_indice_pairs(torch.from_numpy(idx).to(DEV), (17, 18, 19), 1, 3, 2, 1)
    ws, nwords, shape, B = I._STRIDED_BITMAPS[fwd.out_indices][:4]
    half = fwd.out_indices[: len(fwd.out_indices) // 2].contiguous()
    n = len(half)
    cols_row = torch.empty(n, dtype=torch.int32, device=DEV)
    nbr = torch.empty((27, n), dtype=torch.int32, device=DEV)
    counts = torch.empty(29, dtype=torch.int32, device=DEV)
    lib = L.lib()
    L.check(lib.tsc_subm_pairs_from_bitmap(half.data_ptr(), n, B, L.i3(shape), L.i3((3, 3, 3)),
                                           L.i3((1, 1, 1)), ws.data_ptr(), nwords,
                                           cols_row.data_ptr(), nbr.data_ptr(),
                                           counts.data_ptr(), 0, L.stream_of(half)), "bitmap build")
    host = counts.cpu()
    assert int(host[27]) & L.FLAG_ROWS_NOT_BITMAP
    assert int(nbr.max()) < n


def test_bitmap_build_on_permuted_rows_raises_at_first_reuse():
    """The strided output coordinates permuted in place through ``.data``
    (same tensor, address and version counter: a write the reuse key cannot
    see).  The build on the strided bitmap checks every row's own cell rank on
    the device, and the first reuse of the pairs under their key reads that
    flag and raises."""
    import trispconv.pytorch as spconv
    idx = _tiny(47, (17, 18, 19), 2, 900)
    fwd = generate_strided_indice_pairs(torch.from_numpy(idx).to(DEV), (17, 18, 19), 2, 3, 2, 1)
    out = fwd.out_indices
    shape = tuple(fwd.output_spatial_shape)
    # unpermuted: the pairs' first reuse reads a clean flag
    ok = generate_subm_indice_pairs(out, shape, 2, 3)
    assert ok._deferred_check
    conv = spconv.SubMConv3d(8, 8, 3, indice_key="s").to(DEV)
    x = spconv.SparseConvTensor(torch.randn(len(out), 8, device=DEV), out, list(shape), 2)
    x.indice_dict["s"] = ok
    conv(conv(x))
    assert not ok._deferred_check
    perm = torch.randperm(len(out), generator=torch.Generator().manual_seed(0)).to(DEV)
    version = out._version
    out.data.copy_(out.data[perm])
    assert out._version == version
    say("bitmap build on permuted rows")
    bad = generate_subm_indice_pairs(out, shape, 2, 3)
    assert bad._deferred_check  # still taken for the registered output set
    x = spconv.SparseConvTensor(torch.randn(len(out), 8, device=DEV), out, list(shape), 2)
    x.indice_dict["s"] = bad
    y = conv(x)
    with pytest.raises(RuntimeError, match="not the rows"):
        conv(y)


def _map_by_rows(lib, L, nbr_cols, cols_row, n, K):
    """A column map in row order (tsc_map_to_rows): comparable across builds
    that place the columns of repeated coordinates in different orders."""
    rows = torch.full((K, n), -7, dtype=torch.int32, device=DEV)
    L.check(lib.tsc_map_to_rows(nbr_cols.data_ptr(), cols_row.data_ptr(), n, n, K, rows.data_ptr(),
                                L.stream_of(rows)), "map_to_rows")
    return rows


@pytest.mark.parametrize("shape,dups,what", [((20, 24, 28), 0, "bitmap"),
                                             ((20, 24, 28), 300, "bitmap, repeats"),
                                             ((640, 320, 200), 300, "hash, repeats")])
def test_checked_build_matches_the_plain_build(shape, dups, what):
    """tsc_subm_pairs_checked (returns at the coordinate check; counts summed
    by tsc_subm_counts) against tsc_subm_pairs, through the C ABI: the same
    map row by row, the same counts, status and column order."""
    import ctypes

    from trispconv_amd import _lib as L
    lib = L.lib()
    B, K = 2, 27
    idx = _clustered_with_duplicates(7, shape, B, 3000, 16, dups)
    say("checked vs plain subm build:", what, idx.shape)
    c = torch.from_numpy(idx).to(DEV)
    n = len(idx)
    args = (L.i3(shape), L.i3((3, 3, 3)), L.i3((1, 1, 1)))
    ws_bytes = lib.tsc_subm_workspace_bytes(n, K, B, args[0], 0)
    out = {}
    for mode in ("plain", "checked"):
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        cols = torch.empty(n, dtype=torch.int32, device=DEV)
        nbr_all = torch.full(((K + 1) * n,), -3, dtype=torch.int32, device=DEV)
        nbr = nbr_all[:K * n].view(K, n)
        counts = torch.full((K + 2,), -5, dtype=torch.int32, device=DEV)
        s = L.stream_of(c)
        if mode == "plain":
            L.check(lib.tsc_subm_pairs(c.data_ptr(), n, B, *args, ws.data_ptr(), ws_bytes,
                                       cols.data_ptr(), nbr.data_ptr(), counts.data_ptr(), s),
                    "plain")
            host = counts.cpu().tolist()
        else:
            blocks = torch.empty(lib.tsc_subm_slot_blocks_len(n, K), dtype=torch.int32, device=DEV)
            result = (ctypes.c_int32 * 2)()
            L.check(lib.tsc_subm_pairs_checked(c.data_ptr(), n, B, *args, ws.data_ptr(), ws_bytes,
                                               None, 0, 0, cols.data_ptr(), nbr.data_ptr(),
                                               counts.data_ptr(),
                                               blocks.data_ptr(), 1, result, s), "checked")
            assert result[0] == 0, what
            if result[1]:  # columns in (b,z,y,x) order: row K holds their slot masks
                bits = (nbr >= 0).to(torch.int64) << torch.arange(K, device=DEV).view(K, 1)
                want = bits.sum(0).to(torch.int32)
                assert torch.equal(nbr_all[K * n:], want), f"{what}: slot-mask row"
            h = (ctypes.c_int32 * (K + 2))()
            L.check(lib.tsc_subm_counts(blocks.data_ptr(), n, K, counts.data_ptr(), h, s),
                    "counts")
            host = list(h)
            assert counts.cpu().tolist() == host, f"{what}: device and host counts"
            assert result[1] == host[K + 1], f"{what}: column order flag"
        out[mode] = (host, _map_by_rows(lib, L, nbr, cols, n, K).cpu())
    assert out["plain"][0] == out["checked"][0], f"{what}: counts"
    assert torch.equal(out["plain"][1], out["checked"][1]), f"{what}: map"
    exp = OP.subm_pairs(idx, shape, B, 3, 1)
    assert out["checked"][0][:K] == exp.pair_num.tolist(), f"{what}: counts vs oracle"


def test_checked_build_reports_bad_coordinates():
    """The early check reports a row outside the grid (and which kind) before
    the build's kernels have finished; the Python build raises IndexError."""
    import ctypes

    from trispconv_amd import _lib as L
    lib = L.lib()
    shape, K = (8, 8, 8), 27
    for bad, flag in (([0, 8, 1, 1], L.FLAG_COORD_OUT_OF_GRID),
                      ([3, 1, 1, 1], L.FLAG_BATCH_OUT_OF_RANGE)):
        idx = np.array([[0, 1, 1, 1], [0, 2, 2, 2], bad, [0, 1, 2, 1]], np.int32)
        say("checked build, bad row:", bad)
        c = torch.from_numpy(idx).to(DEV)
        n = len(idx)
        args = (L.i3(shape), L.i3((3, 3, 3)), L.i3((1, 1, 1)))
        ws_bytes = lib.tsc_subm_workspace_bytes(n, K, 1, args[0], 0)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        cols = torch.empty(n, dtype=torch.int32, device=DEV)
        nbr = torch.empty((K, n), dtype=torch.int32, device=DEV)
        counts = torch.empty(K + 2, dtype=torch.int32, device=DEV)
        blocks = torch.empty(lib.tsc_subm_slot_blocks_len(n, K), dtype=torch.int32, device=DEV)
        result = (ctypes.c_int32 * 2)()
        L.check(lib.tsc_subm_pairs_checked(c.data_ptr(), n, 1, *args, ws.data_ptr(), ws_bytes,
                                           None, 0, 0, cols.data_ptr(), nbr.data_ptr(),
                                           counts.data_ptr(),
                                           blocks.data_ptr(), 0, result, L.stream_of(c)),
                "checked")
        assert result[0] == flag, bad
        with pytest.raises(IndexError):
            generate_subm_indice_pairs(c, shape, 1, 3, 1)
    torch.cuda.synchronize()


@pytest.mark.parametrize("name", ["inverse_blob4x150k", "strided64_lidar2x200k"])
def test_inverse_from_forward_ids_matches_the_counted_inverse(name):
    """tsc_inverse_fill_ids (the ids the strided fill wrote) against
    tsc_inverse_count + tsc_inverse_fill, through the C ABI, on a reduced
    workload: out_coords, the map and the remapped ids bit for bit."""
    from trispconv_amd import _lib as L
    lib = L.lib()
    w = workloads.make_workload(name, scale=0.05)
    lay = w.layers[0]
    say("inverse from forward ids:", name, w.indices.shape)
    x = torch.from_numpy(w.indices).to(DEV)
    fwd = generate_strided_indice_pairs(x, w.spatial_shape, w.batch_size, lay["kernel_size"],
                                        lay["stride"], lay["padding"], lay["dilation"])
    assert fwd._in_ids is not None
    K, cap, n_in = fwd.K, fwd._pin.shape[1], len(w.indices)
    s = L.stream_of(x)
    ws = torch.empty(lib.tsc_inverse_workspace_bytes(n_in), dtype=torch.uint8, device=DEV)
    counts = torch.empty(1, dtype=torch.int32, device=DEV)
    L.check(lib.tsc_inverse_count(fwd._pin.data_ptr(), fwd._cnt.data_ptr(), K, cap, n_in,
                                  ws.data_ptr(), ws.numel(), counts.data_ptr(), s), "count")
    n_out = int(counts.cpu()[0])
    assert n_out == fwd._n_in_paired
    ids = fwd._in_ids.cpu().numpy()
    assert int((ids >= 0).sum()) == n_out
    assert np.array_equal(ids[ids >= 0], np.arange(n_out)), "ids ascend with the rows"
    res = {}
    for mode in ("count", "ids"):
        oc = torch.empty((n_out, 4), dtype=torch.int32, device=DEV)
        nbr = torch.empty((K, n_out), dtype=torch.int32, device=DEV)
        ipo = torch.full((K, cap), -9, dtype=torch.int32, device=DEV)
        if mode == "count":
            L.check(lib.tsc_inverse_fill(fwd._pin.data_ptr(), fwd._pout.data_ptr(),
                                         fwd._cnt.data_ptr(), K, cap, x.data_ptr(), n_in,
                                         ws.data_ptr(), ws.numel(), n_out, oc.data_ptr(),
                                         nbr.data_ptr(), ipo.data_ptr(), s), "fill")
        else:
            L.check(lib.tsc_inverse_fill_ids(fwd._pin.data_ptr(), fwd._pout.data_ptr(),
                                             fwd._cnt.data_ptr(), K, cap, fwd._in_ids.data_ptr(),
                                             x.data_ptr(), n_in, n_out, oc.data_ptr(),
                                             nbr.data_ptr(), ipo.data_ptr(), s), "fill_ids")
        res[mode] = (oc.cpu(), nbr.cpu(), ipo.cpu())
    pn = fwd.pair_num.tolist()
    for a, b, what in zip(res["count"], res["ids"], ("out_coords", "map", "ids")):
        if what == "ids":  # only each slot's first pair_num[k] entries are written
            a = torch.cat([a[k, :pn[k]] for k in range(K)])
            b = torch.cat([b[k, :pn[k]] for k in range(K)])
        assert torch.equal(a, b), f"{name}: {what}"


def test_pair_counts_read_on_the_build_stream():
    """A submanifold build leaves its counts on the device; pair_num, read
    later while another stream is current (and busy), sums and reads them on
    the stream the build ran on, and equals the oracle's."""
    w = workloads.make_workload("subm128_surface500k", scale=0.05)
    idx = w.indices
    say("pair counts across streams:", idx.shape)
    s_build, s_other = torch.cuda.Stream(), torch.cuda.Stream()
    x = torch.from_numpy(idx).to(DEV)
    torch.cuda.synchronize()
    with torch.cuda.stream(s_build):
        got = generate_subm_indice_pairs(x, w.spatial_shape, 1, 3, 1)
    with torch.cuda.stream(s_other):
        torch.cuda._sleep(2_000_000)  # keep the other stream busy meanwhile
        pn = got.pair_num
    exp = OP.subm_pairs(idx, w.spatial_shape, 1, 3, 1)
    assert pn.tolist() == exp.pair_num.tolist()
    torch.cuda.synchronize()


def test_sparse_bitmap_skips_untouched_tiles():
    """A grid sparse enough for the atomically marked bitmap (more than 64
    cells per voxel): only the 1024-word tiles holding a row's cell are
    zeroed, scanned and ranked, and probes read the others as empty.  Small
    clusters straddle tile boundaries (y = 64k and z planes), with repeated
    rows on top; the pairs must equal the oracle's."""
    shape, B = (64, 512, 512), 2
    cells = B * shape[0] * shape[1] * shape[2]
    rng = np.random.default_rng(17)
    parts = []
    for b in range(B):
        for _ in range(12):
            # a 6^3 box around a tile boundary (y multiple of 64) or a z plane
            z0 = int(rng.integers(1, shape[0] - 7))
            y0 = int(rng.choice([63, 127, 255, 447])) - 3
            x0 = int(rng.integers(0, shape[2] - 6))
            zz, yy, xx = np.meshgrid(np.arange(6), np.arange(6), np.arange(6), indexing="ij")
            box = np.stack([np.full(216, b), (z0 + zz).ravel(), (y0 + yy).ravel(),
                            (x0 + xx).ravel()], 1)
            parts.append(box[rng.random(216) < 0.6])
    idx = np.unique(np.concatenate(parts).astype(np.int32), axis=0)
    idx = np.concatenate([idx, idx[rng.choice(len(idx), 50)]])
    idx = idx[rng.permutation(len(idx))]
    n = len(idx)
    words = -(-cells // 32)
    assert cells > 64 * n and words <= 64 * n + (1 << 20)  # the atomically marked bitmap
    _subm(idx, shape, B, 3, 1, "sparse bitmap, untouched tiles")
    _subm(idx, shape, B, 3, (2, 2, 1), "sparse bitmap, dilated")
