"""tsc_subm_pairs_noalloc against tsc_subm_pairs, through the C ABI.

The no-allocation entry point runs the same submanifold build on a fixed
device array instead of a caller's workspace.  Its outputs (the neighbour map
by columns, the column -> row table and the counts with their status flags)
must equal tsc_subm_pairs' bit for bit: two calls in a row, the second on a
smaller input (the array keeps the first call's contents, which the build
must clear), both on a bitmap-sized grid and on a sparse grid (the hash
build), then a grid whose bitmap is larger than the array (the build falls
back to the hash and agrees with the workspace build's row-order map), and a
build larger than the array in either form (an argument error, nothing
launched).
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import DEV, needs_gpu, say
from oracle import pairs as OP
from trispconv_amd import _lib as L

pytestmark = [pytest.mark.gpu, needs_gpu]


def _cloud(seed, shape, B, n):
    rng = np.random.default_rng(seed)
    total = shape[0] * shape[1] * shape[2]
    parts = []
    for b in range(B):
        cells = rng.choice(total, size=n, replace=False)
        z, r = np.divmod(cells, shape[1] * shape[2])
        y, x = np.divmod(r, shape[2])
        parts.append(np.stack([np.full(n, b), z, y, x], 1))
    idx = np.concatenate(parts).astype(np.int32)
    return idx[rng.permutation(len(idx))]


def _outputs(n, K):
    return (torch.full((max(n, 1),), -7, dtype=torch.int32, device=DEV),
            torch.full((K, max(n, 1)), -7, dtype=torch.int32, device=DEV),
            torch.full((K + 2,), -7, dtype=torch.int32, device=DEV))


def _with_workspace(c, B, shape, ks, dil):
    lib = L.lib()
    n, K = c.shape[0], ks[0] * ks[1] * ks[2]
    ws = L.workspace(lib.tsc_subm_workspace_bytes(n, K, B, L.i3(shape), 0), DEV)
    cols_row, nbr, counts = _outputs(n, K)
    L.check(lib.tsc_subm_pairs(c.data_ptr(), n, B, L.i3(shape), L.i3(ks), L.i3(dil),
                               ws.data_ptr(), ws.numel(), cols_row.data_ptr(), nbr.data_ptr(),
                               counts.data_ptr(), L.stream_of(c)), "subm")
    return cols_row, nbr, counts


def _no_alloc(c, B, shape, ks, dil):
    lib = L.lib()
    n, K = c.shape[0], ks[0] * ks[1] * ks[2]
    cols_row, nbr, counts = _outputs(n, K)
    L.check(lib.tsc_subm_pairs_noalloc(c.data_ptr(), n, B, L.i3(shape), L.i3(ks), L.i3(dil),
                                       cols_row.data_ptr(), nbr.data_ptr(), counts.data_ptr(),
                                       L.stream_of(c)), "subm noalloc")
    return cols_row, nbr, counts


def _rows_map(cols_row, nbr, n):
    """The map in row order (columns may be cells in raster order)."""
    out = torch.full((nbr.shape[0], n), -1, dtype=torch.int32, device=DEV)
    cr = cols_row[:n].long()
    ok = cr >= 0
    out[:, cr[ok]] = nbr[:, :n][:, ok]
    return out


# (shape, batch, voxels first, voxels second, kernel, dilation)
CASES = [
    ((40, 40, 40), 2, 9000, 3000, (3, 3, 3), (1, 1, 1)),     # bitmap, 3x3x3 rows probe
    ((30, 36, 33), 1, 4000, 1500, (3, 1, 3), (2, 1, 1)),     # bitmap, other 3-wide kernel
    ((25, 22, 28), 2, 2500, 800, (5, 3, 2), (1, 1, 1)),      # bitmap, generic probe
    ((600, 700, 800), 2, 6000, 2500, (3, 3, 3), (1, 1, 1)),  # sparse: the hash build
]


@pytest.mark.parametrize("shape,B,n1,n2,ks,dil", CASES)
def test_noalloc_equals_workspace_build_twice(shape, B, n1, n2, ks, dil):
    for call, n in enumerate((n1, n2)):
        idx = _cloud(100 + call + n, shape, B, n // B)
        c = torch.from_numpy(idx).to(DEV)
        say("noalloc call", call, shape, B, len(idx), ks, dil)
        a = _with_workspace(c, B, shape, ks, dil)
        b = _no_alloc(c, B, shape, ks, dil)
        torch.cuda.synchronize()
        for x, y, what in zip(a, b, ("cols_row", "map", "counts")):
            assert torch.equal(x, y), what
        exp = OP.subm_pairs(idx, shape, B, ks, dil)
        assert b[2][: len(exp.pair_num)].cpu().numpy().tolist() == exp.pair_num.tolist()


def test_noalloc_falls_back_to_the_hash_when_the_bitmap_does_not_fit():
    lib = L.lib()
    limit = lib.tsc_subm_pairs_noalloc_limit()
    assert limit > 0
    # 4 x 41 x 1600 x 1408 cells (a 92 MiB bitmap) with enough voxels that
    # the workspace build takes the bitmap: the fixed scratch only holds the
    # hash
    shape, B = (41, 1600, 1408), 4
    for call, n in enumerate((200000, 170000)):
        idx = _cloud(7 + call, shape, B, n // B)
        c = torch.from_numpy(idx).to(DEV)
        say("noalloc fallback call", call, len(idx))
        cr_a, nbr_a, cnt_a = _with_workspace(c, B, shape, (3, 3, 3), (1, 1, 1))
        cr_b, nbr_b, cnt_b = _no_alloc(c, B, shape, (3, 3, 3), (1, 1, 1))
        assert int(cnt_a[28]) == 1 and int(cnt_b[28]) == 0  # raster columns / rows
        assert torch.equal(cnt_a[:28], cnt_b[:28])
        n_rows = len(idx)
        assert torch.equal(_rows_map(cr_a, nbr_a, n_rows), _rows_map(cr_b, nbr_b, n_rows))


def test_noalloc_rejects_builds_beyond_its_scratch():
    lib = L.lib()
    limit = lib.tsc_subm_pairs_noalloc_limit()
    # a hash table of 16 bytes per slot and at least 2n slots: past the limit
    n = int(limit // 16) + 1024
    B, shape = 1, (1 << 12, 1 << 12, 1 << 12)
    c = torch.zeros((n, 4), dtype=torch.int32, device=DEV)
    # outputs sized for the n rows: were the size check ever to let the call
    # through, the kernels would still write inside them
    cols_row, nbr, counts = _outputs(n, 27)
    rc = lib.tsc_subm_pairs_noalloc(c.data_ptr(), n, B, L.i3(shape), L.i3((3, 3, 3)),
                                    L.i3((1, 1, 1)), cols_row.data_ptr(), nbr.data_ptr(),
                                    counts.data_ptr(), L.stream_of(c))
    assert rc > 0
    assert b"scratch" in lib.tsc_last_error()
