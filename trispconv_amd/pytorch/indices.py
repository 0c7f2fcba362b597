"""Indice-pair generation on the GPU (submanifold, strided, inverse).

Public names and semantics follow trispconv/pytorch/indices.py:10-259 and the
inverse remap of modules.py:175-212; the work runs in libtrispconv_hip.so.

``IndiceData`` keeps the reference's fields.  Pair lists are stored on the
device as padded int32 tables (slot k owns ``[k, :pair_num[k]]``) next to the
output-major neighbour map the convolution reads; the reference-style lists
of K int64 tensors are materialised on first access to ``pairs_in`` /
``pairs_out``.  ``pair_num`` is a CPU int64 tensor, as in the reference
(indices.py:131), read with the one device-to-host copy each build makes.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch
from torch.utils.weak import WeakIdKeyDictionary

from .. import _lib as L

__all__ = [
    "IndiceData",
    "generate_subm_indice_pairs",
    "generate_strided_indice_pairs",
    "generate_inverse_indice_pairs",
]

# The execution-order sort pays off on large layers only.  Measured: it halves
# the 166k-row 64-channel fp32 strided layer and cuts the 500k-row 128-channel
# SubM layer by 20% and the 674k-row 32-channel one by 30% (gathered input
# 43-128 MiB), but leaves layers of up to 240k rows with 16-64 channels
# (gathered input up to 16 MiB) no faster or slower, while its own cost
# (tens of launches) dominates a network's first pass over new coordinates.
_PLAN_MIN_ROWS = 2048
_PLAN_MIN_BYTES = 24 << 20  # output rows x gathered row bytes
# Half of MI355X's 256 MiB Infinity Cache: the execution order sorts rows by
# slot mask within regions whose gathered input rows fit in it.  Measured on
# the 500k-voxel 128-channel layer: larger regions group rows with equal slot
# sets better and beat L2-sized (4 MiB) regions despite the longer reuse
# distance, since the cache behind L2 still holds the gathered rows.
_REGION_BYTES = 128 << 20


def _to3(x) -> Tuple[int, int, int]:
    """indices.py:26-29."""
    if isinstance(x, int):
        return (x, x, x)
    return tuple(int(v) for v in x)


def _output_spatial_shape(in_shape, kernel_size, stride, padding, dilation) -> Tuple[int, int, int]:
    """(S + 2p - d(k-1) - 1) // s + 1 per axis — indices.py:32-42."""
    return tuple((s + 2 * p - d * (k - 1) - 1) // st + 1
                 for s, k, st, p, d in zip(in_shape, kernel_size, stride, padding, dilation))


def _encode_coords(indices: torch.Tensor, D: int, H: int, W: int) -> torch.Tensor:
    """(b, z, y, x) -> b*DHW + z*HW + y*W + x as int64 — indices.py:45-51."""
    i = indices.long()
    return i[:, 0] * (D * H * W) + i[:, 1] * (H * W) + i[:, 2] * W + i[:, 3]


class IndiceData:
    """Pairs of one layer (indices.py:10-23), backed by device tables."""

    def __init__(self, out_indices: torch.Tensor, pairs_in: Optional[List[torch.Tensor]],
                 pairs_out: Optional[List[torch.Tensor]], pair_num: torch.Tensor,
                 input_indices: torch.Tensor, input_spatial_shape, output_spatial_shape,
                 kernel_size, stride, padding, dilation, subm: bool):
        self.out_indices = out_indices
        self.input_indices = input_indices
        self.input_spatial_shape = tuple(input_spatial_shape)
        self.output_spatial_shape = tuple(output_spatial_shape)
        self.kernel_size = tuple(kernel_size)
        self.stride = tuple(stride)
        self.padding = tuple(padding)
        self.dilation = tuple(dilation)
        self.subm = subm
        self.pair_num = pair_num
        # a build whose counts stay on the device until pair_num is read:
        # (counts [K + 1] int32, K); counts[K] holds the build's status flags
        self._counts_pending: Optional[Tuple[torch.Tensor, int]] = None
        self._pairs_in = pairs_in
        self._pairs_out = pairs_out
        # device tables
        self._pin: Optional[torch.Tensor] = None    # [K][cap] int32
        self._pout: Optional[torch.Tensor] = None   # [K][cap] int32
        self._cnt: Optional[torch.Tensor] = None    # [K] int32 on the device
        self._nbr: Optional[torch.Tensor] = None    # [K][n_out] int32, by output row
        # the builder's map by columns: column t belongs to row _cols_row[t];
        # _raster says the columns are in (b,z,y,x) order
        self._map_cols: Optional[torch.Tensor] = None
        self._cols_row: Optional[torch.Tensor] = None
        self._raster = False
        # the output rows themselves are in (b,z,y,x) order (strided builds
        # emit the sorted unique output set)
        self._rows_raster = False
        self._order: Optional[torch.Tensor] = None  # [n_out] int32 execution order
        self._inverse_cache: Optional["IndiceData"] = None
        self._order_region = 0
        self._nbr_ordered: Optional[torch.Tensor] = None
        self._batch_size: Optional[int] = None
        # strided builds: input rows with at least one pair, i.e. the row
        # count of this layer's inverse, read with the build's counts
        self._n_in_paired: Optional[int] = None

    @property
    def pair_num(self) -> torch.Tensor:
        """Pairs per slot, a CPU int64 tensor (indices.py:131).  A build that
        left its counts on the device (a submanifold build on a strided
        layer's bitmap, which has no coordinates to check) is read here, on
        first access, so the forward pass does not wait for it."""
        if self._pair_num is None and self._counts_pending is not None:
            counts, K = self._counts_pending
            host = counts.cpu()
            if int(host[K]) & L.FLAG_ROWS_NOT_BITMAP:
                raise RuntimeError("generate_subm_indice_pairs: coordinates are not the rows of "
                                   "the strided build they were registered with")
            self._pair_num = host[:K].long()
            self._counts_pending = None
        return self._pair_num

    @pair_num.setter
    def pair_num(self, value: torch.Tensor) -> None:
        self._pair_num = value
        self._counts_pending = None

    # --------------------------------------------------- construction
    @classmethod
    def _from_tables(cls, *, out_indices, input_indices, input_spatial_shape, output_spatial_shape,
                     kernel_size, stride, padding, dilation, subm, pin, pout, cnt_dev,
                     pair_num, nbr, batch_size, map_cols=None, cols_row=None,
                     raster=False, rows_raster=False) -> "IndiceData":
        d = cls(out_indices, None, None, pair_num, input_indices, input_spatial_shape,
                output_spatial_shape, kernel_size, stride, padding, dilation, subm)
        d._pin, d._pout, d._cnt, d._nbr = pin, pout, cnt_dev, nbr
        d._map_cols, d._cols_row, d._raster = map_cols, cols_row, bool(raster)
        d._rows_raster = bool(rows_raster)
        d._batch_size = batch_size
        return d

    # --------------------------------------------------- reference fields
    @property
    def K(self) -> int:
        k = self.kernel_size
        return int(k[0]) * int(k[1]) * int(k[2])

    @property
    def pairs_in(self) -> List[torch.Tensor]:
        if self._pairs_in is None:
            self._ensure_tables()
            self._pairs_in = self._slot_views(self._pin)
        return self._pairs_in

    @pairs_in.setter
    def pairs_in(self, value: List[torch.Tensor]) -> None:
        self._pairs_in = value
        self._drop_tables()

    @property
    def pairs_out(self) -> List[torch.Tensor]:
        if self._pairs_out is None:
            self._ensure_tables()
            self._pairs_out = self._slot_views(self._pout)
        return self._pairs_out

    @pairs_out.setter
    def pairs_out(self, value: List[torch.Tensor]) -> None:
        self._pairs_out = value
        self._drop_tables()

    def _slot_views(self, table: Optional[torch.Tensor]) -> List[torch.Tensor]:
        if table is None:
            raise RuntimeError("IndiceData has neither pair lists nor device tables")
        counts = [int(c) for c in self.pair_num.tolist()]
        return [table[k, :c].long() for k, c in enumerate(counts)]

    def _ensure_tables(self) -> None:
        """Padded pair tables from the builder's map (made on first use: the
        convolution itself reads the map)."""
        if self._pin is not None or self._map_cols is None:
            return
        n_out = len(self.out_indices)
        nbr = self.neighbour_map(n_out, self._map_cols.device)
        lib = L.lib()
        K = self.K
        ws = L.workspace(lib.tsc_pairs_from_map_workspace_bytes(n_out, K), nbr.device)
        pin = torch.empty((K, max(n_out, 1)), dtype=torch.int32, device=nbr.device)
        pout = torch.empty_like(pin)
        L.check(lib.tsc_pairs_from_map(nbr.data_ptr(), n_out, K, pin.shape[1], ws.data_ptr(),
                                       ws.numel(), pin.data_ptr(), pout.data_ptr(),
                                       L.stream_of(nbr)), "pair lists")
        self._pin, self._pout = pin, pout
        self._cnt = self.pair_num.to(device=nbr.device, dtype=torch.int32)

    def _drop_tables(self) -> None:
        self._pin = self._pout = self._cnt = self._nbr = self._order = None
        self._map_cols = self._cols_row = None
        self._raster = False
        self._nbr_ordered = None
        self._inverse_cache = None

    # --------------------------------------------------- convolution inputs
    def neighbour_map(self, n_out: int, device) -> torch.Tensor:
        """[K][n_out] int32: input row feeding output row o through slot k, or -1."""
        if self._nbr is None and self._map_cols is not None:
            if not self._raster:  # the builder's columns are the rows in order
                self._nbr = self._map_cols
            else:
                nbr = torch.full((self.K, n_out), -1, dtype=torch.int32, device=device)
                L.check(L.lib().tsc_map_to_rows(self._map_cols.data_ptr(), self._cols_row.data_ptr(),
                                                self._map_cols.shape[1], n_out, self.K,
                                                nbr.data_ptr(), L.stream_of(nbr)), "map to rows")
                self._nbr = nbr
        if self._nbr is None:
            # user-built lists: scatter them into a map (each slot maps an
            # output at most once, as every generator guarantees)
            K = self.K
            nbr = torch.full((K, n_out), -1, dtype=torch.int32, device=device)
            for k, (pi, po) in enumerate(zip(self.pairs_in, self.pairs_out)):
                if pi.numel():
                    nbr[k, po.to(device).long()] = pi.to(device).int()
            self._nbr = nbr
        return self._nbr

    def execution_order(self, n_out: int, device, row_bytes: int = 256) -> Optional[torch.Tensor]:
        """Processing order of the output rows for the fused convolution.

        Morton order cut into regions whose gathered input rows (``row_bytes``
        each) fit in half the Infinity Cache, each region sorted by slot mask,
        then its whole 256-row tiles put in decreasing number of slots used
        (the partial tile last).  Built once per region size and cached; None
        for small layers.
        """
        if n_out < _PLAN_MIN_ROWS or n_out * int(row_bytes) < _PLAN_MIN_BYTES:
            return None
        region = int(min(max(_REGION_BYTES // max(int(row_bytes), 1), 2048), 1 << 30))
        if self._order is None or self._order_region != region:
            if self._map_cols is not None:  # the builder's columns, maybe in spatial order
                nbr, cols_row, raster = self._map_cols, self._cols_row, self._raster
            else:
                nbr, cols_row, raster = self.neighbour_map(n_out, device), None, self._rows_raster
            coords = None if raster else _coords(self.out_indices, "conv plan")
            lib = L.lib()
            ws = L.workspace(lib.tsc_plan_workspace_bytes(n_out, self.K), device)
            order = torch.empty(n_out, dtype=torch.int32, device=device)
            nbr_ordered = torch.empty_like(nbr)
            L.check(lib.tsc_conv_plan(nbr.data_ptr(), L.ptr(cols_row), int(raster), L.ptr(coords),
                                      n_out, self.K, self._batch_bound(),
                                      L.i3(self.output_spatial_shape), region, ws.data_ptr(),
                                      ws.numel(), order.data_ptr(), nbr_ordered.data_ptr(),
                                      L.stream_of(nbr)), "conv plan")
            self._order, self._order_region, self._nbr_ordered = order, region, nbr_ordered
        return self._order

    def conv_operands(self, n_out: int, device, row_bytes: int = 256):
        """(map, order, ordered) for the fused convolution: the planned order
        and its permuted map; for small layers the builder's own spatial
        column order when it has one; else the row-major map."""
        order = self.execution_order(n_out, device, row_bytes)
        if order is not None:
            return self._nbr_ordered, order, True
        if self._map_cols is not None and self._raster:
            return self._map_cols, self._cols_row, True
        return self.neighbour_map(n_out, device), None, False

    def ordered_map(self) -> Optional[torch.Tensor]:
        """The neighbour map permuted into the execution order (None without one)."""
        return self._nbr_ordered if self._order is not None else None

    def _batch_bound(self) -> int:
        if self._batch_size is None:
            oi = self.out_indices
            self._batch_size = int(oi[:, 0].max()) + 1 if len(oi) else 1
        return max(int(self._batch_size), 1)

    def __repr__(self) -> str:
        return (f"IndiceData(subm={self.subm}, K={self.K}, n_out={len(self.out_indices)}, "
                f"pairs={int(self.pair_num.sum()) if self.pair_num.numel() else 0})")


def _coords(indices: torch.Tensor, what: str) -> torch.Tensor:
    L.require_gpu(indices, what)
    if indices.ndim != 2 or indices.shape[1] != 4:
        raise ValueError(f"{what}: indices must be (N, 4) (b, z, y, x), got {tuple(indices.shape)}")
    coords = indices.to(torch.int32).contiguous()
    if coords.data_ptr() % 16:
        coords = coords.clone()  # the kernels read each row as one 16-byte vector
    return coords


def _raise_status(status: int, what: str) -> None:
    if status & L.FLAG_BATCH_OUT_OF_RANGE:
        raise IndexError(f"{what}: batch index outside [0, batch_size)")
    if status & L.FLAG_COORD_OUT_OF_GRID:
        raise IndexError(f"{what}: coordinate outside the spatial shape")


# Output coordinates of strided builds -> (workspace, which begins with the
# output grid's occupancy bitmap, its 32-cell words, output shape, batch size,
# the coordinates' version counter).  A submanifold build on exactly those
# coordinates probes that bitmap instead of building its own.
_STRIDED_BITMAPS = WeakIdKeyDictionary()


def _subm_on_strided_bitmap(indices, coords, shape, batch_size, ks, dil):
    """The submanifold build on a strided build's output set, through its
    bitmap, or None when ``indices`` is not such an output (unchanged)."""
    bm = _STRIDED_BITMAPS.get(indices)
    if bm is None:
        return None
    ws, nwords, out_shape, batch, version = bm
    if (out_shape != shape or batch != int(batch_size) or version != indices._version
            or ks[2] != 3 or 2 * dil[2] >= 32):
        return None
    K = ks[0] * ks[1] * ks[2]
    n = coords.shape[0]
    dev = coords.device
    cols_row = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    map_cols = torch.empty((K, n), dtype=torch.int32, device=dev)
    counts = torch.empty(K + 2, dtype=torch.int32, device=dev)
    L.check(L.lib().tsc_subm_pairs_from_bitmap(
        coords.data_ptr(), n, int(batch_size), L.i3(shape), L.i3(ks), L.i3(dil), ws.data_ptr(),
        nwords, cols_row.data_ptr(), map_cols.data_ptr(), counts.data_ptr(), L.stream_of(coords)),
        "generate_subm_indice_pairs")
    # No read-back here: the rows are the registered output set (same tensor,
    # same version), so there is nothing to validate before the convolution.
    # The counts and the status flag (rows that are not the bitmap's cells,
    # whose neighbours the kernel leaves out of the map) are read with
    # pair_num.
    d = IndiceData._from_tables(
        out_indices=indices, input_indices=indices, input_spatial_shape=shape,
        output_spatial_shape=shape, kernel_size=ks, stride=(1, 1, 1), padding=(0, 0, 0),
        dilation=dil, subm=True, pin=None, pout=None, cnt_dev=None, pair_num=None,
        nbr=None, batch_size=int(batch_size), map_cols=map_cols, cols_row=cols_row[:n],
        raster=True)
    d._counts_pending = (counts, K)
    return d


def generate_subm_indice_pairs(indices: torch.Tensor, spatial_shape, batch_size: int, kernel_size,
                               dilation=1) -> IndiceData:
    """Submanifold pairs: output set == input set (indices.py:67-140)."""
    coords = _coords(indices, "generate_subm_indice_pairs")
    ks, dil = _to3(kernel_size), _to3(dilation)
    shape = tuple(int(v) for v in spatial_shape)
    on_bitmap = _subm_on_strided_bitmap(indices, coords, shape, batch_size, ks, dil)
    if on_bitmap is not None:
        return on_bitmap
    K = ks[0] * ks[1] * ks[2]
    n = coords.shape[0]
    dev = coords.device
    lib = L.lib()
    ws_bytes = lib.tsc_subm_workspace_bytes(n, K, int(batch_size), L.i3(shape))
    if ws_bytes < 0:
        raise ValueError(f"generate_subm_indice_pairs: invalid batch size {batch_size} or "
                         f"spatial shape {shape}")
    ws = L.workspace(ws_bytes, dev)
    # the map by columns (in (b,z,y,x) order when the bitmap path runs); the
    # reference's pair lists are derived from it on first access
    cols_row = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    map_cols = torch.empty((K, n), dtype=torch.int32, device=dev)
    counts = torch.empty(K + 2, dtype=torch.int32, device=dev)
    L.check(lib.tsc_subm_pairs(coords.data_ptr(), n, int(batch_size), L.i3(shape), L.i3(ks),
                               L.i3(dil), ws.data_ptr(), ws.numel(), cols_row.data_ptr(),
                               map_cols.data_ptr(), counts.data_ptr(), L.stream_of(coords)),
            "generate_subm_indice_pairs")
    host = counts.cpu()
    _raise_status(int(host[K]), "generate_subm_indice_pairs")
    return IndiceData._from_tables(
        out_indices=indices, input_indices=indices, input_spatial_shape=spatial_shape,
        output_spatial_shape=spatial_shape, kernel_size=ks, stride=(1, 1, 1),
        padding=(0, 0, 0), dilation=dil, subm=True, pin=None, pout=None, cnt_dev=None,
        pair_num=host[:K].long(), nbr=None, batch_size=int(batch_size), map_cols=map_cols,
        cols_row=cols_row[:n], raster=bool(host[K + 1]))


def generate_strided_indice_pairs(indices: torch.Tensor, spatial_shape, batch_size: int,
                                  kernel_size, stride=1, padding=0, dilation=1) -> IndiceData:
    """Strided pairs and the sorted new active set (indices.py:143-259)."""
    coords = _coords(indices, "generate_strided_indice_pairs")
    ks, st, pd, dil = _to3(kernel_size), _to3(stride), _to3(padding), _to3(dilation)
    shape = tuple(int(v) for v in spatial_shape)
    out_shape = _output_spatial_shape(shape, ks, st, pd, dil)
    K = ks[0] * ks[1] * ks[2]
    n = coords.shape[0]
    dev = coords.device
    if min(out_shape) <= 0:
        raise ValueError(f"generate_strided_indice_pairs: empty output shape {out_shape}")
    lib = L.lib()
    ws = L.workspace(lib.tsc_strided_workspace_bytes(n, K, int(batch_size), L.i3(out_shape)), dev)
    counts = torch.empty(K + 3, dtype=torch.int32, device=dev)
    geo = (L.i3(shape), L.i3(ks), L.i3(st), L.i3(pd), L.i3(dil), L.i3(out_shape))
    stream = L.stream_of(coords)
    L.check(lib.tsc_strided_count(coords.data_ptr(), n, int(batch_size), *geo, ws.data_ptr(),
                                  ws.numel(), counts.data_ptr(), stream),
            "generate_strided_indice_pairs")
    host = counts.cpu()
    _raise_status(int(host[K + 1]), "generate_strided_indice_pairs")
    n_out = int(host[K])
    out_coords = torch.empty((n_out, 4), dtype=torch.int32, device=dev)
    nbr = torch.empty((K, n_out), dtype=torch.int32, device=dev)
    pin = torch.empty((K, n), dtype=torch.int32, device=dev)
    pout = torch.empty((K, n), dtype=torch.int32, device=dev)
    L.check(lib.tsc_strided_fill(coords.data_ptr(), n, int(batch_size), *geo, ws.data_ptr(),
                                 ws.numel(), n_out, out_coords.data_ptr(), nbr.data_ptr(),
                                 pin.data_ptr(), pout.data_ptr(), stream),
            "generate_strided_indice_pairs")
    data = IndiceData._from_tables(
        out_indices=out_coords, input_indices=indices, input_spatial_shape=shape,
        output_spatial_shape=out_shape, kernel_size=ks, stride=st, padding=pd, dilation=dil,
        subm=False, pin=pin, pout=pout, cnt_dev=counts[:K], pair_num=host[:K].long(), nbr=nbr,
        batch_size=int(batch_size), rows_raster=True)
    data._n_in_paired = int(host[K + 2])
    cells = int(batch_size) * out_shape[0] * out_shape[1] * out_shape[2]
    _STRIDED_BITMAPS[out_coords] = (ws, (cells + 31) // 32, tuple(out_shape), int(batch_size),
                                    out_coords._version)
    return data


def generate_inverse_indice_pairs(fwd: IndiceData) -> IndiceData:
    """Pairs of the inverse of a strided layer (modules.py:175-212).

    Output rows: forward input rows with at least one forward pair, ascending;
    slot k reads forward outputs pairs_out[k] and writes the compact id of
    forward input pairs_in[k]; pair_num is the forward's.
    """
    fwd._ensure_tables()
    if fwd._pin is None:
        raise ValueError("inverse pairs need a forward IndiceData built on the GPU")
    dev = fwd._pin.device
    K = fwd.K
    cap = fwd._pin.shape[1]
    n_in = len(fwd.input_indices)
    lib = L.lib()
    ws = L.workspace(lib.tsc_inverse_workspace_bytes(n_in), dev)
    counts = torch.empty(1, dtype=torch.int32, device=dev)
    stream = L.stream_of(fwd._pin)
    L.check(lib.tsc_inverse_count(fwd._pin.data_ptr(), fwd._cnt.data_ptr(), K, cap, n_in,
                                  ws.data_ptr(), ws.numel(), counts.data_ptr(), stream),
            "inverse pairs")
    # a forward built here counted its paired input rows with its own pair
    # counts, so the inverse needs no host read of its own
    n_out = fwd._n_in_paired if fwd._n_in_paired is not None else int(counts.cpu()[0])
    in_coords = _coords(fwd.input_indices, "inverse pairs")
    out_coords = torch.empty((n_out, 4), dtype=torch.int32, device=dev)
    nbr = torch.empty((K, n_out), dtype=torch.int32, device=dev)
    inv_pout = torch.empty((K, cap), dtype=torch.int32, device=dev)
    L.check(lib.tsc_inverse_fill(fwd._pin.data_ptr(), fwd._pout.data_ptr(), fwd._cnt.data_ptr(), K,
                                 cap, in_coords.data_ptr(), n_in, ws.data_ptr(), ws.numel(), n_out,
                                 out_coords.data_ptr(), nbr.data_ptr(), inv_pout.data_ptr(),
                                 stream), "inverse pairs")
    return IndiceData._from_tables(
        out_indices=out_coords, input_indices=fwd.out_indices,
        input_spatial_shape=fwd.output_spatial_shape,
        output_spatial_shape=fwd.input_spatial_shape, kernel_size=fwd.kernel_size,
        stride=fwd.stride, padding=fwd.padding, dilation=fwd.dilation, subm=False,
        pin=fwd._pout, pout=inv_pout, cnt_dev=fwd._cnt, pair_num=fwd.pair_num, nbr=nbr,
        batch_size=fwd._batch_size)
