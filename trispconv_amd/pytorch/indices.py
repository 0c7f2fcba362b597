"""Indice-pair generation on the GPU (submanifold, strided, inverse).

Public names and semantics follow trispconv/pytorch/indices.py:10-259 and the
inverse remap of modules.py:175-212; the work runs in libtrispconv_hip.so.

``IndiceData`` keeps the reference's fields.  Pair lists are stored on the
device as padded int32 tables (slot k owns ``[k, :pair_num[k]]``) next to the
output-major neighbour map the convolution reads; the reference-style lists
of K int64 tensors are materialised on first access to ``pairs_in`` /
``pairs_out``.  ``pair_num`` is a CPU int64 tensor, as in the reference
(indices.py:131): strided builds read it with the one device-to-host copy
they make (their output count), submanifold builds on its first access.
"""
from __future__ import annotations

import ctypes
import functools
import threading
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional, Sequence, Tuple

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
# Gathered row bytes from which a spatially ordered map is planned on its
# first use (see IndiceData.execution_order).
_PLAN_FIRST_USE_ROW_BYTES = 256


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


@dataclass(init=False, repr=False)
class IndiceData:
    """Pairs of one layer (indices.py:10-23), backed by device tables.

    A dataclass with the reference's twelve fields in its order, so
    ``dataclasses.fields``, ``replace``, ``asdict`` and field-wise ``==``
    behave as on the reference's.  ``pairs_in``, ``pairs_out`` and
    ``pair_num`` are properties over the device tables (made on first
    access); the tables and caches are plain attributes, not fields."""

    out_indices: torch.Tensor           # (N_out, 4) int32
    pairs_in: List[torch.Tensor]        # K int64 tensors
    pairs_out: List[torch.Tensor]       # K int64 tensors
    pair_num: torch.Tensor              # (K,) int64, CPU
    input_indices: torch.Tensor         # (N_in, 4) int32
    input_spatial_shape: Tuple[int, ...]
    output_spatial_shape: Tuple[int, ...]
    kernel_size: Tuple[int, ...]
    stride: Tuple[int, ...]
    padding: Tuple[int, ...]
    dilation: Tuple[int, ...]
    subm: bool

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
        # (counts [K + 2] int32, K, a function that returns them on the host,
        # reading them on the build's stream, or None);
        # counts[K] holds the build's status flags
        self._counts_pending: Optional[Tuple[torch.Tensor, int, Optional[Callable[[], None]]]] = None
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
        # the convolution's nbr_ordered flag for it: 2 when the slot masks
        # of the positions follow the map as its row K, else 1
        self._ordered_flag = 1
        # the builder's map by columns has each column's slot mask as row K
        self._map_masks = False
        self._batch_size: Optional[int] = None
        # strided builds: input rows with at least one pair, i.e. the row
        # count of this layer's inverse, read with the build's counts
        self._n_in_paired: Optional[int] = None
        # strided builds: each input row's id among the rows with a pair (-1
        # for the others), the inverse's output ids
        self._in_ids: Optional[torch.Tensor] = None
        # input rows the pairs may name: ids lie in [0, _in_bound) (the
        # builders' input rows; for user-assigned lists their largest id + 1)
        self._in_bound: Optional[int] = None
        # convolutions run on these pairs so far without an execution order
        self._conv_uses = 0
        # map rows per slot (user-assigned lists with repeated outputs)
        self._slot_repeat = 1
        # a build whose status flags are read on its first reuse (a
        # submanifold build on a strided layer's bitmap: its rows are checked
        # against that bitmap on the device, with no read-back at build time)
        self._deferred_check = False
        self._uses = 0
        # for such a build: (an event recorded right behind it, a pinned host
        # copy of its status word made before that event)
        self._status_copy: Optional[Tuple[torch.cuda.Event, torch.Tensor]] = None

    def _get_pair_num(self) -> torch.Tensor:
        """Pairs per slot, a CPU int64 tensor (indices.py:131).  Submanifold
        builds leave their counts on the device (their coordinates are
        checked before the build returns, or, on a strided layer's bitmap,
        need no check); they are read here, on first access, so the forward
        pass does not wait for them."""
        if self._pair_num is None and self._counts_pending is not None:
            counts, K, read = self._counts_pending
            host = read() if read is not None else counts.cpu()
            if int(host[K]) & L.FLAG_ROWS_NOT_BITMAP:
                raise RuntimeError("generate_subm_indice_pairs: coordinates are not the rows of "
                                   "the strided build they were registered with")
            self._pair_num = host[:K].long()
            self._counts_pending = None
        return self._pair_num

    def _set_pair_num(self, value: torch.Tensor) -> None:
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

    def _get_pairs_in(self) -> List[torch.Tensor]:
        if self._pairs_in is None:
            self._ensure_tables()
            self._pairs_in = self._slot_views(self._pin)
        return self._pairs_in

    def _set_pairs_in(self, value: List[torch.Tensor]) -> None:
        if self._pairs_out is None and (self._pout is not None or self._map_cols is not None):
            self.pairs_out  # keep the other list: the tables it comes from go
        self._pairs_in = value
        self._drop_tables()

    def _get_pairs_out(self) -> List[torch.Tensor]:
        if self._pairs_out is None:
            self._ensure_tables()
            self._pairs_out = self._slot_views(self._pout)
        return self._pairs_out

    def _set_pairs_out(self, value: List[torch.Tensor]) -> None:
        if self._pairs_in is None and (self._pin is not None or self._map_cols is not None):
            self.pairs_in  # keep the other list: the tables it comes from go
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
        self._map_masks = False
        self._nbr_ordered = None
        self._inverse_cache = None
        self._in_bound = None
        self._in_ids = None
        self._slot_repeat = 1

    # --------------------------------------------------- convolution inputs
    def neighbour_map(self, n_out: int, device, n_in: Optional[int] = None) -> torch.Tensor:
        """[K][n_out] int32: input row feeding output row o through slot k, or -1.
        ``n_in``: the rows of the features the map will gather from (checked
        against user-assigned lists)."""
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
            self._nbr = self._user_map(n_out, n_in, device)
        return self._nbr

    def _user_lists(self, n_in: Optional[int], n_out: int, device):
        """The user-assigned pair lists as flat device tensors (slot of each
        pair, input ids, output ids) and the per-slot sizes, after the checks
        the reference's own indexing makes: ``features[in_ids]`` and
        ``out.index_add_(0, out_ids, ...)`` (functional.py:46) raise
        IndexError for ids outside the rows.  Ids must lie in [0, n_in) and
        [0, n_out)."""
        K = self.K
        pin, pout = self.pairs_in, self.pairs_out
        if len(pin) != K or len(pout) != K:
            raise ValueError(f"IndiceData: {len(pin)} pairs_in and {len(pout)} pairs_out lists "
                             f"for a kernel of {K} slots")
        sizes = [int(p.numel()) for p in pin]
        if sizes != [int(p.numel()) for p in pout]:
            raise ValueError("IndiceData: pairs_in[k] and pairs_out[k] differ in length")
        total = sum(sizes)
        if total == 0:
            e = torch.empty(0, dtype=torch.long, device=device)
            return e, e, e, sizes
        cat_in = torch.cat([p.reshape(-1).to(device=device, dtype=torch.long) for p in pin])
        cat_out = torch.cat([p.reshape(-1).to(device=device, dtype=torch.long) for p in pout])
        slot = torch.repeat_interleave(torch.arange(K, device=device),
                                       torch.tensor(sizes, device=device))
        return slot, cat_in, cat_out, sizes

    @staticmethod
    def _range_error(lo_in, hi_in, lo_out, hi_out, n_in, n_out, what):
        if n_in is not None and (lo_in < 0 or hi_in >= n_in):
            raise IndexError(f"{what}: pairs_in holds ids in [{lo_in}, {hi_in}], outside the "
                             f"{n_in} input rows")
        if lo_out < 0 or hi_out >= n_out:
            raise IndexError(f"{what}: pairs_out holds ids in [{lo_out}, {hi_out}], outside the "
                             f"{n_out} output rows")

    def _user_map(self, n_out: int, n_in: Optional[int], device) -> torch.Tensor:
        """[K*m][n_out] map of user-assigned lists, checked with one host read
        (ids in range).

        The reference adds every pair of a slot with ``index_add_``
        (functional.py:46), so a list that names an output row twice within a
        slot adds both contributions.  The map holds one input per (row,
        output): the j-th occurrence of an output within slot k (in list
        order) goes to map row k*m + j, m the largest multiplicity, and the
        convolution runs with each slot's weight repeated m times
        (``slot_repeat``).  Slot k's contributions stay together and in list
        order, so the sums keep the slot-ascending order; m is 1 for lists
        without repeats (every generator's)."""
        K = self.K
        slot, cat_in, cat_out, sizes = self._user_lists(n_in, n_out, device)
        self._slot_repeat = 1
        if not slot.numel():
            self._in_bound = 0
            return torch.full((K, n_out), -1, dtype=torch.int32, device=device)
        # clamped ids, so that the scatter below stays in bounds whatever the
        # lists hold (out-of-range ids raise after the one host read)
        hi_in = (n_in if n_in is not None else 1 << 31) - 1
        out_c = cat_out.clamp(0, max(n_out - 1, 0))
        # occurrence rank of each pair among the pairs of its (slot, output):
        # a stable sort keeps list order within a run of equal keys
        key = slot * max(n_out, 1) + out_c
        skey, perm = torch.sort(key, stable=True)
        pos = torch.arange(len(key), device=device)
        run_start = torch.ones_like(skey, dtype=torch.bool)
        run_start[1:] = skey[1:] != skey[:-1]
        first = torch.where(run_start, pos, torch.zeros_like(pos)).cummax(0).values
        rank = torch.empty_like(pos)
        rank[perm] = pos - first
        stats = torch.stack([cat_in.min(), cat_in.max(), cat_out.min(), cat_out.max(),
                             rank.max()]).cpu().tolist()
        self._range_error(*stats[:4], n_in, n_out, "sparse_conv_forward")
        m = int(stats[4]) + 1
        nbr = torch.full((K * m, n_out), -1, dtype=torch.int32, device=device)
        nbr[slot * m + rank, out_c] = cat_in.clamp(0, hi_in).int()
        self._slot_repeat = m
        self._in_bound = int(stats[1]) + 1
        return nbr

    @property
    def slot_repeat(self) -> int:
        """How many map rows each slot has: 1, or for user-assigned lists that
        name an output row more than once within a slot, the largest such
        count (the map's row k*m + j is the j-th occurrence in slot k)."""
        return self._slot_repeat

    def _tables_from_lists(self, device) -> None:
        """Padded device tables (and counts) from user-assigned lists, for the
        inverse remap (modules.py:175-212 reads the forward's lists)."""
        K = self.K
        n_in, n_out = len(self.input_indices), len(self.out_indices)
        slot, cat_in, cat_out, sizes = self._user_lists(n_in, n_out, device)
        cap = max([n_in, 1] + sizes)
        pin = torch.full((K, cap), -1, dtype=torch.int32, device=device)
        pout = torch.full((K, cap), -1, dtype=torch.int32, device=device)
        if slot.numel():
            starts = torch.tensor([0] + sizes[:-1], device=device).cumsum(0)
            pos = torch.arange(len(slot), device=device) - starts[slot]
            stats = torch.stack([cat_in.min(), cat_in.max(), cat_out.min(),
                                 cat_out.max()]).cpu().tolist()
            self._range_error(*stats, n_in, n_out, "SparseInverseConv3d")
            pin[slot, pos] = cat_in.int()
            pout[slot, pos] = cat_out.int()
        self._pin, self._pout = pin, pout
        self._cnt = torch.tensor(sizes, dtype=torch.int32, device=device)

    def execution_order(self, n_out: int, device, row_bytes: int = 256,
                        eager: bool = False) -> Optional[torch.Tensor]:
        """Processing order of the output rows for the fused convolution.

        Morton order cut into regions whose gathered input rows (``row_bytes``
        each) fit in half the Infinity Cache, each region sorted by slot mask,
        then its whole 256-row tiles put in decreasing number of slots used
        (the partial tile last).  Built once per region size and cached; None
        for small layers.

        The order never changes an output bit.  When the map's columns are
        already in (b,z,y,x) order (a bitmap build's columns, a strided
        build's output rows) and the gathered rows are wide (at least 256
        bytes), the plan pays for itself on its first use (measured: the
        500k-row 128-channel SubM layer 0.55 ms unplanned against 0.17 +
        0.37 ms, the 166k-row 64-channel fp32 strided layer 0.36 against
        0.11 + 0.16 ms), so it is built then.  Otherwise it costs more than
        one use saves (the 600k-row 64-channel bf16 inverse layer: 0.16 ms
        unplanned against 0.145 + 0.065 ms; the 674k-row 32-channel bf16
        strided layer: about 0.12 against 0.20 + 0.076 ms): the first
        convolution runs without one and the order is built when the pairs
        are used again (the next layer with this indice_key, or the next
        forward).  ``eager`` builds it at once.
        """
        if n_out < _PLAN_MIN_ROWS or n_out * int(row_bytes) < _PLAN_MIN_BYTES \
                or self._slot_repeat != 1:
            return None
        region = int(min(max(_REGION_BYTES // max(int(row_bytes), 1), 2048), 1 << 30))
        if self._order is None or self._order_region != region:
            self._conv_uses += 1
            raster = self._raster if self._map_cols is not None else self._rows_raster
            first_use = raster and int(row_bytes) >= _PLAN_FIRST_USE_ROW_BYTES
            if self._conv_uses < 2 and not eager and not first_use:
                return None
            if self._map_cols is not None:  # the builder's columns, maybe in spatial order
                nbr, cols_row = self._map_cols, self._cols_row
            else:
                nbr, cols_row = self.neighbour_map(n_out, device), None
            coords = None if raster else _coords(self.out_indices, "conv plan")
            lib = L.lib()
            ws = L.workspace(lib.tsc_plan_workspace_bytes(n_out, self.K), device)
            order = torch.empty(n_out, dtype=torch.int32, device=device)
            # with K <= 32 the permuted map gets one more row: each position's
            # slot mask, so the convolution learns a tile's slots from one
            # word per row instead of all of its entries
            masks = self.K <= 32
            ordered = torch.empty((self.K + int(masks)) * n_out, dtype=torch.int32,
                                  device=device)
            nbr_ordered = ordered[:self.K * n_out].view(self.K, n_out)
            L.check(lib.tsc_conv_plan(nbr.data_ptr(), L.ptr(cols_row), int(raster), L.ptr(coords),
                                      n_out, self.K, self._batch_bound(),
                                      L.i3(self.output_spatial_shape), region, ws.data_ptr(),
                                      ws.numel(), order.data_ptr(), nbr_ordered.data_ptr(),
                                      ordered.data_ptr() + 4 * self.K * n_out if masks else None,
                                      L.stream_of(nbr)), "conv plan")
            self._order, self._order_region, self._nbr_ordered = order, region, nbr_ordered
            self._ordered_flag = 2 if masks else 1
        return self._order

    def conv_operands(self, n_out: int, device, row_bytes: int = 256,
                      n_in: Optional[int] = None):
        """(map, order, ordered) for the fused convolution: the planned order
        and its permuted map (ordered 2 when the map has the plan's row of
        slot masks after it, else 1); for small layers the builder's own
        spatial column order when it has one (ordered 1); else the row-major
        map (ordered 0).  ``n_in``, the
        feature rows, must cover every input id the pairs name (IndexError,
        as the reference's ``features[in_ids]``)."""
        if self._deferred_check:
            self._uses += 1
            if self._uses >= 2:
                # the first reuse under the key reads the build's status
                # flags once and raises when the rows were not the registered
                # strided output set; it waits for the build alone (its event),
                # so the convolutions queued after the build keep the GPU busy
                self._deferred_check = False
                if self._status_copy is not None:
                    done, flag = self._status_copy
                    done.synchronize()
                    self._status_copy = None
                    if int(flag[0]) & L.FLAG_ROWS_NOT_BITMAP:
                        raise RuntimeError("generate_subm_indice_pairs: coordinates are not the "
                                           "rows of the strided build they were registered with")
                else:
                    self.pair_num  # noqa: B018
        if self._map_cols is None and self._nbr is None:
            self.neighbour_map(n_out, device, n_in)  # user-assigned lists: checked here
        if n_in is not None:
            bound = self._in_bound if self._in_bound is not None else len(self.input_indices)
            if n_in < bound:
                raise IndexError(f"sparse_conv_forward: the pairs read input rows up to "
                                 f"{bound - 1}, the features have {n_in} rows")
        order = self.execution_order(n_out, device, row_bytes)
        if order is not None:
            return self._nbr_ordered, order, self._ordered_flag
        if self._map_cols is not None and self._raster:
            return self._map_cols, self._cols_row, 2 if self._map_masks else 1
        return self.neighbour_map(n_out, device), None, 0

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


# The three lazy fields are properties over the device tables.  They are set
# on the class after the dataclass decorator has recorded the fields, so that
# the fields carry no default (a property in the class body would be taken
# for one).
IndiceData.pair_num = property(IndiceData._get_pair_num, IndiceData._set_pair_num)
IndiceData.pairs_in = property(IndiceData._get_pairs_in, IndiceData._set_pairs_in)
IndiceData.pairs_out = property(IndiceData._get_pairs_out, IndiceData._set_pairs_out)


def _coords(indices: torch.Tensor, what: str) -> torch.Tensor:
    L.require_gpu(indices, what)
    if indices.ndim != 2 or indices.shape[1] != 4:
        raise ValueError(f"{what}: indices must be (N, 4) (b, z, y, x), got {tuple(indices.shape)}")
    coords = indices
    if coords.dtype != torch.int32 or not coords.is_contiguous():
        coords = indices.to(torch.int32).contiguous()
    if coords.data_ptr() % 16:
        coords = coords.clone()  # the kernels read each row as one 16-byte vector
    return coords


def _align64(count: int) -> int:
    """count rounded up to a multiple of 64 int32 elements (256 bytes)."""
    return (int(count) + 63) // 64 * 64


def _raise_status(status: int, what: str) -> None:
    if status & L.FLAG_BATCH_OUT_OF_RANGE:
        raise IndexError(f"{what}: batch index outside [0, batch_size)")
    if status & L.FLAG_COORD_OUT_OF_GRID:
        raise IndexError(f"{what}: coordinate outside the spatial shape")


# Output coordinates of strided builds -> (workspace, which begins with the
# output grid's occupancy bitmap, its 32-cell words, output shape, batch size,
# the coordinates' version counter, their address and storage offset).  A submanifold build on exactly those
# coordinates probes that bitmap instead of building its own.
_STRIDED_BITMAPS = WeakIdKeyDictionary()


class _Marks:
    """Byte marks (a byte per grid cell, then a few status words) that the
    bitmap pair builds one host thread launches on one stream share.  Each
    build marks with a value of its own, 1..255, and reads only that value,
    so no build zeroes them first; they are zeroed when the values run out,
    and replaced by a larger, zeroed buffer when a build needs more."""

    __slots__ = ("buf", "gen")

    def __init__(self):
        self.buf: Optional[torch.Tensor] = None
        self.gen = 0

    def take(self, nbytes: int, device) -> Tuple[int, int, int]:
        """(address, size, value) for the next build on this stream."""
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = None
            self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            self.gen = 0
        if self.gen == 255:
            self.buf.zero_()
            self.gen = 0
        self.gen += 1
        return self.buf.data_ptr(), self.buf.numel(), self.gen


class _ThreadMarks(threading.local):
    """Per host thread: (device index, stream) -> the marks of the builds
    this thread launches on that stream.  One thread's builds on one stream
    run one after another and can share marks.  Builds on two streams may
    overlap, and two threads' launches on one stream may interleave (one
    build's mark between another's mark and scan), so each pair gets marks
    of its own.  Each is as large as the largest grid built there, and is
    freed with its thread."""

    def __init__(self):
        self.by_stream: Dict[Tuple[int, int], _Marks] = {}


_MARKS = _ThreadMarks()


def _marks_for(device, stream: int, nbytes: int) -> Tuple[Optional[int], int, int]:
    """Marks for a build of nbytes of byte marks on ``stream`` (None when the
    build marks no bytes)."""
    if nbytes <= 0:
        return None, 0, 0
    key = (device.index, stream)
    m = _MARKS.by_stream.get(key)
    if m is None:
        m = _MARKS.by_stream[key] = _Marks()
    return m.take(nbytes, device)


# A submanifold build on a bitmap packs cell ids in 32 bits: grids of this
# many cells or more take the 64-bit-key hash build instead.
_NARROW_CELLS = (1 << 32) - 1


def _counts_to_host(counts: torch.Tensor, K: int, stream: int,
                    slot_blocks: Optional[torch.Tensor] = None, n: int = 0) -> torch.Tensor:
    """A submanifold build's counts [K + 2] on the host, read on the build's
    stream (which need not be the current one any more); with slot_blocks,
    the per-slot sums of the probe's block counts are made first."""
    host = (ctypes.c_int32 * (K + 2))()
    L.check(L.lib().tsc_subm_counts(slot_blocks.data_ptr() if slot_blocks is not None else None,
                                    n if slot_blocks is not None else 0, K, counts.data_ptr(),
                                    host, stream), "generate_subm_indice_pairs")
    return torch.tensor(list(host), dtype=torch.int32)


# The ctypes shape arrays are only read during a call, so one set serves
# every build of a shape.
@functools.lru_cache(maxsize=64)
def _shape_args(shape, ks, dil):
    return L.i3(shape), L.i3(ks), L.i3(dil)


def _subm_on_strided_bitmap(indices, coords, shape, batch_size, ks, dil):
    """The submanifold build on a strided build's output set, through its
    bitmap, or None when ``indices`` is not such an output (unchanged)."""
    bm = _STRIDED_BITMAPS.get(indices)
    if bm is None:
        return None
    ws, nwords, out_shape, batch, version, ptr = bm
    if (out_shape != shape or batch != int(batch_size) or version != indices._version
            or ptr != (indices.data_ptr(), indices.storage_offset())
            or ks[2] != 3 or 2 * dil[2] >= 32 or nwords * 32 >= _NARROW_CELLS):
        return None
    K = ks[0] * ks[1] * ks[2]
    n = coords.shape[0]
    dev = coords.device
    masks = K <= 32  # each column's slot mask as row K, for the convolution's set-up
    # cols_row, the map (with its mask row) and the counts in one allocation
    # at 256-byte aligned offsets; raw addresses for the launch, views after
    o_map = _align64(max(n, 1))
    o_counts = o_map + _align64((K + int(masks)) * n)
    tables = torch.empty(o_counts + K + 2, dtype=torch.int32, device=dev)
    base = tables.data_ptr()
    stream = L.stream_of(coords)
    L.check(L.lib().tsc_subm_pairs_from_bitmap(
        coords.data_ptr(), n, int(batch_size), *_shape_args(shape, ks, dil), ws.data_ptr(),
        nwords, base, base + 4 * o_map, base + 4 * o_counts, int(masks), stream),
        "generate_subm_indice_pairs")
    cols_row = tables[:n]
    map_cols = tables[o_map:o_map + K * n].view(K, n)
    counts = tables[o_counts:o_counts + K + 2]
    # No read-back here: the rows are the registered output set (same tensor,
    # same version), so there is nothing to validate before the convolution.
    # The probe checks on the device that every row is the bitmap's cell of
    # its own rank and that no neighbour lies beyond the rows; that status
    # flag is read with pair_num, or at the build's first reuse (the second
    # convolution on it), whichever comes first.  For the reuse its word is
    # copied to pinned host memory right behind the build, with an event.
    flag = torch.empty(1, dtype=torch.int32, pin_memory=True)
    flag.copy_(counts[K:K + 1], non_blocking=True)
    done = torch.cuda.Event()
    done.record(torch.cuda.current_stream(dev))
    d = IndiceData._from_tables(
        out_indices=indices, input_indices=indices, input_spatial_shape=shape,
        output_spatial_shape=shape, kernel_size=ks, stride=(1, 1, 1), padding=(0, 0, 0),
        dilation=dil, subm=True, pin=None, pout=None, cnt_dev=None, pair_num=None,
        nbr=None, batch_size=int(batch_size), map_cols=map_cols, cols_row=cols_row,
        raster=True)
    d._map_masks = masks
    d._counts_pending = (counts, K, lambda: _counts_to_host(counts, K, stream))
    d._deferred_check = True
    d._status_copy = (done, flag)
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
    sz = _subm_sizes(n, K, int(batch_size), shape, ks, dil)
    if sz.ws_bytes < 0:
        raise ValueError(f"generate_subm_indice_pairs: invalid batch size {batch_size} or "
                         f"spatial shape {shape}")
    # The workspace, and one allocation for the map by columns (in (b,z,y,x)
    # order when the bitmap path runs; the reference's pair lists are derived
    # from it on first access), the column -> row table, the counts and the
    # probe's per-(slot, block) counts, at 256-byte aligned offsets.  Only
    # raw addresses are made before the launch; the views after it, while the
    # GPU works.
    ws = L.workspace(sz.ws_bytes, dev)
    tables = torch.empty(sz.words, dtype=torch.int32, device=dev)
    base = tables.data_ptr()
    stream = L.stream_of(coords)
    marks, marks_size, gen = _marks_for(dev, stream, sz.marks_bytes)
    result = (ctypes.c_int32 * 2)()
    # Returns once the coordinates are checked (a row outside the grid raises
    # here, as in the reference); the map is still being built on the stream,
    # and the per-slot counts are summed and read only when pair_num is.
    L.check(lib.tsc_subm_pairs_checked(coords.data_ptr(), n, int(batch_size), sz.shape, sz.ks,
                                       sz.dil, ws.data_ptr(), sz.ws_bytes, marks, marks_size,
                                       gen, base,
                                       base + 4 * sz.o_map, base + 4 * sz.o_counts,
                                       base + 4 * sz.o_blocks, int(sz.masks), result, stream),
            "generate_subm_indice_pairs")
    _raise_status(int(result[0]), "generate_subm_indice_pairs")
    cols_row = tables[:n]
    map_cols = tables[sz.o_map:sz.o_map + K * n].view(K, n)
    counts = tables[sz.o_counts:sz.o_counts + K + 2]
    slot_blocks = tables[sz.o_blocks:]
    d = IndiceData._from_tables(
        out_indices=indices, input_indices=indices, input_spatial_shape=spatial_shape,
        output_spatial_shape=spatial_shape, kernel_size=ks, stride=(1, 1, 1),
        padding=(0, 0, 0), dilation=dil, subm=True, pin=None, pout=None, cnt_dev=None,
        pair_num=None, nbr=None, batch_size=int(batch_size), map_cols=map_cols,
        cols_row=cols_row)
    d._counts_pending = (counts, K, lambda: _counts_to_host(counts, K, stream, slot_blocks, n))
    d._raster = bool(result[1])
    d._map_masks = sz.masks and d._raster  # the bitmap path's probe wrote them
    return d


class _SubmSizes:
    """Sizes and ABI arguments of a submanifold build of one shape."""

    def __init__(self, n, K, batch_size, shape, ks, dil):
        lib = L.lib()
        self.shape, self.ks, self.dil = L.i3(shape), L.i3(ks), L.i3(dil)
        # byte marks, when the build uses them, are kept per stream (_Marks)
        self.marks_bytes = int(lib.tsc_subm_marks_bytes(n, K, batch_size, self.shape))
        self.ws_bytes = int(lib.tsc_subm_workspace_bytes(n, K, batch_size, self.shape,
                                                         int(self.marks_bytes > 0)))
        n_al = _align64(max(n, 1))
        self.masks = K <= 32  # each column's slot mask after the map, as its row K
        self.o_map = n_al
        self.o_counts = n_al + _align64((K + int(self.masks)) * n)
        self.o_blocks = self.o_counts + _align64(K + 2)
        self.words = self.o_blocks + int(lib.tsc_subm_slot_blocks_len(n, K))


# The ctypes argument arrays are only read during a call, so one set serves
# every build of a shape (a network builds the same shapes every pass).
@functools.lru_cache(maxsize=64)
def _subm_sizes(n, K, batch_size, shape, ks, dil) -> _SubmSizes:
    return _SubmSizes(n, K, batch_size, shape, ks, dil)


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
    sz = _strided_sizes(n, int(batch_size), shape, ks, st, pd, dil, out_shape)
    ws = L.workspace(sz.ws_bytes, dev)
    counts = torch.empty(K + 3, dtype=torch.int32, device=dev)
    stream = L.stream_of(coords)
    marks, marks_size, gen = _marks_for(dev, stream, sz.marks_bytes)
    L.check(lib.tsc_strided_count(coords.data_ptr(), n, int(batch_size), *sz.geo, ws.data_ptr(),
                                  sz.ws_bytes, marks, marks_size, gen, counts.data_ptr(), stream),
            "generate_strided_indice_pairs")
    # the counts go to the host behind the count pass; the fill is queued
    # before they arrive, with room for the rows this geometry's largest
    # output ratio so far predicts, and is queued again at the exact size in
    # the rare build that outgrows it
    host = torch.empty(K + 3, dtype=torch.int32, pin_memory=True)
    host.copy_(counts, non_blocking=True)
    counted = torch.cuda.Event()
    counted.record(torch.cuda.current_stream(dev))
    geo_key = (int(batch_size), shape, ks, st, pd, dil)
    cap = _strided_out_cap(geo_key, n, sz.cells)

    def fill(out_cap: int):
        # the output coordinates (the next tensor's indices, with their own
        # storage and version counter); the map and the two pair tables in
        # one allocation at 256-byte aligned offsets, passed as raw
        # addresses, the views made after the launch
        out_coords = torch.empty((out_cap, 4), dtype=torch.int32, device=dev)
        o_pin = _align64(K * out_cap)
        tables = torch.empty(max(o_pin + 2 * _align64(K * n) + n, 1), dtype=torch.int32,
                             device=dev)
        base = tables.data_ptr()
        L.check(lib.tsc_strided_fill(coords.data_ptr(), n, int(batch_size), *sz.geo,
                                     ws.data_ptr(), sz.ws_bytes, counts.data_ptr(), out_cap,
                                     out_coords.data_ptr(), base, base + 4 * o_pin,
                                     base + 4 * (o_pin + _align64(K * n)),
                                     base + 4 * (o_pin + 2 * _align64(K * n)), stream),
                "generate_strided_indice_pairs")
        return out_coords, tables, o_pin

    out_coords, tables, o_pin = fill(cap)
    counted.synchronize()
    _raise_status(int(host[K + 1]), "generate_strided_indice_pairs")
    n_out = int(host[K])
    if n > 0:
        _STRIDED_OUT_RATIO[geo_key] = max(_STRIDED_OUT_RATIO.get(geo_key, 0.0), n_out / n)
    if n_out > cap:
        out_coords, tables, o_pin = fill(n_out)
    out_coords = out_coords[:n_out]
    o_pout = o_pin + _align64(K * n)
    o_ids = o_pout + _align64(K * n)
    nbr = tables[:K * n_out].view(K, n_out)
    pin = tables[o_pin:o_pin + K * n].view(K, n)
    pout = tables[o_pout:o_pout + K * n].view(K, n)
    data = IndiceData._from_tables(
        out_indices=out_coords, input_indices=indices, input_spatial_shape=shape,
        output_spatial_shape=out_shape, kernel_size=ks, stride=st, padding=pd, dilation=dil,
        subm=False, pin=pin, pout=pout, cnt_dev=counts[:K], pair_num=host[:K].long(), nbr=nbr,
        batch_size=int(batch_size), rows_raster=True)
    data._n_in_paired = int(host[K + 2])
    data._in_ids = tables[o_ids:o_ids + n]
    _STRIDED_BITMAPS[out_coords] = (ws, sz.out_words, tuple(out_shape), int(batch_size),
                                    out_coords._version,
                                    (out_coords.data_ptr(), out_coords.storage_offset()))
    return data


class _StridedSizes:
    """Workspace size and ABI arguments of a strided build of one shape."""

    def __init__(self, n, batch_size, shape, ks, st, pd, dil, out_shape):
        K = ks[0] * ks[1] * ks[2]
        self.geo = (L.i3(shape), L.i3(ks), L.i3(st), L.i3(pd), L.i3(dil), L.i3(out_shape))
        # byte marks, when the build uses them, are kept per stream (_Marks)
        self.marks_bytes = int(L.lib().tsc_strided_marks_bytes(n, K, batch_size, self.geo[5]))
        self.ws_bytes = max(int(L.lib().tsc_strided_workspace_bytes(
            n, K, batch_size, self.geo[5], int(self.marks_bytes > 0))), 1)
        self.cells = batch_size * out_shape[0] * out_shape[1] * out_shape[2]
        self.out_words = (self.cells + 31) // 32


# Largest n_out / n each strided geometry (batch size, input shape, kernel,
# stride, padding, dilation) has given in this process.  A build sizes its
# output coordinates and map for that ratio (n rows while it is unknown)
# before its count reaches the host; a build that outgrows it is filled again.
_STRIDED_OUT_RATIO: Dict[tuple, float] = {}


def _strided_out_cap(geo_key: tuple, n: int, cells: int) -> int:
    """Rows of room for a strided build's outputs before its count is known:
    1/16 above the geometry's largest ratio so far, and never more than the
    output grid's cells."""
    if n == 0:
        return 0
    ratio = _STRIDED_OUT_RATIO.get(geo_key, 1.0)
    return int(min(cells, (1 << 31) - 1, int(n * ratio * 1.0625) + 256))


@functools.lru_cache(maxsize=64)
def _strided_sizes(n, batch_size, shape, ks, st, pd, dil, out_shape) -> _StridedSizes:
    return _StridedSizes(n, batch_size, shape, ks, st, pd, dil, out_shape)


def generate_inverse_indice_pairs(fwd: IndiceData) -> IndiceData:
    """Pairs of the inverse of a strided layer (modules.py:175-212).

    Output rows: forward input rows with at least one forward pair, ascending;
    slot k reads forward outputs pairs_out[k] and writes the compact id of
    forward input pairs_in[k]; pair_num is the forward's.
    """
    fwd._ensure_tables()
    from_lists = fwd._pin is None
    if from_lists:
        # lists assigned by the user: the reference remaps whatever lists it
        # finds (modules.py:175-212); check them and lay them out as tables
        dev = fwd.input_indices.device
        L.require_gpu(fwd.input_indices, "SparseInverseConv3d")
        fwd._tables_from_lists(dev)
    dev = fwd._pin.device
    K = fwd.K
    cap = fwd._pin.shape[1]
    n_in = len(fwd.input_indices)
    lib = L.lib()
    stream = L.stream_of(fwd._pin)
    in_coords = _coords(fwd.input_indices, "inverse pairs")
    if fwd._in_ids is not None and fwd._n_in_paired is not None and not from_lists:
        # a forward built here: its fill gave every input row its output id
        # and its count read gave the row count, so the inverse is one fill
        n_out = fwd._n_in_paired
        out_coords = torch.empty((n_out, 4), dtype=torch.int32, device=dev)
        nbr = torch.empty((K, n_out), dtype=torch.int32, device=dev)
        inv_pout = torch.empty((K, cap), dtype=torch.int32, device=dev)
        L.check(lib.tsc_inverse_fill_ids(fwd._pin.data_ptr(), fwd._pout.data_ptr(),
                                         fwd._cnt.data_ptr(), K, cap, fwd._in_ids.data_ptr(),
                                         in_coords.data_ptr(), n_in, n_out, out_coords.data_ptr(),
                                         nbr.data_ptr(), inv_pout.data_ptr(), stream),
                "inverse pairs")
    else:
        ws = L.workspace(lib.tsc_inverse_workspace_bytes(n_in), dev)
        counts = torch.empty(1, dtype=torch.int32, device=dev)
        L.check(lib.tsc_inverse_count(fwd._pin.data_ptr(), fwd._cnt.data_ptr(), K, cap, n_in,
                                      ws.data_ptr(), ws.numel(), counts.data_ptr(), stream),
                "inverse pairs")
        # a forward built here counted its paired input rows with its own
        # pair counts, so the inverse needs no host read of its own
        n_out = fwd._n_in_paired if (fwd._n_in_paired is not None and not from_lists) \
            else int(counts.cpu()[0])
        out_coords = torch.empty((n_out, 4), dtype=torch.int32, device=dev)
        nbr = torch.empty((K, n_out), dtype=torch.int32, device=dev)
        inv_pout = torch.empty((K, cap), dtype=torch.int32, device=dev)
        L.check(lib.tsc_inverse_fill(fwd._pin.data_ptr(), fwd._pout.data_ptr(),
                                     fwd._cnt.data_ptr(), K, cap, in_coords.data_ptr(), n_in,
                                     ws.data_ptr(), ws.numel(), n_out, out_coords.data_ptr(),
                                     nbr.data_ptr(), inv_pout.data_ptr(), stream),
                "inverse pairs")
    if from_lists and int((nbr >= 0).sum()) != int(fwd._cnt.sum()):
        # a forward pairs_in list names an input row twice within a slot, so
        # the inverse's pairs_out names that output twice: the reference adds
        # both (index_add_, functional.py:46).  The remapped lists become the
        # inverse's own lists, whose map runs repeats as slots of their own.
        cnt = fwd._cnt.tolist()
        inv_in = [fwd._pout[k, :int(c)].long() for k, c in enumerate(cnt)]
        inv_out = [inv_pout[k, :int(c)].long() for k, c in enumerate(cnt)]
        d = IndiceData(out_coords, inv_in, inv_out, fwd.pair_num, fwd.out_indices,
                       fwd.output_spatial_shape, fwd.input_spatial_shape, fwd.kernel_size,
                       fwd.stride, fwd.padding, fwd.dilation, False)
        d._batch_size = fwd._batch_size
        return d
    return IndiceData._from_tables(
        out_indices=out_coords, input_indices=fwd.out_indices,
        input_spatial_shape=fwd.output_spatial_shape,
        output_spatial_shape=fwd.input_spatial_shape, kernel_size=fwd.kernel_size,
        stride=fwd.stride, padding=fwd.padding, dilation=fwd.dilation, subm=False,
        pin=fwd._pout, pout=inv_pout, cnt_dev=fwd._cnt, pair_num=fwd.pair_num, nbr=nbr,
        batch_size=fwd._batch_size)
