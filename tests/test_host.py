"""Host-side behaviour that needs no GPU: the tensor carrier, constructors,
error paths, weight layout, the C-ABI library's exports and the workloads.

Mirrors the CPU-checkable parts of the reference's tests/test_tensor.py,
test_indices_strided.py:119-127 and modules.py:46-51 / :149-155.
"""
import ctypes
import os
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import trispconv.pytorch as spconv
from trispconv.pytorch.weight import normalize_spconv_weight
from trispconv_amd import _lib as L
from trispconv_amd import workloads

ROOT = Path(__file__).resolve().parent.parent


def make_sparse(B=1, N=8, C=4, D=8, H=8, W=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    coords = torch.randint(0, min(D, H, W), (N, 3), dtype=torch.int32, generator=g)
    idx = torch.cat([torch.zeros(N, 1, dtype=torch.int32), coords], dim=1)
    return spconv.SparseConvTensor(torch.randn(N, C, generator=g), idx, [D, H, W], B)


# ----------------------------------------------------------- tensor carrier
def test_construction():
    x = make_sparse()
    assert x.features.shape == (8, 4)
    assert x.indices.shape == (8, 4)
    assert x.spatial_shape == [8, 8, 8]
    assert x.batch_size == 1


def test_constructor_asserts():
    with pytest.raises(AssertionError):
        spconv.SparseConvTensor(torch.zeros(3), torch.zeros(3, 4, dtype=torch.int32), [2, 2, 2], 1)
    with pytest.raises(AssertionError):
        spconv.SparseConvTensor(torch.zeros(3, 2), torch.zeros(3, 4, dtype=torch.int64), [2, 2, 2], 1)


def test_replace_feature_shares_indices_and_dict():
    x = make_sparse()
    y = x.replace_feature(torch.ones(8, 4))
    assert torch.equal(y.features, torch.ones(8, 4))
    assert y.indices is x.indices
    assert y.indice_dict is x.indice_dict
    assert not torch.equal(x.features, torch.ones(8, 4))


def test_features_setter_raises():
    x = make_sparse()
    with pytest.raises(AttributeError):
        x.features = torch.zeros(8, 4)


def test_dense_has_no_cpu_path():
    """dense() runs on the GPU only (tensor.py:72-99 runs in
    libtrispconv_hip.so); a CPU tensor fails loudly instead of falling back."""
    x = make_sparse(B=2, N=10, C=3, D=4, H=5, W=6)
    with pytest.raises(RuntimeError, match="CPU"):
        x.dense()


def test_find_indice_pair():
    x = make_sparse()
    assert x.find_indice_pair("nonexistent") is None
    assert x.find_indice_pair(None) is None
    x.indice_dict["k"] = "sentinel"
    assert x.find_indice_pair("k") == "sentinel"


# ----------------------------------------------------------- constructors
def test_constructor_errors():
    with pytest.raises(NotImplementedError):
        spconv.SparseConvolution(2, 4, 4, 3)
    with pytest.raises(NotImplementedError):
        spconv.SparseConvolution(3, 4, 4, 3, groups=2)
    with pytest.raises(NotImplementedError):
        spconv.SparseConvolution(3, 4, 4, 3, transposed=True)


def test_module_parameters_krsc_and_forced_fields():
    m = spconv.SubMConv3d(4, 6, 3, stride=2, padding=1)
    assert m.weight.shape == (6, 3, 3, 3, 4)
    assert m.stride == (1, 1, 1) and m.padding == (0, 0, 0) and m.subm
    assert torch.equal(m.bias, torch.zeros(6))
    inv = spconv.SparseInverseConv3d(4, 6, (3, 1, 3), bias=False)
    assert inv.inverse and inv.bias is None and inv.kernel_size == (3, 1, 3)
    # kaiming-uniform bound over the (C_out, K*C_in) view
    bound = (6.0 / (27 * 4)) ** 0.5
    assert float(m.weight.abs().max()) <= bound + 1e-7


def test_inverse_requires_key_before_any_gpu_work():
    x = spconv.SparseConvTensor(torch.randn(5, 4), torch.zeros(5, 4, dtype=torch.int32), [8, 8, 8], 1)
    with pytest.raises(ValueError):
        spconv.SparseInverseConv3d(4, 4, 3)(x)
    with pytest.raises(KeyError):
        spconv.SparseInverseConv3d(4, 4, 3, indice_key="missing")(x)


def test_cpu_tensors_are_refused():
    x = make_sparse(C=4)
    with pytest.raises(RuntimeError, match="GPU"):
        spconv.SubMConv3d(4, 4, 3)(x)


def test_sparse_sequential_names():
    from collections import OrderedDict
    seq = spconv.SparseSequential(OrderedDict(a=torch.nn.ReLU(), b=torch.nn.Identity()))
    assert [n for n, _ in seq.named_children()] == ["a", "b"]
    seq2 = spconv.SparseSequential(torch.nn.ReLU(), extra=torch.nn.Identity())
    assert [n for n, _ in seq2.named_children()] == ["0", "extra"]
    # dense modules act on features, the carrier keeps its coordinates
    x = make_sparse()
    y = seq2(x)
    assert torch.equal(y.features, torch.relu(x.features)) and y.indices is x.indices


# ----------------------------------------------------------- weight layout
def test_normalize_weight_layouts():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(6, 3, 2, 3, 4, generator=g)
    W = normalize_spconv_weight(w, (3, 2, 3), 4, 6)
    assert W.shape == (18, 4, 6)
    assert torch.equal(W[(2 * 2 + 1) * 3 + 2], w[:, 2, 1, 2, :].T)
    w1 = torch.randn(6, 1, 1, 1, 4, generator=g)
    assert torch.equal(normalize_spconv_weight(w1, (1, 1, 1), 4, 6)[0], w1.reshape(-1).view(4, 6))
    assert torch.equal(normalize_spconv_weight(w1.reshape(6, 4), (1, 1, 1), 4, 6)[0],
                       w1.reshape(-1).view(4, 6))
    assert torch.equal(normalize_spconv_weight(W, (3, 2, 3), 4, 6), W)
    with pytest.raises(ValueError):
        normalize_spconv_weight(torch.zeros(5, 5), (3, 3, 3), 4, 6)


# ----------------------------------------------------------- C ABI
def _declared_symbols():
    text = (ROOT / "include" / "trispconv_abi.h").read_text()
    return sorted(set(re.findall(r"TSC_API\s+[\w\s\*]+?\b(tsc_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    declared = _declared_symbols()
    assert declared, "no declarations parsed"
    assert declared == L.exported_symbols()
    for name in declared:
        assert getattr(lib, name) is not None
    assert lib.tsc_abi_version() == L.ABI_VERSION


def test_indice_data_is_a_dataclass_with_the_reference_fields():
    """IndiceData is a dataclass with the reference's twelve fields in its
    order (indices.py:10-23): fields, replace, asdict and field-wise ==."""
    import dataclasses
    from trispconv.pytorch.indices import IndiceData
    names = [f.name for f in dataclasses.fields(IndiceData)]
    assert names == ["out_indices", "pairs_in", "pairs_out", "pair_num", "input_indices",
                     "input_spatial_shape", "output_spatial_shape", "kernel_size", "stride",
                     "padding", "dilation", "subm"]
    assert all(f.default is dataclasses.MISSING for f in dataclasses.fields(IndiceData))
    idx = torch.zeros(3, 4, dtype=torch.int32)
    pin = [torch.tensor([0, 1]), torch.tensor([2])]
    pout = [torch.tensor([1, 2]), torch.tensor([0])]
    d = IndiceData(idx, pin, pout, torch.tensor([2, 1]), idx, (4, 4, 4), (4, 4, 4), (2, 1, 1),
                   (1, 1, 1), (0, 0, 0), (1, 1, 1), False)
    assert dataclasses.is_dataclass(d)
    d2 = dataclasses.replace(d, subm=True)
    assert d2.subm and not d.subm and d2.pairs_in is d.pairs_in
    assert d == dataclasses.replace(d)
    assert d != d2
    a = dataclasses.asdict(d)
    assert list(a) == names
    assert torch.equal(a["pairs_out"][0], pout[0]) and torch.equal(a["pair_num"], d.pair_num)
    # the lazy fields are still settable, as plain dataclass fields are
    d.pair_num = torch.tensor([1, 1])
    assert d.pair_num.tolist() == [1, 1]


def test_integration_load_snippet_runs_as_written():
    """The 'Build and load' snippet of the boundary document, executed as written
    from the repository root: it loads the built library and asserts its ABI
    version (no GPU call)."""
    text = (ROOT / "INTEGRATION.md").read_text()
    section = text.split("## Build and load", 1)[1]
    blocks = re.findall(r"```python\n(.*?)```", section, flags=re.S)
    assert blocks, "no python block under 'Build and load'"
    snippet = blocks[0]
    assert "tsc_abi_version()" in snippet
    cwd = os.getcwd()
    try:
        os.chdir(ROOT)
        scope: dict = {}
        exec(compile(snippet, "INTEGRATION.md", "exec"), scope)
    finally:
        os.chdir(cwd)
    assert scope["lib"].tsc_abi_version() == L.ABI_VERSION


def test_workspace_queries_are_host_only():
    lib = L.lib()
    # dense enough for the occupancy bitmap: a word and its rank per 32 cells
    assert lib.tsc_subm_workspace_bytes(500_000, 27, 1, L.i3((256, 256, 256)), 0) >= \
        2 * (256 ** 3 // 32) * 4
    assert lib.tsc_pairs_from_map_workspace_bytes(500_000, 27) >= 2 * 27 * (500_000 // 256) * 4
    # very sparse grid: the hash (2N..4N 8-byte slots), far below the bitmap
    sparse = lib.tsc_subm_workspace_bytes(60_000, 27, 4, L.i3((41, 1600, 1408)), 0)
    assert 1 << 20 <= sparse < 4 * 41 * 1600 * 1408 // 8
    assert lib.tsc_subm_workspace_bytes(10, 27, 0, L.i3((4, 4, 4)), 0) == -1
    assert lib.tsc_strided_workspace_bytes(1000, 27, 2, L.i3((21, 800, 704)), 0) > \
        2 * 21 * 800 * 704 // 8
    # byte marks: a byte per cell of a dense grid plus status words, else none;
    # a workspace without them is smaller by their size
    dense = L.i3((256, 256, 256))
    mb = lib.tsc_subm_marks_bytes(500_000, 27, 1, dense)
    assert mb >= 256 ** 3 and mb % 16 == 0
    assert lib.tsc_subm_workspace_bytes(500_000, 27, 1, dense, 0) - \
        lib.tsc_subm_workspace_bytes(500_000, 27, 1, dense, 1) >= 256 ** 3
    assert lib.tsc_subm_marks_bytes(60_000, 27, 4, L.i3((41, 1600, 1408))) == 0
    lidar = L.i3((21, 800, 704))
    assert lib.tsc_strided_marks_bytes(400_000, 27, 2, lidar) >= 2 * 21 * 800 * 704
    assert lib.tsc_strided_marks_bytes(1000, 27, 2, lidar) == 0  # sparse: atomic marks
    assert lib.tsc_strided_workspace_bytes(400_000, 27, 2, lidar, 0) - \
        lib.tsc_strided_workspace_bytes(400_000, 27, 2, lidar, 1) >= 2 * 21 * 800 * 704
    assert lib.tsc_inverse_workspace_bytes(1000) >= 8000
    assert lib.tsc_plan_workspace_bytes(1000, 27) >= 16000
    # MFMA-eligible layers pack 2-byte weights, others fp32
    assert lib.tsc_packed_weight_bytes(27, 128, 128, L.F16) == 27 * 128 * 128 * 2
    assert lib.tsc_packed_weight_bytes(27, 16, 16, L.F32) == 27 * 16 * 16 * 4
    # C_in an odd multiple of 16 packs a 32-channel chunk whose upper half is zero
    assert lib.tsc_packed_weight_bytes(27, 16, 32, L.F16) == 27 * 32 * 32 * 2
    assert lib.tsc_packed_weight_bytes(27, 48, 64, L.F32) == 27 * 64 * 64 * 4
    # narrow layers pack 16-byte reduction steps per lane quad: 32 values for
    # f16/bf16 (27 * 4 -> 4 steps, the last padded), 16 for f32 (27 * 4 -> 7);
    # C_in not a multiple of 4 stays on the fp32 VALU layout
    assert lib.tsc_packed_weight_bytes(27, 4, 16, L.F16) == 4 * 32 * 16 * 2
    assert lib.tsc_packed_weight_bytes(125, 16, 32, L.BF16) == 63 * 32 * 32 * 2
    assert lib.tsc_packed_weight_bytes(27, 4, 16, L.F32) == 7 * 16 * 16 * 4
    assert lib.tsc_packed_weight_bytes(27, 3, 16, L.F16) == 27 * 3 * 16 * 4


def test_argument_errors_return_codes_without_gpu():
    lib = L.lib()
    rc = lib.tsc_subm_pairs(None, -1, 1, L.i3((4, 4, 4)), L.i3((3, 3, 3)), L.i3((1, 1, 1)), None,
                            0, None, None, None, None)
    assert rc == 1 and b"out of range" in lib.tsc_last_error()
    rc = lib.tsc_strided_count(None, 10, 1, L.i3((8, 8, 8)), L.i3((3, 3, 3)), L.i3((2, 2, 2)),
                               L.i3((1, 1, 1)), L.i3((1, 1, 1)), L.i3((5, 5, 5)), None, 0, None,
                               0, 0, None, None)
    assert rc == 1 and b"output shape" in lib.tsc_last_error()
    rc = lib.tsc_conv_forward(None, 7, 1, 1, None, None, 0, None, None, 0, 1, 1, 1, None, None)
    assert rc == 1 and b"dtype" in lib.tsc_last_error()
    # byte marks kept by the caller: too few bytes for the grid, or a mark
    # value outside 1..255, are refused before anything is launched (the
    # marks address is never touched)
    geo = (L.i3((8, 8, 8)), L.i3((3, 3, 3)), L.i3((2, 2, 2)), L.i3((1, 1, 1)), L.i3((1, 1, 1)),
           L.i3((4, 4, 4)))
    need = lib.tsc_strided_marks_bytes(10, 27, 1, geo[5])
    assert need >= 64 and need % 16 == 0
    rc = lib.tsc_strided_count(None, 10, 1, *geo, None, 0, 16, need - 1, 1, None, None)
    assert rc == 1 and b"marks of" in lib.tsc_last_error()
    for gen in (0, 256):
        rc = lib.tsc_strided_count(None, 10, 1, *geo, None, 0, 16, need, gen, None, None)
        assert rc == 1 and b"mark value" in lib.tsc_last_error()
    # a build on an existing bitmap: 3-wide kernels only, and a bitmap that
    # covers the grid
    rc = lib.tsc_subm_pairs_from_bitmap(None, 10, 1, L.i3((8, 8, 8)), L.i3((5, 5, 5)),
                                        L.i3((1, 1, 1)), None, 0, None, None, None, 0, None)
    assert rc == 1 and b"3 cells wide" in lib.tsc_last_error()
    rc = lib.tsc_subm_pairs_from_bitmap(None, 10, 1, L.i3((8, 8, 8)), L.i3((3, 3, 3)),
                                        L.i3((1, 1, 1)), None, 0, None, None, None, 0, None)
    assert rc == 1 and b"bitmap" in lib.tsc_last_error()
    with pytest.raises(ValueError):
        L.check(1, "probe")


# ----------------------------------------------------------- workloads
@pytest.mark.parametrize("name", workloads.WORKLOAD_NAMES)
def test_workloads_unique_in_grid(name):
    w = workloads.make_workload(name, scale=0.02)
    idx = w.indices
    assert idx.dtype == np.int32 and idx.shape[1] == 4
    D, H, W = w.spatial_shape
    assert (idx[:, 0] >= 0).all() and (idx[:, 0] < w.batch_size).all()
    assert (idx[:, 1] < D).all() and (idx[:, 2] < H).all() and (idx[:, 3] < W).all()
    assert (idx >= 0).all()
    keys = ((idx[:, 0].astype(np.int64) * D + idx[:, 1]) * H + idx[:, 2]) * W + idx[:, 3]
    assert len(np.unique(keys)) == len(keys)


# ----------------------------------------------------------- weight tracking
def test_conv_weight_state_follows_every_kind_of_write():
    """The packed-weight cache key changes on in-place updates, on writes
    through ``.data`` (which leave the version counter alone), on
    load_state_dict and on dtype conversion; a plain Parameter has no key."""
    import copy
    import io
    from trispconv_amd.pytorch.weight import ConvWeight, weight_state
    m = spconv.SubMConv3d(4, 8, 3)
    w = m.weight
    assert type(w) is ConvWeight and isinstance(w, torch.nn.Parameter)
    k0 = weight_state(w, torch.float16)
    assert k0 == weight_state(w, torch.float16)        # stable while untouched
    assert k0 != weight_state(w, torch.float32)        # per compute dtype
    w.data.copy_(torch.ones_like(w))
    k1 = weight_state(w, torch.float16)
    assert k1 != k0 and w._version == 0                # .data write: counted, not versioned
    with torch.no_grad():
        w.mul_(2)
    k2 = weight_state(w, torch.float16)
    assert k2 != k1
    m.load_state_dict({"weight": torch.zeros(8, 3, 3, 3, 4), "bias": torch.zeros(8)})
    assert weight_state(m.weight, torch.float16) != k2 and m.weight is w
    m.half()
    assert type(m.weight) is ConvWeight and m.weight.dtype == torch.float16
    # deepcopy and pickling keep the class (and so the tracking)
    assert type(copy.deepcopy(m).weight) is ConvWeight
    buf = io.BytesIO()
    torch.save(m, buf)
    buf.seek(0)
    assert type(torch.load(buf, weights_only=False).weight) is ConvWeight
    assert repr(w).startswith("Parameter containing:\ntensor(")
    m.weight = torch.nn.Parameter(torch.zeros(8, 3, 3, 3, 4))
    assert weight_state(m.weight, torch.float16) is None


def test_anigen_shaped_weights_load_and_normalize():
    """The reference's checkpoint test without the checkpoint
    (tests/test_anigen_weights.py:43-91): KRSC tensors of the AniGen decoder's
    shapes load into the modules (through .data, and through load_state_dict)
    and normalize to (K, C_in, C_out)."""
    shapes = {"inv3": ((192, 3, 3, 3, 768), (3, 3, 3), 768, 192),
              "subm3": ((192, 3, 3, 3, 192), (3, 3, 3), 192, 192),
              "inv1": ((192, 1, 1, 1, 768), (1, 1, 1), 768, 192)}
    mods = {"inv3": spconv.SparseInverseConv3d(768, 192, 3, bias=False, indice_key="up0"),
            "subm3": spconv.SubMConv3d(192, 192, 3, bias=False),
            "inv1": spconv.SparseInverseConv3d(768, 192, 1, bias=False, indice_key="up0_skip")}
    g = torch.Generator().manual_seed(0)
    for name, (shape, ks, c_in, c_out) in shapes.items():
        w = torch.randn(*shape, generator=g)
        m = mods[name]
        m.weight.data.copy_(w)
        assert torch.equal(m.weight, w)
        W = normalize_spconv_weight(m.weight, ks, c_in, c_out)
        K = ks[0] * ks[1] * ks[2]
        assert W.shape == (K, c_in, c_out)
        m.load_state_dict({"weight": w * 2})
        assert torch.equal(m.weight, w * 2)
    # the 1x1x1 fold re-reads the flat KRSC storage as (C_in, C_out)
    w1 = mods["inv1"].weight
    assert torch.equal(normalize_spconv_weight(w1, (1, 1, 1), 768, 192)[0],
                       w1.reshape(-1).view(768, 192))


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    """Without the built HIP library there is no fallback: the first call that
    needs it raises and names the build command."""
    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", tmp_path / "libtrispconv_hip.so")
    with pytest.raises(RuntimeError, match="trispconv_amd.build"):
        L.lib()


def test_pending_pair_counts_are_read_and_checked_on_first_access():
    """A submanifold build on a strided layer's bitmap leaves its counts on the
    device; pair_num reads them on first access and raises if the build
    flagged rows that are not the bitmap's cells."""
    from trispconv_amd.pytorch.indices import IndiceData

    def data(counts):
        d = IndiceData(torch.zeros((1, 4), dtype=torch.int32), None, None, None,
                       torch.zeros((1, 4), dtype=torch.int32), (4, 4, 4), (4, 4, 4), (3, 1, 1),
                       (1, 1, 1), (0, 0, 0), (1, 1, 1), True)
        d._counts_pending = (torch.tensor(counts, dtype=torch.int32), 3, None)
        return d

    d = data([3, 0, 5, 0])
    assert d.pair_num.dtype == torch.int64 and d.pair_num.tolist() == [3, 0, 5]
    assert d._counts_pending is None
    d.pair_num = torch.tensor([1, 1, 1])
    assert d.pair_num.tolist() == [1, 1, 1]
    with pytest.raises(RuntimeError, match="not the rows"):
        data([1, 1, 1, L.FLAG_ROWS_NOT_BITMAP]).pair_num


# Instructions that read M0 implicitly on gfx9-family targets, besides the
# direct-to-LDS loads themselves.
_M0_READERS = re.compile(r"\b(s_movrel|v_movrel|s_sendmsg|ds_gws|v_interp|ds_\w*addtid)\w*|"
                         r"\bbuffer_load\w*\b.*\blds\b")


@pytest.mark.skipif(not Path("/opt/rocm/bin/hipcc").exists(), reason="needs ROCm's hipcc")
def test_dma_kernels_own_m0(tmp_path):
    """conv_dma_kernel sets M0 in inline assembly right before each
    direct-to-LDS load, without telling the compiler; that is sound only while
    nothing else in those kernels uses M0.  The gfx950 assembly of every
    instantiation, built with the library's own flags, must show each
    global_load_lds right after its own M0 write and no other M0 user.  No
    global_load_lds may carry an immediate offset either: the offset moves
    the LDS destination as well as the global address, so a load meant for
    the next 64 bytes of a row lands 64 bytes past its slot."""
    import subprocess

    from trispconv_amd import build as B
    asm = tmp_path / "conv.s"
    cmd = [B.hipcc(), *B.HIPCC_FLAGS, "--cuda-device-only", "-S", str(B.CSRC / "conv.hip"),
           "-o", str(asm)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    text = asm.read_text()
    names = re.findall(r"^(_Z\S*conv_dma_kernel\S*):", text, re.M)
    assert len(names) >= 6, "expected the f16, bf16 and f32 instantiations"
    for name in names:
        body = text[text.index(name + ":"):]
        body = body[:body.index(".Lfunc_end")]  # the whole function, every exit
        lines = [ln.split(";")[0].strip() for ln in body.splitlines()]
        lines = [ln for ln in lines if ln and not ln.startswith((".", "#"))]
        n_dma = 0
        for i, ln in enumerate(lines):
            assert not _M0_READERS.search(ln), (name, ln)
            if ln.startswith("global_load_lds"):
                n_dma += 1
                assert lines[i - 1].startswith("s_mov_b32 m0,"), (name, lines[i - 1], ln)
                assert "offset" not in ln, (name, ln)
            elif re.search(r"\bm0\b", ln):
                assert ln.startswith("s_mov_b32 m0,") and lines[i + 1].startswith("global_load_lds"), \
                    (name, ln)
        assert n_dma > 0, name
