"""The reference-side bindings shown in the boundary document, executed as
written on the GPU.

Seam 1 (``sparse_conv_forward`` over the reference's pair lists), seam 2
(``generate_subm_indice_pairs`` with its pair lists), seam 3
(``generate_strided_indice_pairs``, the fill queued before the count is
read), seam 4 (the inverse's pair swap) and seam 5 (``dense()``) are taken
from the document's code blocks and run with a small ``_tsc`` module in
place of the binding module they call: the library, its error check, the
shape arrays and the current stream.  Their outputs must equal this
package's: the same pair lists, pair counts and output coordinates bit for
bit, and the same convolution bits (the kernel sums each output in the same
order whatever map it is given).
"""
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from gpu_util import DEV, needs_gpu, say
from trispconv.pytorch import functional as Fn
from trispconv.pytorch.indices import IndiceData, generate_subm_indice_pairs
from trispconv_amd import _lib as L
from trispconv_amd.pytorch.indices import _to3
from trispconv_amd.pytorch.weight import normalize_spconv_weight

pytestmark = [pytest.mark.gpu, needs_gpu]
ROOT = Path(__file__).resolve().parent.parent
BOUNDARY_DOC = ROOT / "INTEGRATION.md"


class _Tsc:
    """What the snippets call ``_tsc``: the ctypes library and helpers."""

    lib = None

    @staticmethod
    def check(rc, what="trispconv"):
        L.check(rc, what)

    @staticmethod
    def i3(v):
        return L.i3(v)

    @staticmethod
    def stream():
        return torch.cuda.current_stream(DEV).cuda_stream

    @staticmethod
    def available():
        return True


def _run_snippet(heading: str, **names) -> dict:
    """Executes the first python block under ``heading`` and returns its
    names; the binding module it calls (and may import) is the ``_tsc``
    above."""
    text = BOUNDARY_DOC.read_text()
    section = text.split(heading, 1)[1]
    block = re.findall(r"```python\n(.*?)```", section, flags=re.S)[0]
    assert "_tsc." in block
    _Tsc.lib = L.lib()
    scope = {"torch": torch, "_tsc": _Tsc, **names}
    exec(compile(block.replace("from . import _tsc", "pass"), str(BOUNDARY_DOC), "exec"), scope)
    return scope


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
    return idx[np.random.default_rng(seed + 1).permutation(len(idx))]


def test_seam_2_subm_pairs_snippet_runs_as_written():
    shape, B = (20, 22, 24), 2
    idx = _tiny(91, shape, B, 1800)
    x = torch.from_numpy(idx).to(DEV)
    scope = _run_snippet("## Seam 2", IndiceData=IndiceData, _to3=_to3)
    say("boundary document, seam 2 snippet:", idx.shape, shape)
    got = scope["generate_subm_indice_pairs"](x, shape, B, 3, 1)
    exp = generate_subm_indice_pairs(x, shape, B, 3, 1)
    assert torch.equal(got.pair_num, exp.pair_num)
    for k in range(27):
        assert torch.equal(got.pairs_in[k].cpu(), exp.pairs_in[k].cpu()), k
        assert torch.equal(got.pairs_out[k].cpu(), exp.pairs_out[k].cpu()), k


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_seam_1_conv_snippet_runs_as_written(dtype):
    shape, B = (20, 22, 24), 2
    idx = _tiny(93, shape, B, 1800)
    x = torch.from_numpy(idx).to(DEV)
    data = generate_subm_indice_pairs(x, shape, B, 3, 1)
    n = len(idx)
    g = torch.Generator().manual_seed(5)
    feats = torch.randn(n, 32, generator=g).to(DEV).to(dtype)
    krsc = (torch.randn(64, 3, 3, 3, 32, generator=g) * 0.1).to(DEV).to(dtype)
    bias = (torch.randn(64, generator=g) * 0.1).to(DEV).to(dtype)
    weight = normalize_spconv_weight(krsc, (3, 3, 3), 32, 64)  # (K, C_in, C_out)
    scope = _run_snippet("## Seam 1 ", )
    say("boundary document, seam 1 snippet:", dtype, n)
    got = scope["sparse_conv_forward"](feats, weight, bias, data, n)
    exp = Fn.sparse_conv_forward(feats, weight, bias, data, n)
    assert got.dtype == dtype and got.shape == (n, 64)
    assert torch.equal(got, exp)


def test_seam_3_and_4_strided_and_inverse_snippets_run_as_written():
    from trispconv.pytorch.indices import generate_inverse_indice_pairs, generate_strided_indice_pairs
    shape, B = (21, 18, 25), 2
    idx = _tiny(95, shape, B, 1500)
    x = torch.from_numpy(idx).to(DEV)
    s3 = _run_snippet("## Seam 3", IndiceData=IndiceData, _to3=_to3)
    s4 = _run_snippet("## Seam 4", IndiceData=IndiceData)
    say("boundary document, seam 3 and 4 snippets:", idx.shape, shape)
    got = s3["generate_strided_indice_pairs"](x, shape, B, 3, 2, 1, 1)
    exp = generate_strided_indice_pairs(x, shape, B, 3, 2, 1, 1)
    assert tuple(got.output_spatial_shape) == tuple(exp.output_spatial_shape)
    assert torch.equal(got.out_indices, exp.out_indices)
    assert torch.equal(got.pair_num, exp.pair_num)
    for k in range(27):
        assert torch.equal(got.pairs_in[k].cpu(), exp.pairs_in[k].cpu()), k
        assert torch.equal(got.pairs_out[k].cpu(), exp.pairs_out[k].cpu()), k
    inv_got = s4["inverse_indice_pairs"](got)
    inv_exp = generate_inverse_indice_pairs(exp)
    assert torch.equal(inv_got.out_indices, inv_exp.out_indices)
    for k in range(27):
        assert torch.equal(inv_got.pairs_in[k].cpu(), inv_exp.pairs_in[k].cpu()), k
        assert torch.equal(inv_got.pairs_out[k].cpu(), inv_exp.pairs_out[k].cpu()), k


@pytest.mark.parametrize("channels_first", [True, False])
def test_seam_5_dense_snippet_runs_as_written(channels_first):
    import trispconv.pytorch as spconv
    shape, B = (9, 10, 11), 2
    idx = _tiny(97, shape, B, 300)
    feats = torch.randn(len(idx), 5, generator=torch.Generator().manual_seed(3)).to(DEV)
    t = spconv.SparseConvTensor(feats, torch.from_numpy(idx).to(DEV), list(shape), B)
    scope = _run_snippet("## Seam 5")
    say("boundary document, seam 5 snippet:", channels_first)
    got = scope["dense"](t, channels_first)
    assert torch.equal(got, t.dense(channels_first))
