"""A network forward captured in a HIP graph (torch.cuda.graph) replays to the
same bits as the eager forward.

Once a SparseSequential's pairs are built and cached under their indice_keys
(the first, eager call), a forward makes no host synchronisation and no
allocation outside torch's allocator, and every kernel goes to torch's current
stream, so torch.cuda.graph captures it as is.  Each replay is checked
against an eager forward, with eager work and synchronisations in between.
"""
import pytest
import torch
import torch.nn as nn

import trispconv.pytorch as spconv
from gpu_util import DEV, needs_gpu, say

pytestmark = [pytest.mark.gpu, needs_gpu]


def _bn(c, seed):
    g = torch.Generator().manual_seed(seed)
    bn = nn.BatchNorm1d(c)
    with torch.no_grad():
        bn.weight.copy_(torch.rand(c, generator=g) + 0.5)
        bn.bias.copy_(torch.randn(c, generator=g) * 0.1)
        bn.running_mean.copy_(torch.randn(c, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(c, generator=g) + 0.5)
    return bn


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("fuse", [True, False])
def test_captured_forward_replays_to_the_eager_bits(dtype, fuse):
    torch.manual_seed(3)
    net = spconv.SparseSequential(
        spconv.SubMConv3d(16, 32, 3, indice_key="a"), _bn(32, 1), nn.ReLU(),
        spconv.SparseConv3d(32, 64, 3, stride=2, padding=1, indice_key="down"), _bn(64, 2),
        nn.ReLU(),
        spconv.SubMConv3d(64, 64, 3, indice_key="b"), nn.ReLU(),
        spconv.SparseInverseConv3d(64, 32, 3, indice_key="down"),
    ).to(DEV).to(dtype).eval()
    net.fuse_epilogues = fuse
    g = torch.Generator().manual_seed(5)
    shape = (40, 40, 40)
    cells = torch.randperm(shape[0] * shape[1] * shape[2], generator=g)[:9000]
    idx = torch.stack([torch.zeros_like(cells), cells // 1600, (cells // 40) % 40, cells % 40],
                      1).int()
    feats = torch.randn(len(idx), 16, generator=g).to(dtype)
    x = spconv.SparseConvTensor(feats.to(DEV), idx.to(DEV), list(shape), 1)
    with torch.no_grad():
        eager = net(x)  # builds and caches every pair set and execution order
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.no_grad(), torch.cuda.stream(side):
        for _ in range(2):
            net(x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        captured = net(x)
    for rep in range(3):
        captured.features.fill_(float("nan"))  # nothing left over from the last replay
        graph.replay()
        torch.cuda.synchronize()
        with torch.no_grad():
            again = net(x)  # eager work between replays
        torch.cuda.synchronize()
        say("replay", rep, dtype, "fused" if fuse else "unfused")
        assert torch.equal(captured.indices, eager.indices)
        assert torch.equal(captured.features, eager.features)
        assert torch.equal(again.features, eager.features)
