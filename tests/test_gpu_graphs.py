"""HIP graph capture of SparseLinear's training step.

The library's entry points are capture-safe: they allocate nothing, read
nothing back on the host and clear nothing with hipMemsetAsync (every output
is written by a kernel). A captured forward + backward of a SparseLinear
layer therefore holds kernel nodes only, and every replay gives the eager
step's bits: replays here alternate with eager steps and synchronizations,
and each one is compared with the eager result. Both layer paths: the
general one (transpose cache, segment dW) and the narrow one (<= 64 outputs).
"""

from __future__ import annotations

import pytest
import torch

import sparsecore_amd as slk
from sparsecore_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(384, 1536, 2048), (512, 10, 256)],
                         ids=["general", "narrow"])
def test_sparselinear_step_graph_is_kernels_only_and_replays_exactly(dev, shape):
    K, M, T = shape
    torch.manual_seed(5)
    layer = slk.SparseLinear(K, M, sparsity=0.9).to(dev)
    params = list(layer.parameters())
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    x = torch.randn(T, K, generator=g, device=dev).requires_grad_(True)
    gy = torch.randn(T, M, generator=g, device=dev)

    def step():
        y = layer(x)
        grads = torch.autograd.grad(y, [x] + params, gy)
        return (y.detach(),) + tuple(grads)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):  # builds the transpose cache and the schedules
            step()
    torch.cuda.current_stream().wait_stream(side)
    want = [t.clone() for t in step()]
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        outs = step()
    nodes = _lib.graph_node_types(graph)
    print(f"[graph {shape}] node types {nodes}", flush=True)
    assert nodes.get("kernel", 0) > 0
    assert set(nodes) <= {"kernel", "empty"}, nodes
    graph.instantiate()

    for r in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, want)):
            assert torch.equal(a, b), f"replay {r}: output {i} differs from the eager step"
        eager = step()  # eager work between replays
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(eager, want))


def test_two_stream_forward_captures_and_replays_exactly(dev, tune):
    """slk_spmm's split forward on two streams (a skewed matrix with phase
    bounds on the LDS-staged path) inside a HIP graph: the fork and join
    become graph edges (kernel nodes only), and every replay gives the eager
    bits, with eager work and synchronizations between the replays."""
    import numpy as np

    import oracle
    from helpers import from_oracle

    tune(spmm_kernel=1)
    c = oracle.zipf_rows(3000, 700, 0.03, 1.1, seed=92, sigma=0.5)
    W = from_oracle(c, dev)
    v = W._view_phased(3)
    assert v.n_heavy_rows > 0 and v.n_phases == 3
    g = torch.Generator(device=dev)
    g.manual_seed(92)
    X = torch.randn(700, 520, generator=g, device=dev)
    Y = torch.empty(3000, 520, device=dev)
    _lib.spmm(v, X, Y)  # eager first: creates the library's side stream
    torch.cuda.synchronize()
    want = Y.clone()
    assert np.array_equal(want.cpu().numpy(), oracle.spmm(c, X.cpu().numpy()))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _lib.spmm(v, X, Y)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        _lib.spmm(v, X, Y)
    nodes = _lib.graph_node_types(graph)
    print(f"[graph two streams] node types {nodes}", flush=True)
    assert nodes.get("kernel", 0) >= 2 and set(nodes) <= {"kernel", "empty"}, nodes
    graph.instantiate()
    for r in range(4):
        Y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(Y, want), f"replay {r}"
        _lib.spmm(v, X, Y)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(Y, want)
