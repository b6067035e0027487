"""The fused autograd boundary under HIP graph capture (torch.cuda.graph).

The reference's training example captures its whole step in a CUDA graph
(example/train_6layer.py), so the fused core must be capturable: the C ABI
neither allocates, synchronizes nor records memsets, outputs come from torch's
graph pool, and every launch goes to torch's current stream (the capture
stream, in forward and in the autograd backward alike).

Each case captures forward + ``torch.autograd.grad`` once, then replays it
several times.  Before each replay new input values are copied into the
captured leaves; after it the program runs the same step eagerly on those
inputs.  Every replay must give the eager step's bits (the kernels are
deterministic), which also checks that nothing captured kept the first call's
values.
"""
from __future__ import annotations

import pytest
import torch

from tests.test_gpu_parity import _case

pytestmark = pytest.mark.gpu


def _inputs(n, t, d, seed, device):
    _, dev = _case(n, t, d, seed=seed, device=device)
    return dev


@pytest.mark.parametrize("d", [1, 2, 4, 8])
def test_graph_replays_match_eager(cuda_device, d):
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    n, t = 80, 48
    print(f"graph capture d={d} n={n} t={t}", flush=True)
    first = _inputs(n, t, d, seed=700 + d, device=cuda_device)
    names = ("k", "v", "q", "d", "p", "r", "m0", "c0")
    leaves = [first[k].clone().requires_grad_(True) for k in names]
    cot = [first[k].clone() for k in ("gy", "gmf", "gcf")]

    def step():
        y, mf, cf = fused_diagonal_bayesian(*leaves, chunk_length=16, denominator_floor=1e-6)
        grads = torch.autograd.grad((y, mf, cf), leaves, cot)
        return (y.detach(), mf.detach(), cf.detach(), *grads)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    torch.cuda.synchronize()

    for rep in range(4):
        fresh = _inputs(n, t, d, seed=710 + 10 * d + rep, device=cuda_device)
        with torch.no_grad():
            for x, k in zip(leaves, names):
                x.copy_(fresh[k])
            for x, k in zip(cot, ("gy", "gmf", "gcf")):
                x.copy_(fresh[k])
        graph.replay()
        torch.cuda.synchronize()
        got = [x.clone() for x in captured]
        expect = step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, expect)):
            assert torch.equal(a, b), f"replay {rep}: output {i} differs from the eager step"
    del graph
