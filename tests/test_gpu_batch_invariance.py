"""The same sequences inside batches of different size (D4M8, float32 ABI, through the autograd boundary).

The library picks the D4M8 kernels from the sequence count N (``bssm_small_batch_limit`` in include/bssm.h):
at N = 2048 (B32 x H64, one GPU's share of config 3 under 8-way data parallelism) the forward and the backward
run the row-per-sequence split kernels; at N = 16384 (config 3, B256 x H64) the row forward and the rotated-
layout backward.  The forward kernels of the row layout are bitwise one another, so outputs and final states
must be identical bits.  The rotated-layout backward replays and reverses each chunk with its own summation
order, so gradients may differ in the last bits between the two batch sizes; they must agree to the north
star's tolerance (1e-5 relative, 1e-4 absolute), and the test prints the largest differences it saw.
The reference keeps one launch shape for every N (persistent_bayes_chunked_d4m8.cu:195-245, :467).
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-4


def _inputs(n, t, device, seed):
    """Config-3 distributions (bench.make_workload), drawn on the device."""
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(n, t, 4, device=device, generator=g).bfloat16().float()
    v = torch.randn(n, t, 8, device=device, generator=g).bfloat16().float()
    q = torch.randn(n, t, 4, device=device, generator=g).bfloat16().float()
    dec = torch.sigmoid(torch.randn(n, t, 4, device=device, generator=g) + 2.0)
    p = torch.nn.functional.softplus(torch.randn(n, t, device=device, generator=g) - 3.0)
    r = 1e-4 + torch.nn.functional.softplus(torch.randn(n, t, device=device, generator=g))
    gy = torch.randn(n, t, 8, device=device, generator=g)
    return [k, v, q, dec, p, r], gy


def _run(xs, gy, rows):
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    leaves = [x[:rows].clone().requires_grad_(True) for x in xs]
    m0 = torch.zeros(rows, 4, 8, device=gy.device)
    c0 = torch.eye(4, device=gy.device).expand(rows, 4, 4).contiguous()
    y, mT, cT = fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=64, denominator_floor=1e-6)
    grads = torch.autograd.grad(y, leaves, gy[:rows])
    return y.detach(), mT, cT, grads


@pytest.mark.parametrize("small", [2048, 32])
def test_same_sequences_in_config3_and_smaller_batch(cuda_device, small):
    n, t = 16384, 512
    print(f"batch invariance N={n} vs N={small}, T={t}", flush=True)
    xs, gy = _inputs(n, t, cuda_device, seed=3)
    big = _run(xs, gy, n)
    part = _run(xs, gy, small)
    torch.cuda.synchronize()
    for name, a, b in zip(("y", "mean_T", "cov_T"), big[:3], part[:3]):
        assert torch.equal(a[:small], b), f"{name}: the forward must be bitwise independent of the batch size"
    worst = []
    for name, a, b in zip(("gk", "gv", "gq", "gd", "gp", "gr"), big[3], part[3]):
        a, b = a[:small].double(), b.double()
        diff = (a - b).abs()
        worst.append(f"{name} max abs {diff.max().item():.2e} max rel "
                     f"{(diff / b.abs().clamp_min(1e-3)).max().item():.2e}")
        torch.testing.assert_close(a, b, rtol=RTOL, atol=ATOL, msg=lambda m: f"{name}: {m}")
    print("; ".join(worst), flush=True)
