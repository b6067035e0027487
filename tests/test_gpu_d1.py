"""GPU parity of the D = 1, M = 8 column-per-lane kernels (bssm_d1.hip) against the CPU oracle.

These kernels take D1 calls whose streams are 16-byte aligned with T and the
checkpoint chunk multiples of 4 (forward), and chunk 16 with T a positive
multiple of 16 (backward); the shapes below are chosen to reach them, with
N = 37 leaving idle sequence slots in the last wave and T values that end
on partial 64-token forward blocks and on half-filled 32-token backward
blocks.  Other D1 shapes take the generic kernels, which serve as a second
reference here.  Tolerance (north star): 1e-5 relative, 1e-4 absolute.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O
from tests.test_gpu_parity import ABIS, _case, _fixed_dynamics, _oracle_forward, close

pytestmark = pytest.mark.gpu

D = 1


@pytest.fixture(scope="module")
def ext(cuda_device):
    from bayes_ssm import fused_cuda

    e = fused_cuda._load_extension(D)
    assert e is not None
    return e


def _forward(ext, dev, fixed, chunk):
    fn = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    return fn(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk, 1e-6)


@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("chunk", [4, 12, 16, 64])
@pytest.mark.parametrize("t", [4, 60, 64, 68, 200])
def test_d1_forward_matches_oracle(ext, cuda_device, fixed, chunk, t):
    print(f"d1 forward fixed={fixed} chunk={chunk} t={t}", flush=True)
    n = 37
    cpu, dev = _case(n, t, D, seed=500 + t + chunk, device=cuda_device)
    y, mT, cT, bm, bc = _forward(ext, dev, fixed, chunk)
    torch.cuda.synchronize()
    ref = _fixed_dynamics(cpu) if fixed else cpu
    ey, em, ec = _oracle_forward(ref, False)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    nb = -(-t // chunk)
    assert bm.shape == (n, nb + 1, D, 8) and bc.shape == (n, nb + 1, D, D)
    f64 = {k: x.double() for k, x in ref.items()}
    ebm, ebc = O.checkpoints(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                             chunk, 1e-6)
    close(bm, ebm, "bmean")
    close(bc, ebc, "bcov")
    assert torch.equal(bm[:, nb].cpu(), mT.cpu()) and torch.equal(bc[:, nb].cpu(), cT.cpu())
    assert torch.equal(bm[:, 0].cpu(), dev["m0"].cpu()) and torch.equal(bc[:, 0].cpu(), dev["c0"].cpu())


def test_d1_forward_matches_generic_kernel(ext, cuda_device):
    """Chunk 13 (not a multiple of 4) takes the generic kernel: same recurrence, same checkpoint indexing."""
    n, t = 45, 104
    _, dev = _case(n, t, D, seed=77, device=cuda_device)
    fast = _forward(ext, dev, False, 52)
    generic = _forward(ext, dev, False, 13)
    torch.cuda.synchronize()
    for name, a, b in zip(("y", "mean_T", "cov_T"), fast[:3], generic[:3]):
        close(a, b, name)
    close(fast[3], generic[3][:, ::4], "bmean")
    close(fast[4], generic[4][:, ::4], "bcov")


@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
@pytest.mark.parametrize("final_grads", [False, True])
@pytest.mark.parametrize("t", [16, 48, 64, 80])
def test_d1_backward_matches_oracle(ext, cuda_device, abi, final_grads, t):
    name, fixed, nout = abi
    print(f"d1 backward {name} final_grads={final_grads} t={t}", flush=True)
    n, chunk = 37, 16
    cpu, dev = _case(n, t, D, seed=600 + t, device=cuda_device)
    ref = _fixed_dynamics(cpu) if fixed else cpu
    _, _, _, bm, bc = _forward(ext, dev, fixed, chunk)
    gmf = dev["gmf"] if final_grads else None
    gcf = dev["gcf"] if final_grads else None
    if hasattr(ext, name):
        grads = getattr(ext, name)(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                   dev["c0"], bm, bc, dev["gy"], gmf, gcf, chunk, 1e-6)
    else:
        grads = ext._backward("bssm_" + name, fixed, nout, dev["k"], dev["v"], dev["q"], dev["d"], dev["p"],
                              dev["r"], dev["m0"], dev["c0"], bm, bc, (), dev["gy"], gmf, gcf, chunk, 1e-6)
    torch.cuda.synchronize()
    assert len(grads) == nout
    f64 = {k: x.double() for k, x in ref.items()}
    _, _, _, eg = O.diagonal_grads(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                                   f64["gy"], f64["gmf"] if final_grads else None,
                                   f64["gcf"] if final_grads else None)
    names = ["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"]
    for i in range(nout):
        if fixed and names[i] in ("gd", "gp", "gr"):
            assert torch.count_nonzero(grads[i]) == 0, f"{names[i]} must be zero for fixed dynamics"
            continue
        close(grads[i], eg[i], names[i])


def test_d1_backward_matches_generic_kernel(ext, cuda_device):
    """Chunk 16 (column-per-lane kernel) against chunk 8 (generic kernel) at T = 112."""
    n, t = 29, 112
    _, dev = _case(n, t, D, seed=91, device=cuda_device)
    out = {}
    for chunk in (16, 8):
        _, _, _, bm, bc = _forward(ext, dev, False, chunk)
        out[chunk] = ext.backward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                          dev["c0"], bm, bc, dev["gy"], dev["gmf"], dev["gcf"], chunk, 1e-6)
    torch.cuda.synchronize()
    for name, a, b in zip(["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"], out[16], out[8]):
        close(a, b, name)


def test_d1_autograd_config2_shape(cuda_device):
    """The autograd boundary at T = 512 (preferred checkpoint 16 for D = 1) against the oracle on a subset."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    n, t = 300, 512
    k, v, q, dec, p, r, gy = O.make_inputs(n, t, D, seed=12)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (k, v, q, dec, p, r)]
    m0 = torch.zeros(n, D, 8, device=cuda_device)
    c0 = torch.ones(n, D, D, device=cuda_device)
    y, _, _ = fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=64, denominator_floor=1e-6)
    y.backward(gy.to(cuda_device))
    torch.cuda.synchronize()
    idx = torch.tensor([0, 7, 8, 150, n - 1])
    sub = [x[idx].double() for x in (k, v, q, dec, p, r)]
    ey, _, _, eg = O.diagonal_grads(*sub, torch.zeros(len(idx), D, 8, dtype=torch.float64),
                                    torch.ones(len(idx), D, D, dtype=torch.float64), gy[idx].double())
    close(y[idx.to(cuda_device)], ey, "y")
    for i, name in enumerate(("k", "v", "q", "d", "p", "r")):
        close(leaves[i].grad[idx.to(cuda_device)], eg[i], "grad " + name)
