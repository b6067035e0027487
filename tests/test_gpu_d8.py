"""GPU parity of the D = 8, M = 8 kernels against the float64 oracle.

Both kernels are bssm_d8.hip for T a positive multiple of 8 (the forward at any chunk, the backward at the
library's preferred checkpoint chunk, 8); other T take the generic kernels (bssm_recurrence.hip; T = 44 below).
Their reference is bayes_ssm/persistent_bayes_chunked_d8.cu:209-419.  Cases: the forward's outputs, final state
and every checkpoint record at chunks that are and are not multiples of 8 (records between and inside 8-token
blocks), with full and partial 16-token tiles, their chunk invariance (bit for bit);
every backward ABI, with and without final-state gradients, T from one chunk to several; N = 13 (a partial
last wave of 8 sequences).  Tolerance (north star): 1e-5 relative, 1e-4 absolute.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O
from tests.test_gpu_parity import ABIS, _case, _fixed_dynamics, close

pytestmark = pytest.mark.gpu

D = 8


@pytest.fixture(scope="module")
def ext(cuda_device):
    from bayes_ssm import _hip, fused_cuda

    assert _hip.preferred_checkpoint(D) == 8
    e = fused_cuda._load_extension(D)
    assert e is not None
    return e


@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("chunk", [1, 5, 8, 13, 16, 64])
@pytest.mark.parametrize("t", [8, 16, 40, 44, 64])
def test_d8_forward_matches_oracle(ext, cuda_device, fixed, chunk, t):
    print(f"d8 forward fixed={fixed} chunk={chunk} t={t}", flush=True)
    n = 13
    cpu, dev = _case(n, t, D, seed=400 + t + chunk, device=cuda_device)
    ref = _fixed_dynamics(cpu) if fixed else cpu
    fwd = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    y, mT, cT, bm, bc = fwd(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"],
                            chunk, 1e-6)
    torch.cuda.synchronize()
    f64 = {k: x.double() for k, x in ref.items()}
    ey, em, ec = O.run_diagonal(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                                1e-6)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    nb = -(-t // chunk)
    assert bm.shape == (n, nb + 1, D, 8) and bc.shape == (n, nb + 1, D, D)
    ebm, ebc = O.checkpoints(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                             chunk, 1e-6)
    close(bm, ebm, "bmean")
    close(bc, ebc, "bcov")
    # Record 0 is the initial state as given; record nb is the final state.
    assert torch.equal(bm[:, 0], dev["m0"]) and torch.equal(bc[:, 0], dev["c0"])
    assert torch.equal(bm[:, nb], mT) and torch.equal(bc[:, nb], cT)


def test_d8_forward_chunk_invariance_bitexact(ext, cuda_device):
    """The chunk only places the records: outputs are the same bits for every chunk, and record c of chunk
    k is record c * k of chunk 1 (records inside an 8-token block and at its end alike)."""
    n, t = 16, 96
    _, dev = _case(n, t, D, seed=433, device=cuda_device)
    runs = {c: ext.forward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                   dev["c0"], c, 1e-6) for c in (1, 3, 8, 12, 24, 96, 200)}
    base = runs[1]
    for c, out in runs.items():
        for a, b in zip(out[:3], base[:3]):
            assert torch.equal(a, b), f"chunk {c} changes the recurrence"
        idx = torch.arange(0, t + 1, c, device=dev["k"].device)
        if idx[-1] != t:
            idx = torch.cat([idx, torch.tensor([t], device=idx.device)])
        assert torch.equal(out[3], base[3][:, idx]), f"bmean records, chunk {c}"
        assert torch.equal(out[4], base[4][:, idx]), f"bcov records, chunk {c}"


@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
@pytest.mark.parametrize("final_grads", [False, True])
@pytest.mark.parametrize("t", [8, 16, 40, 64])
def test_d8_backward_matches_oracle(ext, cuda_device, abi, final_grads, t):
    name, fixed, nout = abi
    print(f"d8 backward {name} final_grads={final_grads} t={t}", flush=True)
    n, chunk = 13, 8
    cpu, dev = _case(n, t, D, seed=300 + t, device=cuda_device)
    ref = _fixed_dynamics(cpu) if fixed else cpu
    fwd = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    _, _, _, bm, bc = fwd(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk,
                          1e-6)
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


def test_d8_backward_sequences_independent(ext, cuda_device):
    """A sequence's outputs, records and gradients are the same bits whichever wave slot it lands in (8
    sequences per wave, forward and backward)."""
    n, t, chunk = 16, 24, 8
    _, dev = _case(n, t, D, seed=321, device=cuda_device)
    perm = torch.roll(torch.arange(n), 3)

    def run(x):
        fwd = ext.forward_chunked(x["k"], x["v"], x["q"], x["d"], x["p"], x["r"], x["m0"], x["c0"], chunk, 1e-6)
        bm, bc = fwd[3], fwd[4]
        return (*fwd, *ext.backward_chunked(x["k"], x["v"], x["q"], x["d"], x["p"], x["r"], x["m0"], x["c0"], bm,
                                            bc, x["gy"], x["gmf"], x["gcf"], chunk, 1e-6))

    base = run(dev)
    moved = run({k: v[perm.to(v.device)].contiguous() for k, v in dev.items()})
    for a, b in zip(base, moved):
        assert torch.equal(a[perm.to(a.device)], b)
