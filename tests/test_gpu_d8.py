"""GPU parity of the D = 8, M = 8 backward kernel (bssm_d8.hip) against the float64 oracle.

The kernel runs for T a positive multiple of 8 with the library's preferred checkpoint chunk (8); its
reference is bayes_ssm/persistent_bayes_chunked_d8.cu:358-419.  Cases: every backward ABI, with and without
final-state gradients, T from one chunk to several, and N = 13 (a partial last wave of 8 sequences).
Tolerance (north star): 1e-5 relative, 1e-4 absolute.
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
    """A sequence's gradients are the same bits whichever wave slot it lands in (8 sequences per wave)."""
    n, t, chunk = 16, 24, 8
    _, dev = _case(n, t, D, seed=321, device=cuda_device)
    perm = torch.roll(torch.arange(n), 3)

    def run(x):
        _, _, _, bm, bc = ext.forward_chunked(x["k"], x["v"], x["q"], x["d"], x["p"], x["r"], x["m0"], x["c0"],
                                              chunk, 1e-6)
        return ext.backward_chunked(x["k"], x["v"], x["q"], x["d"], x["p"], x["r"], x["m0"], x["c0"], bm, bc,
                                    x["gy"], x["gmf"], x["gcf"], chunk, 1e-6)

    base = run(dev)
    moved = run({k: v[perm.to(v.device)].contiguous() for k, v in dev.items()})
    for a, b in zip(base, moved):
        assert torch.equal(a[perm.to(a.device)], b)
