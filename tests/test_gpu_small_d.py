"""GPU parity of the D = 1 and D = 2 (M = 8) column-per-lane kernels (bssm_d1.hip, bssm_d2.hip).

The forwards take calls whose streams are 16-byte aligned with T a multiple
of 4 (and, for D = 1, the checkpoint chunk too); the backwards take the
library's preferred checkpoint chunk (16 for D = 1, 8 for D = 2), and for
D = 1 also T a multiple of 16.  The shapes
below are chosen to reach them, with N = 37 leaving idle sequence slots in
the last wave and T values that end on partial forward blocks and on partly
filled backward blocks.  Other shapes take the generic kernels, which serve
as a second reference here.  Tolerance (north star): 1e-5 relative, 1e-4
absolute.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O
from tests.test_gpu_parity import ABIS, _case, _fixed_dynamics, _oracle_forward, close

pytestmark = pytest.mark.gpu

DIMS = [1, 2]
CHUNK = {1: 16, 2: 8}  # the backward's checkpoint chunk
# D = 2: T = 20, 36 and 44 give 3, 5 and 6 backward blocks, so the last block
# is alone in its pair of whole-row k/d/q loads (odd counts), with full and
# partial last blocks.
BWD_TIMES = {1: [16, 48, 64, 80], 2: [4, 12, 16, 20, 36, 44, 60]}
BWD_CASES = [(D, t) for D in DIMS for t in BWD_TIMES[D]]


def _ext(d):
    from bayes_ssm import fused_cuda

    e = fused_cuda._load_extension(d)
    assert e is not None
    return e


def _forward(ext, dev, fixed, chunk):
    fn = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    return fn(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk, 1e-6)


@pytest.mark.parametrize("D", DIMS)
@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("chunk", [4, 12, 16, 64])
@pytest.mark.parametrize("t", [4, 60, 64, 68, 200])
def test_small_d_forward_matches_oracle(cuda_device, D, fixed, chunk, t):
    print(f"small-D forward D={D} fixed={fixed} chunk={chunk} t={t}", flush=True)
    ext = _ext(D)
    n = 37
    cpu, dev = _case(n, t, D, seed=500 + 7 * D + t + chunk, device=cuda_device)
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


@pytest.mark.parametrize("D", DIMS)
def test_small_d_forward_matches_generic_kernel(cuda_device, D):
    """Chunk 13 (not a multiple of 4) takes the generic kernel: same recurrence, same checkpoint indexing."""
    ext = _ext(D)
    n, t = 45, 104
    _, dev = _case(n, t, D, seed=77, device=cuda_device)
    fast = _forward(ext, dev, False, 52)
    generic = _forward(ext, dev, False, 13)
    torch.cuda.synchronize()
    for name, a, b in zip(("y", "mean_T", "cov_T"), fast[:3], generic[:3]):
        close(a, b, name)
    close(fast[3], generic[3][:, ::4], "bmean")
    close(fast[4], generic[4][:, ::4], "bcov")


@pytest.mark.parametrize("D,t", BWD_CASES)
@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
@pytest.mark.parametrize("final_grads", [False, True])
def test_small_d_backward_matches_oracle(cuda_device, D, t, abi, final_grads):
    name, fixed, nout = abi
    print(f"small-D backward D={D} {name} final_grads={final_grads} t={t}", flush=True)
    ext = _ext(D)
    n, chunk = 37, CHUNK[D]
    cpu, dev = _case(n, t, D, seed=600 + 11 * D + t, device=cuda_device)
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


@pytest.mark.parametrize("D", DIMS)
def test_small_d_backward_matches_generic_kernel(cuda_device, D):
    """The preferred chunk (column-per-lane kernel) against chunk 4 (generic kernel) at T = 112."""
    ext = _ext(D)
    n, t = 29, 112
    _, dev = _case(n, t, D, seed=91, device=cuda_device)
    out = {}
    for chunk in (CHUNK[D], 4):
        _, _, _, bm, bc = _forward(ext, dev, False, chunk)
        out[chunk] = ext.backward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                          dev["c0"], bm, bc, dev["gy"], dev["gmf"], dev["gcf"], chunk, 1e-6)
    torch.cuda.synchronize()
    for name, a, b in zip(["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"], out[CHUNK[D]], out[4]):
        close(a, b, name)


@pytest.mark.parametrize("D", DIMS)
def test_small_d_autograd_config_shape(cuda_device, D):
    """The autograd boundary at T = 512 (the preferred checkpoint chunk) against the oracle on a subset."""
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


@pytest.mark.parametrize("D", DIMS)
def test_small_d_unaligned_streams_take_generic_kernels(cuda_device, D):
    """Streams that start off a 16-byte boundary fail the column-per-lane kernels' preconditions: same results."""
    ext = _ext(D)
    n, t, chunk = 9, 64, CHUNK[D]
    cpu, dev = _case(n, t, D, seed=300 + D, device=cuda_device)
    shifted = {}
    for name, x in dev.items():
        flat = torch.empty(x.numel() + 1, device=cuda_device)
        view = flat[1:].view(x.shape)  # contiguous, 4 bytes past an aligned start
        view.copy_(x)
        shifted[name] = view
    assert shifted["k"].data_ptr() % 16 != 0
    outs = {}
    for label, src in (("aligned", dev), ("shifted", shifted)):
        y, mT, cT, bm, bc = _forward(ext, src, False, chunk)
        grads = ext.backward_chunked(src["k"], src["v"], src["q"], src["d"], src["p"], src["r"], src["m0"],
                                     src["c0"], bm, bc, src["gy"], src["gmf"], src["gcf"], chunk, 1e-6)
        outs[label] = [y, mT, cT, bm, bc, *grads]
    torch.cuda.synchronize()
    names = ["y", "mean_T", "cov_T", "bmean", "bcov", "gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"]
    for name, a, b in zip(names, outs["aligned"], outs["shifted"]):
        close(a, b, name)


@pytest.mark.parametrize("D", DIMS)
def test_small_d_single_sequence_and_long_chunk(cuda_device, D):
    """N = 1 (one sequence in the wave) and a forward chunk longer than T."""
    ext = _ext(D)
    n, t = 1, 32
    cpu, dev = _case(n, t, D, seed=410 + D, device=cuda_device)
    y, mT, cT, bm, bc = _forward(ext, dev, False, 64)
    torch.cuda.synchronize()
    ey, em, ec = _oracle_forward(cpu, False)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    assert bm.shape == (1, 2, D, 8)
    assert torch.equal(bm[:, 1].cpu(), mT.cpu()) and torch.equal(bm[:, 0].cpu(), dev["m0"].cpu())
    chunk = CHUNK[D]
    _, _, _, bm, bc = _forward(ext, dev, False, chunk)
    grads = ext.backward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"],
                                 bm, bc, dev["gy"], dev["gmf"], dev["gcf"], chunk, 1e-6)
    torch.cuda.synchronize()
    f64 = {k: x.double() for k, x in cpu.items()}
    _, _, _, eg = O.diagonal_grads(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                                   f64["gy"], f64["gmf"], f64["gcf"])
    for name, a, e in zip(["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"], grads, eg):
        close(a, e, name)
