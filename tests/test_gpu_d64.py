"""GPU parity of the D = M = 64 kernels (bssm_d64.hip) against the CPU oracle.

The reference extension for this shape is bayes_ssm/persistent_bayes_chunked.cu
(exports at :436).  Calls go through the C ABI via the ``fused_cuda``
extension object or the autograd boundary.  Tolerance (north star): 1e-5
relative, 1e-4 absolute against the float64 oracle; chunk invariance and the
checkpoint layout are bit-exact.  Keys and queries are drawn N(0, 1/D).

Conventions of the D = 64 reference kernels reproduced here:
* the initial-covariance gradient is symmetric: the u = P'k adjoint enters as
  sym(gu k^T) (persistent_bayes_chunked.cu:329-333), so it equals the
  symmetric part of the oracle's (autograd) gradient;
* the first covariance update mirrors the initial covariance's upper triangle
  (:221-241), while u of the first token reads its rows as given -- the two
  agree for a symmetric initial covariance, and the asymmetric case is pinned
  by a restatement of that first step below.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-4
D = 64


def close(actual, expected, name="", rtol=RTOL, atol=ATOL):
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    torch.testing.assert_close(actual, expected, rtol=rtol, atol=atol, msg=lambda m: f"{name}: {m}")


@pytest.fixture(scope="module")
def ext(cuda_device):
    from bayes_ssm import fused_cuda

    e = fused_cuda._load_extension(D)
    assert e is not None and e.value_dim == D
    return e


def _case(n, t, seed, device, asymmetric=False):
    k, v, q, dec, p, r, gy = O.make_inputs(n, t, D, D, seed=seed)
    k = k / D ** 0.5
    q = q / D ** 0.5
    g = torch.Generator().manual_seed(seed + 100)
    m0 = 0.2 * torch.randn(n, D, D, generator=g)
    a = torch.randn(n, D, D, generator=g)
    c0 = a @ a.transpose(-1, -2) / D + 0.5 * torch.eye(D)
    c0 = 0.5 * (c0 + c0.transpose(-1, -2))
    if asymmetric:
        c0 = c0 + 0.05 * torch.randn(n, D, D, generator=g)
    gmf = torch.randn(n, D, D, generator=g)
    gcf = torch.randn(n, D, D, generator=g)
    cpu = dict(k=k, v=v, q=q, d=dec, p=p, r=r, m0=m0, c0=c0, gy=gy, gmf=gmf, gcf=gcf)
    dev = {name: x.to(device).contiguous() for name, x in cpu.items()}
    return cpu, dev


def _fixed(c):
    out = dict(c)
    out["d"] = torch.full_like(c["d"], O.FIXED_DECAY)
    out["p"] = torch.full_like(c["p"], O.FIXED_PROCESS)
    out["r"] = torch.full_like(c["r"], O.FIXED_OBSERVATION)
    return out


def _f64(c):
    return {k: x.double() for k, x in c.items()}


def _sym(x):
    return 0.5 * (x + x.transpose(-1, -2))


@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("chunk", [1, 8, 13, 64])
@pytest.mark.parametrize("t", [1, 24])
def test_forward_matches_oracle(ext, cuda_device, fixed, chunk, t):
    print(f"d64 forward fixed={fixed} chunk={chunk} t={t}", flush=True)
    n = 5
    cpu, dev = _case(n, t, seed=chunk + t, device=cuda_device)
    fn = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    y, mT, cT, bm, bc = fn(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk,
                           1e-6)
    torch.cuda.synchronize()
    ref = _f64(_fixed(cpu) if fixed else cpu)
    ey, em, ec = O.run_diagonal(ref["k"], ref["v"], ref["q"], ref["d"], ref["p"], ref["r"], ref["m0"], ref["c0"],
                                1e-6)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    nb = -(-t // chunk)
    assert bm.shape == (n, nb + 1, D, D) and bc.shape == (n, nb + 1, D, D)
    ebm, ebc = O.checkpoints(ref["k"], ref["v"], ref["q"], ref["d"], ref["p"], ref["r"], ref["m0"], ref["c0"],
                             chunk, 1e-6)
    close(bm, ebm, "bmean")
    close(bc, ebc, "bcov")
    assert torch.equal(bm[:, nb].cpu(), mT.cpu()) and torch.equal(bc[:, nb].cpu(), cT.cpu())
    assert torch.equal(bm[:, 0].cpu(), cpu["m0"]) and torch.equal(bc[:, 0].cpu(), cpu["c0"])
    # The covariance stays bitwise symmetric (mirrored update).
    assert torch.equal(cT, cT.transpose(-1, -2))


def test_forward_chunk_invariance_bitexact(ext, cuda_device):
    """Outputs are bitwise identical for every chunk; bm/bc index c is the state before token c*chunk."""
    n, t = 4, 32
    _, dev = _case(n, t, seed=3, device=cuda_device)
    runs = {c: ext.forward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"],
                                   c, 1e-6) for c in (4, 8, 16, 32, 50)}
    base = runs[8]
    for c, out in runs.items():
        for a, b in zip(out[:3], base[:3]):
            assert torch.equal(a, b), f"chunk {c} changes the recurrence"
    for c in (8, 16):
        step = c // 4
        assert torch.equal(runs[c][3], runs[4][3][:, ::step]), f"bmean layout chunk {c}"
        assert torch.equal(runs[c][4], runs[4][4][:, ::step]), f"bcov layout chunk {c}"


def _first_step_mirrored(c, floor=1e-6):
    """The first token as the D = 64 reference kernel computes it for any P0:
    u from P0's rows, the update from P0's upper triangle mirrored
    (persistent_bayes_chunked.cu:207-241); later tokens by the oracle."""
    k, v, q, d, p, r, m0, c0 = (c[x] for x in ("k", "v", "q", "d", "p", "r", "m0", "c0"))
    d0 = d[:, 0]
    eye = torch.eye(D, dtype=c0.dtype)
    pred = d0[:, :, None] * c0 * d0[:, None, :] + p[:, 0, None, None] * eye
    upper = torch.triu(pred) + torch.triu(pred, 1).transpose(-1, -2)
    u = (pred @ k[:, 0, :, None]).squeeze(-1)
    s = (r[:, 0] + (k[:, 0] * u).sum(-1)).clamp_min(floor)
    e = v[:, 0] - ((d0[:, :, None] * m0) * k[:, 0, :, None]).sum(-2)
    m1 = d0[:, :, None] * m0 + (u / s[:, None])[:, :, None] * e[:, None, :]
    c1 = upper - (u / s[:, None])[:, :, None] * u[:, None, :]
    y1 = (m1 * q[:, 0, :, None]).sum(-2)
    y, mT, cT = O.run_diagonal(k[:, 1:], v[:, 1:], q[:, 1:], d[:, 1:], p[:, 1:], r[:, 1:], m1, c1, floor)
    return torch.cat([y1[:, None], y], 1), mT, cT


def test_forward_asymmetric_initial_covariance(ext, cuda_device):
    n, t = 4, 12
    cpu, dev = _case(n, t, seed=5, device=cuda_device, asymmetric=True)
    y, mT, cT, bm, bc = ext.forward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                            dev["c0"], 4, 1e-6)
    ey, em, ec = _first_step_mirrored(_f64(cpu))
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    assert torch.equal(bc[:, 0].cpu(), cpu["c0"])


ABIS = [
    ("backward_chunked", False, 8),
    ("backward_chunked_lean", False, 3),
    ("backward_chunked_fixed", True, 8),
    ("backward_chunked_lean_fixed", True, 3),
]


@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
@pytest.mark.parametrize("final_grads", [False, True])
@pytest.mark.parametrize("chunk", [8, 5])
@pytest.mark.parametrize("t", [1, 13])
def test_backward_matches_oracle(ext, cuda_device, abi, final_grads, chunk, t):
    name, fixed, nout = abi
    print(f"d64 backward {name} final_grads={final_grads} chunk={chunk} t={t}", flush=True)
    n = 4
    cpu, dev = _case(n, t, seed=7 + chunk + t, device=cuda_device)
    ref = _f64(_fixed(cpu) if fixed else cpu)
    fwd = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    _, _, _, bm, bc = fwd(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk,
                          1e-6)
    gmf = dev["gmf"] if final_grads else None
    gcf = dev["gcf"] if final_grads else None
    grads = getattr(ext, name)(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], bm,
                               bc, dev["gy"], gmf, gcf, chunk, 1e-6)
    torch.cuda.synchronize()
    assert len(grads) == nout
    _, _, _, eg = O.diagonal_grads(ref["k"], ref["v"], ref["q"], ref["d"], ref["p"], ref["r"], ref["m0"], ref["c0"],
                                   ref["gy"], ref["gmf"] if final_grads else None,
                                   ref["gcf"] if final_grads else None)
    eg[7] = _sym(eg[7])
    names = ["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"]
    for i in range(nout):
        if fixed and names[i] in ("gd", "gp", "gr"):
            assert torch.count_nonzero(grads[i]) == 0, f"{names[i]} must be zero for fixed dynamics"
            continue
        close(grads[i], eg[i], names[i])
    if nout == 8:
        assert torch.equal(grads[7], grads[7].transpose(-1, -2)), "gc0 must be bitwise symmetric"


def test_sequence_results_independent_of_batch(ext, cuda_device):
    """A sequence's outputs, checkpoints and gradients are bitwise the same in a batch of 300 (more workgroups
    than the device runs at once) as alone: each sequence is one workgroup with fixed arithmetic."""
    print("d64 batch invariance n=300 t=20 chunk=8", flush=True)
    n, t, chunk = 300, 20, 8
    _, dev = _case(n, t, seed=41, device=cuda_device)
    names = ("k", "v", "q", "d", "p", "r", "m0", "c0", "gy", "gmf", "gcf")

    def run(c):
        fwd = ext.forward_chunked(c["k"], c["v"], c["q"], c["d"], c["p"], c["r"], c["m0"], c["c0"], chunk, 1e-6)
        bm, bc = fwd[3], fwd[4]
        grads = ext.backward_chunked(c["k"], c["v"], c["q"], c["d"], c["p"], c["r"], c["m0"], c["c0"], bm, bc,
                                     c["gy"], c["gmf"], c["gcf"], chunk, 1e-6)
        return list(fwd) + list(grads)

    whole = run(dev)
    for i in (0, 137, n - 1):
        alone = run({name: dev[name][i:i + 1].contiguous() for name in names})
        for j, (a, b) in enumerate(zip(alone, whole)):
            assert torch.equal(a, b[i:i + 1]), f"sequence {i}, result {j} differs between N = 1 and N = {n}"


@pytest.mark.parametrize("t", [160, 512])
def test_long_sequence_matches_oracle(ext, cuda_device, t):
    """T = 160 and T = 512 (the length bench.py times; 64 checkpoint chunks): forward and full backward against
    the float64 oracle, with the symmetric initial-covariance adjoint of the D = 64 reference."""
    n, chunk = 2, 8
    print(f"d64 long t={t}", flush=True)
    cpu, dev = _case(n, t, seed=99, device=cuda_device)
    ref = _f64(cpu)
    y, mT, cT, bm, bc = ext.forward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                            dev["c0"], chunk, 1e-6)
    grads = ext.backward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"],
                                 bm, bc, dev["gy"], dev["gmf"], dev["gcf"], chunk, 1e-6)
    torch.cuda.synchronize()
    ey, em, ec, eg = O.diagonal_grads(ref["k"], ref["v"], ref["q"], ref["d"], ref["p"], ref["r"], ref["m0"],
                                      ref["c0"], ref["gy"], ref["gmf"], ref["gcf"])
    eg[7] = _sym(eg[7])
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    for i, name in enumerate(["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"]):
        close(grads[i], eg[i], name)


@pytest.mark.parametrize("t", [20, 16, 512])
def test_autograd_boundary(cuda_device, t):
    """fused_diagonal_bayesian at D = M = 64 under autograd (checkpoint interval of the library), up to the
    T = 512 that bench.py times."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    n = 3
    cpu, dev = _case(n, t, seed=11 + t, device=cuda_device)
    leaves = {k: dev[k].clone().requires_grad_(True) for k in ("k", "v", "q", "d", "p", "r")}
    y, mT, cT = fused_diagonal_bayesian(leaves["k"], leaves["v"], leaves["q"], leaves["d"], leaves["p"],
                                        leaves["r"], dev["m0"], dev["c0"], chunk_length=64, denominator_floor=1e-6)
    torch.autograd.backward([y, mT], [dev["gy"], dev["gmf"]])
    f = _f64(cpu)
    ey, em, ec, eg = O.diagonal_grads(f["k"], f["v"], f["q"], f["d"], f["p"], f["r"], f["m0"], f["c0"], f["gy"],
                                      f["gmf"], None)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    for i, key in enumerate(("k", "v", "q", "d", "p", "r")):
        close(leaves[key].grad, eg[i], "grad " + key)


def test_bayesian_layer_routes_d64_to_hip(cuda_device, monkeypatch):
    """bayesian_layer sends (64, 64) diagonal dynamics to the fused kernels (bayesian_layer.py:1047-1051)."""
    import bayes_ssm
    from bayes_ssm import fused_cuda

    calls = []
    real = fused_cuda._ChunkedBayesianFunction.apply
    monkeypatch.setattr(fused_cuda._ChunkedBayesianFunction, "apply",
                        staticmethod(lambda *a: calls.append(a[0].shape) or real(*a)))
    n, t = 2, 9
    cpu, dev = _case(n, t, seed=31, device=cuda_device)
    y, _, _ = bayes_ssm.bayesian_layer(dev["k"], dev["v"], dev["q"], transition_diagonals=dev["d"],
                                       process_variances=dev["p"], observation_variances=dev["r"],
                                       initial_mean=dev["m0"], initial_covariance=dev["c0"], optimized=True)
    assert calls and calls[0][-1] == D
    f = _f64(cpu)
    ey, _, _ = O.run_diagonal(f["k"], f["v"], f["q"], f["d"], f["p"], f["r"], f["m0"], f["c0"], 1e-6)
    close(y, ey, "y")


def test_edge_sizes(ext, cuda_device):
    """N = 0 launches nothing; T = 0 returns the initial belief (forward) and the final-state adjoints (backward)."""
    _, dev = _case(2, 3, seed=1, device=cuda_device)
    empty = {k: x[:0].contiguous() for k, x in dev.items()}
    out = ext.forward_chunked(empty["k"], empty["v"], empty["q"], empty["d"], empty["p"], empty["r"],
                              empty["m0"], empty["c0"], 8, 1e-6)
    assert out[0].shape == (0, 3, D)
    zt = {k: dev[k][:, :0].contiguous() for k in ("k", "v", "q", "d", "p", "r", "gy")}
    y, mT, cT, bm, bc = ext.forward_chunked(zt["k"], zt["v"], zt["q"], zt["d"], zt["p"], zt["r"], dev["m0"],
                                            dev["c0"], 8, 1e-6)
    grads = ext.backward_chunked(zt["k"], zt["v"], zt["q"], zt["d"], zt["p"], zt["r"], dev["m0"], dev["c0"], bm,
                                 bc, zt["gy"], dev["gmf"], dev["gcf"], 8, 1e-6)
    torch.cuda.synchronize()
    assert y.shape == (2, 0, D)
    assert torch.equal(mT, dev["m0"]) and torch.equal(cT, dev["c0"])
    assert torch.equal(bm[:, 0], dev["m0"]) and torch.equal(bc[:, 0], dev["c0"])
    assert torch.equal(grads[6], dev["gmf"])
    close(grads[7], _sym(dev["gcf"]), "gc0")
