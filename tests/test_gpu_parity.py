"""GPU parity of the HIP kernels against the CPU oracle (run on an MI355X).

Every call goes through the C ABI (via the ``fused_cuda`` extension object or
the autograd boundary).  Tolerance (north star): 1e-5 relative, 1e-4 absolute
on outputs and gradients against the float64 oracle and against the
reference's float32 CPU path; checkpoint indexing and chunk invariance are
bit-exact.
"""
from __future__ import annotations

import os

import pytest
import torch

from oracle import bssm_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-4
DIMS = [1, 2, 4, 8]


def close(actual, expected, name="", rtol=RTOL, atol=ATOL):
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    torch.testing.assert_close(actual, expected, rtol=rtol, atol=atol, msg=lambda m: f"{name}: {m}")


@pytest.fixture(scope="module")
def ext_for(cuda_device):
    from bayes_ssm import fused_cuda

    def get(d):
        ext = fused_cuda._load_extension(d)
        assert ext is not None
        return ext

    return get


def _case(n, t, d, seed, device, m=8):
    k, v, q, dec, p, r, gy = O.make_inputs(n, t, d, m, seed=seed)
    g = torch.Generator().manual_seed(seed + 100)
    m0 = 0.2 * torch.randn(n, d, m, generator=g)
    a = torch.randn(n, d, d, generator=g)
    c0 = a @ a.transpose(-1, -2) / d + 0.5 * torch.eye(d)
    c0 = 0.5 * (c0 + c0.transpose(-1, -2))
    gmf = torch.randn(n, d, m, generator=g)
    gcf = torch.randn(n, d, d, generator=g)
    cpu = dict(k=k, v=v, q=q, d=dec, p=p, r=r, m0=m0, c0=c0, gy=gy, gmf=gmf, gcf=gcf)
    dev = {name: x.to(device).contiguous() for name, x in cpu.items()}
    return cpu, dev


def _oracle_forward(c, fixed, floor=1e-6):
    f64 = {k: x.double() for k, x in c.items()}
    if fixed:
        return O.run_fixed(f64["k"], f64["v"], f64["q"], f64["m0"], f64["c0"], floor)
    return O.run_diagonal(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"], floor)


def _fixed_dynamics(c):
    out = dict(c)
    out["d"] = torch.full_like(c["d"], O.FIXED_DECAY)
    out["p"] = torch.full_like(c["p"], O.FIXED_PROCESS)
    out["r"] = torch.full_like(c["r"], O.FIXED_OBSERVATION)
    return out


# T = 45 takes the generic kernels; T = 52 (a multiple of 4 that is not a
# multiple of the 16-token forward tile) takes the D4 rotated-layout kernels
# with a partial last tile (their backward needs the library's preferred
# checkpoint chunk, 8).  N = 37 leaves idle sequence slots in the last wave.
TIMES = [45, 52]


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("chunk", [1, 8, 13, 64])
@pytest.mark.parametrize("t", TIMES)
def test_forward_matches_oracle(ext_for, cuda_device, d, fixed, chunk, t):
    print(f"forward d={d} fixed={fixed} chunk={chunk} t={t}", flush=True)
    n = 37
    cpu, dev = _case(n, t, d, seed=d * 10 + chunk, device=cuda_device)
    ext = ext_for(d)
    fn = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    y, mT, cT, bm, bc = fn(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk,
                           1e-6)
    torch.cuda.synchronize()
    ref = _fixed_dynamics(cpu) if fixed else cpu
    ey, em, ec = _oracle_forward(ref, False)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    nb = -(-t // chunk)
    assert bm.shape == (n, nb + 1, d, 8) and bc.shape == (n, nb + 1, d, d)
    f64 = {k: x.double() for k, x in ref.items()}
    ebm, ebc = O.checkpoints(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                             chunk, 1e-6)
    close(bm, ebm, "bmean")
    close(bc, ebc, "bcov")
    # The final checkpoint and the final state are the same numbers.
    assert torch.equal(bm[:, nb].cpu(), mT.cpu()) and torch.equal(bc[:, nb].cpu(), cT.cpu())
    assert torch.equal(bm[:, 0].cpu(), dev["m0"].cpu())


@pytest.mark.parametrize("d", DIMS)
def test_forward_chunk_invariance_bitexact(ext_for, cuda_device, d):
    """Outputs are bitwise identical for every chunk; bm/bc index c is the state before token c*chunk."""
    print(f"chunk invariance d={d}", flush=True)
    n, t = 40, 96
    _, dev = _case(n, t, d, seed=3, device=cuda_device)
    ext = ext_for(d)
    runs = {c: ext.forward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"],
                                   c, 1e-6) for c in (4, 8, 16, 96, 200)}
    base = runs[8]
    for c, out in runs.items():
        for a, b in zip(out[:3], base[:3]):
            assert torch.equal(a, b), f"chunk {c} changes the recurrence"
    for c in (4, 16):
        bm, bc = runs[c][3], runs[c][4]
        step = c // 4
        assert torch.equal(bm, runs[4][3][:, ::step]), f"bmean layout chunk {c}"
        assert torch.equal(bc, runs[4][4][:, ::step]), f"bcov layout chunk {c}"


ABIS = [
    ("backward_chunked", False, 8),
    ("backward_chunked_lean", False, 3),
    ("backward_chunked_noinitial", False, 6),
    ("backward_chunked_fixed", True, 8),
    ("backward_chunked_lean_fixed", True, 3),
    ("backward_chunked_noinitial_fixed", True, 6),
]


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
@pytest.mark.parametrize("final_grads", [False, True])
@pytest.mark.parametrize("chunk", [8, 13, 16])
@pytest.mark.parametrize("t", TIMES)
def test_backward_matches_oracle(ext_for, cuda_device, d, abi, final_grads, chunk, t):
    name, fixed, nout = abi
    print(f"backward {name} d={d} final_grads={final_grads} chunk={chunk} t={t}", flush=True)
    n = 37
    cpu, dev = _case(n, t, d, seed=7 * d + chunk, device=cuda_device)
    ref = _fixed_dynamics(cpu) if fixed else cpu
    ext_name = name
    ext = ext_for(d)
    # noinitial is exported for D2 only (as in the reference); call the C ABI for other D.
    fwd = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    _, _, _, bm, bc = fwd(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk,
                          1e-6)
    gmf = dev["gmf"] if final_grads else None
    gcf = dev["gcf"] if final_grads else None
    if hasattr(ext, ext_name):
        grads = getattr(ext, ext_name)(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                       dev["c0"], bm, bc, dev["gy"], gmf, gcf, chunk, 1e-6)
    else:
        grads = ext._backward("bssm_" + ext_name, fixed, nout, dev["k"], dev["v"], dev["q"], dev["d"], dev["p"],
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


@pytest.mark.parametrize("t", [4, 8, 12, 16, 20, 24, 28, 56, 60])
@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("chunk", [8, 16])
def test_rot4_backward_tails(ext_for, cuda_device, rotated_layout, t, fixed, chunk):
    """D4 rotated-layout backward at checkpoint chunks 8 (a record per 8-token chunk) and 16 (a record per
    16-token tile, the second chunk's start advanced on chip): every shape of the last tiles."""
    print(f"rot4 backward tails t={t} fixed={fixed} chunk={chunk}", flush=True)
    n, d = 21, 4
    cpu, dev = _case(n, t, d, seed=100 + t, device=cuda_device)
    ref = _fixed_dynamics(cpu) if fixed else cpu
    ext = ext_for(d)
    fwd = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    bwd = ext.backward_chunked_fixed if fixed else ext.backward_chunked
    _, _, _, bm, bc = fwd(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk,
                          1e-6)
    grads = bwd(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], bm, bc, dev["gy"],
                dev["gmf"], dev["gcf"], chunk, 1e-6)
    torch.cuda.synchronize()
    f64 = {k: x.double() for k, x in ref.items()}
    _, _, _, eg = O.diagonal_grads(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                                   f64["gy"], f64["gmf"], f64["gcf"])
    for i, name in enumerate(["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"]):
        if fixed and name in ("gd", "gp", "gr"):
            assert torch.count_nonzero(grads[i]) == 0, f"{name} must be zero for fixed dynamics"
            continue
        close(grads[i], eg[i], name)


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("t", [70, 64])
def test_autograd_boundary(cuda_device, d, t):
    """fused_diagonal_bayesian under autograd: values and all input gradients."""
    print(f"autograd d={d} t={t}", flush=True)
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    n = 20
    cpu, dev = _case(n, t, d, seed=11 + d, device=cuda_device)
    leaves = {k: dev[k].clone().requires_grad_(True) for k in ("k", "v", "q", "d", "p", "r")}
    y, mT, cT = fused_diagonal_bayesian(leaves["k"], leaves["v"], leaves["q"], leaves["d"], leaves["p"],
                                        leaves["r"], dev["m0"], dev["c0"], chunk_length=64, denominator_floor=1e-6)
    torch.autograd.backward([y, mT], [dev["gy"], dev["gmf"]])
    f64 = {k: x.double() for k, x in cpu.items()}
    ey, em, ec, eg = O.diagonal_grads(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"],
                                      f64["c0"], f64["gy"], f64["gmf"], None)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    for i, key in enumerate(("k", "v", "q", "d", "p", "r")):
        close(leaves[key].grad, eg[i], "grad " + key)


@pytest.mark.parametrize("d", DIMS)
def test_lean_autograd_readout_only(cuda_device, d):
    """Readout-only loss with constant dynamics takes the lean ABI (3 gradients)."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    n, t = 24, 33
    cpu, dev = _case(n, t, d, seed=21 + d, device=cuda_device)
    leaves = {k: dev[k].clone().requires_grad_(True) for k in ("k", "v", "q")}
    y, _, _ = fused_diagonal_bayesian(leaves["k"], leaves["v"], leaves["q"], dev["d"], dev["p"], dev["r"],
                                      dev["m0"], dev["c0"], chunk_length=16, denominator_floor=1e-6)
    y.backward(dev["gy"])
    f64 = {k: x.double() for k, x in cpu.items()}
    _, _, _, eg = O.diagonal_grads(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"],
                                   f64["c0"], f64["gy"])
    for i, key in enumerate(("k", "v", "q")):
        close(leaves[key].grad, eg[i], "grad " + key)


def test_d1_saved_history_abi(ext_for, cuda_device):
    """forward_chunked_saved + backward_chunked_saved{,_lean,_d1} (reference D1 ABI)."""
    n, t = 30, 50
    cpu, dev = _case(n, t, 1, seed=5, device=cuda_device)
    ext = ext_for(1)
    out = ext.forward_chunked_saved(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                    dev["c0"], t, 1e-6)
    y, mT, cT, bm, bc, mp, pp, uh, bh, eh = out
    assert bm.shape == (n, 2, 1, 8)
    ey, em, ec = _oracle_forward(cpu, False)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    f64 = {k: x.double() for k, x in cpu.items()}
    _, _, _, eg = O.diagonal_grads(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"],
                                   f64["c0"], f64["gy"], f64["gmf"], f64["gcf"])
    for name in ("backward_chunked_saved", "backward_chunked_saved_d1"):
        grads = getattr(ext, name)(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"],
                                   bm, bc, mp, pp, uh, bh, eh, dev["gy"], dev["gmf"], dev["gcf"], t, 1e-6)
        for g, e, nm in zip(grads, eg, ["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"]):
            close(g, e, f"{name} {nm}")
    lean = ext.backward_chunked_saved_lean(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                           dev["c0"], bm, bc, mp, pp, uh, bh, eh, dev["gy"], dev["gmf"],
                                           dev["gcf"], t, 1e-6)
    for g, e, nm in zip(lean, eg, ["gk", "gv", "gq"]):
        close(g, e, f"saved_lean {nm}")


def test_bayesian_layer_routes_to_hip(cuda_device, monkeypatch):
    """bayesian_layer(optimized=True) on the GPU takes the fused HIP path and matches the CPU reference path."""
    import bayes_ssm
    from bayes_ssm import fused_cuda

    calls = []
    real = fused_cuda._ChunkedBayesianFunction.apply
    monkeypatch.setattr(fused_cuda._ChunkedBayesianFunction, "apply",
                        staticmethod(lambda *a: calls.append(1) or real(*a)))
    n, t, d = 16, 40, 4
    cpu, dev = _case(n, t, d, seed=31, device=cuda_device)
    y, mT, cT = bayes_ssm.bayesian_layer(dev["k"], dev["v"], dev["q"], transition_diagonals=dev["d"],
                                         process_variances=dev["p"], observation_variances=dev["r"],
                                         chunk_length=16, optimized=True)
    assert calls, "fused HIP path was not taken"
    ry, rm, rc = bayes_ssm.bayesian_layer(cpu["k"], cpu["v"], cpu["q"], transition_diagonals=cpu["d"],
                                          process_variances=cpu["p"], observation_variances=cpu["r"],
                                          chunk_length=16, optimized=False)
    close(y, ry, "y vs reference fp32 path")
    close(mT, rm, "mean")
    close(cT, rc, "cov")
    # Both against the float64 oracle (the CPU path above is this package's own code).
    f64 = {k: x.double() for k, x in cpu.items()}
    ey, em, ec = O.run_diagonal(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"],
                                torch.zeros(n, d, 8, dtype=torch.float64),
                                torch.eye(d, dtype=torch.float64).expand(n, d, d), 1e-6)
    for name, a, b, e in (("y", y, ry, ey), ("mean", mT, rm, em), ("cov", cT, rc, ec)):
        close(a, e, name + " vs oracle")
        close(b, e, name + " (CPU path) vs oracle")


@pytest.mark.parametrize("cfg", [(1, 16, 4, 4), (4, 64, 16, 16)])
def test_associative_scan_configs(cuda_device, cfg):
    """Configs 0 and 1: HIP information-form scan vs oracle scan and the dense recurrence."""
    import bayes_ssm

    b, t, d, m = cfg
    k, v, q, r = O.make_scan_inputs(b, t, d, m, seed=0)
    y, mT, cT = bayes_ssm.associative_static_bayesian_cuda(k.to(cuda_device), v.to(cuda_device),
                                                           q.to(cuda_device), observation_variances=r.to(cuda_device))
    ey, em, ec = O.associative_static(k.double(), v.double(), q.double(), r.double())
    close(y, ey, "y")
    close(mT, em, "mean")
    close(cT, ec, "cov")
    # Dense-recurrence equivalence (the reference benchmark's check).
    ones = torch.ones(b, t, d, dtype=torch.float64)
    zeros = torch.zeros(b, t, dtype=torch.float64)
    m0 = torch.zeros(b, d, m, dtype=torch.float64)
    c0 = torch.eye(d, dtype=torch.float64).expand(b, d, d).clone()
    dy, dm, dc = O.run_diagonal(k.double(), v.double(), q.double(), ones, zeros, r.double(), m0, c0, 1e-6)
    close(y, dy, "y vs dense")


@pytest.mark.parametrize("cfg", [(3, 5, 1, 8), (2, 9, 3, 5), (2, 12, 5, 7), (3, 20, 12, 33), (2, 10, 20, 9),
                                 (1, 6, 32, 64)])
def test_associative_scan_priors_and_sizes(cuda_device, cfg):
    """Key dims padded to the register kernel's sizes and the LDS kernel (D > 16), with a random SPD prior."""
    import bayes_ssm

    b, t, d, m = cfg
    print(f"associative scan b={b} t={t} d={d} m={m}", flush=True)
    k, v, q, r = O.make_scan_inputs(b, t, d, m, seed=d + m)
    gen = torch.Generator().manual_seed(7)
    a = torch.randn(b, d, d, generator=gen) / d ** 0.5
    c0 = a @ a.transpose(-1, -2) + 0.5 * torch.eye(d)
    m0 = torch.randn(b, d, m, generator=gen)
    y, mT, cT = bayes_ssm.associative_static_bayesian_cuda(
        k.to(cuda_device), v.to(cuda_device), q.to(cuda_device), observation_variances=r.to(cuda_device),
        initial_mean=m0.to(cuda_device), initial_covariance=c0.to(cuda_device))
    ey, em, ec = O.associative_static(k.double(), v.double(), q.double(), r.double(), m0.double(), c0.double())
    close(y, ey, "y")
    close(mT, em, "mean")
    close(cT, ec, "cov")


@pytest.mark.parametrize("d", [4, 2, 8])
def test_config3_full_size_subset(cuda_device, d):
    """Config 3 at full size (B256 x T512 x H64; D4M8 and the D2M8 / D8M8 variants): fwd+bwd on the GPU,
    a seeded subset of sequences against the oracle."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    n, t = 256 * 64, 512
    print(f"config3 full size d={d}", flush=True)
    k, v, q, dec, p, r, gy = O.make_inputs(n, t, d, seed=0)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (k, v, q, dec, p, r)]
    m0 = torch.zeros(n, d, 8, device=cuda_device)
    c0 = torch.eye(d, device=cuda_device).expand(n, d, d).contiguous()
    y, _, _ = fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=64, denominator_floor=1e-6)
    y.backward(gy.to(cuda_device))
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    idx = torch.tensor([0, 1, 15, 16, 17, 1000, 8191, 12345, n - 2, n - 1])
    sub = [x[idx].double() for x in (k, v, q, dec, p, r)]
    ey, _, _, eg = O.diagonal_grads(*sub, torch.zeros(len(idx), d, 8, dtype=torch.float64),
                                    torch.eye(d, dtype=torch.float64).expand(len(idx), d, d).clone(),
                                    gy[idx].double())
    close(y[idx.to(cuda_device)], ey, "y")
    for i, name in enumerate(("k", "v", "q", "d", "p", "r")):
        close(leaves[i].grad[idx.to(cuda_device)], eg[i], "grad " + name)


@pytest.mark.parametrize("b", [32, 2])
def test_config3_per_gpu_share_subset(cuda_device, b):
    """Config 3's batch divided over GPUs (B32: one GPU's share under 8-way data parallelism; B2 x H64 = 128
    sequences), D4M8 at T512, through the autograd boundary: the default dispatch takes the split row kernels
    (two-wave forward, three-wave backward); a seeded subset of sequences against the oracle."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    n, t, d = b * 64, 512, 4
    print(f"config3 share b={b}", flush=True)
    k, v, q, dec, p, r, gy = O.make_inputs(n, t, d, seed=1)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (k, v, q, dec, p, r)]
    m0 = torch.zeros(n, d, 8, device=cuda_device)
    c0 = torch.eye(d, device=cuda_device).expand(n, d, d).contiguous()
    y, _, _ = fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=64, denominator_floor=1e-6)
    y.backward(gy.to(cuda_device))
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    idx = torch.tensor(sorted({0, 1, 3, 4, 63, 64, n // 2 + 5, n - 5, n - 2, n - 1}))
    sub = [x[idx].double() for x in (k, v, q, dec, p, r)]
    ey, _, _, eg = O.diagonal_grads(*sub, torch.zeros(len(idx), d, 8, dtype=torch.float64),
                                    torch.eye(d, dtype=torch.float64).expand(len(idx), d, d).clone(),
                                    gy[idx].double())
    close(y[idx.to(cuda_device)], ey, "y")
    for i, name in enumerate(("k", "v", "q", "d", "p", "r")):
        close(leaves[i].grad[idx.to(cuda_device)], eg[i], "grad " + name)


def test_config2_d1_full_size_subset(cuda_device):
    """Config 2 (B64 x T512 x H64, D1M8)."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    n, t, d = 64 * 64, 512, 1
    k, v, q, dec, p, r, gy = O.make_inputs(n, t, d, seed=2)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (k, v, q, dec, p, r)]
    m0 = torch.zeros(n, d, 8, device=cuda_device)
    c0 = torch.ones(n, d, d, device=cuda_device)
    y, _, _ = fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=64, denominator_floor=1e-6)
    y.backward(gy.to(cuda_device))
    idx = torch.tensor([0, 7, 8, 2047, n - 1])
    sub = [x[idx].double() for x in (k, v, q, dec, p, r)]
    ey, _, _, eg = O.diagonal_grads(*sub, torch.zeros(len(idx), d, 8, dtype=torch.float64),
                                    torch.ones(len(idx), d, d, dtype=torch.float64), gy[idx].double())
    close(y[idx.to(cuda_device)], ey, "y")
    for i, name in enumerate(("k", "v", "q", "d", "p", "r")):
        close(leaves[i].grad[idx.to(cuda_device)], eg[i], "grad " + name)


def test_edge_sizes(ext_for, cuda_device):
    """Empty batch, empty time axis, and a single token."""
    ext = ext_for(4)
    for n, t in ((0, 10), (5, 0), (3, 1)):
        cpu, dev = _case(n, t, 4, seed=1, device=cuda_device)
        y, mT, cT, bm, bc = ext.forward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"],
                                                dev["m0"], dev["c0"], 8, 1e-6)
        grads = ext.backward_chunked(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"],
                                     dev["c0"], bm, bc, dev["gy"], dev["gmf"], dev["gcf"], 8, 1e-6)
        torch.cuda.synchronize()
        assert y.shape == (n, t, 8)
        if n and t == 0:
            close(mT, cpu["m0"], "mean passthrough", rtol=0, atol=0)
            close(grads[6], cpu["gmf"], "gm0 passthrough", rtol=0, atol=0)
            close(grads[7], cpu["gcf"], "gc0 passthrough", rtol=0, atol=0)
        if n and t:
            ey, em, ec = _oracle_forward(cpu, False)
            close(y, ey, "y")


def _bf16_case(n, t, seed, device):
    cpu, dev = _case(n, t, 4, seed=seed, device=device)
    for name in ("k", "v", "q"):
        dev[name + "h"] = dev[name].bfloat16().contiguous()
        dev[name] = dev[name + "h"].float().contiguous()
    return cpu, dev


@pytest.mark.parametrize("t", [4, 8, 12, 16, 20, 52, 64])
@pytest.mark.parametrize("fixed", [False, True])
def test_bf16_abi_matches_float32_kernels(cuda_device, rotated_layout, t, fixed):
    """bf16 k/v/q C ABI: outputs bit-identical to the float32 kernels on the widened values;
    gk/gv/gq are the float32 gradients rounded to bfloat16, the other gradients bit-identical."""
    from bayes_ssm import _hip, fused_cuda

    print(f"bf16 abi t={t} fixed={fixed}", flush=True)
    n = 37
    _, dev = _bf16_case(n, t, seed=500 + t, device=cuda_device)
    ext = fused_cuda._load_extension(4)
    chunk = _hip.preferred_checkpoint(4)
    nb = -(-t // chunk)
    P = _hip.ptr
    fwd = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    bwd = ext.backward_chunked_fixed if fixed else ext.backward_chunked
    args = [dev[x] for x in ("k", "v", "q", "d", "p", "r", "m0", "c0")]
    y, mT, cT, bm, bc = fwd(*args, chunk, 1e-6)
    ref = bwd(*args, bm, bc, dev["gy"], dev["gmf"], dev["gcf"], chunk, 1e-6)

    yh, mh, ch = torch.empty_like(y), torch.empty_like(mT), torch.empty_like(cT)
    bmh, bch = torch.empty_like(bm), torch.empty_like(bc)
    assert bmh.shape[1] == nb + 1
    stream = _hip.stream_of(cuda_device)
    _hip.call("bssm_forward_chunked_bf16", 4, 8, int(fixed), P(dev["kh"]), P(dev["vh"]), P(dev["qh"]),
              P(dev["d"]), P(dev["p"]), P(dev["r"]), P(dev["m0"]), P(dev["c0"]), P(yh), P(mh), P(ch), P(bmh),
              P(bch), n, t, chunk, 1e-6, stream)
    gk, gv, gq = (torch.empty_like(dev[x]) for x in ("kh", "vh", "qh"))
    gd, gp, gr = torch.empty_like(dev["d"]), torch.empty_like(dev["p"]), torch.empty_like(dev["r"])
    gm0, gc0 = torch.empty_like(dev["m0"]), torch.empty_like(dev["c0"])
    _hip.call("bssm_backward_chunked_bf16", 4, 8, int(fixed), P(dev["kh"]), P(dev["vh"]), P(dev["qh"]),
              P(dev["d"]), P(dev["p"]), P(dev["r"]), P(dev["m0"]), P(dev["c0"]), P(bmh), P(bch), P(dev["gy"]),
              P(dev["gmf"]), P(dev["gcf"]), P(gk), P(gv), P(gq), P(gd), P(gp), P(gr), P(gm0), P(gc0), n, t, chunk,
              1e-6, stream)
    torch.cuda.synchronize()
    for name, a, b in (("y", yh, y), ("mean_T", mh, mT), ("cov_T", ch, cT), ("bmean", bmh, bm), ("bcov", bch, bc)):
        assert torch.equal(a, b), f"{name} differs from the float32 kernels"
    for name, a, b in (("gk", gk, ref[0]), ("gv", gv, ref[1]), ("gq", gq, ref[2])):
        assert a.dtype == torch.bfloat16
        assert torch.equal(a, b.bfloat16()), f"{name} is not the float32 gradient rounded to bfloat16"
    for name, a, b in (("gd", gd, ref[3]), ("gp", gp, ref[4]), ("gr", gr, ref[5]), ("gm0", gm0, ref[6]),
                       ("gc0", gc0, ref[7])):
        assert torch.equal(a, b), f"{name} differs from the float32 kernels"


@pytest.mark.parametrize("t", [64, 45])
@pytest.mark.parametrize("leaves", ["all", "kqv"])
def test_bf16_autograd_boundary(cuda_device, rotated_layout, t, leaves):
    """fused_diagonal_bayesian with bf16 k/v/q leaves equals the float32 path on the widened values
    (T = 45 is not a multiple of 4: the bf16 inputs are widened and take the float32 kernels)."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    print(f"bf16 autograd t={t} leaves={leaves}", flush=True)
    n = 24
    _, dev = _bf16_case(n, t, seed=700 + t, device=cuda_device)
    names = ("k", "v", "q", "d", "p", "r") if leaves == "all" else ("k", "v", "q")
    lh = {x: (dev[x + "h"] if x in "kvq" else dev[x]).clone().requires_grad_(x in names) for x in "kvqdpr"}
    lf = {x: dev[x].clone().requires_grad_(x in names) for x in "kvqdpr"}
    outs = []
    for lv in (lh, lf):
        y, mT, cT = fused_diagonal_bayesian(lv["k"], lv["v"], lv["q"], lv["d"], lv["p"], lv["r"], dev["m0"],
                                            dev["c0"], chunk_length=64, denominator_floor=1e-6)
        torch.autograd.backward([y, mT], [dev["gy"], dev["gmf"]])
        outs.append((y, mT, cT))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
    for x in names:
        expected = lf[x].grad.bfloat16() if x in "kvq" else lf[x].grad
        assert lh[x].grad.dtype == expected.dtype
        assert torch.equal(lh[x].grad, expected), f"grad {x}"


def test_bf16_bayesian_layer_routes_to_bf16_kernels(cuda_device, monkeypatch):
    """bayesian_layer passes bf16 keys/values/queries to the bf16 kernels (no float32 copies on that path)."""
    import bayes_ssm
    from bayes_ssm import fused_cuda

    calls = []
    orig = fused_cuda._ChunkedBayesianBF16Function.apply
    monkeypatch.setattr(fused_cuda._ChunkedBayesianBF16Function, "apply",
                        staticmethod(lambda *a: calls.append(1) or orig(*a)))
    n, t = 16, 32
    cpu, dev = _bf16_case(n, t, seed=9, device=cuda_device)
    y, mT, cT = bayes_ssm.bayesian_layer(dev["kh"], dev["vh"], dev["qh"], transition_diagonals=dev["d"],
                                         process_variances=dev["p"], observation_variances=dev["r"],
                                         chunk_length=16, optimized=True)
    assert calls, "bf16 kernels were not used"
    ry, rm, rc = bayes_ssm.bayesian_layer(dev["k"].cpu(), dev["v"].cpu(), dev["q"].cpu(),
                                          transition_diagonals=cpu["d"], process_variances=cpu["p"],
                                          observation_variances=cpu["r"], chunk_length=16, optimized=False)
    close(y, ry, "y vs reference fp32 path")
    close(mT, rm, "mean")
    close(cT, rc, "cov")
