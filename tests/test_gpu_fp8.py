"""float8 keys, values and queries on the D4M8 kernels (C ABI ``bssm_*_chunked_fp8``).

The kernels widen float8 (OCP e4m3fn / e5m2) on chip, exactly, so every
output and every float32 gradient must equal, bit for bit, the float32
kernels' results on the widened values; the float8 gradients of keys, values
and queries must be those float32 gradients rounded as torch rounds them
(``.to(float8_*)``: the gradient autograd gives through the reference's
promotion of float8 inputs, bayesian_layer.py:823-827).  The float32 kernels
are checked against the float64 oracle in test_gpu_parity.py; here the
forward is also checked against the oracle directly.  Comparisons are on the
bit patterns, so NaN and infinity codes count too.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O
from tests.test_gpu_parity import _case, close

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("rotated_layout")]

FMTS = {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}


def _bits(x: torch.Tensor) -> torch.Tensor:
    return x.view(torch.uint8) if x.element_size() == 1 else x.view(torch.int32)


def _same(a: torch.Tensor, b: torch.Tensor, name: str):
    assert a.dtype == b.dtype, f"{name}: dtype {a.dtype} != {b.dtype}"
    bad = (_bits(a) != _bits(b)).sum().item()
    assert bad == 0, f"{name}: {bad} of {a.numel()} entries differ"


def _fp8_case(n, t, fmt, seed, device, codes=False):
    cpu, dev = _case(n, t, 4, seed=seed, device=device)
    g = torch.Generator().manual_seed(seed + 7)
    for name in "kvq":
        if codes:
            # Uniform over the finite float8 codes (every exponent, subnormals and both zeros).
            finite = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(FMTS[fmt]).float().isfinite()
            pool = torch.nonzero(finite).flatten().to(torch.uint8)
            pick = pool[torch.randint(len(pool), dev[name].shape, generator=g)]
            dev[name + "h"] = pick.view(FMTS[fmt]).to(device).contiguous()
        else:
            dev[name + "h"] = dev[name].to(FMTS[fmt]).contiguous()
        dev[name] = dev[name + "h"].float().contiguous()
    return cpu, dev


def _run_abi(dev, n, t, fmt, fixed, dyn, device):
    """The float32 kernels on the widened values, and the float8 entry points."""
    from bayes_ssm import _hip, fused_cuda

    ext = fused_cuda._load_extension(4)
    chunk = _hip.preferred_checkpoint(4)
    P = _hip.ptr
    fwd = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    bwd = ext.backward_chunked_fixed if fixed else ext.backward_chunked
    args = [dev[x] for x in ("k", "v", "q", "d", "p", "r", "m0", "c0")]
    y, mT, cT, bm, bc = fwd(*args, chunk, 1e-6)
    ref = bwd(*args, bm, bc, dev["gy"], dev["gmf"], dev["gcf"], chunk, 1e-6)

    yh, mh, ch = torch.empty_like(y), torch.empty_like(mT), torch.empty_like(cT)
    bmh, bch = torch.empty_like(bm), torch.empty_like(bc)
    stream = _hip.stream_of(device)
    _hip.call("bssm_forward_chunked_fp8", 4, 8, int(fixed), fmt, P(dev["kh"]), P(dev["vh"]), P(dev["qh"]),
              P(dev["d"]), P(dev["p"]), P(dev["r"]), P(dev["m0"]), P(dev["c0"]), P(yh), P(mh), P(ch), P(bmh),
              P(bch), n, t, chunk, 1e-6, stream)
    gk, gv, gq = (torch.empty_like(dev[x]) for x in ("kh", "vh", "qh"))
    gd, gp, gr = ((torch.empty_like(dev[x]) for x in "dpr") if dyn else (None, None, None))
    gm0, gc0 = torch.empty_like(dev["m0"]), torch.empty_like(dev["c0"])
    _hip.call("bssm_backward_chunked_fp8", 4, 8, int(fixed), fmt, P(dev["kh"]), P(dev["vh"]), P(dev["qh"]),
              P(dev["d"]), P(dev["p"]), P(dev["r"]), P(dev["m0"]), P(dev["c0"]), P(bmh), P(bch), P(dev["gy"]),
              P(dev["gmf"]), P(dev["gcf"]), P(gk), P(gv), P(gq), P(gd), P(gp), P(gr), P(gm0), P(gc0), n, t, chunk,
              1e-6, stream)
    torch.cuda.synchronize()
    return (y, mT, cT, bm, bc), ref, (yh, mh, ch, bmh, bch), (gk, gv, gq, gd, gp, gr, gm0, gc0)


def _check(f32_out, ref, f8_out, f8_grads, fmt, dyn):
    for name, a, b in zip(("y", "mean_T", "cov_T", "bmean", "bcov"), f8_out, f32_out):
        _same(a, b, name)
    for name, a, b in zip(("gk", "gv", "gq"), f8_grads[:3], ref[:3]):
        assert a.dtype == FMTS[fmt]
        _same(a, b.to(FMTS[fmt]), name + " (the float32 gradient rounded to float8)")
    rest = zip(("gd", "gp", "gr", "gm0", "gc0"), f8_grads[3:], ref[3:])
    for name, a, b in rest:
        if a is None:
            assert not dyn
            continue
        _same(a, b, name)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("t,fixed,dyn", [(4, False, True), (20, False, True), (64, False, False), (52, True, False),
                                         (16, True, False)])
def test_fp8_abi_matches_float32_kernels(cuda_device, fmt, t, fixed, dyn):
    print(f"fp8 abi fmt={fmt} t={t} fixed={fixed} dyn={dyn}", flush=True)
    n = 37
    _, dev = _fp8_case(n, t, fmt, seed=900 + t, device=cuda_device)
    f32_out, ref, f8_out, f8_grads = _run_abi(dev, n, t, fmt, fixed, dyn, cuda_device)
    _check(f32_out, ref, f8_out, f8_grads, fmt, dyn)


@pytest.mark.parametrize("fmt", [0, 1])
def test_fp8_every_finite_code(cuda_device, fmt):
    """k, v, q drawn uniformly from every finite float8 code: widening and rounding of the whole range."""
    print(f"fp8 every code fmt={fmt}", flush=True)
    n, t = 37, 64
    _, dev = _fp8_case(n, t, fmt, seed=950, device=cuda_device, codes=True)
    seen = torch.unique(torch.cat([dev[x + "h"].view(torch.uint8).flatten() for x in "kvq"]))
    assert len(seen) == 256 - (2 if fmt == 0 else 8), "not every finite code was drawn"
    f32_out, ref, f8_out, f8_grads = _run_abi(dev, n, t, fmt, False, True, cuda_device)
    _check(f32_out, ref, f8_out, f8_grads, fmt, True)


@pytest.mark.parametrize("fmt", [0, 1])
def test_fp8_autograd_boundary_and_oracle(cuda_device, fmt):
    """fused_diagonal_bayesian with float8 k/v/q leaves: the float32 path on the widened values, bit for bit,
    and the float64 oracle on them within the float32 tolerance."""
    from bayes_ssm import fused_cuda
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    print(f"fp8 autograd fmt={fmt}", flush=True)
    n, t = 24, 64
    cpu, dev = _fp8_case(n, t, fmt, seed=960, device=cuda_device)
    lh = {x: (dev[x + "h"] if x in "kvq" else dev[x]).clone().requires_grad_(True) for x in "kvqdpr"}
    lf = {x: dev[x].clone().requires_grad_(True) for x in "kvqdpr"}
    calls = []
    orig = fused_cuda._ChunkedBayesianBF16Function.apply
    fused_cuda._ChunkedBayesianBF16Function.apply = staticmethod(lambda *a: calls.append(1) or orig(*a))
    try:
        outs = []
        for lv in (lh, lf):
            y, mT, cT = fused_diagonal_bayesian(lv["k"], lv["v"], lv["q"], lv["d"], lv["p"], lv["r"], dev["m0"],
                                                dev["c0"], chunk_length=64, denominator_floor=1e-6)
            torch.autograd.backward([y, mT], [dev["gy"], dev["gmf"]])
            outs.append((y, mT, cT))
    finally:
        fused_cuda._ChunkedBayesianBF16Function.apply = orig
    assert len(calls) == 1, "the float8 kernels were not used"
    for name, a, b in zip(("y", "mean_T", "cov_T"), *outs):
        _same(a, b, name)
    for x in "kvqdpr":
        expected = lf[x].grad.to(FMTS[fmt]) if x in "kvq" else lf[x].grad
        _same(lh[x].grad, expected, f"grad {x}")
    f64 = {k: v.double() for k, v in cpu.items()}
    wide = {x: dev[x].double().cpu() for x in "kvq"}
    ey, em, ec = O.run_diagonal(wide["k"], wide["v"], wide["q"], f64["d"], f64["p"], f64["r"], f64["m0"],
                                f64["c0"], 1e-6)
    close(outs[0][0], ey, "y vs oracle")
    close(outs[0][1], em, "mean vs oracle")
    close(outs[0][2], ec, "cov vs oracle")


@pytest.mark.parametrize("fmt", [0, 1])
def test_fp8_bayesian_layer_routes_to_fp8_kernels(cuda_device, monkeypatch, fmt):
    import bayes_ssm
    from bayes_ssm import fused_cuda

    calls = []
    orig = fused_cuda._ChunkedBayesianBF16Function.apply
    monkeypatch.setattr(fused_cuda._ChunkedBayesianBF16Function, "apply",
                        staticmethod(lambda *a: calls.append(a[0].dtype) or orig(*a)))
    n, t = 16, 32
    cpu, dev = _fp8_case(n, t, fmt, seed=970, device=cuda_device)
    y, mT, cT = bayes_ssm.bayesian_layer(dev["kh"], dev["vh"], dev["qh"], transition_diagonals=dev["d"],
                                         process_variances=dev["p"], observation_variances=dev["r"],
                                         chunk_length=16, optimized=True)
    assert calls == [FMTS[fmt]], "float8 kernels were not used"
    ry, rm, rc = bayes_ssm.bayesian_layer(dev["k"].cpu(), dev["v"].cpu(), dev["q"].cpu(),
                                          transition_diagonals=cpu["d"], process_variances=cpu["p"],
                                          observation_variances=cpu["r"], chunk_length=16, optimized=False)
    close(y, ry, "y vs reference fp32 path")
    close(mT, rm, "mean")
    close(cT, rc, "cov")


def test_fp8_config3_full_size(cuda_device):
    """Config 3 (B256 x T512 x H64, D4M8) with e4m3fn k/v/q: bit for bit the float32 kernels on the widened values."""
    print("fp8 config3 full size", flush=True)
    n, t = 256 * 64, 512
    g = torch.Generator(device=cuda_device).manual_seed(11)
    k, v, q, dec, p, r, gy = O.make_inputs(n, t, 4, seed=0)
    dev = {"d": dec.to(cuda_device), "p": p.to(cuda_device), "r": r.to(cuda_device), "gy": gy.to(cuda_device),
           "m0": torch.zeros(n, 4, 8, device=cuda_device),
           "c0": torch.eye(4, device=cuda_device).expand(n, 4, 4).contiguous(),
           "gmf": torch.randn(n, 4, 8, device=cuda_device, generator=g),
           "gcf": torch.randn(n, 4, 4, device=cuda_device, generator=g)}
    for name, x in (("k", k), ("v", v), ("q", q)):
        dev[name + "h"] = x.to(cuda_device).to(torch.float8_e4m3fn).contiguous()
        dev[name] = dev[name + "h"].float()
    del k, v, q, dec, p, r, gy
    f32_out, ref, f8_out, f8_grads = _run_abi(dev, n, t, 0, False, True, cuda_device)
    _check(f32_out, ref, f8_out, f8_grads, 0, True)
