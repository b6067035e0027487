"""The public API on the GPU: which kernels each entry point reaches, checked against the float64 oracle.

ReplaySSM (bayes_ssm/replay_ssm.py:34-145) and BayesianLayer
(bayes_ssm/bayesian_layer.py:1185-1274) never reach the fused kernels in the
reference (a replayed or learned-initial-state call keeps the dense path,
:987-993, :1047-1061); their scan and the scalar-noise / low-precision /
fixed-dynamics calls of ``bayesian_layer`` do.  Tolerance (north star): 1e-5
relative, 1e-4 absolute.
"""
from __future__ import annotations

import importlib

import pytest
import torch

import bayes_ssm
from oracle import bssm_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-4
F64 = torch.float64


def close(actual, expected, name="", rtol=RTOL, atol=ATOL):
    torch.testing.assert_close(actual.detach().double().cpu(), expected.detach().double().cpu(), rtol=rtol,
                               atol=atol, msg=lambda m: f"{name}: {m}")


def _count(monkeypatch, owner, attr="apply"):
    calls = []
    orig = getattr(owner, attr)
    monkeypatch.setattr(owner, attr, staticmethod(lambda *a, **k: calls.append(1) or orig(*a, **k)))
    return calls


def test_replay_ssm_associative_scan_reaches_hip(cuda_device, monkeypatch):
    rs = importlib.import_module("bayes_ssm.replay_ssm")
    calls = _count(monkeypatch, rs._StaticScanFunction)
    layer = bayes_ssm.ReplaySSM(16, 16, process_variance=0.0, observation_variance=0.4).to(cuda_device)
    k, v, q, _ = O.make_scan_inputs(4, 64, 16, 16, seed=3)
    y, mT, cT = layer.associative_scan(k.to(cuda_device), v.to(cuda_device), q.to(cuda_device))
    assert calls, "the HIP scan was not used"
    r = torch.full((4, 64), 0.4, dtype=F64)
    ey, em, ec = O.associative_static(k.double(), v.double(), q.double(), r)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")


def test_associative_scan_cuda_gradients(cuda_device):
    """associative_static_bayesian_cuda is differentiable (replay_ssm.py:276-339): all six gradients."""
    b, t, d, m = 3, 24, 4, 5
    k, v, q, r = O.make_scan_inputs(b, t, d, m, seed=8)
    g = torch.Generator().manual_seed(9)
    a = torch.randn(b, d, d, generator=g) / d ** 0.5
    c0 = a @ a.transpose(-1, -2) + 0.5 * torch.eye(d)
    m0 = torch.randn(b, d, m, generator=g)
    gy = torch.randn(b, t, m, generator=g)
    gm = torch.randn(b, d, m, generator=g)
    gc = torch.randn(b, d, d, generator=g)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (k, v, q, r, m0, c0)]
    y, mT, cT = bayes_ssm.associative_static_bayesian_cuda(
        leaves[0], leaves[1], leaves[2], observation_variances=leaves[3], initial_mean=leaves[4],
        initial_covariance=leaves[5])
    torch.autograd.backward([y, mT, cT], [gy.to(cuda_device), gm.to(cuda_device), gc.to(cuda_device)])
    el = [x.double().requires_grad_(True) for x in (k, v, q, r, m0, c0)]
    ey, em, ec = O.associative_static(*el[:4], el[4], el[5])
    torch.autograd.backward([ey, em, ec], [gy.double(), gm.double(), gc.double()])
    close(y, ey, "y")
    for name, x, e in zip(("k", "v", "q", "r", "mean0", "cov0"), leaves, el):
        close(x.grad, e.grad, "grad " + name)


@pytest.mark.parametrize("b,t,d,m,with_final", [
    (2, 1, 4, 8, True), (2, 33, 1, 1, True), (3, 17, 3, 7, True), (2, 9, 2, 64, True), (2, 40, 8, 8, False),
    (1, 20, 16, 33, True), (2, 12, 13, 20, False), (2, 65, 5, 64, True), (4, 64, 16, 16, True),
    (2, 300, 4, 8, True)])
def test_associative_scan_hip_backward_shapes(cuda_device, monkeypatch, b, t, d, m, with_final):
    """The HIP scan backward (key dims <= 16, exact and padded) against the oracle's autograd; without
    final-state gradients the kernel takes null pointers for them."""
    rs = importlib.import_module("bayes_ssm.replay_ssm")
    calls = _count(monkeypatch, rs._StaticScanFunction, "_hip_backward")
    print(f"scan backward b={b} t={t} d={d} m={m} final={with_final}", flush=True)
    k, v, q, r = O.make_scan_inputs(b, t, d, m, seed=40 + d + t)
    g = torch.Generator().manual_seed(41 + m)
    a = torch.randn(b, d, d, generator=g) / d ** 0.5
    c0 = a @ a.transpose(-1, -2) + 0.5 * torch.eye(d)
    m0 = torch.randn(b, d, m, generator=g)
    gy = torch.randn(b, t, m, generator=g)
    gm = torch.randn(b, d, m, generator=g)
    gc = torch.randn(b, d, d, generator=g)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (k, v, q, r, m0, c0)]
    y, mT, cT = bayes_ssm.associative_static_bayesian_cuda(
        leaves[0], leaves[1], leaves[2], observation_variances=leaves[3], initial_mean=leaves[4],
        initial_covariance=leaves[5])
    el = [x.double().requires_grad_(True) for x in (k, v, q, r, m0, c0)]
    ey, em, ec = O.associative_static(*el[:4], el[4], el[5])
    if with_final:
        torch.autograd.backward([y, mT, cT], [gy.to(cuda_device), gm.to(cuda_device), gc.to(cuda_device)])
        torch.autograd.backward([ey, em, ec], [gy.double(), gm.double(), gc.double()])
    else:
        y.backward(gy.to(cuda_device))
        ey.backward(gy.double())
    assert calls, "the HIP scan backward was not used"
    for name, x, e in zip(("k", "v", "q", "r", "mean0", "cov0"), leaves, el):
        close(x.grad, e.grad, "grad " + name)


def test_associative_scan_hip_backward_partial_inputs(cuda_device):
    """Only some inputs need gradients; an empty sequence passes the final-state gradients to the prior."""
    k, v, q, r = O.make_scan_inputs(2, 10, 4, 6, seed=50)
    gy = torch.randn(2, 10, 6, generator=torch.Generator().manual_seed(51))
    kk = k.to(cuda_device).requires_grad_(True)
    y, _, _ = bayes_ssm.associative_static_bayesian_cuda(kk, v.to(cuda_device), q.to(cuda_device),
                                                         observation_variances=r.to(cuda_device))
    y.backward(gy.to(cuda_device))
    ek = k.double().requires_grad_(True)
    ey, _, _ = O.associative_static(ek, v.double(), q.double(), r.double())
    ey.backward(gy.double())
    close(kk.grad, ek.grad, "grad k")

    m0 = torch.randn(2, 4, 6, device=cuda_device, requires_grad=True)
    c0 = (2.0 * torch.eye(4, device=cuda_device)).expand(2, 4, 4).contiguous().requires_grad_(True)
    empty_k = torch.zeros(2, 0, 4, device=cuda_device, requires_grad=True)
    y0, mT, cT = bayes_ssm.associative_static_bayesian_cuda(empty_k, torch.zeros(2, 0, 6, device=cuda_device),
                                                            torch.zeros(2, 0, 4, device=cuda_device),
                                                            initial_mean=m0, initial_covariance=c0)
    assert y0.shape == (2, 0, 6)
    gm, gc = torch.randn_like(mT), torch.randn_like(cT)
    torch.autograd.backward([mT, cT], [gm, gc])
    close(m0.grad, gm, "grad mean0 (T = 0)")
    close(c0.grad, gc, "grad cov0 (T = 0)")


def test_scalar_noise_reaches_the_fused_kernels(cuda_device, monkeypatch):
    """Scalar process/observation noise expand to stride-0 [N, T] views that the gate makes contiguous."""
    from bayes_ssm import fused_cuda

    calls = _count(monkeypatch, fused_cuda._ChunkedBayesianFunction)
    n, t, d = 32, 48, 4
    k, v, q, dec, _, _, gy = O.make_inputs(n, t, d, seed=31)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (k, v, q, dec)]
    y, mT, cT = bayes_ssm.bayesian_layer(*leaves[:3], transition_diagonals=leaves[3], process_variances=0.03,
                                         observation_variances=0.6, chunk_length=16, optimized=True)
    assert calls, "fused HIP path was not taken"
    y.backward(gy.to(cuda_device))
    el = [x.double().requires_grad_(True) for x in (k, v, q, dec)]
    ey, em, ec = O.run_diagonal(*el, torch.full((n, t), 0.03, dtype=F64), torch.full((n, t), 0.6, dtype=F64),
                                torch.zeros(n, d, 8, dtype=F64), torch.eye(d, dtype=F64).expand(n, d, d), 1e-6)
    ey.backward(gy.double())
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    for name, x, e in zip(("k", "v", "q", "decay"), leaves, el):
        close(x.grad, e.grad, "grad " + name)


def test_fp16_inputs_and_fixed_dynamics_reach_the_fused_kernels(cuda_device, monkeypatch):
    """fp16 keys/values/queries are promoted (bayesian_layer.py:823-827); fixed_dynamics selects the
    constant-dynamics kernels (A = 0.97 I, Q = 0.1 I, R = 1; :366-369)."""
    from bayes_ssm import fused_cuda

    calls = _count(monkeypatch, fused_cuda._ChunkedBayesianFunction)
    n, t, d = 24, 40, 2
    k, v, q, _, _, _, gy = O.make_inputs(n, t, d, seed=32)
    kh, vh, qh = (x.half().to(cuda_device).requires_grad_(True) for x in (k, v, q))
    dec = torch.full((n, t, d), O.FIXED_DECAY, device=cuda_device)
    y, mT, cT = bayes_ssm.bayesian_layer(kh, vh, qh, transition_diagonals=dec, process_variances=O.FIXED_PROCESS,
                                         observation_variances=O.FIXED_OBSERVATION, chunk_length=8,
                                         optimized=True, fixed_dynamics=True)
    assert calls, "fused HIP path was not taken"
    assert y.dtype == torch.float32
    y.backward(gy.to(cuda_device))
    el = [x.half().double().requires_grad_(True) for x in (k, v, q)]
    ey, em, ec = O.run_fixed(*el, torch.zeros(n, d, 8, dtype=F64), torch.eye(d, dtype=F64).expand(n, d, d), 1e-6)
    ey.backward(gy.double())
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    for name, x, e in zip(("k", "v", "q"), (kh, vh, qh), el):
        assert x.grad.dtype == torch.float16
        close(x.grad, e.grad, "grad " + name, rtol=2 ** -10, atol=1e-3)


def test_replay_ssm_and_bayesian_layer_modules_on_gpu(cuda_device):
    """The modules on the GPU take the dense replay / chunk paths and match the oracle, gradients included."""
    n, t, d, m = 6, 30, 4, 8
    k, v, q, dec, _, _, gy = O.make_inputs(n, t, d, m, seed=33)
    layer = bayes_ssm.ReplaySSM(d, m, chunk_length=8).to(cuda_device)
    leaves = [x.to(cuda_device).requires_grad_(True) for x in (k, v, q, dec)]
    y, _, _ = layer(*leaves[:3], transition_diagonals=leaves[3])
    y.backward(gy.to(cuda_device))
    el = [x.double().requires_grad_(True) for x in (k, v, q, dec)]
    ey, _, _ = O.run_diagonal(*el, torch.full((n, t), 0.05, dtype=F64), torch.full((n, t), 0.2, dtype=F64),
                              torch.zeros(n, d, m, dtype=F64), torch.eye(d, dtype=F64).expand(n, d, d), 1e-6,
                              strict=False)
    ey.backward(gy.double())
    close(y, ey, "ReplaySSM y")
    for name, x, e in zip(("k", "v", "q", "decay"), leaves, el):
        close(x.grad, e.grad, "ReplaySSM grad " + name)

    bl = bayes_ssm.BayesianLayer(d, m, learn_noise=True).to(cuda_device)
    g = torch.Generator().manual_seed(34)
    A = 0.9 * torch.eye(d) + 0.05 * torch.randn(n, t, d, d, generator=g)
    y2, _, _ = bl(k.to(cuda_device), v.to(cuda_device), q.to(cuda_device), transitions=A.to(cuda_device),
                  optimized=True)
    y2.backward(gy.to(cuda_device))
    raw = torch.tensor(bl._process_raw.item(), dtype=F64, requires_grad=True)
    qv = torch.nn.functional.softplus(raw)
    rv = torch.nn.functional.softplus(torch.tensor(bl._observation_raw.item(), dtype=F64))
    ey2, _, _ = O.run_dense(k.double(), v.double(), q.double(), A.double(),
                            qv * torch.eye(d, dtype=F64).expand(n, t, d, d), rv.expand(n, t),
                            torch.zeros(n, d, m, dtype=F64), 3.0 * torch.eye(d, dtype=F64).expand(n, d, d), 1e-6)
    ey2.backward(gy.double())
    close(y2, ey2, "BayesianLayer y")
    close(bl._process_raw.grad, raw.grad, "BayesianLayer grad process raw")


def test_value_stats_kernel_matches_torch(cuda_device):
    """bssm_value_stats (the batched argument checks): min / max over the finite entries and the non-finite flag,
    float32 and float64, lengths that are not multiples of 4 or of the block chunk, unaligned views, more than
    16 tensors (two launches)."""
    from bayes_ssm.bayesian_layer import _device_value_stats

    g = torch.Generator(device=cuda_device).manual_seed(5)
    base = torch.randn(3 * 16384 + 7, device=cuda_device, generator=g)
    xs = [base, base[1:], base[:5], base[3:40001], torch.full((1,), -2.5, device=cuda_device)]
    bad = base.clone()
    bad[12345] = float("nan")
    xs.append(bad)
    inf = base[:1000].clone()
    inf[999] = float("-inf")
    xs.append(inf)
    d = torch.randn(20001, device=cuda_device, dtype=torch.float64, generator=g)
    d[7] = 1e300
    d[8] = -1e-320
    xs.append(d)
    pos = torch.full((33,), 1e-320, device=cuda_device, dtype=torch.float64)
    xs.append(pos)
    for j in range(10):
        xs.append(torch.rand(1000 + j, device=cuda_device, generator=g) + j)
    out = torch.cat([_device_value_stats(xs[c:c + 16]) for c in range(0, len(xs), 16)]).cpu()
    assert out.shape == (len(xs), 3)
    for i, x in enumerate(xs):
        finite = x[torch.isfinite(x)]
        flag = float(not bool(torch.isfinite(x).all()))
        assert out[i, 2].item() == flag, f"tensor {i}: non-finite flag"
        lo, hi = finite.min().item(), finite.max().item()
        if x.dtype == torch.float32:
            assert out[i, 0].item() == lo and out[i, 1].item() == hi, f"tensor {i}: min / max"
        else:
            # float64: the sign and (within float32) the value are kept.
            assert (out[i, 0].item() > 0) == (lo > 0) and (out[i, 0].item() < 0) == (lo < 0), f"tensor {i}: min sign"
            assert (out[i, 1].item() > 0) == (hi > 0), f"tensor {i}: max sign"
    assert out[-11, 0].item() > 0, "a positive float64 below the float32 range must stay positive"


def test_gpu_argument_checks_use_the_stats_kernel(cuda_device):
    """bayesian_layer on CUDA inputs: the value checks raise the reference's errors, in its order."""
    n, t, d = 4, 12, 4
    k, v, q, dec, p, r, _ = O.make_inputs(n, t, d, seed=61)
    dev = [x.to(cuda_device) for x in (k, v, q, dec, p, r)]
    kk = dev[0].clone()
    kk[1, 2, 3] = float("nan")
    with pytest.raises(ValueError, match="keys must contain only finite"):
        bayes_ssm.bayesian_layer(kk, dev[1], dev[2], transition_diagonals=dev[3], process_variances=dev[4],
                                 observation_variances=dev[5])
    with pytest.raises(ValueError, match="strictly positive"):
        bayes_ssm.bayesian_layer(*dev[:3], transition_diagonals=dev[3], process_variances=dev[4],
                                 observation_variances=torch.zeros_like(dev[5]))
    with pytest.raises(ValueError, match="nonnegative"):
        bayes_ssm.bayesian_layer(*dev[:3], transition_diagonals=dev[3], process_variances=-dev[4],
                                 observation_variances=torch.zeros_like(dev[5]))
    with pytest.raises(ValueError, match="transition_diagonals must contain only finite"):
        bad = dev[3].clone()
        bad[0, 0, 0] = float("inf")
        bayes_ssm.bayesian_layer(*dev[:3], transition_diagonals=bad, process_variances=dev[4],
                                 observation_variances=torch.zeros_like(dev[5]))
    y, _, _ = bayes_ssm.bayesian_layer(*dev[:3], transition_diagonals=dev[3], process_variances=dev[4],
                                       observation_variances=dev[5])
    assert torch.isfinite(y).all()


def test_gpu_checks_read_back_after_the_fused_launch(cuda_device):
    """The value checks are read back once the fused kernels are queued: the errors, and their order
    (a tensor's value error before a bad denominator_floor), stay the reference's, on every fused path."""
    n, t, d = 4, 12, 4
    k, v, q, dec, p, r, _ = O.make_inputs(n, t, d, seed=62)
    dev = [x.to(cuda_device) for x in (k, v, q, dec, p, r)]
    kk = dev[0].clone()
    kk[0, 5, 1] = float("inf")
    with pytest.raises(ValueError, match="keys must contain only finite"):
        bayes_ssm.bayesian_layer(kk, *dev[1:3], transition_diagonals=dev[3], process_variances=dev[4],
                                 observation_variances=dev[5], denominator_floor=-1.0)
    with pytest.raises(ValueError, match="denominator_floor must be positive"):
        bayes_ssm.bayesian_layer(*dev[:3], transition_diagonals=dev[3], process_variances=dev[4],
                                 observation_variances=dev[5], denominator_floor=-1.0)
    # Rotation dynamics (fused rotation kernels).
    rad = torch.full((n, t, d // 2), 0.9, device=cuda_device)
    ang = torch.full((n, t, d // 2), 0.3, device=cuda_device)
    with pytest.raises(ValueError, match="keys must contain only finite"):
        bayes_ssm.bayesian_layer(kk, *dev[1:3], rotation_radii=rad, rotation_angles=ang,
                                 process_variances=dev[4].unsqueeze(-1).expand(n, t, d // 2).contiguous(),
                                 observation_variances=dev[5])
    # The associative scan's kernel is queued before its checks are read back.
    rr = torch.full((1, 16), 1e-9, device=cuda_device)
    kk0, vv0, qq0 = (torch.randn(1, 16, w, device=cuda_device) for w in (4, 4, 4))
    with pytest.raises(ValueError, match="greater than or equal to denominator_floor"):
        bayes_ssm.associative_static_bayesian_cuda(kk0, vv0, qq0, observation_variances=rr)
    with pytest.raises(ValueError, match="initial_mean must contain only finite"):
        bayes_ssm.associative_static_bayesian_cuda(kk0, vv0, qq0,
                                                   initial_mean=torch.full((1, 4, 4), float("nan"),
                                                                           device=cuda_device))
    # Valid calls after the failures still run and agree with the oracle.
    y, _, _ = bayes_ssm.bayesian_layer(*dev[:3], transition_diagonals=dev[3], process_variances=dev[4],
                                       observation_variances=dev[5])
    ref = O.run_diagonal(*(x.double() for x in (k, v, q, dec, p, r)), torch.zeros(n, d, 8, dtype=torch.float64),
                         torch.eye(d, dtype=torch.float64).expand(n, d, d), 1e-6)[0]
    assert torch.allclose(y.double().cpu(), ref, rtol=1e-5, atol=1e-4)
    y0, _, _ = bayes_ssm.associative_static_bayesian_cuda(kk0, vv0, qq0)
    assert torch.isfinite(y0).all()
