"""GPU parity of the rotation-dynamics kernels (C ABI bssm_*_chunked_rotation) against the CPU oracle.

The oracle restates the reference's rotation core (bayes_ssm/bayesian_layer.py:254-323) in float64;
tolerance 1e-5 relative / 1e-4 absolute on outputs, checkpoints and all gradients.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-4


def close(actual, expected, name=""):
    torch.testing.assert_close(actual.detach().double().cpu(), expected.detach().double().cpu(), rtol=RTOL,
                               atol=ATOL, msg=lambda m: f"{name}: {m}")


def _case(n, t, d, seed, angle_scale=2.0):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(n, t, d, generator=g) / d ** 0.5
    v = torch.randn(n, t, 8, generator=g)
    q = torch.randn(n, t, d, generator=g)
    rad = 0.6 + 0.5 * torch.rand(n, t, d // 2, generator=g)  # about a fifth above 1 (clamped)
    ang = angle_scale * torch.randn(n, t, d // 2, generator=g)
    p = 0.02 + 0.2 * torch.rand(n, t, d // 2, generator=g)
    r = 0.3 + torch.rand(n, t, generator=g)
    m0 = 0.2 * torch.randn(n, d, 8, generator=g)
    a = torch.randn(n, d, d, generator=g)
    c0 = a @ a.transpose(-1, -2) / d + 0.5 * torch.eye(d)
    c0 = 0.5 * (c0 + c0.transpose(-1, -2))
    gy = torch.randn(n, t, 8, generator=g)
    gmf = torch.randn(n, d, 8, generator=g)
    gcf = torch.randn(n, d, d, generator=g)
    return [k, v, q, rad, ang, p, r, m0, c0], gy, gmf, gcf


def _run(ins, gy, gmf, gcf, chunk, device, floor=1e-6):
    from bayes_ssm import _hip

    k, v, q, rad, ang, p, r, m0, c0 = [x.to(device).contiguous() for x in ins]
    n, t, d = k.shape
    nb = -(-t // chunk)
    y = torch.empty(n, t, 8, device=device)
    mT, cT = torch.empty(n, d, 8, device=device), torch.empty(n, d, d, device=device)
    bm, bc = torch.empty(n, nb + 1, d, 8, device=device), torch.empty(n, nb + 1, d, d, device=device)
    P = _hip.ptr
    s = _hip.stream_of(device)
    _hip.call("bssm_forward_chunked_rotation", d, 8, P(k), P(v), P(q), P(rad), P(ang), P(p), P(r), P(m0), P(c0),
              P(y), P(mT), P(cT), P(bm), P(bc), n, t, chunk, floor, s)
    grads = [torch.empty_like(x) for x in (k, v, q, rad, ang, p, r, m0, c0)]
    gy_d, gmf_d, gcf_d = gy.to(device), gmf.to(device), gcf.to(device)
    _hip.call("bssm_backward_chunked_rotation", d, 8, P(k), P(v), P(q), P(rad), P(ang), P(p), P(r), P(m0), P(c0),
              P(bm), P(bc), P(gy_d), P(gmf_d), P(gcf_d), *map(P, grads), n, t, chunk, floor, s)
    torch.cuda.synchronize()
    return y, mT, cT, bm, bc, grads


@pytest.mark.parametrize("d", [2, 4, 8])
# T = 52 (a multiple of 4, several 16-token forward tiles and a partial
# last one) takes the register-staged prefetch of the forward and, for D = 8,
# of the backward; T = 37 and 21 stage synchronously.
@pytest.mark.parametrize("n,t,chunk", [(13, 37, 0), (5, 16, 0), (9, 21, 5), (3, 1, 0), (7, 52, 0)])
def test_rotation_abi_matches_oracle(cuda_device, d, n, t, chunk):
    from bayes_ssm import _hip

    chunk = chunk or _hip.load().bssm_rotation_checkpoint(d)
    print(f"rotation d={d} n={n} t={t} chunk={chunk}", flush=True)
    ins, gy, gmf, gcf = _case(n, t, d, seed=100 * d + t)
    y, mT, cT, bm, bc, grads = _run(ins, gy, gmf, gcf, chunk, cuda_device)
    leaves = [x.double().requires_grad_(True) for x in ins]
    ey, em, ec = O.run_rotation(*leaves, 1e-6)
    loss = (ey * gy.double()).sum() + (em * gmf.double()).sum() + (ec * gcf.double()).sum()
    eg = torch.autograd.grad(loss, leaves)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    names = ["gk", "gv", "gq", "g_radii", "g_angles", "g_process", "g_observation", "gm0", "gc0"]
    for name, a, e in zip(names, grads, eg):
        close(a, e, name)
    # Checkpoints: the belief before token c * chunk.
    with torch.no_grad():
        for c in range(bm.shape[1] - 1):
            stop = c * chunk
            _, mc, cc = O.run_rotation(*(x.double()[:, :stop] for x in ins[:7]), ins[7].double(), ins[8].double(),
                                       1e-6) if stop else (None, ins[7].double(), ins[8].double())
            close(bm[:, c], mc, f"bmean[{c}]")
            close(bc[:, c], cc, f"bcov[{c}]")


@pytest.mark.parametrize("lay", ["row", "quad"])
# T multiple of 4 with aligned streams: the row-per-sequence forward (row) or
# the quad-per-sequence one (quad) for D = 4.  Chunk 4 and the partial tiles
# (T = 52, 36, 4, 8) take the row kernel's token-by-token path; n = 65 leaves
# one sequence in the last wave of four.
@pytest.mark.parametrize("n,t,chunk", [(5, 16, 0), (7, 52, 0), (9, 20, 4), (65, 36, 0), (3, 4, 0), (2, 8, 8)])
def test_rotation_d4_forward_layouts(cuda_device, lay, n, t, chunk):
    from bayes_ssm import _hip
    from tests._layouts import layout

    chunk = chunk or _hip.load().bssm_rotation_checkpoint(4)
    print(f"rotation d4 layout={lay} n={n} t={t} chunk={chunk}", flush=True)
    ins, gy, gmf, gcf = _case(n, t, 4, seed=300 + t + n)
    with layout(lay):
        y, mT, cT, bm, bc, grads = _run(ins, gy, gmf, gcf, chunk, cuda_device)
    leaves = [x.double().requires_grad_(True) for x in ins]
    ey, em, ec = O.run_rotation(*leaves, 1e-6)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    assert torch.equal(cT, cT.transpose(-1, -2)), "cov_T not bitwise symmetric"
    if t:
        loss = (ey * gy.double()).sum() + (em * gmf.double()).sum() + (ec * gcf.double()).sum()
        eg = torch.autograd.grad(loss, leaves)
        names = ["gk", "gv", "gq", "g_radii", "g_angles", "g_process", "g_observation", "gm0", "gc0"]
        for name, a, e in zip(names, grads, eg):
            close(a, e, name)
    with torch.no_grad():
        for c in range(bm.shape[1]):
            stop = min(c * chunk, t)
            _, mc, cc = O.run_rotation(*(x.double()[:, :stop] for x in ins[:7]), ins[7].double(), ins[8].double(),
                                       1e-6) if stop else (None, ins[7].double(), ins[8].double())
            close(bm[:, c], mc, f"bmean[{c}]")
            close(bc[:, c], cc, f"bcov[{c}]")
            assert torch.equal(bc[:, c], bc[:, c].transpose(-1, -2)), f"bcov[{c}] not bitwise symmetric"


def test_rotation_large_angles(cuda_device):
    """Angles of tens of radians: the kernels' own sin/cos reduction stays within tolerance."""
    ins, gy, gmf, gcf = _case(8, 24, 4, seed=7, angle_scale=40.0)
    from bayes_ssm import _hip

    y, mT, cT, _, _, grads = _run(ins, gy, gmf, gcf, _hip.load().bssm_rotation_checkpoint(4), cuda_device)
    leaves = [x.double().requires_grad_(True) for x in ins]
    ey, em, ec = O.run_rotation(*leaves, 1e-6)
    loss = (ey * gy.double()).sum() + (em * gmf.double()).sum() + (ec * gcf.double()).sum()
    eg = torch.autograd.grad(loss, leaves)
    close(y, ey, "y")
    close(cT, ec, "cov_T")
    close(grads[4], eg[4], "g_angles")
    close(grads[3], eg[3], "g_radii")


def test_bayesian_layer_routes_rotation_to_kernels(cuda_device, monkeypatch):
    """bayesian_layer(rotation_radii=..., rotation_angles=..., optimized=True) runs the HIP kernels."""
    import bayes_ssm
    from bayes_ssm import fused_cuda

    calls = []
    orig = fused_cuda._ChunkedRotationFunction.apply
    monkeypatch.setattr(fused_cuda._ChunkedRotationFunction, "apply",
                        staticmethod(lambda *a: calls.append(1) or orig(*a)))
    ins, gy, _, _ = _case(6, 20, 4, seed=3)
    k, v, q, rad, ang, p, r, _, _ = [x.to(cuda_device) for x in ins]
    leaves = [x.clone().requires_grad_(True) for x in (k, v, q, rad, ang)]
    y, mT, cT = bayes_ssm.bayesian_layer(*leaves[:3], rotation_radii=leaves[3], rotation_angles=leaves[4],
                                         process_variances=p, observation_variances=r, chunk_length=16,
                                         optimized=True)
    assert calls, "rotation kernels were not used"
    y.backward(gy.to(cuda_device))
    cpu = [x.double() for x in ins]
    cl = [x.clone().requires_grad_(True) for x in cpu[:5]]
    m0 = torch.zeros(6, 4, 8, dtype=torch.float64)
    c0 = torch.eye(4, dtype=torch.float64).expand(6, 4, 4)
    ey, _, _ = O.run_rotation(*cl, cpu[5], cpu[6], m0, c0, 1e-6)
    ey.backward(gy.double())
    close(y, ey, "y")
    for name, a, e in zip(["gk", "gv", "gq", "g_radii", "g_angles"], leaves, cl):
        close(a.grad, e.grad, name)


@pytest.mark.parametrize("d", [2, 4, 8])
def test_rotation_long_sequences(cuda_device, d):
    """T = 512 (the config-3 length): 64 checkpoint chunks of float32 drift against the float64 oracle."""
    from bayes_ssm import _hip

    chunk = _hip.load().bssm_rotation_checkpoint(d)
    n, t = 20, 512
    print(f"rotation long d={d} n={n} t={t}", flush=True)
    ins, gy, gmf, gcf = _case(n, t, d, seed=700 + d, angle_scale=1.0)
    y, mT, cT, _, _, grads = _run(ins, gy, gmf, gcf, chunk, cuda_device)
    leaves = [x.double().requires_grad_(True) for x in ins]
    ey, em, ec = O.run_rotation(*leaves, 1e-6)
    loss = (ey * gy.double()).sum() + (em * gmf.double()).sum() + (ec * gcf.double()).sum()
    eg = torch.autograd.grad(loss, leaves)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    names = ["gk", "gv", "gq", "g_radii", "g_angles", "g_process", "g_observation", "gm0", "gc0"]
    for name, a, e in zip(names, grads, eg):
        close(a, e, name)


@pytest.mark.parametrize("lay", ["row", "quad"])
def test_rotation_config3_full_size_rows(cuda_device, lay):
    """Config 3's shape (16384 sequences x T512, D4M8) on the rotation kernels, the forward in either layout
    (the default picks by sequence count, so both runs are pinned to one): rows run alone match the full run's
    rows bit for bit (sequences are independent), and those rows match the oracle."""
    from bayes_ssm import _hip
    from tests._layouts import layout

    d, n, t = 4, 256 * 64, 512
    chunk = _hip.load().bssm_rotation_checkpoint(d)
    print(f"rotation config3 full size layout={lay}", flush=True)
    ins, gy, gmf, gcf = _case(n, t, d, seed=733, angle_scale=1.0)
    rows = torch.tensor([0, 4097, 9999, n - 1])
    sub_ins = [x[rows].contiguous() for x in ins]
    with layout(lay):
        full = _run(ins, gy, gmf, gcf, chunk, cuda_device)
        sub = _run(sub_ins, gy[rows], gmf[rows], gcf[rows], chunk, cuda_device)
    rows_d = rows.to(cuda_device)
    for name, a, b in zip(("y", "mean_T", "cov_T", "bmean", "bcov"), sub[:5], full[:5]):
        assert torch.equal(a, b[rows_d]), f"{name}: subset rows differ from the full run"
    for i, (a, b) in enumerate(zip(sub[5], full[5])):
        assert torch.equal(a, b[rows_d]), f"gradient {i}: subset rows differ from the full run"
    del full
    leaves = [x.double().requires_grad_(True) for x in sub_ins]
    ey, em, ec = O.run_rotation(*leaves, 1e-6)
    loss = (ey * gy[rows].double()).sum() + (em * gmf[rows].double()).sum() + (ec * gcf[rows].double()).sum()
    eg = torch.autograd.grad(loss, leaves)
    close(sub[0], ey, "y")
    close(sub[1], em, "mean_T")
    close(sub[2], ec, "cov_T")
    names = ["gk", "gv", "gq", "g_radii", "g_angles", "g_process", "g_observation", "gm0", "gc0"]
    for name, a, e in zip(names, sub[5], eg):
        close(a, e, name)
