"""GPU parity with the innovation floor active (every kernel family, every backward ABI).

``denominator_floor`` is raised so that a share of tokens has r + k.u below it:
there the gain uses 1/floor, and dL/dr and the s-path of dL/dk vanish.  Token
0 of some sequences is built so that r + k.u equals the floor exactly in
binary (P0 = I, d = 1, p = 0, dyadic k and r): there the diagonal kernels'
strict gate ``s > floor`` (persistent_bayes_chunked_d4m8.cu:315) zeroes dL/dr,
as the oracle's ``floor_clamp`` does, while the rotation kernels follow the
reference's torch core (clamp_min passes the gradient at equality).

Other tokens whose float64 r + k.u lies within 2e-4 (relative) of the floor
are moved away from it first (r raised, or k scaled for fixed dynamics), so
float32 rounding cannot put the GPU and the oracle on different sides of the
gate.  Tolerance (north star): 1e-5 relative, 1e-4 absolute.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O
from tests.test_gpu_parity import ABIS, _case, _fixed_dynamics, close

pytestmark = pytest.mark.gpu

# Exactly representable floors near the 30-40 % quantile of r + k.u for each
# key dimension (fixed dynamics have r = 1, so there s >= 1).
FLOORS = {1: 0.75, 2: 0.875, 4: 1.25, 8: 2.0}
FLOORS_FIXED = {1: 1.125, 2: 1.375, 4: 2.25, 8: 4.5}
FLOOR = 0.75  # D = 64, the mixer and the rotation cases
BAND = 2e-4
NAMES = ["gk", "gv", "gq", "gd", "gp", "gr", "gm0", "gc0"]


def _innovations(c, floor):
    f = {k: x.double() for k, x in c.items()}
    seen = []
    O.run_diagonal(f["k"], f["v"], f["q"], f["d"], f["p"], f["r"], f["m0"], f["c0"], floor, innovations=seen)
    return torch.stack(seen, dim=-1)


def _build_equality(cpu, rows, floor):
    """Token 0 of `rows`: P0 = I, d = 1, p = 0, k = (0.5, 0.5, 0, ...) -> u = k, r + k.u == floor exactly."""
    d = cpu["k"].shape[-1]
    nz = min(d, 2)
    for i in rows:
        cpu["c0"][i] = torch.eye(d)
        cpu["d"][i, 0] = 1.0
        cpu["p"][i, 0] = 0.0
        cpu["k"][i, 0] = 0.0
        cpu["k"][i, 0, :nz] = 0.5
        cpu["r"][i, 0] = floor - 0.25 * nz


def _settle(cpu, floor, fixed, protect):
    """Move tokens off the floor band (not the protected, deliberately equal ones); returns r + k.u."""
    for _ in range(200):
        ref = _fixed_dynamics(cpu) if fixed else cpu
        s = _innovations(ref, floor)
        near = ((s - floor).abs() < BAND * floor) & ~protect
        if not near.any():
            return s
        rows = near.any(-1).nonzero().flatten()
        first = near.float().argmax(-1)
        for i in rows.tolist():
            t = int(first[i])
            if fixed:
                cpu["k"][i, t] *= 1.05
            else:
                cpu["r"][i, t] += 5 * BAND * floor
    raise AssertionError("could not move the innovations off the floor band")


def _floor_case(n, t, d, seed, device, fixed, eq_rows=(0, 5, 17)):
    cpu, _ = _case(n, t, d, seed, "cpu")
    floor = (FLOORS_FIXED if fixed else FLOORS)[d]
    protect = torch.zeros(n, t, dtype=torch.bool)
    if not fixed and t:
        rows = [i for i in eq_rows if i < n]
        _build_equality(cpu, rows, floor)
        protect[rows, 0] = True
    s = _settle(cpu, floor, fixed, protect)
    below = (s < floor).float().mean()
    assert 0.05 < below < 0.95, f"floor active on {below:.2f} of the tokens"
    if not fixed:
        assert bool((s[protect] == floor).all()), "equality tokens are not exactly at the floor"
    dev = {name: x.to(device).contiguous() for name, x in cpu.items()}
    return cpu, dev, floor


def _run_abi(ext, name, fixed, nout, dev, chunk, floor):
    fwd = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    y, mT, cT, bm, bc = fwd(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"],
                            chunk, floor)
    args = (dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], bm, bc, dev["gy"],
            dev["gmf"], dev["gcf"], chunk, floor)
    if hasattr(ext, name):
        grads = getattr(ext, name)(*args)
    else:  # noinitial is exported for D2 only (as in the reference); the C ABI has it for every D
        grads = ext._backward("bssm_" + name, fixed, nout, *args[:8], bm, bc, (), dev["gy"], dev["gmf"],
                              dev["gcf"], chunk, floor)
    torch.cuda.synchronize()
    return (y, mT, cT), grads


def _check(cpu, fixed, floor, outs, grads, nout, eq_rows_checked=True):
    ref = _fixed_dynamics(cpu) if fixed else cpu
    f = {k: x.double() for k, x in ref.items()}
    ey, em, ec, eg = O.diagonal_grads(f["k"], f["v"], f["q"], f["d"], f["p"], f["r"], f["m0"], f["c0"], f["gy"],
                                      f["gmf"], f["gcf"], floor=floor)
    for name, a, e in zip(("y", "mean_T", "cov_T"), outs, (ey, em, ec)):
        close(a, e, name)
    for i in range(nout):
        if fixed and NAMES[i] in ("gd", "gp", "gr"):
            assert torch.count_nonzero(grads[i]) == 0, f"{NAMES[i]} must be zero for fixed dynamics"
            continue
        close(grads[i], eg[i], NAMES[i])
    if nout >= 6 and not fixed and eq_rows_checked:
        # The strict gate at the equality tokens: dL/dr is exactly zero.
        gr = grads[5].cpu()
        assert float(gr[0, 0]) == 0.0 and float(gr[5, 0]) == 0.0


def _ext(d):
    from bayes_ssm import fused_cuda

    e = fused_cuda._load_extension(d)
    assert e is not None
    return e


# T = 64 with the library's preferred checkpoint chunk takes the dedicated
# kernels for D = 1, 2, 4 (rotated layout for D = 4); T = 45 with chunk 13
# takes the generic kernels (also D = 8 at T = 64).
@pytest.mark.parametrize("d", [1, 2, 4, 8])
@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
@pytest.mark.parametrize("shape", ["dedicated", "generic"])
def test_floor_active_every_abi(cuda_device, d, abi, shape):
    from bayes_ssm import _hip

    name, fixed, nout = abi
    t, chunk = (64, _hip.preferred_checkpoint(d)) if shape == "dedicated" else (45, 13)
    print(f"floor d={d} {name} {shape} t={t} chunk={chunk}", flush=True)
    cpu, dev, floor = _floor_case(37, t, d, seed=40 + d + t, device=cuda_device, fixed=fixed)
    outs, grads = _run_abi(_ext(d), name, fixed, nout, dev, chunk, floor)
    assert len(grads) == nout
    _check(cpu, fixed, floor, outs, grads, nout)


@pytest.mark.parametrize("d", [1, 2, 4, 8])
def test_floor_autograd_boundary_config_length(cuda_device, d):
    """fused_diagonal_bayesian at T = 512 with the floor active: the checkpoint-interval path of every D."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    print(f"floor autograd d={d}", flush=True)
    cpu, dev, floor = _floor_case(20, 512, d, seed=60 + d, device=cuda_device, fixed=False)
    leaves = {k: dev[k].clone().requires_grad_(True) for k in ("k", "v", "q", "d", "p", "r")}
    y, mT, cT = fused_diagonal_bayesian(leaves["k"], leaves["v"], leaves["q"], leaves["d"], leaves["p"],
                                        leaves["r"], dev["m0"], dev["c0"], chunk_length=64, denominator_floor=floor)
    torch.autograd.backward([y, mT, cT], [dev["gy"], dev["gmf"], dev["gcf"]])
    grads = [leaves[k].grad for k in ("k", "v", "q", "d", "p", "r")]
    _check(cpu, False, floor, (y, mT, cT), grads, 6)


@pytest.mark.parametrize("t", [64, 52])
def test_floor_bf16_kernels_equal_float32_kernels(cuda_device, rotated_layout, t):
    """The bf16 k/v/q D4M8 kernels with the floor active: bitwise the float32 kernels' results."""
    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    print(f"floor bf16 t={t}", flush=True)
    cpu, dev, floor = _floor_case(24, t, 4, seed=80 + t, device=cuda_device, fixed=False)
    outs = []
    grads = []
    for bf16 in (True, False):
        lv = {x: (dev[x].bfloat16() if (bf16 and x in "kvq") else dev[x]).clone().requires_grad_(True)
              for x in "kvqdpr"}
        y, mT, cT = fused_diagonal_bayesian(lv["k"], lv["v"], lv["q"], lv["d"], lv["p"], lv["r"], dev["m0"],
                                            dev["c0"], chunk_length=64, denominator_floor=floor)
        torch.autograd.backward([y, mT, cT], [dev["gy"], dev["gmf"], dev["gcf"]])
        outs.append((y, mT, cT))
        grads.append([lv[x].grad for x in "kvqdpr"])
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
    for i, x in enumerate("kvqdpr"):
        expected = grads[1][i].bfloat16() if x in "kvq" else grads[1][i]
        assert torch.equal(grads[0][i], expected), f"grad {x}"
    _check(cpu, False, floor, outs[1], grads[1], 6)


def test_floor_d64(cuda_device):
    """D = M = 64 (bssm_d64.hip) forward and full backward with the floor active and equality tokens."""
    print("floor d64", flush=True)
    from bayes_ssm import _hip

    n, t, d = 6, 16, 64
    cpu, _ = _case(n, t, d, seed=90, device="cpu", m=d)
    cpu["k"] = cpu["k"] / d ** 0.5
    cpu["q"] = cpu["q"] / d ** 0.5
    protect = torch.zeros(n, t, dtype=torch.bool)
    _build_equality(cpu, [0, 3], FLOOR)
    protect[[0, 3], 0] = True
    s = _settle(cpu, FLOOR, False, protect)
    assert 0.05 < (s < FLOOR).float().mean() < 0.95
    assert bool((s[protect] == FLOOR).all())
    dev = {name: x.to(cuda_device).contiguous() for name, x in cpu.items()}
    ext = _ext(64)
    chunk = _hip.preferred_checkpoint(64)
    outs, grads = _run_abi(ext, "backward_chunked", False, 8, dev, chunk, FLOOR)
    f = {k: x.double() for k, x in cpu.items()}
    ey, em, ec, eg = O.diagonal_grads(f["k"], f["v"], f["q"], f["d"], f["p"], f["r"], f["m0"], f["c0"], f["gy"],
                                      f["gmf"], f["gcf"], floor=FLOOR)
    eg[7] = 0.5 * (eg[7] + eg[7].transpose(-1, -2))  # the D = 64 kernels' symmetric gc0 convention
    for name, a, e in zip(("y", "mean_T", "cov_T"), outs, (ey, em, ec)):
        close(a, e, name)
    for name, a, e in zip(NAMES, grads, eg):
        close(a, e, name)
    gr = grads[5].cpu()
    assert float(gr[0, 0]) == 0.0 and float(gr[3, 0]) == 0.0


def _mixer_case(b, t, h, seed, floor):
    """Mixer inputs whose float64 innovations stay off the floor band (the seed is checked, not adjusted)."""
    views, g_read = O.make_mixer_inputs(b, t, h, seed=seed)
    seen = []
    O.mixer_core(*views, h, floor=floor, innovations=seen)
    s = torch.stack(seen, dim=-1)
    assert 0.05 < (s < floor).float().mean() < 0.95
    assert float(((s - floor).abs() / floor).min()) > BAND, "seed puts a token on the floor band"
    return views, g_read


def test_floor_mixer_core(cuda_device):
    """The producer-fused mixer kernels with the floor active: readout and all gradients."""
    from tests.test_gpu_mixer import _backward, _device_views, _forward, _lds, _state

    print("floor mixer", flush=True)
    b, t, h = 2, 36, 16
    views, g_read = _mixer_case(b, t, h, seed=2024, floor=FLOOR)
    m0, c0, gmf, gcf = _state(b * h, seed=3)
    dv = _device_views(views, cuda_device)
    lds = _lds(views)
    d = {k: x.to(cuda_device) for k, x in dict(m0=m0, c0=c0, gmf=gmf, gcf=gcf, gy=g_read).items()}
    read, mT, cT, bm, bc = _forward(dv, lds, d["m0"], d["c0"], b, t, h, floor=FLOOR)
    g32 = _backward(dv, lds, d["m0"], d["c0"], bm, bc, d["gy"], d["gmf"], d["gcf"], b, t, h, f32=True, floor=FLOOR)
    torch.cuda.synchronize()
    e_read, e_mT, e_cT, e_grads = O.mixer_grads(*views, h, m0, c0, g_read, gmf, gcf, floor=FLOOR)
    close(read.view(b, t, h, 8), e_read, "read")
    close(mT, e_mT, "mean_T")
    close(cT, e_cT, "cov_T")
    for name, a, e in zip(["g_q", "g_k", "g_v", "g_decay_logits", "g_noise", "g_mean0", "g_cov0"], g32, e_grads):
        close(a, e, name)


def test_floor_mixer_gated(cuda_device):
    """The gated readout kernels with the floor active."""
    from tests.test_gpu_mixer import (EPS32, _device_views, _gate_inputs, _gated_backward, _gated_forward, _lds,
                                      _state)

    print("floor mixer gated", flush=True)
    b, t, h = 2, 36, 16
    views, _ = _mixer_case(b, t, h, seed=2024, floor=FLOOR)
    gate, w, gout = _gate_inputs(b, t, h, seed=5, gate_pad=0)
    m0, c0, gmf, gcf = _state(b * h, seed=6)
    dv = _device_views(views, cuda_device)
    lds = _lds(views)
    d = {k: x.to(cuda_device) for k, x in dict(m0=m0, c0=c0, gmf=gmf, gcf=gcf, w=w, gout=gout,
                                                gate=gate).items()}
    o32, yb, mT, cT, bm, bc = _gated_forward(dv, lds, d["gate"], d["w"], d["m0"], d["c0"], b, t, h, True,
                                             floor=FLOOR)
    g32 = _gated_backward(dv, lds, d["gate"], d["w"], d["m0"], d["c0"], bm, bc, yb, d["gout"], d["gmf"], d["gcf"],
                          b, t, h, True, floor=FLOOR)
    torch.cuda.synchronize()
    leaves = [x.detach().double().requires_grad_(True) for x in (*views, gate, w, m0, c0)]
    read, e_mT, e_cT = O.mixer_core(*leaves[:5], h, leaves[7], leaves[8], floor=FLOOR)
    e_out = O.mixer_readout(read, leaves[5], leaves[6], EPS32, read_bf16=yb.cpu())
    close(yb.view(b, t, h, 8), read, "read_bf16", rtol=2 ** -8, atol=1e-6)
    close(o32, e_out, "out")
    close(mT, e_mT, "mean_T")
    close(cT, e_cT, "cov_T")
    loss = (e_out * gout.double()).sum() + (e_mT * gmf.double()).sum() + (e_cT * gcf.double()).sum()
    e_grads = torch.autograd.grad(loss, leaves)
    for name, a, e in zip(["g_q", "g_k", "g_v", "g_decay_logits", "g_noise", "g_gate"], g32[:6], e_grads[:6]):
        close(a, e, name)
    close(g32[6].sum(0), e_grads[6], "g_norm_weight")
    close(g32[7], e_grads[7], "g_mean0")
    close(g32[8], e_grads[8], "g_cov0")


@pytest.mark.parametrize("d", [2, 4, 8])
def test_floor_rotation(cuda_device, d):
    """Rotation kernels with the floor active; at r + k.u == floor they pass dL/dr (clamp_min, as the
    reference's torch core), unlike the diagonal kernels' strict gate."""
    from bayes_ssm import _hip
    from tests.test_gpu_rotation import _case as rot_case
    from tests.test_gpu_rotation import _run

    print(f"floor rotation d={d}", flush=True)
    n, t = 9, 40
    ins, gy, gmf, gcf = rot_case(n, t, d, seed=300 + d)
    k, v, q, rad, ang, p, r, m0, c0 = ins
    r.copy_(0.1 + torch.rand(n, t, generator=torch.Generator().manual_seed(d)))
    eq = [0, 4]
    for i in eq:  # rho = 0.5, angle 0, p = 0, P0 = I: P' = I/4, u = k/4, k = (1, 1, 0..): k.u = 0.5
        rad[i, 0] = 0.5
        ang[i, 0] = 0.0
        p[i, 0] = 0.0
        c0[i] = torch.eye(d)
        k[i, 0] = 0.0
        k[i, 0, :2] = 1.0
        r[i, 0] = FLOOR - 0.5
    protect = torch.zeros(n, t, dtype=torch.bool)
    protect[eq, 0] = True
    for _ in range(200):
        seen = []
        O.run_rotation(*(x.double() for x in (k, v, q, rad, ang, p, r, m0, c0)), FLOOR, innovations=seen)
        s = torch.stack(seen, dim=-1)
        near = ((s - FLOOR).abs() < BAND * FLOOR) & ~protect
        if not near.any():
            break
        first = near.float().argmax(-1)
        for i in near.any(-1).nonzero().flatten().tolist():
            r[i, int(first[i])] += 5 * BAND * FLOOR
    else:
        raise AssertionError("could not move the innovations off the floor band")
    assert bool((s[protect] == FLOOR).all())
    assert 0.05 < (s < FLOOR).float().mean() < 0.95
    chunk = _hip.load().bssm_rotation_checkpoint(d)
    y, mT, cT, bm, bc, grads = _run([k, v, q, rad, ang, p, r, m0, c0], gy, gmf, gcf, chunk, cuda_device,
                                    floor=FLOOR)
    leaves = [x.double().requires_grad_(True) for x in (k, v, q, rad, ang, p, r, m0, c0)]
    ey, em, ec = O.run_rotation(*leaves, FLOOR)
    loss = (ey * gy.double()).sum() + (em * gmf.double()).sum() + (ec * gcf.double()).sum()
    eg = torch.autograd.grad(loss, leaves)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    names = ["gk", "gv", "gq", "g_radii", "g_angles", "g_process", "g_observation", "gm0", "gc0"]
    for name, a, e in zip(names, grads, eg):
        close(a, e, name)
    assert float(grads[6][0, 0]) != 0.0, "clamp_min passes dL/dr at s == floor"
