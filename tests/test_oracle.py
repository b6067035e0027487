"""Pins of the CPU oracle (oracle/bssm_oracle.py) — CPU only.

The reference ships no golden vectors; its tests assert self-consistency
(diagonal == dense at 1e-12, replay/dense gradients at 1e-10,
tests/test_bayesian_layer_diagonal.py:54-123).  Here the oracle is pinned by
those cross-formulation checks plus closed forms that a plausible mistake
(dropped process noise, wrong decay placement, transposed operand, missing
symmetrisation, wrong floor gate) would fail, plus fp64 gradcheck.
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import bssm_oracle as O


@pytest.fixture(autouse=True)
def _float64_default():
    previous = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(previous)


def _rand(n, t, d, m, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(n, t, d, generator=g, dtype=dtype)
    v = torch.randn(n, t, m, generator=g, dtype=dtype)
    q = torch.randn(n, t, d, generator=g, dtype=dtype)
    dec = 0.6 + 0.39 * torch.rand(n, t, d, generator=g, dtype=dtype)
    p = 0.05 + 0.2 * torch.rand(n, t, generator=g, dtype=dtype)
    r = 0.2 + torch.rand(n, t, generator=g, dtype=dtype)
    m0 = 0.3 * torch.randn(n, d, m, generator=g, dtype=dtype)
    a = torch.randn(n, d, d, generator=g, dtype=dtype)
    c0 = a @ a.transpose(-1, -2) / d + 0.5 * torch.eye(d, dtype=dtype)
    return k, v, q, dec, p, r, m0, c0


def test_scalar_kalman_textbook():
    """D = M = 1 is the scalar Kalman filter; compare with its textbook gain form."""
    k, v, q, dec, p, r, m0, c0 = _rand(1, 12, 1, 1, seed=3)
    y, mT, cT = O.run_diagonal(k, v, q, dec, p, r, m0, c0, 1e-6)
    x, P = float(m0[0, 0, 0]), float(c0[0, 0, 0])
    for t in range(12):
        a, h, z = float(dec[0, t, 0]), float(k[0, t, 0]), float(v[0, t, 0])
        x_pred, P_pred = a * x, a * a * P + float(p[0, t])
        S = h * h * P_pred + float(r[0, t])
        K = P_pred * h / S
        x = x_pred + K * (z - h * x_pred)
        P = (1.0 - K * h) * P_pred
        assert math.isclose(float(y[0, t, 0]), x * float(q[0, t, 0]), rel_tol=1e-12, abs_tol=1e-12)
    assert math.isclose(float(mT[0, 0, 0]), x, rel_tol=1e-12)
    assert math.isclose(float(cT[0, 0, 0]), P, rel_tol=1e-12)


def test_first_step_closed_form():
    """From M0 = 0, P0 = I one step gives u = (d^2 + p) k, M1 = u v^T / (r + k.u)."""
    k, v, q, dec, p, r, _, _ = _rand(3, 1, 4, 5, seed=4)
    m0 = torch.zeros(3, 4, 5)
    c0 = torch.eye(4).expand(3, 4, 4).clone()
    y, mT, cT = O.run_diagonal(k, v, q, dec, p, r, m0, c0, 1e-6)
    u = (dec[:, 0] ** 2 + p[:, 0, None]) * k[:, 0]
    s = r[:, 0] + (k[:, 0] * u).sum(-1)
    M1 = u[:, :, None] * v[:, 0, None, :] / s[:, None, None]
    P1 = torch.diag_embed(dec[:, 0] ** 2 + p[:, 0, None]) - u[:, :, None] * u[:, None, :] / s[:, None, None]
    torch.testing.assert_close(mT, M1, rtol=1e-13, atol=1e-13)
    torch.testing.assert_close(cT, P1, rtol=1e-13, atol=1e-13)
    torch.testing.assert_close(y[:, 0], (M1 * q[:, 0, :, None]).sum(-2), rtol=1e-13, atol=1e-13)


def test_no_observation_limit():
    """k = 0 (or r -> inf) leaves only the prediction: M <- d M, P <- d P d + p I."""
    k, v, q, dec, p, r, m0, c0 = _rand(2, 5, 3, 2, seed=5)
    for variant in ("zero_key", "huge_r"):
        kk = torch.zeros_like(k) if variant == "zero_key" else k
        rr = r if variant == "zero_key" else torch.full_like(r, 1e30)
        _, mT, cT = O.run_diagonal(kk, v, q, dec, p, rr, m0, c0, 1e-6)
        M, P = m0.clone(), c0.clone()
        for t in range(5):
            M = dec[:, t, :, None] * M
            P = dec[:, t, :, None] * P * dec[:, t, None, :] + p[:, t, None, None] * torch.eye(3)
        torch.testing.assert_close(mT, M, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(cT, P, rtol=1e-12, atol=1e-12)


def test_static_closed_form_and_associative_scan():
    """A = I, Q = 0 is Bayesian linear regression; recurrence and information-form scan agree."""
    k, v, q, _, _, r, m0, c0 = _rand(3, 9, 4, 3, seed=6)
    ones = torch.ones_like(k)
    zeros = torch.zeros(k.shape[:-1])
    y, mT, cT = O.run_diagonal(k, v, q, ones, zeros, r, m0, c0, 1e-6)
    M_cf, P_cf = O.closed_form_static(k, v, r, m0, c0)
    torch.testing.assert_close(mT, M_cf, rtol=1e-10, atol=1e-11)
    torch.testing.assert_close(cT, P_cf, rtol=1e-10, atol=1e-11)
    ys, ms, cs = O.associative_static(k, v, q, r, m0, c0)
    torch.testing.assert_close(ys, y, rtol=1e-10, atol=1e-11)
    torch.testing.assert_close(ms, mT, rtol=1e-10, atol=1e-11)
    torch.testing.assert_close(cs, cT, rtol=1e-10, atol=1e-11)
    # Every prefix matches the closed form of that prefix.
    for t in (0, 4, 8):
        M_t, _ = O.closed_form_static(k[:, : t + 1], v[:, : t + 1], r[:, : t + 1], m0, c0)
        torch.testing.assert_close(y[:, t], (M_t * q[:, t, :, None]).sum(-2), rtol=1e-10, atol=1e-11)


@pytest.mark.parametrize("chunk", [1, 2, 3, 7, 64])
def test_dense_diagonal_chunked_agree(chunk):
    """The three recurrence formulations agree (reference tests use 1e-12 / 1e-10)."""
    k, v, q, dec, p, r, m0, c0 = _rand(2, 11, 4, 3, seed=7)
    yd, md, cd = O.run_diagonal(k, v, q, dec, p, r, m0, c0, 1e-6)
    A, Q = O.diagonal_as_dense(dec, p)
    ye, me, ce = O.run_dense(k, v, q, A, Q, r, m0, c0, 1e-6)
    yc, mc, cc = O.run_chunked(k, v, q, A, Q, r, m0, c0, chunk, 1e-6)
    for a, b in ((yd, ye), (md, me), (cd, ce)):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
    for a, b in ((yd, yc), (md, mc), (cd, cc)):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-11)


def test_covariance_invariants():
    """Posterior covariance stays symmetric PSD and below the prediction (P_post <= P_pred)."""
    k, v, q, dec, p, r, m0, c0 = _rand(4, 20, 4, 2, seed=8)
    mean, cov = m0, c0
    for t in range(20):
        P_pred = dec[:, t, :, None] * cov * dec[:, t, None, :] + p[:, t, None, None] * torch.eye(4)
        _, mean, cov = O.run_diagonal(k[:, t:t + 1], v[:, t:t + 1], q[:, t:t + 1], dec[:, t:t + 1],
                                      p[:, t:t + 1], r[:, t:t + 1], mean, cov, 1e-6)
        assert torch.equal(cov, cov.transpose(-1, -2))
        assert torch.linalg.eigvalsh(cov).min() > 0
        assert torch.linalg.eigvalsh(P_pred - cov).min() > -1e-12


def test_fixed_dynamics_is_constant_diagonal():
    k, v, q, _, _, _, m0, c0 = _rand(2, 8, 4, 3, seed=9)
    yf, mf, cf = O.run_fixed(k, v, q, m0, c0, 1e-6)
    dec = torch.full_like(k, O.FIXED_DECAY)
    p = torch.full(k.shape[:-1], O.FIXED_PROCESS)
    r = torch.full(k.shape[:-1], O.FIXED_OBSERVATION)
    yd, md, cd = O.run_diagonal(k, v, q, dec, p, r, m0, c0, 1e-6)
    for a, b in ((yf, yd), (mf, md), (cf, cd)):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_floor_clamps_innovation():
    """With r + k.u below the floor the gain uses 1/floor (bayesian_layer.py:243)."""
    k = torch.full((1, 1, 1), 1e-4)
    v = torch.ones(1, 1, 1)
    q = torch.ones(1, 1, 1)
    dec = torch.ones(1, 1, 1)
    p = torch.zeros(1, 1)
    r = torch.full((1, 1), 1e-9)
    m0 = torch.zeros(1, 1, 1)
    c0 = torch.ones(1, 1, 1)
    floor = 1e-3
    y, _, cT = O.run_diagonal(k, v, q, dec, p, r, m0, c0, floor)
    u = 1e-4
    assert math.isclose(float(y), u / floor, rel_tol=1e-12)
    assert math.isclose(float(cT), 1.0 - u * u / floor, rel_tol=1e-12)


def _equality_token(r_value):
    """One D = 1 token with exact dyadic arithmetic: u = (d^2 P0 + p) k = 0.5, k.u = 0.25, s = r + 0.25."""
    k = torch.full((1, 1, 1), 0.5)
    v = torch.full((1, 1, 1), 1.5)
    q = torch.full((1, 1, 1), 2.0)
    dec = torch.ones(1, 1, 1)
    p = torch.zeros(1, 1)
    r = torch.full((1, 1), r_value)
    m0 = torch.full((1, 1, 1), 0.25)
    c0 = torch.ones(1, 1, 1)
    return k, v, q, dec, p, r, m0, c0


def test_strict_floor_gate_is_the_left_derivative():
    """At r + k.u == floor exactly, the kernels' gate (s > floor) gives dL/dr = 0: the left-sided
    finite difference.  torch's clamp_min passes the gradient (the right-sided one).  Away from the
    floor both equal the central difference; below it both are zero."""
    floor = 1.0
    gy = torch.full((1, 1, 1), 0.75)

    def loss(r_value):
        k, v, q, dec, p, r, m0, c0 = _equality_token(r_value)
        y, _, _ = O.run_diagonal(k, v, q, dec, p, r, m0, c0, floor)
        return float((y * gy).sum())

    def grad_r(r_value, strict):
        k, v, q, dec, p, r, m0, c0 = _equality_token(r_value)
        _, _, _, g = O.diagonal_grads(k, v, q, dec, p, r, m0, c0, gy, floor=floor, strict=strict)
        return float(g[5])

    eq = 0.75  # s = 0.75 + 0.25 == floor, every operation exact in binary
    seen = []
    k, v, q, dec, p, r, m0, c0 = _equality_token(eq)
    O.run_diagonal(k, v, q, dec, p, r, m0, c0, floor, innovations=seen)
    assert float(seen[0]) == floor
    h = 1e-7
    left = (loss(eq) - loss(eq - h)) / h
    right = (loss(eq + h) - loss(eq)) / h
    assert abs(left) < 1e-9 and abs(right) > 1e-2
    assert grad_r(eq, strict=True) == 0.0
    assert math.isclose(grad_r(eq, strict=False), right, rel_tol=1e-5)
    for r_value in (0.9, 1.4):  # above the floor: both conventions are the derivative
        central = (loss(r_value + h) - loss(r_value - h)) / (2 * h)
        for strict in (True, False):
            assert math.isclose(grad_r(r_value, strict), central, rel_tol=1e-6)
    for strict in (True, False):  # below: clamped, no dependence on r
        assert grad_r(0.5, strict) == 0.0
    # A planted mistake (the gate written as s >= floor) is what clamp_min computes: caught above.
    assert grad_r(eq, strict=False) != grad_r(eq, strict=True)


def test_strict_floor_gate_gradcheck_away_from_floor():
    """With the floor active on some tokens (none at equality), the gated oracle passes gradcheck."""
    k, v, q, dec, p, r, m0, c0 = _rand(1, 5, 2, 2, seed=14)
    floor = 1.3
    seen = []
    O.run_diagonal(k, v, q, dec, p, r, m0, c0, floor, innovations=seen)
    s = torch.stack(seen)
    assert (s < floor).any() and (s > floor).any()
    assert ((s - floor).abs() > 1e-3).all()
    leaves = [x.clone().requires_grad_(True) for x in (k, v, q, dec, p, r, m0, c0)]
    assert torch.autograd.gradcheck(lambda *xs: O.run_diagonal(*xs, floor), leaves, eps=1e-7, atol=1e-7,
                                    rtol=1e-5)


def test_checkpoint_layout():
    """bm[:, c] is the belief before token c*chunk, bm[:, nb] the final belief."""
    k, v, q, dec, p, r, m0, c0 = _rand(2, 10, 2, 3, seed=10)
    bm, bc = O.checkpoints(k, v, q, dec, p, r, m0, c0, 4, 1e-6)
    assert bm.shape == (2, 4, 2, 3) and bc.shape == (2, 4, 2, 2)
    torch.testing.assert_close(bm[:, 0], m0, rtol=0, atol=0)
    for c, stop in ((1, 4), (2, 8), (3, 10)):
        _, mt, ct = O.run_diagonal(k[:, :stop], v[:, :stop], q[:, :stop], dec[:, :stop], p[:, :stop],
                                   r[:, :stop], m0, c0, 1e-6)
        torch.testing.assert_close(bm[:, c], mt, rtol=1e-13, atol=1e-13)
        torch.testing.assert_close(bc[:, c], ct, rtol=1e-13, atol=1e-13)


def test_gradcheck_diagonal():
    k, v, q, dec, p, r, m0, c0 = _rand(1, 3, 2, 2, seed=11)
    leaves = [x.clone().requires_grad_(True) for x in (k, v, q, dec, p, r, m0, c0)]

    def f(*xs):
        return O.run_diagonal(*xs, 1e-6)

    assert torch.autograd.gradcheck(f, leaves, eps=1e-6, atol=1e-7, rtol=1e-5)


def test_gradients_agree_across_formulations():
    """Autograd of diagonal vs transported-history oracle (reference: 1e-10 / 1e-11)."""
    k, v, q, dec, p, r, m0, c0 = _rand(2, 9, 3, 2, seed=12)
    g = torch.Generator().manual_seed(1)
    gy = torch.randn(2, 9, 2, generator=g)
    gmf = torch.randn(2, 3, 2, generator=g)
    gcf = torch.randn(2, 3, 3, generator=g)
    _, _, _, ga = O.diagonal_grads(k, v, q, dec, p, r, m0, c0, gy, gmf, gcf)
    _, _, _, gb = O.diagonal_grads(k, v, q, dec, p, r, m0, c0, gy, gmf, gcf, chunk=4)
    # The transported-history path symmetrises the prediction before u = P' k,
    # so only the symmetric part of the initial-covariance gradient is shared.
    for i, (a, b) in enumerate(zip(ga, gb)):
        if i == 7:
            a, b = 0.5 * (a + a.transpose(-1, -2)), 0.5 * (b + b.transpose(-1, -2))
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-10)


def test_asymmetric_initial_covariance_gradient():
    """dL/dP0 keeps the row-wise (asymmetric) term from u = P' k: (S + gu k^T) * d d^T."""
    k, v, q, dec, p, r, m0, c0 = _rand(1, 1, 3, 2, seed=13)
    g = torch.Generator().manual_seed(2)
    gy = torch.randn(1, 1, 2, generator=g)
    _, _, _, grads = O.diagonal_grads(k, v, q, dec, p, r, m0, c0, gy)
    gc0 = grads[7]
    assert (gc0 - gc0.transpose(-1, -2)).abs().max() > 1e-6
    # Finite difference along an antisymmetric direction matches.
    direction = torch.zeros(1, 3, 3)
    direction[0, 0, 1], direction[0, 1, 0] = 1.0, -1.0
    eps = 1e-6

    def loss(c):
        y, _, _ = O.run_diagonal(k, v, q, dec, p, r, m0, c, 1e-6)
        return float((y * gy).sum())

    fd = (loss(c0 + eps * direction) - loss(c0 - eps * direction)) / (2 * eps)
    assert math.isclose(fd, float((gc0 * direction).sum()), rel_tol=1e-6, abs_tol=1e-9)


def test_mutation_is_detected():
    """A planted oracle mistake (process noise dropped) fails the textbook pin."""
    k, v, q, dec, p, r, m0, c0 = _rand(1, 6, 1, 1, seed=3)
    _, good, _ = O.run_diagonal(k, v, q, dec, p, r, m0, c0, 1e-6)
    _, bad, _ = O.run_diagonal(k, v, q, dec, torch.zeros_like(p), r, m0, c0, 1e-6)
    assert (good - bad).abs().max() > 1e-3


# ------------------------------------------------------------- Bayes mixer
def test_mixer_transforms_satisfy_identities():
    """exp(-softplus(x)) = sigmoid(-x); softplus(x) - softplus(-x) = x; unit heads along silu(x)."""
    b, t, h = 1, 7, 2
    x = torch.linspace(-30.0, 30.0, b * t * h * 4).reshape(b, t, h * 4)
    nz = torch.linspace(-25.0, 25.0, b * t * h * 2).reshape(b, t, h * 2)
    v = torch.linspace(-6.0, 6.0, b * t * h * 8).reshape(b, t, h * 8)
    k, vv, q, d, p, r = O.mixer_inputs(x, x, v, x, nz, h)
    _, _, _, _, p_neg, r_neg = O.mixer_inputs(x, x, v, x, -nz, h)
    xs = x.reshape(b, t, h, 4).transpose(1, 2).reshape(b * h, t, 4)
    torch.testing.assert_close(d, torch.sigmoid(-xs), rtol=1e-8, atol=0)
    nzs = nz.reshape(b, t, h, 2).transpose(1, 2).reshape(b * h, t, 2)
    # Exact below the threshold (20); above it softplus(x) = x drops log1p(e^-x) < 2.1e-9.
    torch.testing.assert_close(p - p_neg, nzs[..., 0], rtol=0, atol=1e-8)
    torch.testing.assert_close(r - r_neg, nzs[..., 1], rtol=0, atol=1e-8)
    inside = nzs.abs() < 20
    torch.testing.assert_close((p - p_neg)[inside[..., 0]], nzs[..., 0][inside[..., 0]], rtol=0, atol=1e-12)
    assert float((p - O.MIXER_NOISE_FLOOR).min()) > 0 and float(r.min()) > O.MIXER_NOISE_FLOOR
    torch.testing.assert_close(k.norm(dim=-1), torch.ones(b * h, t), rtol=0, atol=1e-12)
    a = xs / (1 + torch.exp(-xs))  # silu
    cos = (k * a).sum(-1) / a.norm(dim=-1)
    torch.testing.assert_close(cos, torch.ones_like(cos), rtol=0, atol=1e-12)
    vs = v.reshape(b, t, h, 8).transpose(1, 2).reshape(b * h, t, 8)
    torch.testing.assert_close(vv, vs / (1 + torch.exp(-vs)), rtol=1e-14, atol=1e-14)
    # All-zero head: normalize's eps keeps it at zero instead of NaN.
    k0, _, _, _, _, _ = O.mixer_inputs(torch.zeros(1, 1, 4), torch.zeros(1, 1, 4), torch.zeros(1, 1, 8),
                                       torch.zeros(1, 1, 4), torch.zeros(1, 1, 2), 1)
    assert torch.equal(k0, torch.zeros_like(k0))


def test_mixer_sequence_map_with_tagged_heads():
    """Sequence b*H + h, token t of every layer input is head h of batch row b at token t."""
    b, t, h = 3, 5, 4
    tag = torch.arange(b).view(b, 1, 1) * 1000.0 + torch.arange(t).view(1, t, 1) * 10.0 \
        + torch.arange(h).view(1, 1, h)
    x4 = 1e-3 * tag.repeat_interleave(4, dim=-1)
    x8 = 1e-3 * tag.repeat_interleave(8, dim=-1)
    x2 = 1e-3 * tag.repeat_interleave(2, dim=-1)
    _, v, _, d, p, _ = O.mixer_inputs(x4, x4, x8, x4, x2, h)
    for bb in range(b):
        for hh in range(h):
            for tt in range(t):
                want = 1e-3 * (bb * 1000.0 + tt * 10.0 + hh)
                n = bb * h + hh
                assert math.isclose(float(v[n, tt, 3]), want / (1 + math.exp(-want)), rel_tol=1e-12)
                assert math.isclose(float(d[n, tt, 0]), 1 / (1 + math.exp(want)), rel_tol=1e-12)
                assert math.isclose(float(p[n, tt]), math.log1p(math.exp(want)) + 1e-4, rel_tol=1e-12)
    # The readout goes back the same way: read[b, t, h] is sequence b*H + h.
    qk = torch.randn(b, t, h * 4)
    read, _, _ = O.mixer_core(qk, qk, x8, x4, x2, h)
    k, vv, q, dd, pp, rr = O.mixer_inputs(qk, qk, x8, x4, x2, h)
    y, _, _ = O.run_diagonal(k[h + 2:h + 3], vv[h + 2:h + 3], q[h + 2:h + 3], dd[h + 2:h + 3], pp[h + 2:h + 3],
                             rr[h + 2:h + 3], torch.zeros(1, 4, 8), torch.eye(4).expand(1, 4, 4), 1e-6)
    torch.testing.assert_close(read[1, :, 2], y[0], rtol=0, atol=0)


def test_mixer_gradcheck():
    views, _ = O.make_mixer_inputs(1, 3, 2, seed=5)
    leaves = [x.double().requires_grad_(True) for x in views]
    m0 = (0.3 * torch.randn(2, 4, 8)).requires_grad_(True)
    c0 = (torch.eye(4) * 0.8).expand(2, 4, 4).clone().requires_grad_(True)

    def fn(*xs):
        read, mT, cT = O.mixer_core(*xs[:5], 2, xs[5], xs[6])
        return read, mT, cT

    assert torch.autograd.gradcheck(fn, (*leaves, m0, c0), eps=1e-6, atol=1e-6)


def test_product_mixer_chain_matches_oracle():
    """The package's unfused op chain (float32) equals the oracle's (float64) transforms."""
    from bayes_ssm.mixer import mixer_layer_inputs

    views, _ = O.make_mixer_inputs(2, 9, 3, seed=6)
    ours = mixer_layer_inputs(*views, 3)
    want = O.mixer_inputs(*views, 3)
    for a, w in zip(ours, want):
        assert a.dtype == torch.float32
        torch.testing.assert_close(a.double(), w, rtol=1e-6, atol=1e-7)


def test_mixer_mutation_is_detected():
    """A planted sign error in the decay (exp(+softplus)) fails the sigmoid identity."""
    x = torch.linspace(-4.0, 4.0, 8).reshape(1, 1, 8)
    bad = torch.exp(O._softplus(x))
    assert not torch.allclose(bad, torch.sigmoid(-x), rtol=1e-8, atol=0)


def _block_inputs(b, t, h, seed):
    g = torch.Generator().manual_seed(seed)
    state, width = 4 * h, 8 * h
    core, aux = 2 * state + width, state + 2 * h
    projected = torch.randn(b, t, core + aux + width, generator=g)
    projected[..., core:core + state] -= 4.0          # decay logits: slow decay, as the learned init
    projected[..., core + state:core + aux:2] -= 2.0  # process logits
    projected = projected.to(torch.bfloat16).double()
    weight = (0.5 * torch.randn(core, 1, 4, generator=g)).to(torch.bfloat16).double()
    norm_w = (1 + 0.2 * torch.randn(8, generator=g)).to(torch.bfloat16).double()
    aux_bias = (0.3 * torch.randn(aux, generator=g)).to(torch.bfloat16).double()
    return projected, weight, norm_w, aux_bias


def _reference_block_ops(projected, weight, norm_w, aux_bias, h, eps):
    """train_6layer.py:583-729 written with torch's own ops (the bf16 tensors' values kept at each boundary)."""
    F = torch.nn.functional
    b, t, _ = projected.shape
    state, width = 4 * h, 8 * h
    core, aux = 2 * state + width, state + 2 * h

    def bf16(x):
        return x.to(torch.bfloat16).double()

    x = projected[..., :core].transpose(1, 2)
    w = weight[:, 0]
    padded = F.pad(x, (3, 0))
    y = padded[..., :t] * w[:, 0].view(1, -1, 1)
    for j in range(1, 4):
        y = y + padded[..., j:t + j] * w[:, j].view(1, -1, 1)
    conv = bf16(y.transpose(1, 2))
    q_in, k_in, v_in = conv.split((state, state, width), dim=-1)
    auxv = bf16(projected[..., core:core + aux] + aux_bias)
    gate = projected[..., core + aux:]
    q = F.normalize(F.silu(q_in).view(b, t, h, 4), dim=-1).permute(0, 2, 1, 3).reshape(b * h, t, 4)
    k = F.normalize(F.silu(k_in).view(b, t, h, 4), dim=-1).permute(0, 2, 1, 3).reshape(b * h, t, 4)
    v = F.silu(v_in).view(b, t, h, 8).permute(0, 2, 1, 3).reshape(b * h, t, 8)
    noise = auxv[..., state:].view(b, t, h, 2)
    process = (F.softplus(noise[..., 0]) + 1e-4).permute(0, 2, 1).reshape(b * h, t)
    observation = (F.softplus(noise[..., 1]) + 1e-4).permute(0, 2, 1).reshape(b * h, t)
    decay = torch.exp(-F.softplus(auxv[..., :state])).view(b, t, h, 4).permute(0, 2, 1, 3).reshape(b * h, t, 4)
    read, _, _ = O.reference_layer(k, v, q, decay, process, observation, chunk=64, floor=1e-6)
    read = read.view(b, h, t, 8).permute(0, 2, 1, 3)
    normed = F.rms_norm(bf16(read), (8,), norm_w, eps)
    return (normed * F.silu(gate.view(b, t, h, 8))).reshape(b, t, width)


def test_mixer_block_matches_reference_op_sequence():
    """mixer_block equals the reference's mixer ops written with torch's own functions (filter as shifted
    products, F.normalize, softplus, the transported-history layer, rms_norm, silu) at float64."""
    h = 2
    projected, weight, norm_w, aux_bias = _block_inputs(2, 11, h, seed=21)
    eps = torch.finfo(torch.float32).eps
    ours, _, _ = O.mixer_block(projected, weight, norm_w, h, aux_bias=aux_bias, eps=eps)
    ref = _reference_block_ops(projected, weight, norm_w, aux_bias, h, eps)
    torch.testing.assert_close(ours, ref, rtol=1e-10, atol=1e-12)
    # A planted mistake (gate and v columns swapped) is detected.
    core = 16 * h
    swapped = projected.clone()
    swapped[..., 8 * h:core], swapped[..., -8 * h:] = projected[..., -8 * h:], projected[..., 8 * h:core]
    bad, _, _ = O.mixer_block(swapped, weight, norm_w, h, aux_bias=aux_bias, eps=eps)
    assert (bad - ref).abs().max() > 1e-2


def test_mixer_block_gradcheck():
    projected, weight, norm_w, aux_bias = _block_inputs(1, 4, 1, seed=22)
    leaves = [x.clone().requires_grad_(True) for x in (projected, weight, norm_w, aux_bias)]

    def fn(p, w, n, a):
        out, mT, cT = O.mixer_block(p, w, n, 1, aux_bias=a, round_bf16=False)
        return out, mT, cT

    assert torch.autograd.gradcheck(fn, leaves, eps=1e-6, atol=1e-6)


def test_mixer_readout_matches_torch_ops_and_invariants():
    """mixer_readout equals torch's bf16 rms_norm * silu chain (the reference's ops) to bf16 rounding;
    the normalized head has unit RMS; the float32-epsilon default matters for tiny heads."""
    g = torch.Generator().manual_seed(8)
    b, t, h = 2, 5, 3
    read = torch.randn(b, t, h, 8, generator=g)
    gate = torch.randn(b, t, h * 8, generator=g).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(8, generator=g)).to(torch.bfloat16)
    ours = O.mixer_readout(read, gate, w)
    rn = torch.nn.functional.rms_norm(read.to(torch.bfloat16), (8,), w, None)
    ref = (rn * torch.nn.functional.silu(gate.view(b, t, h, 8))).reshape(b, t, h * 8)
    # The torch chain rounds to bf16 three times (norm, silu, product), each within 2^-8 relative.
    torch.testing.assert_close(ours, ref.double(), rtol=3 * 2 ** -8, atol=0)
    unit = O.mixer_readout(read, torch.full((b, t, h * 8), 30.0), torch.ones(8), eps=0.0)  # silu(30) = 30
    rms = (unit / 30.0).reshape(b, t, h, 8).square().mean(-1).sqrt()
    torch.testing.assert_close(rms, torch.ones_like(rms), rtol=1e-12, atol=0)
    tiny = 1e-4 * read
    a = O.mixer_readout(tiny, gate, w)
    rn_t = torch.nn.functional.rms_norm(tiny.to(torch.bfloat16), (8,), w, None)
    ref_t = (rn_t * torch.nn.functional.silu(gate.view(b, t, h, 8))).reshape(b, t, h * 8)
    torch.testing.assert_close(a, ref_t.double(), rtol=3 * 2 ** -8, atol=1e-6)
    bad = O.mixer_readout(tiny, gate, w, eps=torch.finfo(torch.bfloat16).eps)
    assert not torch.allclose(bad, ref_t.double(), rtol=3 * 2 ** -8, atol=1e-6)


def test_mixer_readout_gradcheck():
    g = torch.Generator().manual_seed(9)
    read = torch.randn(1, 2, 2, 8, generator=g, dtype=torch.float64).requires_grad_(True)
    gate = torch.randn(1, 2, 16, generator=g, dtype=torch.float64).requires_grad_(True)
    w = (1 + 0.2 * torch.randn(8, generator=g, dtype=torch.float64)).requires_grad_(True)
    # The bf16 rounding of read is value-only; with the rounded values taken as read itself the
    # map is smooth and its autograd gradient is the one the rounding passes through.
    assert torch.autograd.gradcheck(lambda r, z, ww: O.mixer_readout(r, z, ww, read_bf16=r), (read, gate, w),
                                     eps=1e-6, atol=1e-6)


# ------------------------------------------------------ causal depthwise filter
def test_causal_depthwise4_matches_conv1d_and_impulse_response():
    g = torch.Generator().manual_seed(10)
    b, c, t = 2, 5, 9
    x = torch.randn(b, c, t, generator=g)
    w = torch.randn(c, 1, 4, generator=g)
    ref = torch.nn.functional.conv1d(torch.nn.functional.pad(x, (3, 0)), w, groups=c)
    torch.testing.assert_close(O.causal_depthwise4(x, w), ref, rtol=1e-12, atol=1e-12)
    # Impulse at tau: y[t] = w[c, 0, 3 - (t - tau)] for 0 <= t - tau <= 3, else 0.
    tau = 4
    imp = torch.zeros(1, c, t)
    imp[..., tau] = 1.0
    y = O.causal_depthwise4(imp, w)
    for tt in range(t):
        want = w[:, 0, 3 - (tt - tau)] if 0 <= tt - tau <= 3 else torch.zeros(c)
        torch.testing.assert_close(y[0, :, tt], want, rtol=0, atol=0)
    # Causality: changing the future leaves the past alone.
    x2 = x.clone()
    x2[..., 6:] += 1.0
    torch.testing.assert_close(O.causal_depthwise4(x2, w)[..., :6], O.causal_depthwise4(x, w)[..., :6], rtol=0, atol=0)
    # Short sequences (T < 4) keep only the taps that fit.
    torch.testing.assert_close(O.causal_depthwise4(x[..., :2], w), ref[..., :2], rtol=1e-12, atol=1e-12)


def test_causal_depthwise4_gradcheck():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 3, 6, generator=g, dtype=torch.float64).requires_grad_(True)
    w = torch.randn(3, 1, 4, generator=g, dtype=torch.float64).requires_grad_(True)
    assert torch.autograd.gradcheck(O.causal_depthwise4, (x, w), eps=1e-6, atol=1e-7)


def test_product_conv_formula_matches_oracle():
    """The package's torch fallback (the reference's shifted products) equals the oracle."""
    from bayes_ssm.conv import CausalDepthwise4

    g = torch.Generator().manual_seed(12)
    m = CausalDepthwise4(6, dtype=torch.float64)
    with torch.no_grad():
        m.weight.copy_(torch.randn(6, 1, 4, generator=g, dtype=torch.float64))
    x = torch.randn(3, 6, 10, generator=g, dtype=torch.float64)
    torch.testing.assert_close(m(x), O.causal_depthwise4(x, m.weight.detach()), rtol=1e-12, atol=1e-12)
    with pytest.raises(ValueError):
        CausalDepthwise4(6, 5)


# ------------------------------------------------------------ rotation core
def _rot_case(n, t, d, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(n, t, d, generator=g)
    v = torch.randn(n, t, 3, generator=g)
    q = torch.randn(n, t, d, generator=g)
    rad = 0.5 + 0.6 * torch.rand(n, t, d // 2, generator=g)  # some above 1: clamped
    ang = 3.0 * torch.randn(n, t, d // 2, generator=g)
    p = 0.05 + 0.2 * torch.rand(n, t, d // 2, generator=g)
    r = 0.2 + torch.rand(n, t, generator=g)
    m0 = 0.3 * torch.randn(n, d, 3, generator=g)
    a = torch.randn(n, d, d, generator=g)
    c0 = a @ a.transpose(-1, -2) / d + 0.5 * torch.eye(d)
    return k, v, q, rad, ang, p, r, m0, c0


def test_rotation_matches_dense_block_rotation():
    """The pairwise rotation core equals run_dense with block-diagonal R_t and Q_t = diag(p on even entries)."""
    k, v, q, rad, ang, p, r, m0, c0 = _rot_case(3, 7, 6, seed=20)
    n, t, d = k.shape
    rho = torch.clamp(rad, max=1.0)
    A = torch.zeros(n, t, d, d)
    Q = torch.zeros(n, t, d, d)
    for j in range(d // 2):
        cj, sj = rho[..., j] * torch.cos(ang[..., j]), rho[..., j] * torch.sin(ang[..., j])
        A[..., 2 * j, 2 * j], A[..., 2 * j, 2 * j + 1] = cj, -sj
        A[..., 2 * j + 1, 2 * j], A[..., 2 * j + 1, 2 * j + 1] = sj, cj
        Q[..., 2 * j, 2 * j] = p[..., j]
    yd, md, cd = O.run_dense(k, v, q, A, Q, r, m0, c0, 1e-6)
    yr, mr, cr = O.run_rotation(k, v, q, rad, ang, p, r, m0, c0, 1e-6)
    for a_, b_ in ((yr, yd), (mr, md), (cr, cd)):
        torch.testing.assert_close(a_, b_, rtol=1e-12, atol=1e-12)


def test_rotation_zero_angle_is_diagonal_with_even_noise():
    """Angle 0: the transition is diag(rho per pair); noise only on even entries (checked via run_dense)."""
    k, v, q, rad, _, p, r, m0, c0 = _rot_case(2, 5, 4, seed=21)
    rad = rad.clamp(max=0.99)
    ang = torch.zeros_like(rad)
    d_full = rad.repeat_interleave(2, dim=-1)
    yr, mr, cr = O.run_rotation(k, v, q, rad, ang, p, r, m0, c0, 1e-6)
    Q = torch.diag_embed(torch.stack((p, torch.zeros_like(p)), dim=-1).reshape(*p.shape[:-1], 4))
    yd, md, cd = O.run_dense(k, v, q, torch.diag_embed(d_full), Q, r, m0, c0, 1e-6)
    torch.testing.assert_close(yr, yd, rtol=1e-12, atol=1e-12)
    # With the same noise on every entry it would differ: the even-only placement matters.
    yw, _, _ = O.run_dense(k, v, q, torch.diag_embed(d_full), torch.diag_embed(p.repeat_interleave(2, dim=-1)), r,
                           m0, c0, 1e-6)
    assert (yw - yr).abs().max() > 1e-6


def test_rotation_gradcheck_and_clamp():
    k, v, q, rad, ang, p, r, m0, c0 = _rot_case(1, 3, 4, seed=22)
    rad = torch.tensor([[[0.7, 1.3], [0.9, 0.5], [1.2, 0.8]]], dtype=torch.float64)  # two clamped entries
    leaves = [x.clone().requires_grad_(True) for x in (k, v, q, rad, ang, p, r)]

    def fn(*xs):
        return O.run_rotation(*xs, m0, c0, 1e-6)

    assert torch.autograd.gradcheck(fn, tuple(leaves), eps=1e-6, atol=1e-6)
    y, mT, cT = fn(*leaves)
    g = torch.autograd.grad(y.sum() + mT.sum(), leaves[3])[0]
    assert g[0, 0, 1] == 0 and g[0, 2, 0] == 0  # radius > 1: clamped, no gradient
