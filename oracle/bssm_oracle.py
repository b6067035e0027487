"""CPU oracle for the bayes-ssm Bayesian recurrence — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker / the timed CPU
baseline.  The product path (``bayes_ssm``) never imports it.

Each function restates one reference routine in plain PyTorch (float64 or
float32, autograd-friendly), written from the equations:

* ``dense_step`` / ``run_dense``     — bayes_ssm/bayesian_layer.py:153-204 (_step, _core_loop)
* ``run_diagonal``                   — bayesian_layer.py:207-251 (_core_loop_diagonal_transition)
* ``run_fixed``                      — bayesian_layer.py:343-397 (_core_loop_fixed_diagonal)
* ``run_rotation``                   — bayesian_layer.py:254-323 (_core_loop_rotation, damped 2-D rotations)
* ``run_chunked``                    — bayesian_layer.py:670-732 (_run_chunked, paper §C.2
                                       transported-history chunk algorithm; the reference
                                       CPU path of ``bayesian_layer(optimized=False)``)
* ``reference_layer``                — bayesian_layer.py:1169-1182 (the optimized=False dispatch:
                                       diag_embed + _run_chunked)
* ``checkpoints``                    — boundary layout of persistent_bayes_chunked_d4m8.cu:208-211, :244
* ``associative_static``             — bayes_ssm/replay_ssm.py:155-270 (information-form scan)
* ``closed_form_static``             — Bayesian linear regression, the A=I, Q=0 closed form
* ``mixer_inputs`` / ``mixer_core``  — the Bayes mixer's producer chain and readout permute
                                       (example/train_6layer.py:627-693, :709-710)
* ``mixer_readout``                  — its gated readout: RMSNorm(bf16(read)) * silu(gate) (:719-729)
* ``mixer_block``                    — the mixer from its fused projection to out_proj's input
                                       (:583-729): filter, producer chain, layer, gated readout
* ``causal_depthwise4``              — the length-four causal depthwise filter (:160-191)
* ``floor_clamp``                    — the innovation floor: the CUDA reverse kernels' strict
                                       ``s > floor`` gate (persistent_bayes_chunked_d4m8.cu:315),
                                       used by run_diagonal / run_fixed / mixer_core, or
                                       torch's clamp_min (the eager and chunked CPU paths)

Pinning (tests/test_oracle.py): closed forms (scalar Kalman filter, one-step
u = (d^2+p)k, no-update limits, Bayesian linear regression), invariants
(symmetric PSD covariance, P_post <= P_pred, chunk-length invariance),
cross-formulation agreement (dense == diagonal == transported-history ==
information-form, as the reference's own tests assert at 1e-12/1e-10), and
fp64 gradcheck of the gradients that the reference obtains by autograd.
The mixer producer chain is pinned by identities the reference's formulas
must satisfy (exp(-softplus(x)) = sigmoid(-x), softplus(x) - softplus(-x) = x,
unit-norm heads, the [B, T, H] -> [B*H, T] sequence map checked with
head-tagged inputs) and by its reduction to ``run_diagonal``.  The readout
epilogue is pinned against torch's own rms_norm / silu on bf16 tensors (the
reference's ops), by unit RMS of the normalized head, and by gradcheck.  The
mixer block is pinned against the reference's op sequence written out with
torch's own ops (pad + shifted products, split, normalize, softplus, rms_norm,
silu) on the same fused projection, and by gradcheck of its float64 chain.  The
causal filter is pinned against torch's conv1d on the left-padded input (the
reference's nn.Conv1d path, :478-480), by its impulse response and causality,
and by gradcheck.
The strict floor gate is pinned at a token built to have r + k.u == floor
exactly: its dL/dr is the one-sided (left) finite difference, zero, while
clamp_min's is the right one.
The rotation core is pinned against run_dense with an independently built
block-rotation transition (the reference's own check,
tests/test_bayesian_layer_diagonal.py:12-51), by the angle = 0 reduction to
the diagonal core and by the radius clamp.
No function here is left "parity unpinned".
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

FIXED_DECAY = 0.97
FIXED_PROCESS = 0.1
FIXED_OBSERVATION = 1.0


def _sym(x: Tensor) -> Tensor:
    return 0.5 * (x + x.transpose(-1, -2))


class _StrictFloor(torch.autograd.Function):
    """max(s, floor) whose derivative is 1 only where s > floor (strictly).

    The reference's CUDA reverse kernels gate the innovation-variance
    adjoint with a strict comparison, ``(s > floor) ? -z beta^2 : 0``
    (persistent_bayes_chunked_d4m8.cu:315, _d2m8.cu:318, _d1m8.cu:339, _d8.cu:381,
    persistent_bayes_chunked.cu:324), while torch's ``clamp_min`` passes the
    gradient at s == floor as well.  The two differ only at equality.
    """

    @staticmethod
    def forward(ctx, s, floor):
        ctx.save_for_backward(s)
        ctx.floor = floor
        return s.clamp_min(floor)

    @staticmethod
    def backward(ctx, grad):
        (s,) = ctx.saved_tensors
        return grad * (s > ctx.floor).to(grad.dtype), None


def floor_clamp(s: Tensor, floor: float, strict: bool = True) -> Tensor:
    """The innovation floor: the fused kernels' strict gate, or torch's clamp_min (strict=False)."""
    return _StrictFloor.apply(s, floor) if strict else s.clamp_min(floor)


def dense_step(mean, cov, k, v, q, A, Q, r, floor):
    """One predict/condition/read step (bayesian_layer.py:153-181).

    mean [..., D, M], cov [..., D, D], k/q [..., D], v [..., M], A/Q [..., D, D], r [...].
    """
    cov_pred = A @ cov @ A.transpose(-1, -2) + Q
    mean_pred = A @ mean
    u = (cov_pred @ k.unsqueeze(-1)).squeeze(-1)
    s = (r + (k * u).sum(-1)).clamp_min(floor)
    beta = 1.0 / s
    e = v - (mean_pred.transpose(-1, -2) @ k.unsqueeze(-1)).squeeze(-1)
    bu = beta[..., None] * u
    mean_new = mean_pred + bu[..., :, None] * e[..., None, :]
    cov_new = _sym(cov_pred - bu[..., :, None] * u[..., None, :])
    y = (mean_new.transpose(-1, -2) @ q.unsqueeze(-1)).squeeze(-1)
    return mean_new, cov_new, y


def run_dense(k, v, q, A, Q, r, mean0, cov0, floor):
    """Token loop over dense dynamics (bayesian_layer.py:184-204).  A, Q: [..., T, D, D]."""
    mean, cov = mean0, cov0
    ys = []
    for t in range(k.shape[-2]):
        mean, cov, y = dense_step(mean, cov, k[..., t, :], v[..., t, :], q[..., t, :], A[..., t, :, :],
                                  Q[..., t, :, :], r[..., t], floor)
        ys.append(y)
    return torch.stack(ys, dim=-2), mean, cov


def run_diagonal(k, v, q, d, p, r, mean0, cov0, floor, strict=True, innovations=None):
    """Diagonal-transition token loop (bayesian_layer.py:207-251).

    The predicted covariance is d_i P_ij d_j + p delta_ij; the initial
    covariance is used as given (not symmetrised), so autograd yields the
    full asymmetric initial-covariance gradient the fused kernels return.
    ``strict`` selects the fused kernels' floor gate (the default; see
    ``_StrictFloor``); ``strict=False`` is the eager loop's clamp_min (:243).
    ``innovations``, a list, receives each token's unclamped r + k.u.
    """
    mean, cov = mean0, cov0
    eye = torch.eye(k.shape[-1], dtype=k.dtype, device=k.device)
    ys = []
    for t in range(k.shape[-2]):
        dt = d[..., t, :]
        mean_pred = dt[..., :, None] * mean
        cov_pred = dt[..., :, None] * cov * dt[..., None, :] + p[..., t, None, None] * eye
        kt = k[..., t, :]
        u = (cov_pred @ kt.unsqueeze(-1)).squeeze(-1)
        s_raw = r[..., t] + (kt * u).sum(-1)
        if innovations is not None:
            innovations.append(s_raw.detach())
        s = floor_clamp(s_raw, floor, strict)
        beta = 1.0 / s
        e = v[..., t, :] - (mean_pred * kt[..., :, None]).sum(-2)
        bu = beta[..., None] * u
        mean = mean_pred + bu[..., :, None] * e[..., None, :]
        cov = _sym(cov_pred - bu[..., :, None] * u[..., None, :])
        ys.append((mean * q[..., t, :, None]).sum(-2))
    return torch.stack(ys, dim=-2), mean, cov


def run_fixed(k, v, q, mean0, cov0, floor, strict=True):
    """Constant dynamics A = 0.97 I, Q = 0.1 I, R = 1 (bayesian_layer.py:343-397; floor gate as run_diagonal)."""
    mean, cov = mean0, cov0
    eye = torch.eye(k.shape[-1], dtype=k.dtype, device=k.device)
    rho, rho2 = FIXED_DECAY, FIXED_DECAY * FIXED_DECAY
    ys = []
    for t in range(k.shape[-2]):
        kt = k[..., t, :]
        mean_pred = rho * mean
        u = rho2 * (cov * kt[..., None, :]).sum(-1) + FIXED_PROCESS * kt
        s = floor_clamp(FIXED_OBSERVATION + (kt * u).sum(-1), floor, strict)
        beta = 1.0 / s
        e = v[..., t, :] - (mean_pred * kt[..., :, None]).sum(-2)
        bu = beta[..., None] * u
        mean = mean_pred + bu[..., :, None] * e[..., None, :]
        cov = _sym(rho2 * cov + FIXED_PROCESS * eye - bu[..., :, None] * u[..., None, :])
        ys.append((mean * q[..., t, :, None]).sum(-2))
    return torch.stack(ys, dim=-2), mean, cov


def rotation_coefficients(radius, angle, tiny: float = 1.1754943508222875e-38):
    """c, s of the damped rotations: rho = min(max(radius, tiny), 1) (bayesian_layer.py:279-281)."""
    rho = radius.clamp_min(tiny)
    rho = torch.where(rho <= 1.0, rho, torch.ones_like(rho))
    return rho * torch.cos(angle), rho * torch.sin(angle)


def run_rotation(k, v, q, radius, angle, p, r, mean0, cov0, floor, innovations=None):
    """Block-diagonal damped 2-D rotations (bayesian_layer.py:254-323), pair by pair.

    Pair j = rows (2j, 2j+1): mean and covariance rows, then covariance
    columns, are turned by [[c, -s], [s, c]]; the pair's process variance p[.., j]
    is added to entry (2j, 2j) only; then the Kalman update of run_dense with
    the covariance symmetrised.  radius, angle, p: [..., T, D/2]; tiny is the
    float32 one, as the reference's float32 covariance uses.  The reference
    runs this core in torch, so the floor is clamp_min's (gradient passes at
    s == floor), not the fused kernels' strict gate.
    """
    D = k.shape[-1]
    J = D // 2
    mean, cov = mean0, cov0

    def turn(x, c, s):  # rows of x [..., D, W] by the pair rotations
        pairs = x.reshape(*x.shape[:-2], J, 2, x.shape[-1])
        a, b = pairs[..., 0, :], pairs[..., 1, :]
        c, s = c[..., None], s[..., None]
        return torch.stack((c * a - s * b, s * a + c * b), dim=-2).reshape(x.shape)

    ys = []
    for t in range(k.shape[-2]):
        c, s = rotation_coefficients(radius[..., t, :], angle[..., t, :])
        mean_pred = turn(mean, c, s)
        cov_pred = turn(turn(cov, c, s).transpose(-1, -2), c, s).transpose(-1, -2)
        noise = torch.stack((p[..., t, :], torch.zeros_like(p[..., t, :])), dim=-1).reshape(*p.shape[:-2], D)
        cov_pred = cov_pred + torch.diag_embed(noise)
        kt = k[..., t, :]
        u = (cov_pred @ kt.unsqueeze(-1)).squeeze(-1)
        s_raw = r[..., t] + (kt * u).sum(-1)
        if innovations is not None:
            innovations.append(s_raw.detach())
        beta = 1.0 / floor_clamp(s_raw, floor, strict=False)
        e = v[..., t, :] - (mean_pred * kt[..., :, None]).sum(-2)
        mean = mean_pred + beta[..., None, None] * u[..., :, None] * e[..., None, :]
        cov = _sym(cov_pred - beta[..., None, None] * u[..., :, None] * u[..., None, :])
        ys.append((mean * q[..., t, :, None]).sum(-2))
    return torch.stack(ys, dim=-2), mean, cov


def run_chunked(k, v, q, A, Q, r, mean0, cov0, chunk, floor):
    """Transported-history chunk algorithm (bayesian_layer.py:670-732).

    Inside a chunk the covariance is kept as Pi_t (the prediction with the
    chunk's own observations removed) plus the transported rank-one update
    directions w_s; the dense posterior is only formed at chunk exit.
    """
    T = k.shape[-2]
    mean, cov = mean0, cov0
    ys = []
    for start in range(0, T, chunk):
        stop = min(T, start + chunk)
        pi = cov
        m = mean
        dirs: list[Tensor] = []
        betas: list[Tensor] = []
        for t in range(start, stop):
            At = A[..., t, :, :]
            pi = _sym(At @ pi @ At.transpose(-1, -2) + Q[..., t, :, :])
            m = At @ m
            dirs = [(At @ w.unsqueeze(-1)).squeeze(-1) for w in dirs]
            kt = k[..., t, :]
            u = (pi @ kt.unsqueeze(-1)).squeeze(-1)
            for w, b in zip(dirs, betas):
                u = u - b[..., None] * w * (w * kt).sum(-1)[..., None]
            s = (r[..., t] + (kt * u).sum(-1)).clamp_min(floor)
            beta = 1.0 / s
            e = v[..., t, :] - (m.transpose(-1, -2) @ kt.unsqueeze(-1)).squeeze(-1)
            m = m + beta[..., None, None] * u[..., :, None] * e[..., None, :]
            ys.append((m.transpose(-1, -2) @ q[..., t, :].unsqueeze(-1)).squeeze(-1))
            dirs.append(u)
            betas.append(beta)
        cov = pi
        for w, b in zip(dirs, betas):
            cov = cov - b[..., None, None] * w[..., :, None] * w[..., None, :]
        cov = _sym(cov)
        mean = m
    return torch.stack(ys, dim=-2), mean, cov


def diagonal_as_dense(d, p):
    """diag_embed(d) and p I as dense [..., T, D, D] dynamics (bayesian_layer.py:1175-1179)."""
    eye = torch.eye(d.shape[-1], dtype=d.dtype, device=d.device)
    return torch.diag_embed(d), p[..., None, None] * eye


def reference_layer(k, v, q, d, p, r, mean0=None, cov0=None, chunk=64, floor=1e-6):
    """The reference CPU path ``bayesian_layer(..., transition_diagonals=d, optimized=False)``."""
    D, M = k.shape[-1], v.shape[-1]
    batch = k.shape[:-2]
    if mean0 is None:
        mean0 = torch.zeros(*batch, D, M, dtype=k.dtype)
    if cov0 is None:
        cov0 = torch.eye(D, dtype=k.dtype).expand(*batch, D, D).clone()
    A, Q = diagonal_as_dense(d, p)
    return run_chunked(k, v, q, A, Q, r, mean0, cov0, chunk, floor)


def checkpoints(k, v, q, d, p, r, mean0, cov0, chunk, floor):
    """Boundary beliefs: index c holds the belief before token c*chunk, index nb the final one."""
    T = k.shape[-2]
    nb = -(-T // chunk)
    means, covs = [mean0], [cov0]
    mean, cov = mean0, cov0
    for c in range(1, nb + 1):
        stop = min(T, c * chunk)
        start = (c - 1) * chunk
        _, mean, cov = run_diagonal(k[..., start:stop, :], v[..., start:stop, :], q[..., start:stop, :],
                                    d[..., start:stop, :], p[..., start:stop], r[..., start:stop], mean, cov, floor)
        means.append(mean)
        covs.append(cov)
    return torch.stack(means, dim=-3), torch.stack(covs, dim=-3)


def associative_static(k, v, q, r, mean0: Optional[Tensor] = None, cov0: Optional[Tensor] = None):
    """Information-form static scan (replay_ssm.py:251-270): prefix precision/natural, Cholesky solve."""
    D, M = k.shape[-1], v.shape[-1]
    batch = k.shape[:-2]
    if cov0 is None:
        cov0 = torch.eye(D, dtype=k.dtype).expand(*batch, D, D)
    if mean0 is None:
        mean0 = torch.zeros(*batch, D, M, dtype=k.dtype)
    lam0 = torch.linalg.inv(cov0)
    nat0 = lam0 @ mean0
    wk = k / r[..., :, None]
    lam = lam0.unsqueeze(-3) + (k[..., :, :, None] * wk[..., :, None, :]).cumsum(-3)
    nat = nat0.unsqueeze(-3) + (wk[..., :, :, None] * v[..., :, None, :]).cumsum(-3)
    lam = _sym(lam)
    chol = torch.linalg.cholesky(lam)
    mean = torch.cholesky_solve(nat, chol)
    y = (mean.transpose(-1, -2) @ q.unsqueeze(-1)).squeeze(-1)
    cov_last = torch.cholesky_inverse(chol[..., -1, :, :])
    return y, mean[..., -1, :, :], cov_last


def closed_form_static(k, v, r, mean0, cov0):
    """A = I, Q = 0 posterior after all tokens: M = (P0^-1 + sum k k^T/r)^-1 (P0^-1 M0 + sum k v^T/r)."""
    lam0 = torch.linalg.inv(cov0)
    lam = lam0 + torch.einsum("...ti,...tj->...ij", k / r[..., :, None], k)
    nat = lam0 @ mean0 + torch.einsum("...ti,...tc->...ic", k / r[..., :, None], v)
    mean = torch.linalg.solve(lam, nat)
    return mean, torch.linalg.inv(lam)


# ----------------------------------------------------------- Bayes mixer
MIXER_NOISE_FLOOR = 1e-4


def _softplus(x: Tensor) -> Tensor:
    """torch.nn.functional.softplus with beta 1 and threshold 20: x above 20, else log(1 + e^x)."""
    return torch.where(x > 20, x, torch.log1p(torch.exp(x.clamp(max=20))))


def _silu(x: Tensor) -> Tensor:
    return x * torch.sigmoid(x)


def mixer_inputs(q_proj, k_proj, v_proj, decay_logits, noise, heads: int, dtype=torch.float64):
    """Layer inputs of the Bayes mixer from its projections (train_6layer.py:627-693).

    q_proj, k_proj, decay_logits [B, T, H*4], v_proj [B, T, H*8], noise
    [B, T, H*2] ((process, observation) logits per head), any float dtype
    (computed in ``dtype``).  Per head: q, k = silu(x) / max(|silu(x)|, 1e-12),
    v = silu(x), d = exp(-softplus(x)), p, r = softplus(x) + 1e-4.  Sequence
    b*H + h of the layer is head h of batch row b.  Returns (k, v, q, d, p, r)
    in the layer's [B*H, T, .] layout.
    """
    b, t, _ = q_proj.shape

    def split(x: Tensor, w: int) -> Tensor:
        return x.to(dtype).reshape(b, t, heads, w)

    def unit(x: Tensor) -> Tensor:
        a = _silu(x)
        return a / a.square().sum(-1, keepdim=True).sqrt().clamp_min(1e-12)

    def seq(x: Tensor) -> Tensor:  # [B, T, H, ...] -> [B*H, T, ...]
        return x.transpose(1, 2).reshape(b * heads, t, *x.shape[3:])

    q = unit(split(q_proj, 4))
    k = unit(split(k_proj, 4))
    v = _silu(split(v_proj, 8))
    d = torch.exp(-_softplus(split(decay_logits, 4)))
    nz = split(noise, 2)
    p = _softplus(nz[..., 0]) + MIXER_NOISE_FLOOR
    r = _softplus(nz[..., 1]) + MIXER_NOISE_FLOOR
    return seq(k), seq(v), seq(q), seq(d), seq(p), seq(r)


def mixer_core(q_proj, k_proj, v_proj, decay_logits, noise, heads: int, mean0=None, cov0=None, floor=1e-6,
               dtype=torch.float64, innovations=None):
    """Readout [B, T, H, 8] of the mixer's layer (train_6layer.py:709-710) and the final belief [B*H, ...].

    The layer runs on the fused kernels in the reference (strict floor gate);
    ``innovations`` as in ``run_diagonal``.
    """
    b, t, _ = q_proj.shape
    k, v, q, d, p, r = mixer_inputs(q_proj, k_proj, v_proj, decay_logits, noise, heads, dtype)
    n = b * heads
    if mean0 is None:
        mean0 = torch.zeros(n, 4, 8, dtype=dtype)
    if cov0 is None:
        cov0 = torch.eye(4, dtype=dtype).expand(n, 4, 4)
    y, mT, cT = run_diagonal(k, v, q, d, p, r, mean0.to(dtype), cov0.to(dtype), floor, innovations=innovations)
    return y.reshape(b, heads, t, 8).transpose(1, 2), mT, cT


def mixer_grads(q_proj, k_proj, v_proj, decay_logits, noise, heads: int, mean0, cov0, g_read, gmf=None, gcf=None,
                floor=1e-6, dtype=torch.float64):
    """Readout, final belief and the gradients of the five projections and the initial belief.

    Autograd through ``mixer_core`` with loss <read, g_read> + <mT, gmf> + <cT, gcf>.
    Returns (read, mT, cT, [g_q, g_k, g_v, g_decay_logits, g_noise, g_mean0, g_cov0]).
    """
    leaves = [x.detach().to(dtype).clone().requires_grad_(True)
              for x in (q_proj, k_proj, v_proj, decay_logits, noise, mean0, cov0)]
    read, mT, cT = mixer_core(*leaves[:5], heads, leaves[5], leaves[6], floor, dtype)
    loss = (read * g_read.to(dtype)).sum()
    if gmf is not None:
        loss = loss + (mT * gmf.to(dtype)).sum()
    if gcf is not None:
        loss = loss + (cT * gcf.to(dtype)).sum()
    grads = torch.autograd.grad(loss, leaves)
    return read.detach(), mT.detach(), cT.detach(), list(grads)


def mixer_readout(read, gate, weight, eps: float = 1.1920928955078125e-07, read_bf16=None):
    """The mixer's gated readout (train_6layer.py:719-729) per head of 8 values, in float64.

    out = rms(r) * w * silu(gate) with r = read.to(bf16) and rms(x) =
    x / sqrt(mean(x^2) + eps) (torch's rms_norm; eps None is the float32
    epsilon).  The bf16 rounding of read is value-only: the gradient passes
    through it to read, as autograd's through ``.to()``.  ``read_bf16``
    (the rounded values, e.g. a kernel's) replaces the rounding done here.
    read, gate: [B, T, H, 8] (or [B, T, H*8] for gate); returns [B, T, H*8].
    """
    b, t, h = read.shape[:3]
    r64 = read.to(torch.float64)
    rb = (read.to(torch.bfloat16) if read_bf16 is None else read_bf16.reshape(b, t, h, 8)).to(torch.float64)
    y = r64 + (rb - r64).detach()
    n = y / (y.square().mean(-1, keepdim=True) + eps).sqrt()
    g = gate.reshape(b, t, h, 8).to(torch.float64)
    return (n * weight.to(torch.float64) * _silu(g)).reshape(b, t, h * 8)


def causal_depthwise4(x, weight):
    """CausalDepthwise4 (train_6layer.py:160-191): x [B, C, T], weight [C, 1, 4].

    y[c, t] = sum_j weight[c, 0, j] x[c, t - 3 + j], with x = 0 before t = 0,
    written as an explicit sum over the taps.
    """
    b, c, t = x.shape
    w = weight.reshape(c, 4).to(x.dtype)
    y = torch.zeros_like(x)
    for j in range(4):
        shift = 3 - j
        if shift == 0:
            y = y + w[:, j].view(1, c, 1) * x
        elif shift < t:
            y = y + torch.cat([torch.zeros(b, c, shift, dtype=x.dtype), w[:, j].view(1, c, 1) * x[..., : t - shift]],
                              dim=-1)
    return y


def _round_bf16(x: Tensor) -> Tensor:
    """x rounded to bfloat16 in value only (the gradient passes, as autograd's through ``.to()``)."""
    return x + (x.to(torch.bfloat16).to(x.dtype) - x).detach()


def mixer_block(projected, conv_weight, norm_weight, heads: int, aux_bias=None, conv_out=None, floor=1e-6,
                eps: float = 1.1920928955078125e-07, round_bf16: bool = True):
    """The Bayes mixer from its fused projection to out_proj's input (train_6layer.py:583-729), float64.

    projected [B, T, H*4 + H*4 + H*8 | H*4 + H*2 | H*8]: the Q/K/V core, the
    aux columns (decay logits, interleaved noise; plus ``aux_bias``, :589-593,
    rounded to bf16 as the reference's bf16 add) and the gate.  The core goes
    through ``causal_depthwise4`` (weight [C, 1, 4]) and is rounded to bf16,
    the reference's tensor dtype there (``conv_out``, a kernel's bf16 filter
    output, replaces the values of that rounding); then ``mixer_core`` and
    ``mixer_readout``.  Returns (out [B, T, H*8], mean_T, cov_T), out unrounded.
    ``round_bf16=False`` drops the bf16 roundings (a smooth chain, for gradcheck).
    """
    rnd = _round_bf16 if round_bf16 else (lambda v: v)
    state, width = heads * 4, heads * 8
    core, aux = 2 * state + width, state + 2 * heads
    x = projected.to(torch.float64)
    filtered = causal_depthwise4(x[..., :core].transpose(1, 2), conv_weight.to(torch.float64)).transpose(1, 2)
    if conv_out is None:
        filtered = rnd(filtered)
    else:
        filtered = filtered + (conv_out.to(torch.float64) - filtered).detach()
    q_in, k_in, v_in = filtered.split((state, state, width), dim=-1)
    aux_in = x[..., core:core + aux]
    if aux_bias is not None:
        aux_in = rnd(aux_in + aux_bias.to(torch.float64))
    read, mean_t, cov_t = mixer_core(q_in, k_in, v_in, aux_in[..., :state], aux_in[..., state:], heads, floor=floor)
    read_b = None if round_bf16 else read
    return mixer_readout(read, x[..., core + aux:], norm_weight, eps, read_bf16=read_b), mean_t, cov_t


def make_mixer_inputs(b: int, t: int, heads: int, *, seed: int = 0, ld_pad: int = 0, scale: float = 1.0):
    """Seeded bf16 projections of the mixer (CPU tensors), drawn as one fused projection.

    Draw order: one [B, T, H*22 + ld_pad] N(0,1) block whose columns are
    q (H*4), k (H*4), v (H*8), decay logits (H*4, shifted by +2) and noise
    (H*2, process logits shifted by -3); the five are returned as column
    views (row stride H*22 + ld_pad), then the readout gradient [B, T, H, 8].
    ``scale`` multiplies the N(0,1) draw (before the shifts): large values
    reach the saturated ends of silu, sigmoid and softplus.
    """
    gen = torch.Generator().manual_seed(seed)
    width = heads * 22 + ld_pad
    fused = scale * torch.randn(b, t, width, generator=gen)
    fused[..., heads * 16:heads * 20] += 2.0
    fused[..., heads * 20:heads * 22:2] -= 3.0
    fused = fused.to(torch.bfloat16)
    cuts = [0, heads * 4, heads * 8, heads * 16, heads * 20, heads * 22]
    views = [fused[..., cuts[i]:cuts[i + 1]] for i in range(5)]
    g_read = torch.randn(b, t, heads, 8, generator=gen)
    return views, g_read


# --------------------------------------------------------------- inputs
def make_inputs(n: int, t: int, d: int, m: int = 8, *, seed: int = 0, dtype=torch.float32,
                bf16_round: bool = True, requires_grad: bool = False):
    """Seeded synthetic inputs of the measurement configs (CPU tensors).

    Draw order k, v, q, decay-logit, process-logit, observation-logit, gy:
    k, v, q ~ N(0,1) (rounded through bf16), decay = sigmoid(N(2,1)),
    p = softplus(N(-3,1)), r = 1e-4 + softplus(N(0,1)), gy ~ N(0,1).
    """
    gen = torch.Generator().manual_seed(seed)
    k = torch.randn(n, t, d, generator=gen)
    v = torch.randn(n, t, m, generator=gen)
    q = torch.randn(n, t, d, generator=gen)
    if bf16_round:
        k, v, q = (x.to(torch.bfloat16).float() for x in (k, v, q))
    dec = torch.sigmoid(torch.randn(n, t, d, generator=gen) + 2.0)
    p = torch.nn.functional.softplus(torch.randn(n, t, generator=gen) - 3.0)
    r = 1e-4 + torch.nn.functional.softplus(torch.randn(n, t, generator=gen))
    gy = torch.randn(n, t, m, generator=gen)
    out = [x.to(dtype) for x in (k, v, q, dec, p, r, gy)]
    if requires_grad:
        for x in out[:6]:
            x.requires_grad_(True)
    return out


def make_scan_inputs(b: int, t: int, d: int, m: int, *, seed: int = 0, dtype=torch.float32):
    """Associative-scan configs: k ~ N(0, 1/D), v, q ~ N(0,1), r = 1e-4 + softplus(N(0,1))."""
    gen = torch.Generator().manual_seed(seed)
    k = torch.randn(b, t, d, generator=gen) / (d ** 0.5)
    v = torch.randn(b, t, m, generator=gen)
    q = torch.randn(b, t, d, generator=gen)
    r = 1e-4 + torch.nn.functional.softplus(torch.randn(b, t, generator=gen))
    return [x.to(dtype) for x in (k, v, q, r)]


def diagonal_grads(k, v, q, d, p, r, mean0, cov0, gy, gmf=None, gcf=None, floor=1e-6, chunk=None, strict=True):
    """Outputs and all eight gradients by autograd through the oracle.

    ``chunk=None`` differentiates ``run_diagonal`` (floor gate per ``strict``);
    an integer differentiates the transported-history ``run_chunked`` (the
    reference CPU path, torch's clamp_min).
    Returns (y, mean_T, cov_T, [gk, gv, gq, gd, gp, gr, gm0, gc0]).
    """
    leaves = [x.detach().clone().requires_grad_(True) for x in (k, v, q, d, p, r, mean0, cov0)]
    k_, v_, q_, d_, p_, r_, m0_, c0_ = leaves
    if chunk is None:
        y, mT, cT = run_diagonal(k_, v_, q_, d_, p_, r_, m0_, c0_, floor, strict)
    else:
        A, Q = diagonal_as_dense(d_, p_)
        y, mT, cT = run_chunked(k_, v_, q_, A, Q, r_, m0_, c0_, chunk, floor)
    loss = (y * gy).sum()
    if gmf is not None:
        loss = loss + (mT * gmf).sum()
    if gcf is not None:
        loss = loss + (cT * gcf).sum()
    grads = torch.autograd.grad(loss, leaves, allow_unused=True)
    grads = [torch.zeros_like(x) if g is None else g for g, x in zip(grads, leaves)]
    return y.detach(), mT.detach(), cT.detach(), grads
