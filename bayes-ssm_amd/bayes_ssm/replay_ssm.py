"""ReplaySSM and the exact static associative scan — MI355X build of the reference API.

Follows bayes_ssm/replay_ssm.py of the reference: ``ReplaySSM`` (:34-145),
``associative_static_bayesian`` (:155-270, information-form prefix scan) and
``associative_static_bayesian_cuda`` (:276-339).  The CUDA variant of the
reference runs the same torch-op chain (cumsum + batched Cholesky) on the
device; here it runs one gfx950 kernel (``bssm_associative_static_scan``) that
sums each token's prefix and does the small Cholesky solves in LDS.
"""
from __future__ import annotations

import math
from numbers import Real
from typing import Optional

import torch
from torch import Tensor, nn

from .bayesian_layer import _broadcastable, _DeferredChecks, _validate_covariance, bayesian_layer


class ReplaySSM(nn.Module):
    """Exact dense Bayesian recurrence with chunk replay in the backward pass.

    ``key_dim``/``value_dim`` give the matrix state; inputs are
    ``[..., T, key_dim]`` keys/queries and ``[..., T, value_dim]`` values.  State
    resets at every call.
    """

    def __init__(self, key_dim: int, value_dim: int, *, process_variance: float = 0.05,
                 observation_variance: float = 0.2, initial_covariance: float = 1.0, chunk_length: int = 64,
                 denominator_floor: float = 1e-6) -> None:
        super().__init__()
        if not isinstance(key_dim, int) or isinstance(key_dim, bool) or key_dim <= 0:
            raise ValueError("key_dim must be a positive integer")
        if not isinstance(value_dim, int) or isinstance(value_dim, bool) or value_dim <= 0:
            raise ValueError("value_dim must be a positive integer")
        if not isinstance(chunk_length, int) or isinstance(chunk_length, bool) or chunk_length <= 0:
            raise ValueError("chunk_length must be a positive integer")
        for name, value in (("process_variance", process_variance), ("observation_variance", observation_variance),
                            ("initial_covariance", initial_covariance), ("denominator_floor", denominator_floor)):
            if not isinstance(value, Real) or not math.isfinite(float(value)):
                raise ValueError(f"{name} must be finite")
        if process_variance < 0 or observation_variance <= 0 or initial_covariance <= 0:
            raise ValueError("process variance must be nonnegative; observation and initial covariance positive")
        if denominator_floor <= 0:
            raise ValueError("denominator_floor must be positive")
        self.key_dim = key_dim
        self.value_dim = value_dim
        self.chunk_length = chunk_length
        self.denominator_floor = float(denominator_floor)
        self.register_buffer("process_variance", torch.tensor(float(process_variance)), persistent=False)
        self.register_buffer("observation_variance", torch.tensor(float(observation_variance)), persistent=False)
        self.register_buffer("initial_covariance", torch.eye(key_dim) * float(initial_covariance), persistent=False)

    def forward(self, keys: Tensor, values: Tensor, queries: Tensor, *, transitions: Optional[Tensor] = None,
                transition_diagonals: Optional[Tensor] = None,
                process_variances: Optional[Tensor | Real] = None,
                observation_variances: Optional[Tensor | Real] = None) -> tuple[Tensor, Tensor, Tensor]:
        if keys.shape[-1] != self.key_dim or queries.shape[-1] != self.key_dim:
            raise ValueError("keys and queries must end in key_dim")
        if values.shape[-1] != self.value_dim:
            raise ValueError("values must end in value_dim")
        return bayesian_layer(
            keys, values, queries, transitions=transitions, transition_diagonals=transition_diagonals,
            process_variances=self.process_variance if process_variances is None else process_variances,
            observation_variances=self.observation_variance if observation_variances is None
            else observation_variances,
            initial_covariance=self.initial_covariance.to(device=keys.device),
            denominator_floor=self.denominator_floor, chunk_length=self.chunk_length,
            optimized=True, replay_ssm=True,
        )

    def associative_scan(self, keys: Tensor, values: Tensor, queries: Tensor, *,
                         observation_variances: Optional[Tensor | Real] = None) -> tuple[Tensor, Tensor, Tensor]:
        """Exact static (A = I, Q = 0) scan; requires ``process_variance == 0``."""
        if bool(self.process_variance.detach().item() != 0.0):
            raise ValueError("associative_scan requires process_variance=0")
        if observation_variances is None:
            observation_variances = self.observation_variance
        scan = associative_static_bayesian_cuda if keys.is_cuda else associative_static_bayesian
        return scan(keys, values, queries, observation_variances=observation_variances,
                    initial_covariance=self.initial_covariance.to(device=keys.device),
                    denominator_floor=self.denominator_floor)


__all__ = ["ReplaySSM", "associative_static_bayesian", "associative_static_bayesian_cuda"]


def _scan_prepare(keys, values, queries, observation_variances, initial_mean, initial_covariance,
                  denominator_floor, checks: Optional[_DeferredChecks] = None):
    """Validation and promotion shared by both scans (replay_ssm.py:183-250).

    With ``checks`` given, the value checks still pending at the end are left
    in it for the caller to read back (after queueing its kernel).
    """
    if keys.ndim < 2 or values.ndim < 2 or queries.ndim < 2:
        raise ValueError("keys, values and queries must have time and feature dimensions")
    if not all(x.is_floating_point() for x in (keys, values, queries)):
        raise TypeError("keys, values and queries must have floating-point dtype")
    if not (keys.device == values.device == queries.device):
        raise ValueError("keys, values and queries must be on the same device")
    if keys.shape[:-1] != queries.shape[:-1] or keys.shape[:-2] != values.shape[:-2]:
        raise ValueError("keys/queries batch-time dimensions must match values")
    t, d = keys.shape[-2:]
    if values.shape[-2] != t:
        raise ValueError("values and keys must have the same sequence length")
    m = values.shape[-1]
    try:
        dtype = torch.promote_types(torch.promote_types(keys.dtype, values.dtype),
                                    torch.promote_types(queries.dtype, torch.float32))
    except (RuntimeError, TypeError):
        dtype = torch.float32
    keys, values, queries = keys.to(dtype), values.to(dtype), queries.to(dtype)
    batch = keys.shape[:-2]
    device = keys.device
    cov0 = (torch.eye(d, device=device, dtype=dtype).expand(*batch, d, d) if initial_covariance is None
            else initial_covariance.to(device=device, dtype=dtype))
    if cov0.shape[-2:] != (d, d):
        raise ValueError("initial_covariance must end in [key_dim, key_dim]")
    if not _broadcastable(cov0.shape[:-2], batch):
        raise ValueError("initial_covariance batch dimensions are not broadcastable to keys")
    cov0 = cov0.expand(*batch, d, d)
    # The default identity prior is finite, symmetric and positive definite:
    # only a caller's covariance needs the checks (and their synchronizations).
    if initial_covariance is not None:
        _validate_covariance(cov0, "initial_covariance", d)
    # The remaining value checks are read back together, in the reference's order.
    defer = checks is not None
    checks = checks if defer else _DeferredChecks()
    try:
        mean0 = (torch.zeros(*batch, d, m, device=device, dtype=dtype) if initial_mean is None
                 else initial_mean.to(device=device, dtype=dtype))
        if mean0.shape[-2:] != (d, m):
            raise ValueError("initial_mean must end in [key_dim, value_dim]")
        if not _broadcastable(mean0.shape[:-2], batch):
            raise ValueError("initial_mean batch dimensions are not broadcastable to keys")
        mean0 = mean0.expand(*batch, d, m)
        if initial_mean is not None:
            checks.finite(mean0, "initial_mean")
        if not isinstance(denominator_floor, Real) or not math.isfinite(float(denominator_floor)) \
                or denominator_floor <= 0:
            raise ValueError("denominator_floor must be finite and positive")
        r2 = torch.broadcast_to(torch.as_tensor(observation_variances, device=device, dtype=dtype), (*batch, t))
        # The information form divides by r itself, so r must not need the
        # innovation floor (replay_ssm.py:239-248).
        checks.at_least(r2, float(denominator_floor), "associative_static_bayesian requires finite "
                        "observation_variances greater than or equal to denominator_floor")
    except (ValueError, TypeError):
        checks.flush()
        raise
    if not defer:
        checks.flush()
    return keys, values, queries, r2, mean0, cov0


def associative_static_bayesian(keys: Tensor, values: Tensor, queries: Tensor, *,
                                observation_variances: Tensor | Real = 1.0, initial_mean: Optional[Tensor] = None,
                                initial_covariance: Optional[Tensor] = None,
                                denominator_floor: float = 1e-6) -> tuple[Tensor, Tensor, Tensor]:
    """Exact prefix scan for A = I, Q = 0 in information form (torch ops, any device, differentiable).

    Precision prefix L_t = inv(P0) + sum k k^T / r, natural prefix
    N_t = inv(P0) M0 + sum k v^T / r; posterior mean M_t = L_t^{-1} N_t by
    Cholesky; returns (readouts, M_T, P_T).
    """
    keys, values, queries, r2, mean0, cov0 = _scan_prepare(keys, values, queries, observation_variances,
                                                           initial_mean, initial_covariance, denominator_floor)
    t = keys.shape[-2]
    if t == 0:
        return keys.new_empty(*keys.shape[:-2], 0, values.shape[-1]), mean0, cov0
    lam0 = torch.linalg.inv(cov0)
    nat0 = lam0 @ mean0
    wk = keys / r2.unsqueeze(-1)
    lam = lam0.unsqueeze(-3) + (keys.unsqueeze(-1) * wk.unsqueeze(-2)).cumsum(dim=-3)
    nat = nat0.unsqueeze(-3) + (wk.unsqueeze(-1) * values.unsqueeze(-2)).cumsum(dim=-3)
    lam = 0.5 * (lam + lam.transpose(-1, -2))
    chol = torch.linalg.cholesky(lam)
    mean = torch.cholesky_solve(nat, chol)
    reads = (mean.transpose(-1, -2) @ queries.unsqueeze(-1)).squeeze(-1)
    return reads, mean[..., -1, :, :], torch.cholesky_inverse(chol[..., -1, :, :])


class _StaticScanFunction(torch.autograd.Function):
    """HIP forward and, for key dims up to 16, HIP backward; larger key dims
    differentiate the torch-op scan (same math)."""

    @staticmethod
    def forward(ctx, keys, values, queries, r2, mean0, cov0):
        from . import _hip

        b, t, d = keys.shape
        m = values.shape[-1]
        out = torch.empty(b, t, m, device=keys.device, dtype=torch.float32)
        mT = torch.empty(b, d, m, device=keys.device, dtype=torch.float32)
        cT = torch.empty(b, d, d, device=keys.device, dtype=torch.float32)
        P = _hip.ptr
        with _hip.on_device(keys.device):
            _hip.call("bssm_associative_static_scan", P(keys), P(values), P(queries), P(r2), P(mean0), P(cov0),
                      P(out), P(mT), P(cT), b, t, d, m, _hip.stream_of(keys.device))
        ctx.save_for_backward(keys, values, queries, r2, mean0, cov0)
        return out, mT, cT

    @staticmethod
    def backward(ctx, g_out, g_mean, g_cov):
        keys, values, queries, r2, mean0, cov0 = ctx.saved_tensors
        b, t, d = keys.shape
        m = values.shape[-1]
        if d <= 16 and b <= 65535:
            return _StaticScanFunction._hip_backward(ctx, keys, values, queries, r2, mean0, cov0, g_out, g_mean,
                                                     g_cov)
        saved = [x.detach().requires_grad_(need) for x, need in zip(ctx.saved_tensors, ctx.needs_input_grad)]
        with torch.enable_grad():
            outs = associative_static_bayesian(saved[0], saved[1], saved[2], observation_variances=saved[3],
                                               initial_mean=saved[4], initial_covariance=saved[5],
                                               denominator_floor=torch.finfo(torch.float32).tiny)
            wanted = [x for x in saved if x.requires_grad]
            grads = torch.autograd.grad(
                outs, wanted, grad_outputs=tuple(torch.zeros_like(o) if g is None else g
                                                 for o, g in zip(outs, (g_out, g_mean, g_cov))),
                allow_unused=True)
        it = iter(grads)
        return tuple(next(it) if x.requires_grad else None for x in saved)

    @staticmethod
    def _hip_backward(ctx, keys, values, queries, r2, mean0, cov0, g_out, g_mean, g_cov):
        from . import _hip

        b, t, d = keys.shape
        m = values.shape[-1]
        dev = keys.device
        f32 = lambda x: None if x is None else x.to(torch.float32).contiguous()  # noqa: E731
        g_mean, g_cov = f32(g_mean), f32(g_cov)
        if t == 0:
            grads = (keys.new_zeros(keys.shape), values.new_zeros(values.shape), queries.new_zeros(queries.shape),
                     r2.new_zeros(r2.shape), torch.zeros_like(mean0) if g_mean is None else g_mean,
                     torch.zeros_like(cov0) if g_cov is None else g_cov)
        else:
            g_out = torch.zeros(b, t, m, device=dev) if g_out is None else f32(g_out)
            grads = (torch.empty_like(keys), torch.empty_like(values), torch.empty_like(queries),
                     torch.empty_like(r2), torch.empty_like(mean0), torch.empty_like(cov0))
            ws = torch.empty(b * t * (d * d + d * m), device=dev, dtype=torch.float32)
            P = _hip.ptr
            with _hip.on_device(dev):
                _hip.call("bssm_associative_static_scan_backward", P(keys), P(values), P(queries), P(r2), P(mean0),
                          P(cov0), P(g_out), P(g_mean), P(g_cov), P(ws), *map(P, grads), b, t, d, m,
                          _hip.stream_of(dev))
        return tuple(g if need else None for g, need in zip(grads, ctx.needs_input_grad))


def associative_static_bayesian_cuda(keys: Tensor, values: Tensor, queries: Tensor, *,
                                     observation_variances: Tensor | Real = 1.0,
                                     initial_mean: Optional[Tensor] = None,
                                     initial_covariance: Optional[Tensor] = None,
                                     denominator_floor: float = 1e-6) -> tuple[Tensor, Tensor, Tensor]:
    """Static scan on the GPU: one gfx950 kernel for fp32 inputs with D <= 32, M <= 64.

    Requires CUDA (ROCm) tensors like the reference (replay_ssm.py:294-299).
    float64 inputs (the reference keeps them in float64) and larger D/M run
    the torch-op scan on the device.
    """
    if not isinstance(keys, Tensor) or not keys.is_cuda:
        raise ValueError("associative_static_bayesian_cuda requires CUDA tensors")
    if not values.is_cuda or not queries.is_cuda:
        raise ValueError("keys, values, and queries must share a CUDA device")
    if keys.device != values.device or keys.device != queries.device:
        raise ValueError("keys, values, and queries must share a CUDA device")
    # The value checks are read back after the scan kernel is queued (it
    # indexes by shape only), so the device->host wait overlaps it.
    checks = _DeferredChecks()
    keys_p, values_p, queries_p, r2, mean0, cov0 = _scan_prepare(
        keys, values, queries, observation_variances, initial_mean, initial_covariance, denominator_floor, checks)
    try:
        d, m, t = keys_p.shape[-1], values_p.shape[-1], keys_p.shape[-2]
        if keys_p.dtype != torch.float32 or d > 32 or m > 64:
            checks.flush()
            return associative_static_bayesian(keys, values, queries, observation_variances=observation_variances,
                                               initial_mean=initial_mean, initial_covariance=initial_covariance,
                                               denominator_floor=denominator_floor)
        batch = keys_p.shape[:-2]
        rows = math.prod(batch)
        flat = lambda x, tail: x.reshape(rows, *tail).contiguous()  # noqa: E731
        out, mT, cT = _StaticScanFunction.apply(flat(keys_p, (t, d)), flat(values_p, (t, m)),
                                                flat(queries_p, (t, d)), flat(r2, (t,)), flat(mean0, (d, m)),
                                                flat(cov0, (d, d)))
        checks.flush()
    except Exception:
        # A failure inside the call: the value checks deferred so far may name its cause (a
        # non-finite input), so they run first. Interrupts and exits propagate untouched.
        checks.flush()
        raise
    return out.reshape(*batch, t, m), mT.reshape(*batch, d, m), cT.reshape(*batch, d, d)
