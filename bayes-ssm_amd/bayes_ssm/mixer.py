"""Producer-fused layer core of the Bayes mixer (key dim 4, value dim 8, learned dynamics).

The reference mixer (example/train_6layer.py:613-709) turns its bfloat16
projections into the inputs of the exact layer with a chain of torch ops::

    q = normalize(silu(q_proj.float()).view(b, t, H, 4))        # :627-639
    k = normalize(silu(k_proj.float()).view(b, t, H, 4))
    v = silu(v_proj.float()).view(b, t, H, 8)
    process, observation = softplus(noise.view(b, t, H, 2)) + 1e-4   # :664-668
    decay = exp(-softplus(decay_logits))                             # :690
    (each permuted to [b * H, t, .])                                 # :648-658, :669-670, :691-693
    read, _, _ = bayesian_layer(k, v, q, ...)                        # :709
    read = read.view(b, H, t, 8).permute(0, 2, 1, 3)                 # :710

which materialises every transformed and permuted tensor in float32 before
the recurrence reads them once.  ``bayes_mixer_core`` returns the same
``read`` ([b, t, H, 8], float32) from one forward and one backward kernel that
read the bfloat16 projections in place (each may be a column view of one
fused projection output) and apply the transforms, and their chain rule, on
chip (C ABI ``bssm_mixer_forward`` / ``bssm_mixer_backward``).  Projection
gradients come back as bfloat16, the float32 gradient rounded to nearest even,
which is what autograd through the reference's ``.float()`` widening yields.

Shapes the kernels do not take (heads not a multiple of 16, T not a multiple
of 4, other dtypes or devices, strided rows the kernels cannot address) run the
reference's op chain through ``bayesian_layer`` instead.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _hip
from .bayesian_layer import bayesian_layer

KEY_DIM = 4
VALUE_DIM = 8
NOISE_FLOOR = 1e-4  # softplus(noise) + 1e-4 (train_6layer.py:667-668)

# Per-head widths of the five projections: q, k, v, decay logits, noise.
_WIDTHS = (KEY_DIM, KEY_DIM, VALUE_DIM, KEY_DIM, 2)


def _aligned(x: Tensor) -> Tensor:
    """``x`` contiguous with a 16-byte aligned base (the C ABI's requirement for weights, biases and belief
    tensors): a contiguous view at an unaligned offset, e.g. a slice of a flattened parameter buffer, is copied."""
    x = x.contiguous()
    return x if x.data_ptr() % 16 == 0 else x.clone()


def _row_stride(x: Tensor, t: int) -> Optional[int]:
    """Row stride (elements) of a [B, T, W] view the kernels can address, else None."""
    if x.ndim != 3 or x.stride(2) != 1:
        return None
    ld = x.stride(1)
    if ld % 8 != 0 or x.data_ptr() % 16 != 0:
        return None
    if x.shape[0] > 1 and x.stride(0) != t * ld:
        return None
    return ld


def _fused_eligible(projections: tuple[Tensor, ...], heads: int) -> Optional[tuple[int, ...]]:
    q = projections[0]
    if q.device.type != "cuda" or q.ndim != 3:
        return None
    b, t, _ = q.shape
    if heads % 16 != 0 or t <= 0 or t % 4 != 0:
        return None
    lds = []
    for x, w in zip(projections, _WIDTHS):
        if x.dtype != torch.bfloat16 or x.device != q.device or tuple(x.shape) != (b, t, w * heads):
            return None
        ld = _row_stride(x, t)
        if ld is None:
            return None
        lds.append(ld)
    return tuple(lds)


class _MixerCoreFunction(torch.autograd.Function):
    """Autograd boundary of the producer-fused kernels (C ABI ``bssm_mixer_*``)."""

    @staticmethod
    def forward(ctx, q_proj, k_proj, v_proj, decay_logits, noise, initial_mean, initial_covariance, heads,
                denominator_floor, lds):
        b, t, _ = q_proj.shape
        n = b * heads
        interval = _hip.preferred_checkpoint(KEY_DIM)
        nb = -(-t // interval)
        dev = q_proj.device
        read = torch.empty(b, t, heads, VALUE_DIM, device=dev, dtype=torch.float32)
        mean_t = torch.empty(n, KEY_DIM, VALUE_DIM, device=dev, dtype=torch.float32)
        cov_t = torch.empty(n, KEY_DIM, KEY_DIM, device=dev, dtype=torch.float32)
        bmean = torch.empty(n, nb + 1, KEY_DIM, VALUE_DIM, device=dev, dtype=torch.float32)
        bcov = torch.empty(n, nb + 1, KEY_DIM, KEY_DIM, device=dev, dtype=torch.float32)
        P = _hip.ptr
        with _hip.on_device(dev):
            _hip.call("bssm_mixer_forward", P(q_proj), lds[0], P(k_proj), lds[1], P(v_proj), lds[2],
                      P(decay_logits), lds[3], P(noise), lds[4], P(initial_mean), P(initial_covariance), P(read),
                      P(mean_t), P(cov_t), P(bmean), P(bcov), b, t, heads, interval, float(denominator_floor),
                      _hip.stream_of(dev))
        ctx.save_for_backward(q_proj, k_proj, v_proj, decay_logits, noise, initial_mean, initial_covariance,
                              bmean, bcov)
        ctx.heads = heads
        ctx.interval = interval
        ctx.lds = lds
        ctx.denominator_floor = float(denominator_floor)
        ctx.set_materialize_grads(False)
        return read, mean_t, cov_t

    @staticmethod
    def backward(ctx, grad_read, grad_mean, grad_covariance):
        q_proj, k_proj, v_proj, decay_logits, noise, mean0, cov0, bmean, bcov = ctx.saved_tensors
        b, t, _ = q_proj.shape
        heads, lds = ctx.heads, ctx.lds
        need = ctx.needs_input_grad
        dev = q_proj.device
        if grad_read is None:
            grad_read = torch.zeros(b, t, heads, VALUE_DIM, device=dev, dtype=torch.float32)
        else:
            grad_read = grad_read.float().contiguous()
        gm = None if grad_mean is None else grad_mean.float().contiguous()
        gc = None if grad_covariance is None else grad_covariance.float().contiguous()

        def empty(x: Tensor) -> Tensor:
            return torch.empty(x.shape, device=dev, dtype=torch.bfloat16)

        gq, gk, gv = empty(q_proj), empty(k_proj), empty(v_proj)
        dyn = need[3] or need[4]
        gdl = empty(decay_logits) if dyn else None
        gnz = empty(noise) if dyn else None
        gm0 = torch.empty_like(mean0) if need[5] else None
        gc0 = torch.empty_like(cov0) if need[6] else None
        P = _hip.ptr
        with _hip.on_device(dev):
            _hip.call("bssm_mixer_backward", P(q_proj), lds[0], P(k_proj), lds[1], P(v_proj), lds[2],
                      P(decay_logits), lds[3], P(noise), lds[4], P(mean0), P(cov0), P(bmean), P(bcov),
                      P(grad_read), P(gm), P(gc), P(gq), P(gk), P(gv), P(gdl), P(gnz), P(gm0), P(gc0), b, t, heads,
                      ctx.interval, ctx.denominator_floor, 0, _hip.stream_of(dev))
        return (gq if need[0] else None, gk if need[1] else None, gv if need[2] else None,
                gdl if need[3] else None, gnz if need[4] else None, gm0, gc0, None, None, None)


# The default prior (zero mean, identity covariance) per (sequence count,
# device): read-only inputs of the kernels, built once instead of by three
# small kernels every step.  A few recent shapes are kept.
_DEFAULT_PRIORS: dict[tuple[int, torch.device], tuple[Tensor, Tensor]] = {}


def _default_prior(n: int, device: torch.device) -> tuple[Tensor, Tensor]:
    key = (n, device)
    prior = _DEFAULT_PRIORS.get(key)
    if prior is None:
        if len(_DEFAULT_PRIORS) >= 4:
            _DEFAULT_PRIORS.pop(next(iter(_DEFAULT_PRIORS)))
        mean0 = torch.zeros(n, KEY_DIM, VALUE_DIM, device=device, dtype=torch.float32)
        cov0 = torch.eye(KEY_DIM, device=device, dtype=torch.float32).expand(n, KEY_DIM, KEY_DIM).contiguous()
        prior = _DEFAULT_PRIORS.setdefault(key, (mean0, cov0))
    return prior


def _initial_state(initial_mean: Optional[Tensor], initial_covariance: Optional[Tensor], n: int,
                   device: torch.device) -> tuple[Tensor, Tensor]:
    if initial_mean is None and initial_covariance is None:
        return _default_prior(n, device)
    if initial_mean is None:
        mean0 = torch.zeros(n, KEY_DIM, VALUE_DIM, device=device, dtype=torch.float32)
    else:
        mean0 = initial_mean.to(device=device, dtype=torch.float32).expand(n, KEY_DIM, VALUE_DIM)
    if initial_covariance is None:
        cov0 = torch.eye(KEY_DIM, device=device, dtype=torch.float32).expand(n, KEY_DIM, KEY_DIM)
    else:
        cov0 = initial_covariance.to(device=device, dtype=torch.float32).expand(n, KEY_DIM, KEY_DIM)
    return _aligned(mean0), _aligned(cov0)


def mixer_layer_inputs(q_proj: Tensor, k_proj: Tensor, v_proj: Tensor, decay_logits: Tensor, noise: Tensor,
                       heads: int) -> tuple[Tensor, ...]:
    """The reference's op chain from projections to layer inputs (train_6layer.py:627-693).

    Returns (keys, values, queries, decay, process, observation) in the
    layer's [B * H, T, .] sequence layout, float32.
    """
    b, t, _ = q_proj.shape

    def heads_first(x: Tensor, w: int) -> Tensor:
        return x.view(b, t, heads, w).permute(0, 2, 1, 3).reshape(b * heads, t, w)

    q = F.normalize(F.silu(q_proj.float()).view(b, t, heads, KEY_DIM), dim=-1)
    k = F.normalize(F.silu(k_proj.float()).view(b, t, heads, KEY_DIM), dim=-1)
    v = F.silu(v_proj.float())
    nz = noise.float().view(b, t, heads, 2)
    process = (F.softplus(nz[..., 0]) + NOISE_FLOOR).permute(0, 2, 1).reshape(b * heads, t)
    observation = (F.softplus(nz[..., 1]) + NOISE_FLOOR).permute(0, 2, 1).reshape(b * heads, t)
    decay = torch.exp(-F.softplus(decay_logits.float()))
    return (heads_first(k.reshape(b, t, -1), KEY_DIM), heads_first(v, VALUE_DIM),
            heads_first(q.reshape(b, t, -1), KEY_DIM), heads_first(decay, KEY_DIM), process, observation)


def bayes_mixer_core(
    q_proj: Tensor,
    k_proj: Tensor,
    v_proj: Tensor,
    decay_logits: Tensor,
    noise: Tensor,
    *,
    heads: int,
    initial_mean: Optional[Tensor] = None,
    initial_covariance: Optional[Tensor] = None,
    chunk_length: Optional[int] = None,
    denominator_floor: float = 1e-6,
    optimized: bool = True,
) -> tuple[Tensor, Tensor, Tensor]:
    """Readout of the mixer's exact Bayes layer from its raw projections.

    q_proj, k_proj, decay_logits: [B, T, H*4]; v_proj: [B, T, H*8]; noise:
    [B, T, H*2] ((process, observation) logits per head).  The initial state
    defaults to the layer's (zero mean, identity covariance) and may be given
    broadcastable to [B*H, 4, 8] / [B*H, 4, 4].  Returns ``read`` [B, T, H, 8]
    (float32; the reference's permuted view, made contiguous) and the final
    mean [B*H, 4, 8] and covariance [B*H, 4, 4].

    Eligible inputs (CUDA, bfloat16, H % 16 == 0, T % 4 == 0, rows
    addressable as described in the module docstring) run the fused kernels;
    others run the reference op chain and ``bayesian_layer`` with
    ``chunk_length`` (which the fused kernels do not need: the recurrence is
    exact for every chunk length) and ``optimized``, the mixer's own switch
    (train_6layer.py:711, true for CUDA runs with --optimize-bayes, :987).
    """
    if q_proj.ndim != 3:
        raise ValueError("q_proj must have shape [B, T, H*4]")
    if heads <= 0:
        raise ValueError("heads must be positive")
    if not (denominator_floor > 0):
        raise ValueError("denominator_floor must be positive")
    b, t, _ = q_proj.shape
    projections = (q_proj, k_proj, v_proj, decay_logits, noise)
    for x, w, name in zip(projections, _WIDTHS, ("q_proj", "k_proj", "v_proj", "decay_logits", "noise")):
        if tuple(x.shape) != (b, t, w * heads):
            raise ValueError(f"{name} must have shape [B, T, H*{w}] = {(b, t, w * heads)}, got {tuple(x.shape)}")
    lds = _fused_eligible(projections, heads)
    if lds is not None:
        _hip.load()  # on a GPU the fused path never degrades silently
        mean0, cov0 = _initial_state(initial_mean, initial_covariance, b * heads, q_proj.device)
        return _MixerCoreFunction.apply(q_proj, k_proj, v_proj, decay_logits, noise, mean0, cov0, int(heads),
                                        float(denominator_floor), lds)
    k, v, q, decay, process, observation = mixer_layer_inputs(*projections, heads)
    read, mean_t, cov_t = bayesian_layer(
        k, v, q, transition_diagonals=decay, process_variances=process, observation_variances=observation,
        initial_mean=initial_mean, initial_covariance=initial_covariance, chunk_length=chunk_length,
        denominator_floor=denominator_floor, optimized=optimized)
    read = read.view(b, heads, t, VALUE_DIM).permute(0, 2, 1, 3).contiguous()
    return read, mean_t, cov_t


class _MixerReadoutFunction(torch.autograd.Function):
    """Autograd boundary of the gated kernels (C ABI ``bssm_mixer_gated_*``)."""

    @staticmethod
    def forward(ctx, q_proj, k_proj, v_proj, decay_logits, noise, gate, norm_weight, initial_mean,
                initial_covariance, heads, norm_eps, denominator_floor, lds):
        b, t, _ = q_proj.shape
        n = b * heads
        interval = _hip.preferred_checkpoint(KEY_DIM)
        nb = -(-t // interval)
        dev = q_proj.device
        out = torch.empty(b, t, heads * VALUE_DIM, device=dev, dtype=torch.bfloat16)
        read_bf16 = torch.empty_like(out)
        mean_t = torch.empty(n, KEY_DIM, VALUE_DIM, device=dev, dtype=torch.float32)
        cov_t = torch.empty(n, KEY_DIM, KEY_DIM, device=dev, dtype=torch.float32)
        bmean = torch.empty(n, nb + 1, KEY_DIM, VALUE_DIM, device=dev, dtype=torch.float32)
        bcov = torch.empty(n, nb + 1, KEY_DIM, KEY_DIM, device=dev, dtype=torch.float32)
        w32 = _aligned(norm_weight.detach().float())
        P = _hip.ptr
        with _hip.on_device(dev):
            _hip.call("bssm_mixer_gated_forward", P(q_proj), lds[0], P(k_proj), lds[1], P(v_proj), lds[2],
                      P(decay_logits), lds[3], P(noise), lds[4], P(gate), lds[5], P(w32), float(norm_eps),
                      P(initial_mean), P(initial_covariance), P(out), P(read_bf16), P(mean_t), P(cov_t), P(bmean),
                      P(bcov), b, t, heads, interval, float(denominator_floor), 0, _hip.stream_of(dev))
        ctx.save_for_backward(q_proj, k_proj, v_proj, decay_logits, noise, gate, w32, initial_mean,
                              initial_covariance, bmean, bcov, read_bf16)
        ctx.heads = heads
        ctx.interval = interval
        ctx.lds = lds
        ctx.norm_eps = float(norm_eps)
        ctx.weight_dtype = norm_weight.dtype
        ctx.denominator_floor = float(denominator_floor)
        ctx.set_materialize_grads(False)
        return out, mean_t, cov_t

    @staticmethod
    def backward(ctx, grad_out, grad_mean, grad_covariance):
        (q_proj, k_proj, v_proj, decay_logits, noise, gate, w32, mean0, cov0, bmean, bcov,
         read_bf16) = ctx.saved_tensors
        b, t, _ = q_proj.shape
        heads, lds = ctx.heads, ctx.lds
        need = ctx.needs_input_grad
        dev = q_proj.device
        if grad_out is None:
            grad_out = torch.zeros(b, t, heads * VALUE_DIM, device=dev, dtype=torch.bfloat16)
        else:
            grad_out = grad_out.to(torch.bfloat16).contiguous()
        gm = None if grad_mean is None else grad_mean.float().contiguous()
        gc = None if grad_covariance is None else grad_covariance.float().contiguous()

        def empty(x: Tensor) -> Tensor:
            return torch.empty(x.shape, device=dev, dtype=torch.bfloat16)

        gq, gk, gv = empty(q_proj), empty(k_proj), empty(v_proj)
        dyn = need[3] or need[4]
        gdl = empty(decay_logits) if dyn else None
        gnz = empty(noise) if dyn else None
        ggate = empty(gate)
        partials = torch.empty(b * heads // 16, VALUE_DIM, device=dev, dtype=torch.float32)
        gm0 = torch.empty_like(mean0) if need[7] else None
        gc0 = torch.empty_like(cov0) if need[8] else None
        P = _hip.ptr
        with _hip.on_device(dev):
            _hip.call("bssm_mixer_gated_backward", P(q_proj), lds[0], P(k_proj), lds[1], P(v_proj), lds[2],
                      P(decay_logits), lds[3], P(noise), lds[4], P(gate), lds[5], P(w32), ctx.norm_eps, P(mean0),
                      P(cov0), P(bmean), P(bcov), P(read_bf16), P(grad_out), P(gm), P(gc), P(gq), P(gk), P(gv),
                      P(gdl), P(gnz), P(ggate), P(partials), P(gm0), P(gc0), b, t, heads, ctx.interval,
                      ctx.denominator_floor, 0, _hip.stream_of(dev))
        gw = partials.sum(0).to(ctx.weight_dtype) if need[6] else None
        return (gq if need[0] else None, gk if need[1] else None, gv if need[2] else None,
                gdl if need[3] else None, gnz if need[4] else None, ggate if need[5] else None, gw, gm0, gc0,
                None, None, None, None)


def bayes_mixer_readout(
    q_proj: Tensor,
    k_proj: Tensor,
    v_proj: Tensor,
    decay_logits: Tensor,
    noise: Tensor,
    gate: Tensor,
    norm_weight: Tensor,
    *,
    heads: int,
    norm_eps: Optional[float] = None,
    initial_mean: Optional[Tensor] = None,
    initial_covariance: Optional[Tensor] = None,
    chunk_length: Optional[int] = None,
    denominator_floor: float = 1e-6,
    optimized: bool = True,
) -> tuple[Tensor, Tensor, Tensor]:
    """The mixer's gated readout from its raw projections (train_6layer.py:627-729, up to ``out_proj``).

    Computes ``bayes_mixer_core`` and then, per head of 8 values,
    ``read_norm(read.to(bf16)) * silu(gate)``: read_norm is an RMSNorm with
    weight ``norm_weight`` [8] and ``norm_eps`` (None: the float32 epsilon,
    as torch's rms_norm with eps None).  gate: [B, T, H*8].  Returns the
    product as [B, T, H*8] (what the reference reshapes and feeds to
    out_proj; bf16) and the final mean and covariance.

    On the fused path (the conditions of ``bayes_mixer_core``, plus a bf16
    gate with rows the kernels can address) the product is formed in float32
    and rounded once, the readout never reaches HBM in float32, and the
    backward forms the readout gradient on chip.  Otherwise the op chain runs
    in torch.
    """
    b, t = q_proj.shape[:2]
    if tuple(gate.shape) != (b, t, VALUE_DIM * heads):
        raise ValueError(f"gate must have shape [B, T, H*8] = {(b, t, VALUE_DIM * heads)}, got {tuple(gate.shape)}")
    if tuple(norm_weight.shape) != (VALUE_DIM,):
        raise ValueError("norm_weight must have shape [8]")
    eps = torch.finfo(torch.float32).eps if norm_eps is None else float(norm_eps)
    projections = (q_proj, k_proj, v_proj, decay_logits, noise)
    lds = _fused_eligible(projections, heads)
    ldg = _row_stride(gate, t) if gate.dtype == torch.bfloat16 and gate.device == q_proj.device else None
    if lds is not None and ldg is not None:
        _hip.load()
        mean0, cov0 = _initial_state(initial_mean, initial_covariance, b * heads, q_proj.device)
        return _MixerReadoutFunction.apply(q_proj, k_proj, v_proj, decay_logits, noise, gate, norm_weight, mean0,
                                           cov0, int(heads), eps, float(denominator_floor), (*lds, ldg))
    read, mean_t, cov_t = bayes_mixer_core(*projections, heads=heads, initial_mean=initial_mean,
                                           initial_covariance=initial_covariance, chunk_length=chunk_length,
                                           denominator_floor=denominator_floor, optimized=optimized)
    normed = F.rms_norm(read.to(gate.dtype), (VALUE_DIM,), norm_weight, eps)
    out = (normed * F.silu(gate.view(b, t, heads, VALUE_DIM))).reshape(b, t, heads * VALUE_DIM)
    return out, mean_t, cov_t


class _MixerBlockFunction(torch.autograd.Function):
    """Autograd boundary of config 4's block kernels (C ABI ``bssm_mixer_block_*``): the filter and the
    gated readout in one call per direction, the projection gradient written in place column by column."""

    @staticmethod
    def forward(ctx, projected, conv_weight, norm_weight, aux_bias, mean0, cov0, heads, norm_eps, denominator_floor,
                ld):
        b, t, _ = projected.shape
        core, aux_w = 16 * heads, 6 * heads
        interval = _hip.preferred_checkpoint(KEY_DIM)
        nb = -(-t // interval)
        dev = projected.device
        # The kernels add the aux bias as they read the aux columns, in bf16
        # as the reference does (one rounding).
        bias = None if aux_bias is None else _aligned(aux_bias.detach())
        convolved = torch.empty(b, t, core, device=dev, dtype=torch.bfloat16)
        out = torch.empty(b, t, heads * VALUE_DIM, device=dev, dtype=torch.bfloat16)
        read_bf16 = torch.empty_like(out)
        n = b * heads
        mean_t = torch.empty(n, KEY_DIM, VALUE_DIM, device=dev, dtype=torch.float32)
        cov_t = torch.empty(n, KEY_DIM, KEY_DIM, device=dev, dtype=torch.float32)
        bmean = torch.empty(n, nb + 1, KEY_DIM, VALUE_DIM, device=dev, dtype=torch.float32)
        bcov = torch.empty(n, nb + 1, KEY_DIM, KEY_DIM, device=dev, dtype=torch.float32)
        cw32 = _aligned(conv_weight.detach().reshape(core, 4).float())
        nw32 = _aligned(norm_weight.detach().float())
        P = _hip.ptr
        with _hip.on_device(dev):
            _hip.call("bssm_mixer_block_forward", P(projected), ld, P(cw32), P(bias), P(nw32), float(norm_eps),
                      P(mean0), P(cov0), P(convolved), P(out), P(read_bf16), P(mean_t), P(cov_t), P(bmean),
                      P(bcov), b, t, heads, interval, float(denominator_floor), _hip.stream_of(dev))
        ctx.save_for_backward(projected, cw32, bias, convolved, nw32, mean0, cov0, bmean, bcov, read_bf16)
        ctx.heads, ctx.interval, ctx.ld = heads, interval, ld
        ctx.norm_eps, ctx.denominator_floor = float(norm_eps), float(denominator_floor)
        ctx.conv_shape, ctx.conv_dtype = tuple(conv_weight.shape), conv_weight.dtype
        ctx.norm_dtype = norm_weight.dtype
        ctx.bias_dtype = None if aux_bias is None else aux_bias.dtype
        ctx.set_materialize_grads(False)
        return out, mean_t, cov_t

    @staticmethod
    def backward(ctx, grad_out, grad_mean, grad_covariance):
        projected, cw32, bias, convolved, nw32, mean0, cov0, bmean, bcov, read_bf16 = ctx.saved_tensors
        b, t, _ = projected.shape
        heads = ctx.heads
        core, aux_w = 16 * heads, 6 * heads
        need = ctx.needs_input_grad
        dev = projected.device
        if grad_out is None:
            grad_out = torch.zeros(b, t, heads * VALUE_DIM, device=dev, dtype=torch.bfloat16)
        else:
            grad_out = grad_out.to(torch.bfloat16).contiguous()
        gm = None if grad_mean is None else grad_mean.float().contiguous()
        gc = None if grad_covariance is None else grad_covariance.float().contiguous()
        gproj = torch.empty(b, t, core + aux_w + heads * VALUE_DIM, device=dev, dtype=torch.bfloat16)
        gconv = torch.empty(b, t, core, device=dev, dtype=torch.bfloat16)
        cpart = torch.empty(b, core, 4, device=dev, dtype=torch.float32)
        npart = torch.empty(b * heads // 16, VALUE_DIM, device=dev, dtype=torch.float32)
        apart = torch.empty(b, aux_w, device=dev, dtype=torch.float32) if need[3] else None
        # The weight gradients are summed from their partials in the same call,
        # in the parameters' dtype when all of them are bf16 (else float32).
        dtypes = [dt for dt, n in zip((ctx.conv_dtype, ctx.norm_dtype, ctx.bias_dtype), need[1:4]) if n]
        wdt = torch.bfloat16 if dtypes and all(dt == torch.bfloat16 for dt in dtypes) else torch.float32
        g_conv = torch.empty(ctx.conv_shape, device=dev, dtype=wdt) if need[1] else None
        g_norm = torch.empty(VALUE_DIM, device=dev, dtype=wdt) if need[2] else None
        g_bias = torch.empty(aux_w, device=dev, dtype=wdt) if need[3] else None
        gm0 = torch.empty_like(mean0) if need[4] else None
        gc0 = torch.empty_like(cov0) if need[5] else None
        P = _hip.ptr
        with _hip.on_device(dev):
            _hip.call("bssm_mixer_block_backward", P(projected), ctx.ld, P(cw32), P(bias), P(convolved),
                      P(nw32), ctx.norm_eps, P(mean0), P(cov0), P(bmean), P(bcov), P(read_bf16), P(grad_out), P(gm),
                      P(gc), P(gconv), P(gproj), gproj.shape[-1], P(cpart), P(npart), P(apart), P(g_conv),
                      P(g_norm), P(g_bias), int(wdt == torch.bfloat16), P(gm0), P(gc0), b, t, heads, ctx.interval,
                      ctx.denominator_floor, _hip.stream_of(dev))
        if g_conv is not None and g_conv.dtype != ctx.conv_dtype:
            g_conv = g_conv.to(ctx.conv_dtype)
        if g_norm is not None and g_norm.dtype != ctx.norm_dtype:
            g_norm = g_norm.to(ctx.norm_dtype)
        if g_bias is not None and g_bias.dtype != ctx.bias_dtype:
            g_bias = g_bias.to(ctx.bias_dtype)
        return gproj if need[0] else None, g_conv, g_norm, g_bias, gm0, gc0, None, None, None, None


def bayes_mixer_block(
    projected: Tensor,
    conv_weight: Tensor,
    norm_weight: Tensor,
    *,
    heads: int,
    aux_bias: Optional[Tensor] = None,
    norm_eps: Optional[float] = None,
    initial_mean: Optional[Tensor] = None,
    initial_covariance: Optional[Tensor] = None,
    chunk_length: Optional[int] = None,
    denominator_floor: float = 1e-6,
    optimized: bool = True,
) -> tuple[Tensor, Tensor, Tensor]:
    """The Bayes mixer from its fused projection to ``out_proj``'s input (train_6layer.py:583-729).

    This is the paper configuration of config 4's Bayes blocks (key dim 4,
    learned dynamics, fused Q/K/V/decay/noise/gate projection,
    :585-600): ``projected`` [B, T, H*4 + H*4 + H*8 + H*4 + H*2 + H*8] holds,
    per token, the Q, K and V core (``qkv_core_width``), the decay logits and
    the interleaved (process, observation) noise logits (``aux_width``, plus
    ``aux_bias`` when given, :589-593) and the gate (:594-597).  The core goes
    through the causal depthwise-4 filter with ``conv_weight`` [2*H*4 + H*8,
    1, 4] (:598, ``_causal_depthwise`` :474-480) and is split into q, k, v
    (:599-601); the rest is ``bayes_mixer_readout``.  Returns the gated
    readout [B, T, H*8] and the final mean and covariance.

    On the GPU (bf16 ``projected`` whose rows the kernels can address, heads a
    multiple of 16, T a positive multiple of 4, an absent or bf16 [H*4 + H*2]
    aux bias) the block is one C call per direction: the filter reads the
    core columns in place and writes one contiguous [B, T, 2*H*4 + H*8]
    tensor, whose column views, with the aux and gate columns of
    ``projected``, feed the producer-fused readout kernels (which add the aux
    bias as they read the aux columns); the backward writes the projection
    gradient column by column into one [B, T, 30 H] tensor and sums the
    weight and bias gradients from their partials.  Other inputs run the same
    stages through ``causal_depthwise4`` and ``bayes_mixer_readout``.
    """
    if projected.ndim != 3:
        raise ValueError("projected must have shape [B, T, width]")
    if heads <= 0:
        raise ValueError("heads must be positive")
    if not (denominator_floor > 0):
        raise ValueError("denominator_floor must be positive")
    state = heads * KEY_DIM
    width = heads * VALUE_DIM
    core = 2 * state + width
    aux = state + 2 * heads
    if projected.shape[-1] != core + aux + width:
        raise ValueError(f"projected must have {core + aux + width} columns for {heads} heads, "
                         f"got {projected.shape[-1]}")
    if tuple(conv_weight.shape) != (core, 1, 4):
        raise ValueError(f"conv_weight must have shape [{core}, 1, 4]")
    b, t = projected.shape[:2]
    ld = _row_stride(projected, t) if projected.is_cuda and projected.dtype == torch.bfloat16 else None
    fused = (ld is not None and heads % 16 == 0 and t > 0 and t % 4 == 0
             and conv_weight.device == projected.device and norm_weight.device == projected.device
             and tuple(norm_weight.shape) == (VALUE_DIM,)
             and (aux_bias is None or (aux_bias.device == projected.device and aux_bias.dtype == torch.bfloat16
                                       and tuple(aux_bias.shape) == (aux,))))
    if fused:
        _hip.load()
        eps = torch.finfo(torch.float32).eps if norm_eps is None else float(norm_eps)
        mean0, cov0 = _initial_state(initial_mean, initial_covariance, b * heads, projected.device)
        return _MixerBlockFunction.apply(projected, conv_weight, norm_weight, aux_bias, mean0, cov0, int(heads), eps,
                                         float(denominator_floor), ld)
    from .conv import causal_depthwise4

    qkv = projected[..., :core]
    convolved = causal_depthwise4(qkv.transpose(1, 2), conv_weight).transpose(1, 2)
    q_in, k_in, v_in = convolved.split((state, state, width), dim=-1)
    aux_in = projected[..., core:core + aux]
    if aux_bias is not None:
        aux_in = aux_in + aux_bias
    gate = projected[..., core + aux:]
    return bayes_mixer_readout(q_in, k_in, v_in, aux_in[..., :state], aux_in[..., state:], gate, norm_weight,
                               heads=heads, norm_eps=norm_eps, initial_mean=initial_mean,
                               initial_covariance=initial_covariance, chunk_length=chunk_length,
                               denominator_floor=denominator_floor, optimized=optimized)


__all__ = ["bayes_mixer_block", "bayes_mixer_core", "bayes_mixer_readout", "mixer_layer_inputs"]
