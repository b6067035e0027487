"""Length-four causal depthwise filter (the mixer's CausalDepthwise4) on HIP kernels.

The reference module (example/train_6layer.py:160-191) keeps a Conv1d-shaped
``[C, 1, 4]`` weight and computes, on ``x [batch, channels, time]``,

    y[t] = w[:,0] x[t-3] + w[:,1] x[t-2] + w[:,2] x[t-1] + w[:,3] x[t]    (x = 0 before t = 0)

as four shifted elementwise products.  The mixer applies it to each projected
stream through a transposed view (``conv(value.transpose(1, 2)).transpose(1,
2)``, :474-480), so in memory every token is a row of C channels.  Here that
channels-last view runs on ``bssm_causal_conv4_forward/backward``: one read and
one write per element, computed in float32 and rounded once, and the weight
gradient reduced without atomics.  The output is returned as the same kind of
transposed view, so the mixer's ``.transpose(1, 2)`` gives back a contiguous
``[B, T, C]`` tensor without a copy.

Inputs the kernels do not take (other devices or dtypes, a contiguous
``[B, C, T]`` layout, rows not 16-byte multiples) run the reference's
elementwise formula in torch.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import _hip


def _taps_formula(x: Tensor, weight: Tensor) -> Tensor:
    """The reference's four shifted products (train_6layer.py:182-191), x [B, C, T]."""
    w = weight[:, 0]
    t = x.shape[-1]
    padded = F.pad(x, (3, 0))
    y = padded[..., :t] * w[:, 0].view(1, -1, 1)
    y = y + padded[..., 1 : t + 1] * w[:, 1].view(1, -1, 1)
    y = y + padded[..., 2 : t + 2] * w[:, 2].view(1, -1, 1)
    return y + padded[..., 3 : t + 3] * w[:, 3].view(1, -1, 1)


def _channels_last_stride(x: Tensor) -> Optional[int]:
    """Row stride (elements) when x [B, C, T] is a view of [B, T, C] rows the kernels can address."""
    if x.device.type != "cuda" or x.dtype not in (torch.bfloat16, torch.float32) or x.ndim != 3:
        return None
    b, c, t = x.shape
    per16 = 16 // x.element_size()
    if x.stride(1) != 1 or c % per16 != 0 or x.data_ptr() % 16 != 0:
        return None
    # With one token the row stride is the batch stride (or free with one row).
    ld = x.stride(2) if t > 1 else (x.stride(0) if b > 1 else c)
    if ld < c or ld % per16 != 0 or (b > 1 and x.stride(0) != t * ld):
        return None
    return ld


class _CausalConv4Function(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, ld):
        b, c, t = x.shape
        bf16 = int(x.dtype == torch.bfloat16)
        w32 = weight.detach().reshape(c, 4).float().contiguous()
        y = torch.empty(b, t, c, device=x.device, dtype=x.dtype)
        with _hip.on_device(x.device):
            _hip.call("bssm_causal_conv4_forward", bf16, x.data_ptr(), ld, w32.data_ptr(), y.data_ptr(), b, t, c,
                      _hip.stream_of(x.device))
        ctx.save_for_backward(x, w32)
        ctx.ld = ld
        ctx.weight_dtype = weight.dtype
        ctx.weight_shape = tuple(weight.shape)
        return y.transpose(1, 2)

    @staticmethod
    def backward(ctx, grad_y):
        x, w32 = ctx.saved_tensors
        b, c, t = x.shape
        bf16 = int(x.dtype == torch.bfloat16)
        gy = grad_y.to(x.dtype).transpose(1, 2).contiguous()  # [B, T, C] rows
        gx = torch.empty(b, t, c, device=x.device, dtype=x.dtype)
        part = torch.empty(b, c, 4, device=x.device, dtype=torch.float32)
        with _hip.on_device(x.device):
            _hip.call("bssm_causal_conv4_backward", bf16, x.data_ptr(), ctx.ld, w32.data_ptr(), gy.data_ptr(),
                      gx.data_ptr(), part.data_ptr(), b, t, c, _hip.stream_of(x.device))
        gw = part.sum(0).reshape(ctx.weight_shape).to(ctx.weight_dtype) if ctx.needs_input_grad[1] else None
        return (gx.transpose(1, 2) if ctx.needs_input_grad[0] else None), gw, None


def causal_depthwise4(x: Tensor, weight: Tensor) -> Tensor:
    """CausalDepthwise4's forward on ``x [batch, channels, time]`` with a ``[C, 1, 4]`` weight."""
    if x.ndim != 3 or tuple(weight.shape) != (x.shape[1], 1, 4):
        raise ValueError("x must be [batch, channels, time] and weight [channels, 1, 4]")
    ld = _channels_last_stride(x)
    if ld is not None and weight.device == x.device and x.shape[0] * x.shape[2] > 0:
        _hip.load()  # on a GPU the kernels never degrade silently
        return _CausalConv4Function.apply(x, weight, ld)
    return _taps_formula(x, weight.to(x.dtype))


class CausalDepthwise4(nn.Module):
    """Drop-in for the reference module (train_6layer.py:160-191): same arguments and ``[C, 1, 4]`` weight."""

    def __init__(self, in_channels: int, out_channels: int | None = None, *, kernel_size: int = 4,
                 groups: int | None = None, bias: bool = False, dtype: torch.dtype = torch.float32,
                 device: torch.device | str | None = None):
        super().__init__()
        out_channels = in_channels if out_channels is None else out_channels
        if out_channels != in_channels or kernel_size != 4 or groups not in (None, in_channels) or bias:
            raise ValueError("CausalDepthwise4 requires equal channels, kernel_size=4, groups=channels, bias=False")
        self.weight = nn.Parameter(torch.empty(in_channels, 1, 4, dtype=dtype, device=device))

    def forward(self, x: Tensor) -> Tensor:
        return causal_depthwise4(x, self.weight)


__all__ = ["CausalDepthwise4", "causal_depthwise4"]
