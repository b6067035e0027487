"""GPU parity of the causal depthwise-4 kernels (C ABI bssm_causal_conv4_*) against the CPU oracle.

float32 streams: 1e-5 relative / 1e-6 absolute against the float64 oracle on
the same inputs.  bfloat16 streams: outputs within one bf16 rounding (2^-8
relative) of the float64 result on the same bf16 inputs; the weight gradient,
accumulated in float32 from exact bf16 products, at 1e-5 / 1e-4.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O

pytestmark = pytest.mark.gpu


def close(actual, expected, name="", rtol=1e-5, atol=1e-6):
    torch.testing.assert_close(actual.detach().double().cpu(), expected.detach().double().cpu(), rtol=rtol,
                               atol=atol, msg=lambda m: f"{name}: {m}")


def _case(b, t, c, pad, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    rows = torch.randn(b, t, c + pad, generator=g).to(dtype)
    x = rows[..., :c]  # [B, T, C] view with row stride c + pad
    w = torch.randn(c, 1, 4, generator=g).to(dtype).float()
    gy = torch.randn(b, t, c, generator=g).to(dtype)
    return rows, x, w, gy


CASES = [  # batch, tokens, channels, row padding, dtype
    (2, 37, 64, 0, torch.float32),
    (1, 3, 16, 8, torch.bfloat16),
    (3, 130, 1024, 32, torch.bfloat16),
    (2, 64, 12, 4, torch.float32),
    (1, 1, 8, 0, torch.bfloat16),
    (4, 257, 200, 8, torch.bfloat16),
]


@pytest.mark.parametrize("b,t,c,pad,dtype", CASES)
def test_conv4_abi_matches_oracle(cuda_device, b, t, c, pad, dtype):
    from bayes_ssm import _hip

    print(f"conv4 b={b} t={t} c={c} pad={pad} {dtype}", flush=True)
    rows, x, w, gy = _case(b, t, c, pad, dtype, seed=t + c)
    bf16 = int(dtype == torch.bfloat16)
    rows_d = rows.to(cuda_device)
    x_d = torch.as_strided(rows_d, x.shape, x.stride(), x.storage_offset())
    w_d = w.reshape(c, 4).contiguous().to(cuda_device)
    gy_d = gy.to(cuda_device)
    y = torch.empty(b, t, c, device=cuda_device, dtype=dtype)
    gx = torch.empty_like(y)
    part = torch.empty(b, c, 4, device=cuda_device)
    s = _hip.stream_of(cuda_device)
    _hip.call("bssm_causal_conv4_forward", bf16, x_d.data_ptr(), x.stride(1), w_d.data_ptr(), y.data_ptr(), b, t, c, s)
    _hip.call("bssm_causal_conv4_backward", bf16, x_d.data_ptr(), x.stride(1), w_d.data_ptr(), gy_d.data_ptr(),
              gx.data_ptr(), part.data_ptr(), b, t, c, s)
    torch.cuda.synchronize()

    xl = x.double().transpose(1, 2).contiguous().requires_grad_(True)
    wl = w.double().requires_grad_(True)
    ey = O.causal_depthwise4(xl, wl)
    egx, egw = torch.autograd.grad(ey, (xl, wl), gy.double().transpose(1, 2))
    tol = dict(rtol=2 ** -8, atol=1e-6) if bf16 else {}
    close(y, ey.transpose(1, 2), "y", **tol)
    close(gx, egx.transpose(1, 2), "grad_x", **tol)
    close(part.sum(0).view(c, 1, 4), egw, "grad_weight", rtol=1e-5, atol=1e-4)
    if bf16:
        # The float32 result rounded once: the kernel's output is the bf16 of a float32 within 1e-5 of exact.
        assert (y.double().cpu() - ey.transpose(1, 2).detach()).abs().max() <= \
            (2 ** -8) * ey.detach().abs().max() + 1e-6


def test_conv4_module_in_the_mixer_pattern(cuda_device, monkeypatch):
    """conv(value.transpose(1, 2)).transpose(1, 2) runs the kernels and returns contiguous [B, T, C] rows."""
    from bayes_ssm import conv

    calls = []
    orig = conv._CausalConv4Function.apply
    monkeypatch.setattr(conv._CausalConv4Function, "apply", staticmethod(lambda *a: calls.append(1) or orig(*a)))
    b, t, c = 2, 50, 128
    g = torch.Generator().manual_seed(3)
    fused = torch.randn(b, t, c + 64, generator=g).to(torch.bfloat16).to(cuda_device)
    value = fused[..., :c].detach().requires_grad_(True)
    m = conv.CausalDepthwise4(c, dtype=torch.bfloat16, device=cuda_device)
    with torch.no_grad():
        m.weight.copy_(torch.randn(c, 1, 4, generator=g).to(torch.bfloat16))
    out = m(value.transpose(1, 2)).transpose(1, 2)
    assert calls, "conv kernels were not used"
    assert out.is_contiguous() and out.shape == (b, t, c)
    gy = torch.randn(b, t, c, generator=g).to(torch.bfloat16).to(cuda_device)
    out.backward(gy)
    xl = value.detach().double().cpu().transpose(1, 2).requires_grad_(True)
    wl = m.weight.detach().double().cpu().requires_grad_(True)
    ey = O.causal_depthwise4(xl, wl)
    egx, egw = torch.autograd.grad(ey, (xl, wl), gy.double().cpu().transpose(1, 2))
    close(out, ey.transpose(1, 2), "y", rtol=2 ** -8, atol=1e-6)
    close(value.grad, egx.transpose(1, 2), "grad_x", rtol=2 ** -8, atol=1e-6)
    assert m.weight.grad.dtype == torch.bfloat16
    close(m.weight.grad, egw, "grad_weight", rtol=2 ** -8, atol=1e-3)


def test_conv4_contiguous_channels_first_takes_torch(cuda_device):
    from bayes_ssm import conv

    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 16, 9, generator=g).to(cuda_device)
    w = torch.randn(16, 1, 4, generator=g).to(cuda_device)
    assert conv._channels_last_stride(x) is None
    close(conv.causal_depthwise4(x, w), O.causal_depthwise4(x.double().cpu(), w.double().cpu()), "y")
