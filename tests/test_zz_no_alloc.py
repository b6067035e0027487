"""The allocation-free entry point bssm_causal_conv4_backward_noalloc against bssm_causal_conv4_backward.

The no-alloc variant keeps the weight-gradient partials in the library's own
device scratch and writes their sum over the batch; grad_x comes from the same
kernel.  Two calls in a row, the second with a smaller input, so stale scratch
contents from the first would show; then T = 0 (all-zero partials).  (Sizes
beyond the scratch are rejected before any launch: tests/test_capi.py.)  Tolerance of
the summed weight gradient (north star): 1e-5 relative, 1e-4 absolute against
the float64 sum of the partials; grad_x bit for bit.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(b, t, c, pad, bf16, seed, device):
    g = torch.Generator().manual_seed(seed)
    dtype = torch.bfloat16 if bf16 else torch.float32
    rows = torch.randn(b, t, c + pad, generator=g).to(dtype).to(device)
    x = rows[..., :c]
    w = (0.5 * torch.randn(c, 4, generator=g)).to(device)
    gy = torch.randn(b, t, c, generator=g).to(dtype).to(device)
    return x, w, gy


def _existing(x, w, gy, b, t, c, bf16, stream):
    from bayes_ssm import _hip

    gx = torch.empty(b, t, c, device=x.device, dtype=gy.dtype)
    part = torch.empty(b, c, 4, device=x.device)
    _hip.call("bssm_causal_conv4_backward", int(bf16), x.data_ptr(), x.stride(1) if t else c, w.data_ptr(),
              gy.data_ptr(), gx.data_ptr(), part.data_ptr(), b, t, c, stream)
    return gx, part


def _noalloc(x, w, gy, b, t, c, bf16, stream):
    from bayes_ssm import _hip

    gx = torch.empty(b, t, c, device=x.device, dtype=gy.dtype)
    gw = torch.full((c, 4), float("nan"), device=x.device)
    _hip.call("bssm_causal_conv4_backward_noalloc", int(bf16), x.data_ptr(), x.stride(1) if t else c,
              w.data_ptr(), gy.data_ptr(), gx.data_ptr(), gw.data_ptr(), b, t, c, stream)
    return gx, gw


@pytest.mark.parametrize("bf16", [True, False])
def test_noalloc_conv_backward_matches_existing_entry_point(cuda_device, bf16):
    from bayes_ssm import _hip

    stream = _hip.stream_of(cuda_device)
    # Call 1 fills most of the scratch; call 2 is smaller, so its reduction
    # reads only slots it rewrote; T = 0 writes zero partials.
    for b, t, c, pad in ((256, 96, 1024, 64), (3, 37, 256, 8), (5, 0, 128, 0)):
        print(f"noalloc conv4 backward bf16={bf16} b={b} t={t} c={c}", flush=True)
        x, w, gy = _case(b, t, c, pad, bf16, seed=b + t + c, device=cuda_device)
        gx_ref, part = _existing(x, w, gy, b, t, c, bf16, stream)
        gx, gw = _noalloc(x, w, gy, b, t, c, bf16, stream)
        torch.cuda.synchronize()
        assert torch.equal(gx, gx_ref), "grad_x differs from the existing entry point"
        expected = part.double().sum(0)
        torch.testing.assert_close(gw.double(), expected, rtol=1e-5, atol=1e-4)
        if t == 0:
            assert torch.count_nonzero(gw) == 0

