"""Config 4's in-scope Bayes block at its shape: the mixer from the fused projection to out_proj's input.

``bayes_mixer_block`` chains the causal depthwise-4 filter, the producer-fused
layer core and the gated readout (example/train_6layer.py:583-729) on the HIP
kernels.  At B256 x T512 x W512 x H64 (D4M8), batch rows are independent
except for the two weight gradients, which sum over them: so the full-shape
run's rows must equal, bit for bit, a run on just those rows, and that small
run is checked against the float64 oracle chain (``O.mixer_block``),
including both weight gradients.

Outputs and gradients here are bfloat16 (the reference's tensor dtype at these
boundaries); the oracle takes the kernel's bf16 filter output as the layer's
input (the filter itself is checked against the oracle within one bf16
rounding), so what remains is the rounding of bf16 results: 2^-7 relative,
with an absolute floor of 2^-8 of the tensor's largest magnitude for entries
near zero.  The float32 pieces are checked at 1e-5 / 1e-4 elsewhere
(test_gpu_mixer.py, test_gpu_conv.py).
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O

pytestmark = pytest.mark.gpu

B, T, H = 256, 512, 64
ROWS = [0, 137, 255]


def _inputs(b, t, h, seed, device):
    g = torch.Generator().manual_seed(seed)
    state, width = 4 * h, 8 * h
    core, aux = 2 * state + width, state + 2 * h
    projected = torch.randn(b, t, core + aux + width, generator=g)
    projected[..., core:core + state] -= 4.0          # decay logits near the learned init (slow decay)
    projected[..., core + state:core + aux:2] -= 2.0  # process-noise logits
    projected = projected.to(torch.bfloat16)
    weight = (0.5 * torch.randn(core, 1, 4, generator=g)).to(torch.bfloat16)
    norm_w = (1 + 0.2 * torch.randn(8, generator=g)).to(torch.bfloat16)
    aux_bias = (0.3 * torch.randn(aux, generator=g)).to(torch.bfloat16)
    gout = torch.randn(b, t, width, generator=g).to(torch.bfloat16)
    return [x.to(device) for x in (projected, weight, norm_w, aux_bias, gout)]


def _run(projected, weight, norm_w, aux_bias, gout, h):
    from bayes_ssm.mixer import bayes_mixer_block

    leaves = [x.detach().clone().requires_grad_(True) for x in (projected, weight, norm_w, aux_bias)]
    out, mT, cT = bayes_mixer_block(leaves[0], leaves[1], leaves[2], heads=h, aux_bias=leaves[3])
    out.backward(gout)
    torch.cuda.synchronize()
    return out.detach(), mT.detach(), cT.detach(), [x.grad for x in leaves]


def _bf16_close(actual, expected, name):
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    torch.testing.assert_close(a, e, rtol=2 ** -7, atol=2 ** -8 * float(e.abs().max()),
                               msg=lambda m: f"{name}: {m}")


def test_config4_block_full_shape(cuda_device, monkeypatch):
    from bayes_ssm import conv, mixer

    calls = {"conv": 0, "readout": 0}
    c_orig, r_orig = conv._CausalConv4Function.apply, mixer._MixerReadoutFunction.apply
    monkeypatch.setattr(conv._CausalConv4Function, "apply",
                        staticmethod(lambda *a: calls.__setitem__("conv", calls["conv"] + 1) or c_orig(*a)))
    monkeypatch.setattr(mixer._MixerReadoutFunction, "apply",
                        staticmethod(lambda *a: calls.__setitem__("readout", calls["readout"] + 1) or r_orig(*a)))
    print("config4 block full shape", flush=True)
    projected, weight, norm_w, aux_bias, gout = _inputs(B, T, H, seed=4, device=cuda_device)
    out, mT, cT, grads = _run(projected, weight, norm_w, aux_bias, gout, H)
    assert calls == {"conv": 1, "readout": 1}, f"HIP kernels not used on every stage: {calls}"
    assert out.shape == (B, T, 8 * H) and out.dtype == torch.bfloat16
    assert torch.isfinite(out.float()).all() and torch.isfinite(grads[0].float()).all()

    # The same rows on their own: bitwise the full-shape rows.
    rows = torch.tensor(ROWS, device=cuda_device)
    seqs = (rows[:, None] * H + torch.arange(H, device=cuda_device)).flatten()
    print("config4 block subset rows", flush=True)
    sub_p = projected[rows].contiguous()
    s_out, s_mT, s_cT, s_grads = _run(sub_p, weight, norm_w, aux_bias, gout[rows].contiguous(), H)
    assert torch.equal(s_out, out[rows])
    assert torch.equal(s_mT, mT[seqs]) and torch.equal(s_cT, cT[seqs])
    assert torch.equal(s_grads[0], grads[0][rows]), "projection gradient rows differ from the full-shape run"

    # The small run against the float64 oracle chain.
    from bayes_ssm.conv import causal_depthwise4

    core = 16 * H
    with torch.no_grad():
        conv_out = causal_depthwise4(sub_p[..., :core].transpose(1, 2), weight).transpose(1, 2).cpu()
    sp = sub_p.cpu()
    leaves = [x.detach().cpu().double().requires_grad_(True) for x in (sub_p, weight, norm_w, aux_bias)]
    e_filter = O.causal_depthwise4(sp[..., :core].double().transpose(1, 2), weight.cpu().double()).transpose(1, 2)
    torch.testing.assert_close(conv_out.double(), e_filter, rtol=2 ** -8, atol=1e-6)
    e_out, e_mT, e_cT = O.mixer_block(leaves[0], leaves[1], leaves[2], H, aux_bias=leaves[3], conv_out=conv_out)
    e_grads = torch.autograd.grad((e_out * gout[rows].cpu().double()).sum(), leaves)
    _bf16_close(s_out, e_out, "out")
    torch.testing.assert_close(s_mT.double().cpu(), e_mT, rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(s_cT.double().cpu(), e_cT, rtol=1e-5, atol=1e-4)
    for name, a, e in zip(("grad projected", "grad conv weight", "grad norm weight", "grad aux bias"), s_grads,
                          e_grads):
        assert a.dtype == torch.bfloat16
        _bf16_close(a, e, name)
