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


def _leaves(projected, weight, norm_w, aux_bias, wide):
    """Fresh leaves; with ``wide`` the projection leaf is a wider tensor and the block sees a column view."""
    w = projected.shape[-1]
    if wide:
        base = torch.zeros(*projected.shape[:2], w + 24, device=projected.device, dtype=projected.dtype)
        base[..., 8:8 + w] = projected
        base.requires_grad_(True)
        view = base[..., 8:8 + w]
    else:
        base = projected.detach().clone().requires_grad_(True)
        view = base
    leaves = [base] + [x.detach().clone().requires_grad_(True) for x in (weight, norm_w)]
    bias = None if aux_bias is None else aux_bias.detach().clone().requires_grad_(True)
    return leaves, view, bias


def _staged(projected, weight, norm_w, aux_bias, gout, h, gm=None, gc=None, wide=False):
    """The same block through its separate stages (filter, then the gated readout on column views)."""
    from bayes_ssm.conv import causal_depthwise4
    from bayes_ssm.mixer import bayes_mixer_readout

    leaves, p, bias = _leaves(projected, weight, norm_w, aux_bias, wide)
    state, width = 4 * h, 8 * h
    core, aux = 2 * state + width, state + 2 * h
    conv = causal_depthwise4(p[..., :core].transpose(1, 2), leaves[1]).transpose(1, 2)
    q, k, v = conv.split((state, state, width), dim=-1)
    a = p[..., core:core + aux] if bias is None else p[..., core:core + aux] + bias
    out, mT, cT = bayes_mixer_readout(q, k, v, a[..., :state], a[..., state:], p[..., core + aux:], leaves[2],
                                      heads=h)
    outs, grads_in = [out], [gout]
    if gm is not None:
        outs += [mT, cT]
        grads_in += [gm, gc]
    torch.autograd.backward(outs, grads_in)
    torch.cuda.synchronize()
    return out.detach(), mT.detach(), cT.detach(), [x.grad for x in leaves], None if bias is None else bias.grad


@pytest.mark.parametrize("b,t,h,wide,with_bias", [(3, 36, 16, False, True), (2, 64, 32, True, False),
                                                   (1, 8, 16, True, True)])
def test_block_call_matches_its_stages(cuda_device, monkeypatch, b, t, h, wide, with_bias):
    """The one-call block kernels against the same kernels stage by stage: bitwise, gradients of the final
    state included; ``projected`` as a column view of a wider tensor when ``wide``."""
    from bayes_ssm import mixer
    from bayes_ssm.mixer import bayes_mixer_block

    calls = []
    orig = mixer._MixerBlockFunction.apply
    monkeypatch.setattr(mixer._MixerBlockFunction, "apply", staticmethod(lambda *a: calls.append(1) or orig(*a)))
    print(f"block vs stages b={b} t={t} h={h} wide={wide} bias={with_bias}", flush=True)
    projected, weight, norm_w, aux_bias, gout = _inputs(b, t, h, seed=5 + h, device=cuda_device)
    aux_bias = aux_bias if with_bias else None
    g = torch.Generator().manual_seed(6)
    gm = torch.randn(b * h, 4, 8, generator=g).to(cuda_device)
    gc = torch.randn(b * h, 4, 4, generator=g).to(cuda_device)
    leaves, view, bias = _leaves(projected, weight, norm_w, aux_bias, wide)
    assert view.is_contiguous() != wide
    out, mT, cT = bayes_mixer_block(view, leaves[1], leaves[2], heads=h, aux_bias=bias)
    assert calls, "the block kernels were not used"
    torch.autograd.backward([out, mT, cT], [gout, gm, gc])
    torch.cuda.synchronize()
    s_out, s_mT, s_cT, s_grads, s_bias = _staged(projected, weight, norm_w, aux_bias, gout, h, gm, gc, wide)
    assert torch.equal(out, s_out) and torch.equal(mT, s_mT) and torch.equal(cT, s_cT)
    grads = [x.grad for x in leaves]
    assert grads[0].dtype == s_grads[0].dtype and torch.equal(grads[0], s_grads[0]), \
        "grad projected differs from the staged run"
    # The weight and bias gradients: the same partials, summed over the batch in the block's own fold kernel
    # (fixed order) rather than by torch's reduction: at most one bf16 rounding apart.
    for name, a, e in zip(("conv weight", "norm weight"), grads[1:], s_grads[1:]):
        assert a.dtype == e.dtype, name
        torch.testing.assert_close(a.float(), e.float(), rtol=2 ** -7, atol=1e-6, msg=lambda m: f"{name}: {m}")
    if with_bias:
        # Summation order over (B, T) differs from autograd's: one bf16 rounding.
        torch.testing.assert_close(bias.grad.float(), s_bias.float(), rtol=2 ** -7, atol=1e-6)


def test_config4_block_full_shape(cuda_device, monkeypatch):
    from bayes_ssm import mixer

    calls = []
    orig = mixer._MixerBlockFunction.apply
    monkeypatch.setattr(mixer._MixerBlockFunction, "apply", staticmethod(lambda *a: calls.append(1) or orig(*a)))
    print("config4 block full shape", flush=True)
    projected, weight, norm_w, aux_bias, gout = _inputs(B, T, H, seed=4, device=cuda_device)
    out, mT, cT, grads = _run(projected, weight, norm_w, aux_bias, gout, H)
    assert calls, "the block kernels were not used"
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
    assert len(s_grads) == 4 and s_grads[3] is not None
    _bf16_close(s_out, e_out, "out")
    torch.testing.assert_close(s_mT.double().cpu(), e_mT, rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(s_cT.double().cpu(), e_cT, rtol=1e-5, atol=1e-4)
    for name, a, e in zip(("grad projected", "grad conv weight", "grad norm weight", "grad aux bias"), s_grads,
                          e_grads):
        assert a.dtype == torch.bfloat16
        _bf16_close(a, e, name)
