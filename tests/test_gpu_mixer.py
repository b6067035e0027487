"""GPU parity of the producer-fused mixer kernels (C ABI bssm_mixer_*) against the CPU oracle.

The oracle composes the mixer's producer chain and readout permute
(example/train_6layer.py:627-710) with the float64 diagonal recurrence.
Tolerance: 1e-5 relative, 1e-4 absolute for outputs and float32 gradients;
the bfloat16 gradients are the float32 ones rounded to nearest even, bit for
bit; checkpoints are the oracle's boundary beliefs.
"""
from __future__ import annotations

import pytest
import torch

from oracle import bssm_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-4
CHUNK = 8


def close(actual, expected, name="", rtol=RTOL, atol=ATOL):
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    torch.testing.assert_close(actual, expected, rtol=rtol, atol=atol, msg=lambda m: f"{name}: {m}")


def _device_views(views, device):
    """The five column views re-created over one device copy of their fused projection."""
    base = views[0]._base
    assert base is not None and all(x._base is base for x in views)
    dev = base.to(device)
    return [torch.as_strided(dev, x.shape, x.stride(), x.storage_offset()) for x in views]


def _state(n, seed):
    g = torch.Generator().manual_seed(seed)
    m0 = 0.2 * torch.randn(n, 4, 8, generator=g)
    a = torch.randn(n, 4, 4, generator=g)
    c0 = a @ a.transpose(-1, -2) / 4 + 0.5 * torch.eye(4)
    c0 = 0.5 * (c0 + c0.transpose(-1, -2))
    gmf = torch.randn(n, 4, 8, generator=g)
    gcf = torch.randn(n, 4, 4, generator=g)
    return m0, c0, gmf, gcf


def _lds(views):
    return [x.stride(1) for x in views]


def _forward(dv, lds, m0, c0, b, t, h, floor=1e-6):
    from bayes_ssm import _hip

    n = b * h
    nb = -(-t // CHUNK)
    dev = dv[0].device
    read = torch.empty(b, t, h * 8, device=dev)
    mT, cT = torch.empty(n, 4, 8, device=dev), torch.empty(n, 4, 4, device=dev)
    bm, bc = torch.empty(n, nb + 1, 4, 8, device=dev), torch.empty(n, nb + 1, 4, 4, device=dev)
    P = _hip.ptr
    args = []
    for x, ld in zip(dv, lds):
        args += [P(x), ld]
    _hip.call("bssm_mixer_forward", *args, P(m0), P(c0), P(read), P(mT), P(cT), P(bm), P(bc), b, t, h, CHUNK,
              floor, _hip.stream_of(dev))
    return read, mT, cT, bm, bc


def _backward(dv, lds, m0, c0, bm, bc, gy, gmf, gcf, b, t, h, *, f32, dyn=True, initial=True, floor=1e-6):
    from bayes_ssm import _hip

    dev = dv[0].device
    dtype = torch.float32 if f32 else torch.bfloat16
    grads = [torch.empty(x.shape, device=dev, dtype=dtype) if (i < 3 or dyn) else None for i, x in enumerate(dv)]
    gm0 = torch.empty_like(m0) if initial else None
    gc0 = torch.empty_like(c0) if initial else None
    P = _hip.ptr
    args = []
    for x, ld in zip(dv, lds):
        args += [P(x), ld]
    _hip.call("bssm_mixer_backward", *args, P(m0), P(c0), P(bm), P(bc), P(gy), P(gmf), P(gcf),
              *[P(g) for g in grads], P(gm0), P(gc0), b, t, h, CHUNK, floor, int(f32), _hip.stream_of(dev))
    return grads + [gm0, gc0]


CASES = [  # batch, tokens, heads, extra row padding of the fused projection (elements), input scale
    (2, 36, 16, 0, 1.0),
    (1, 64, 32, 8, 1.0),
    (3, 20, 16, 24, 1.0),
    (1, 4, 16, 0, 1.0),
    (2, 100, 48, 16, 1.0),
    (2, 24, 16, 8, 6.0),  # logits beyond +-20: saturated sigmoid/silu, softplus threshold
]


@pytest.mark.parametrize("b,t,h,pad,scale", CASES)
def test_mixer_abi_matches_oracle(cuda_device, b, t, h, pad, scale):
    print(f"mixer abi b={b} t={t} h={h} pad={pad} scale={scale}", flush=True)
    views, g_read = O.make_mixer_inputs(b, t, h, seed=900 + t, ld_pad=pad, scale=scale)
    n = b * h
    m0, c0, gmf, gcf = _state(n, seed=t)
    dv = _device_views(views, cuda_device)
    lds = _lds(views)
    assert lds[0] == 22 * h + pad
    d = {name: x.to(cuda_device) for name, x in dict(m0=m0, c0=c0, gmf=gmf, gcf=gcf, gy=g_read).items()}

    read, mT, cT, bm, bc = _forward(dv, lds, d["m0"], d["c0"], b, t, h)
    g32 = _backward(dv, lds, d["m0"], d["c0"], bm, bc, d["gy"], d["gmf"], d["gcf"], b, t, h, f32=True)
    g16 = _backward(dv, lds, d["m0"], d["c0"], bm, bc, d["gy"], d["gmf"], d["gcf"], b, t, h, f32=False)
    lean = _backward(dv, lds, d["m0"], d["c0"], bm, bc, d["gy"], None, None, b, t, h, f32=True, dyn=False,
                     initial=False)
    torch.cuda.synchronize()

    e_read, e_mT, e_cT, e_grads = O.mixer_grads(*views, h, m0, c0, g_read, gmf, gcf)
    close(read.view(b, t, h, 8), e_read, "read")
    close(mT, e_mT, "mean_T")
    close(cT, e_cT, "cov_T")
    inputs = O.mixer_inputs(*views, h)
    e_bm, e_bc = O.checkpoints(*inputs, m0.double(), c0.double(), CHUNK, 1e-6)
    close(bm, e_bm, "bmean")
    close(bc, e_bc, "bcov")
    names = ["g_q", "g_k", "g_v", "g_decay_logits", "g_noise", "g_mean0", "g_cov0"]
    for name, a, e in zip(names, g32, e_grads):
        close(a, e, name)
    for name, a, e in zip(names[:5], g16[:5], g32[:5]):
        assert a.dtype == torch.bfloat16
        assert torch.equal(a, e.bfloat16()), f"{name} (bf16) is not the float32 gradient rounded"
    for name, a, e in zip(names[5:], g16[5:], g32[5:]):
        assert torch.equal(a, e), name
    # Without final-state gradients and dynamics gradients: the readout-only
    # loss's q/k/v gradients.
    _, _, _, e_lean = O.mixer_grads(*views, h, m0, c0, g_read)
    for name, a, e in zip(names[:3], lean[:3], e_lean[:3]):
        close(a, e, f"lean {name}")


def test_mixer_matches_reference_float32_chain(cuda_device):
    """Same readout as the reference's own op chain run in float32 on the CPU (bayesian_layer, optimized=False)."""
    import bayes_ssm

    from bayes_ssm.mixer import bayes_mixer_core, mixer_layer_inputs

    b, t, h = 2, 48, 16
    views, _ = O.make_mixer_inputs(b, t, h, seed=31)
    dv = _device_views(views, cuda_device)
    read, mT, cT = bayes_mixer_core(*dv, heads=h)
    k, v, q, dec, p, r = mixer_layer_inputs(*views, h)
    ry, rm, rc = bayes_ssm.bayesian_layer(k, v, q, transition_diagonals=dec, process_variances=p,
                                          observation_variances=r, chunk_length=16, optimized=False)
    close(read, ry.view(b, h, t, 8).permute(0, 2, 1, 3), "read vs reference float32 path")
    close(mT, rm, "mean_T")
    close(cT, rc, "cov_T")


@pytest.mark.parametrize("leaves", ["all", "qkv"])
def test_mixer_autograd_boundary(cuda_device, monkeypatch, leaves):
    """bayes_mixer_core on bf16 column views runs the fused kernels; its gradients are the C ABI's."""
    from bayes_ssm import mixer

    calls = []
    orig = mixer._MixerCoreFunction.apply
    monkeypatch.setattr(mixer._MixerCoreFunction, "apply", staticmethod(lambda *a: calls.append(1) or orig(*a)))
    b, t, h = 2, 40, 32
    views, g_read = O.make_mixer_inputs(b, t, h, seed=77, ld_pad=8)
    base = views[0]._base.to(cuda_device)
    dv = [torch.as_strided(base, x.shape, x.stride(), x.storage_offset()) for x in views]
    # Leaves: the column views of one fused projection (gradients accumulate into it).
    leaf_views = [x.detach().requires_grad_(leaves == "all" or i < 3) for i, x in enumerate(dv)]
    m0 = torch.zeros(b * h, 4, 8, device=cuda_device, requires_grad=True)
    read, mT, cT = mixer.bayes_mixer_core(*leaf_views, heads=h, initial_mean=m0)
    assert calls, "fused mixer kernels were not used"
    gy = g_read.to(cuda_device)
    torch.autograd.backward([read], [gy])

    lds = _lds(views)
    c0 = torch.eye(4, device=cuda_device).expand(b * h, 4, 4).contiguous()
    r2, m2, c2, bm, bc = _forward(dv, lds, m0.detach(), c0, b, t, h)
    g32 = _backward([x.detach() for x in dv], lds, m0.detach(), c0, bm, bc, gy, None, None, b, t, h, f32=True)
    torch.cuda.synchronize()
    assert torch.equal(read.view(b, t, h * 8), r2)
    assert torch.equal(mT, m2) and torch.equal(cT, c2)
    for i, x in enumerate(leaf_views):
        if x.requires_grad:
            assert x.grad.dtype == torch.bfloat16
            assert torch.equal(x.grad, g32[i].bfloat16()), f"grad of projection {i}"
        else:
            assert x.grad is None
    assert torch.equal(m0.grad, g32[5])


def test_mixer_unsupported_shapes_take_the_op_chain(cuda_device):
    """Heads not a multiple of 16 or T not a multiple of 4: the reference op chain + bayesian_layer."""
    from bayes_ssm import mixer

    for b, t, h in ((1, 24, 8), (2, 30, 16)):
        views, _ = O.make_mixer_inputs(b, t, h, seed=5)
        dv = _device_views(views, cuda_device)
        assert mixer._fused_eligible(tuple(dv), h) is None
        read, mT, cT = mixer.bayes_mixer_core(*dv, heads=h)
        e_read, e_mT, e_cT = O.mixer_core(*views, h)
        close(read, e_read, f"read b={b} t={t} h={h}")
        close(mT, e_mT, "mean_T")
        close(cT, e_cT, "cov_T")


# ------------------------------------------------------- gated readout epilogue
EPS32 = torch.finfo(torch.float32).eps


def _gate_inputs(b, t, h, seed, gate_pad):
    g = torch.Generator().manual_seed(seed)
    gate_full = torch.randn(b, t, h * 8 + gate_pad, generator=g).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(8, generator=g)).to(torch.bfloat16).float()
    gout = torch.randn(b, t, h * 8, generator=g).to(torch.bfloat16)
    return gate_full[..., : h * 8], w, gout


def _gated_forward(dv, lds, gate, w, m0, c0, b, t, h, precise, floor=1e-6):
    from bayes_ssm import _hip

    n, nb, dev = b * h, -(-t // CHUNK), dv[0].device
    out = torch.empty(b, t, h * 8, device=dev, dtype=torch.float32 if precise else torch.bfloat16)
    yb = torch.empty(b, t, h * 8, device=dev, dtype=torch.bfloat16)
    mT, cT = torch.empty(n, 4, 8, device=dev), torch.empty(n, 4, 4, device=dev)
    bm, bc = torch.empty(n, nb + 1, 4, 8, device=dev), torch.empty(n, nb + 1, 4, 4, device=dev)
    P = _hip.ptr
    args = []
    for x, ld in zip(dv, lds):
        args += [P(x), ld]
    _hip.call("bssm_mixer_gated_forward", *args, P(gate), gate.stride(1), P(w), EPS32, P(m0), P(c0), P(out), P(yb),
              P(mT), P(cT), P(bm), P(bc), b, t, h, CHUNK, floor, int(precise), _hip.stream_of(dev))
    return out, yb, mT, cT, bm, bc


def _gated_backward(dv, lds, gate, w, m0, c0, bm, bc, yb, gout, gmf, gcf, b, t, h, precise, floor=1e-6):
    from bayes_ssm import _hip

    dev = dv[0].device
    dtype = torch.float32 if precise else torch.bfloat16
    grads = [torch.empty(x.shape, device=dev, dtype=dtype) for x in dv]
    ggate = torch.empty(b, t, h * 8, device=dev, dtype=dtype)
    part = torch.empty(b * h // 16, 8, device=dev)
    gm0, gc0 = torch.empty_like(m0), torch.empty_like(c0)
    P = _hip.ptr
    args = []
    for x, ld in zip(dv, lds):
        args += [P(x), ld]
    _hip.call("bssm_mixer_gated_backward", *args, P(gate), gate.stride(1), P(w), EPS32, P(m0), P(c0), P(bm), P(bc),
              P(yb), P(gout), P(gmf), P(gcf), *[P(g) for g in grads], P(ggate), P(part), P(gm0), P(gc0), b, t, h,
              CHUNK, floor, int(precise), _hip.stream_of(dev))
    return grads + [ggate, part, gm0, gc0]


GATED_CASES = [  # batch, tokens, heads, projection row padding, gate row padding
    (2, 36, 16, 0, 0),
    (1, 4, 16, 8, 8),
    (2, 100, 32, 16, 24),
]


@pytest.mark.parametrize("b,t,h,pad,gpad", GATED_CASES)
def test_mixer_gated_abi_matches_oracle(cuda_device, b, t, h, pad, gpad):
    print(f"mixer gated b={b} t={t} h={h} pad={pad} gpad={gpad}", flush=True)
    views, _ = O.make_mixer_inputs(b, t, h, seed=1300 + t, ld_pad=pad)
    gate, w, gout = _gate_inputs(b, t, h, seed=t, gate_pad=gpad)
    n = b * h
    m0, c0, gmf, gcf = _state(n, seed=t + 1)
    dv = _device_views(views, cuda_device)
    lds = _lds(views)
    gate_d = _device_views([gate], cuda_device)[0] if gpad else gate.to(cuda_device)
    d = {k: x.to(cuda_device) for k, x in dict(m0=m0, c0=c0, gmf=gmf, gcf=gcf, w=w, gout=gout).items()}

    o32, yb, mT, cT, bm, bc = _gated_forward(dv, lds, gate_d, d["w"], d["m0"], d["c0"], b, t, h, True)
    o16, yb2, *_ = _gated_forward(dv, lds, gate_d, d["w"], d["m0"], d["c0"], b, t, h, False)
    g32 = _gated_backward(dv, lds, gate_d, d["w"], d["m0"], d["c0"], bm, bc, yb, d["gout"], d["gmf"], d["gcf"],
                          b, t, h, True)
    g16 = _gated_backward(dv, lds, gate_d, d["w"], d["m0"], d["c0"], bm, bc, yb, d["gout"], d["gmf"], d["gcf"],
                          b, t, h, False)
    torch.cuda.synchronize()

    # Forward: bf16(read) within rounding of the oracle's read; the epilogue on those values.
    leaves = [x.detach().double().requires_grad_(True) for x in (*views, gate, w, m0, c0)]
    read, e_mT, e_cT = O.mixer_core(*leaves[:5], h, leaves[7], leaves[8])
    e_out = O.mixer_readout(read, leaves[5], leaves[6], EPS32, read_bf16=yb.cpu())
    close(yb.view(b, t, h, 8), read, "read_bf16", rtol=2 ** -8, atol=1e-6)
    close(o32, e_out, "out")
    # Not conditioned on the kernel: the oracle's own bf16 rounding of its read.  Heads whose 8 rounded values
    # agree with the kernel's (all but those where a value sits within float32 noise, about 1e-6 relative, of a
    # bf16 tie: a few per thousand heads) must give the oracle's out at the float32 tolerance; the rest within
    # the bf16 step of one rounding flip.
    own = O.mixer_readout(read, leaves[5], leaves[6], EPS32).detach()
    same = (read.detach().to(torch.bfloat16) == yb.cpu().view(b, t, h, 8)).all(-1)
    flips = int((~same).sum())
    assert flips <= max(2, same.numel() // 50), f"bf16(read) disagrees with the oracle's rounding on {flips} heads"
    sel = same.unsqueeze(-1).expand(b, t, h, 8).reshape(b, t, h * 8)
    close(o32.cpu()[sel], own[sel], "out vs the oracle's own rounding (heads that round alike)")
    close(o32.cpu()[~sel], own[~sel], "out vs the oracle's own rounding (rounding flips)", rtol=2 ** -6, atol=2 ** -6)
    close(mT, e_mT, "mean_T")
    close(cT, e_cT, "cov_T")
    assert torch.equal(yb, yb2)
    assert torch.equal(o16, o32.bfloat16()), "bf16 out is not the float32 product rounded"

    # Backward: every gradient against autograd through the oracle.
    loss = (e_out * gout.double()).sum() + (e_mT * gmf.double()).sum() + (e_cT * gcf.double()).sum()
    e_grads = torch.autograd.grad(loss, leaves)
    names = ["g_q", "g_k", "g_v", "g_decay_logits", "g_noise", "g_gate"]
    for name, a, e in zip(names, g32[:6], e_grads[:6]):
        close(a, e, name)
    close(g32[6].sum(0), e_grads[6], "g_norm_weight")
    close(g32[7], e_grads[7], "g_mean0")
    close(g32[8], e_grads[8], "g_cov0")
    for name, a, e in zip(names, g16[:6], g32[:6]):
        assert a.dtype == torch.bfloat16
        assert torch.equal(a, e.bfloat16()), f"{name} (bf16) is not the float32 gradient rounded"
    for a, e in zip(g16[6:], g32[6:]):
        assert torch.equal(a, e)


def test_mixer_readout_autograd_boundary(cuda_device, monkeypatch):
    """bayes_mixer_readout on bf16 inputs runs the gated kernels; results and gradients are the C ABI's."""
    from bayes_ssm import mixer

    calls = []
    orig = mixer._MixerReadoutFunction.apply
    monkeypatch.setattr(mixer._MixerReadoutFunction, "apply", staticmethod(lambda *a: calls.append(1) or orig(*a)))
    b, t, h = 2, 40, 16
    views, _ = O.make_mixer_inputs(b, t, h, seed=41, ld_pad=8)
    gate, w, gout = _gate_inputs(b, t, h, seed=42, gate_pad=0)
    dv = _device_views(views, cuda_device)
    leaves = [x.detach().requires_grad_(True) for x in dv]
    gate_l = gate.to(cuda_device).requires_grad_(True)
    w_l = w.to(cuda_device).to(torch.bfloat16).requires_grad_(True)
    out, mT, cT = mixer.bayes_mixer_readout(*leaves, gate_l, w_l, heads=h)
    assert calls, "gated kernels were not used"
    gout_d = gout.to(cuda_device)
    torch.autograd.backward([out], [gout_d])

    lds = _lds(views)
    m0 = torch.zeros(b * h, 4, 8, device=cuda_device)
    c0 = torch.eye(4, device=cuda_device).expand(b * h, 4, 4).contiguous()
    w32 = w_l.detach().float()
    o16, yb, m2, c2, bm, bc = _gated_forward(dv, lds, gate_l.detach(), w32, m0, c0, b, t, h, False)
    g16 = _gated_backward([x.detach() for x in dv], lds, gate_l.detach(), w32, m0, c0, bm, bc, yb, gout_d, None,
                          None, b, t, h, False)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and torch.equal(out, o16)
    assert torch.equal(mT, m2) and torch.equal(cT, c2)
    for i, x in enumerate(leaves):
        assert torch.equal(x.grad, g16[i]), f"grad of projection {i}"
    assert torch.equal(gate_l.grad, g16[5])
    assert w_l.grad.dtype == torch.bfloat16
    assert torch.equal(w_l.grad, g16[6].sum(0).bfloat16())


def test_mixer_readout_fallback_matches_oracle(cuda_device):
    """Heads not a multiple of 16: the op chain (torch rms_norm and silu in bf16) within bf16 rounding."""
    from bayes_ssm import mixer

    b, t, h = 2, 20, 8
    views, _ = O.make_mixer_inputs(b, t, h, seed=12)
    gate, w, _ = _gate_inputs(b, t, h, seed=13, gate_pad=0)
    dv = _device_views(views, cuda_device)
    out, _, _ = mixer.bayes_mixer_readout(*dv, gate.to(cuda_device), w.to(cuda_device).bfloat16(), heads=h)
    read, _, _ = O.mixer_core(*views, h)
    close(out, O.mixer_readout(read, gate, w), "out", rtol=3 * 2 ** -8, atol=1e-3)


# ------------------------------------------------- the benchmarked shape (H64 x T512)
def _rows_views(views, rows):
    """The five column views over a copy of just `rows` of their fused projection."""
    base = views[0]._base[rows].contiguous()
    return [torch.as_strided(base, (len(rows), *x.shape[1:]), x.stride(), x.storage_offset()) for x in views]


def test_mixer_config3_shape_rows_match_subset_and_oracle(cuda_device):
    """The core and the gated readout at B256 x T512 x H64: batch rows are independent, so the full-shape
    rows equal a run on just those rows bit for bit, and that run matches the float64 oracle (1e-5 / 1e-4)."""
    b, t, h = 256, 512, 64
    rows = [0, 129, 255]
    print("mixer config3 shape", flush=True)
    views, g_read = O.make_mixer_inputs(b, t, h, seed=4242)
    gate, w, gout = _gate_inputs(b, t, h, seed=4243, gate_pad=0)
    n = b * h
    m0 = torch.zeros(n, 4, 8)
    c0 = torch.eye(4).expand(n, 4, 4).contiguous()
    dv = _device_views(views, cuda_device)
    lds = _lds(views)
    d = {k: x.to(cuda_device) for k, x in dict(m0=m0, c0=c0, gy=g_read, gate=gate, w=w, gout=gout).items()}
    read, mT, cT, bm, bc = _forward(dv, lds, d["m0"], d["c0"], b, t, h)
    g32 = _backward(dv, lds, d["m0"], d["c0"], bm, bc, d["gy"], None, None, b, t, h, f32=True)
    o32, yb, _, _, gbm, gbc = _gated_forward(dv, lds, d["gate"], d["w"], d["m0"], d["c0"], b, t, h, True)
    gg = _gated_backward(dv, lds, d["gate"], d["w"], d["m0"], d["c0"], gbm, gbc, yb, d["gout"], None, None, b, t, h,
                         True)
    torch.cuda.synchronize()
    assert torch.isfinite(read).all() and torch.isfinite(g32[0]).all()

    print("mixer config3 shape: subset rows", flush=True)
    ri = torch.tensor(rows)
    seqs = (ri[:, None] * h + torch.arange(h)).flatten()
    sv = _rows_views(views, ri)
    sdv = _device_views(sv, cuda_device)
    bs = len(rows)
    sd = {k: x.to(cuda_device) for k, x in dict(m0=m0[seqs], c0=c0[seqs], gy=g_read[ri], gate=gate[ri],
                                                gout=gout[ri]).items()}
    s_read, s_mT, s_cT, s_bm, s_bc = _forward(sdv, lds, sd["m0"], sd["c0"], bs, t, h)
    s_g32 = _backward(sdv, lds, sd["m0"], sd["c0"], s_bm, s_bc, sd["gy"], None, None, bs, t, h, f32=True)
    s_o32, s_yb, _, _, s_gbm, s_gbc = _gated_forward(sdv, lds, sd["gate"], d["w"], sd["m0"], sd["c0"], bs, t, h,
                                                     True)
    s_gg = _gated_backward(sdv, lds, sd["gate"], d["w"], sd["m0"], sd["c0"], s_gbm, s_gbc, s_yb, sd["gout"], None,
                           None, bs, t, h, True)
    torch.cuda.synchronize()
    rd = ri.to(cuda_device)
    sq = seqs.to(cuda_device)
    assert torch.equal(s_read, read[rd]) and torch.equal(s_mT, mT[sq]) and torch.equal(s_cT, cT[sq])
    for i in range(5):
        assert torch.equal(s_g32[i], g32[i][rd]), f"core gradient {i}"
    assert torch.equal(s_o32, o32[rd]) and torch.equal(s_yb, yb[rd])
    for i in range(6):
        assert torch.equal(s_gg[i], gg[i][rd]), f"gated gradient {i}"

    # The subset run against the oracle.
    e_read, e_mT, e_cT, e_grads = O.mixer_grads(*sv, h, m0[seqs], c0[seqs], g_read[ri])
    close(s_read.view(bs, t, h, 8), e_read, "read")
    close(s_mT, e_mT, "mean_T")
    close(s_cT, e_cT, "cov_T")
    names = ["g_q", "g_k", "g_v", "g_decay_logits", "g_noise"]
    for name, a, e in zip(names, s_g32, e_grads):
        close(a, e, name)
    leaves = [x.detach().double().requires_grad_(True) for x in (*sv, gate[ri], w)]
    e_r2, _, _ = O.mixer_core(*leaves[:5], h, m0[seqs].double(), c0[seqs].double())
    e_out = O.mixer_readout(e_r2, leaves[5], leaves[6], EPS32, read_bf16=s_yb.cpu())
    close(s_yb.view(bs, t, h, 8), e_r2, "read_bf16", rtol=2 ** -8, atol=1e-6)
    close(s_o32, e_out, "out")
    eg = torch.autograd.grad((e_out * gout[ri].double()).sum(), leaves)
    for name, a, e in zip(names + ["g_gate"], s_gg[:6], eg[:6]):
        close(a, e, "gated " + name)
    close(s_gg[6].sum(0), eg[6], "gated g_norm_weight")
