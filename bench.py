#!/usr/bin/env python3
"""Bayes-layer fwd+bwd throughput on one MI355X (BASELINE.json metric).

Workload (config 3): B=256, T=512, H=64 heads -> N = B*H = 16384 sequences,
D=4 key dims, M=8 value columns, chunk length 64, fp32 state.  Inputs are
synthetic (seeded): k, v, q ~ N(0,1) rounded through bf16, decay =
sigmoid(N(2,1)), process = softplus(N(-3,1)), observation = 1e-4 +
softplus(N(0,1)); all six require grad (full 8-gradient ABI), gy ~ N(0,1).

One step = the fused forward plus the full backward of
``bayes_ssm.fused_cuda.fused_diagonal_bayesian`` (inputs resident in HBM).
Prints one JSON line.  ``--gpus`` above 1 is rejected: this build measures
one GPU (sequences are independent, so a multi-GPU run would shard them
with no exchange between GPUs).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "bayes-ssm_amd"))
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

METRIC = "Bayes-layer fwd+bwd tokens/s at B256×T512×H64 D4M8; % HBM roofline"
HBM_PEAK = 8.0e12  # MI355X spec peak, bytes/s
FP32_PEAK = 157.3e12  # MI355X spec peak of fp32 vector arithmetic, flop/s


def algorithmic_bytes(d: int, m: int) -> tuple[int, int]:
    """(forward, backward) bytes per (sequence, token) at the fp32 ABI.

    forward reads k, q, d (D each), v (M), p, r and writes y (M);
    backward reads the same inputs plus gy (M) and writes their 3D+M+2 gradients.
    """
    inputs = 3 * d + m + 2
    return (inputs + m) * 4, (2 * inputs + m) * 4


def dense_flops(d: int, m: int) -> tuple[int, int]:
    """(forward, backward) arithmetic per (sequence, token) of the dense-covariance recurrence, counting a fused
    multiply-add as two operations.

    forward: wk = d k (D), z = P wk (2 D^2), u = d z + p k (3 D), s = k.u (2 D), e = v - M^T wk (2 D M),
    M <- d M + u (beta e)^T (3 D M), P <- P d d^T - beta u u^T (4 D^2), y = M^T q (2 D M);
    backward: the replay (the forward without y) plus the reverse: 16 D M for the mean adjoint, the row sums of
    dL/dq, dL/dk, dL/dd and a = gM e, and 14 D^2 for S u, P' gu, sym(gu k^T), the decay term and S d d^T.
    """
    fwd = d + 2 * d * d + 3 * d + 2 * d + 2 * d * m + 3 * d * m + 4 * d * d + 2 * d * m
    return fwd, (fwd - 2 * d * m) + 16 * d * m + 14 * d * d


def dispatched_kernels(d: int, m: int, n: int, t: int, interval: int) -> tuple[str, str]:
    """Names of the forward and backward kernels the C ABI launches for float32 streams of this shape
    (D4M8: the row-per-sequence kernels up to the library's small-batch limits, else the rotated layout)."""
    from bayes_ssm import _hip

    if (d, m) != (4, 8) or t % 4:
        return f"bssm forward kernel (D{d}M{m})", f"bssm backward kernel (D{d}M{m})"
    lib = _hip.load()
    lim = [lib.bssm_small_batch_limit(k, -1) for k in range(4)]
    groups = 2 if n > 4 * 256 else 1  # 4-sequence groups per workgroup of the split kernels
    if n <= lim[2]:
        fwd = f"bssm::sn::forward_split_kernel<false, 0, {groups}> (row layout, two waves per 4 sequences)"
    elif n <= lim[0]:
        fwd = "bssm::sn::forward_kernel<false, 0> (row layout, 16 lanes per sequence)"
    else:
        fwd = "bssm::r4::forward_kernel<false, 0> (rotated layout, 4 lanes per sequence)"
    row_bwd = t % 16 == 0 and interval == _hip.preferred_checkpoint(4)
    if row_bwd and n <= lim[3]:
        bwd = f"bssm::sn::backward_split_kernel<false, true, 0, {groups}> (row layout, three waves per 4 sequences)"
    elif row_bwd and n <= lim[1]:
        bwd = "bssm::sn::backward_kernel<false, true> (row layout, 16 lanes per sequence)"
    else:
        bwd = (f"bssm::r4::backward_tile_kernel<false, true, 0, {interval}> (rotated layout, 4 lanes per sequence, "
               "16-token tiles)")
    return fwd, bwd


def make_workload(b, t, h, d, m, device, seed=0, kqv_dtype=None):
    """Synthetic config-3 inputs; k, v, q are bf16 values (kept as tensors of kqv_dtype when given:
    bfloat16, or a float8 dtype, rounded from the bf16 values)."""
    n = b * h
    g = torch.Generator(device=device).manual_seed(seed)
    cast = (lambda x: x.bfloat16().to(kqv_dtype)) if kqv_dtype is not None else (lambda x: x.bfloat16().float())
    k = cast(torch.randn(n, t, d, device=device, generator=g))
    v = cast(torch.randn(n, t, m, device=device, generator=g))
    q = cast(torch.randn(n, t, d, device=device, generator=g))
    dec = torch.sigmoid(torch.randn(n, t, d, device=device, generator=g) + 2.0)
    p = torch.nn.functional.softplus(torch.randn(n, t, device=device, generator=g) - 3.0)
    r = 1e-4 + torch.nn.functional.softplus(torch.randn(n, t, device=device, generator=g))
    gy = torch.randn(n, t, m, device=device, generator=g)
    leaves = [x.requires_grad_(True) for x in (k, v, q, dec, p, r)]
    m0 = torch.zeros(n, d, m, device=device)
    c0 = torch.eye(d, device=device).expand(n, d, d).contiguous()
    return leaves, m0, c0, gy


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def _settle(step, warmup: int, min_ms: float = 40.0) -> float:
    """Warm-up calls of a secondary workload's step: at least `warmup`, and after the first call (whose host
    work, new shapes and new allocations can leave the device idle for over 10 ms) enough back-to-back calls to
    keep the device busy for `min_ms`.  An idle of 10 ms or more sends the next ~20 steps through a
    power-management dip of up to 25 %; the timed calls then start at the sustained rate.  Returns the wall
    time of one synchronized call (seconds)."""
    step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step()
    torch.cuda.synchronize()
    per = time.perf_counter() - t0
    for _ in range(max(warmup, int(min_ms * 1e-3 / max(per, 1e-5)) + 1)):
        step()
    torch.cuda.synchronize()
    return per


def time_layer(b, t, h, d, m, chunk, steps, warmup, device, kqv_dtype=None) -> dict:
    """fwd+bwd of fused_diagonal_bayesian at one shape: ms/step, tokens/s, step roofline fraction.

    With kqv_dtype (bfloat16 or a float8 dtype) the keys, values and queries
    are tensors of that dtype (read as such by the kernels; their gradients
    have it too) and the roofline bytes count the dtypes actually streamed.
    """
    from bayes_ssm import fused_cuda

    leaves, m0, c0, gy = make_workload(b, t, h, d, m, device, seed=1, kqv_dtype=kqv_dtype)

    def step():
        y, _, _ = fused_cuda.fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=chunk, denominator_floor=1e-6)
        return torch.autograd.grad(y, leaves, gy)

    per = _settle(step, warmup)
    # At least ~20 ms of timed steps, so that short steps are not dominated by
    # the host's latency to the first launch.
    steps = max(steps, int(20e-3 / max(per, 1e-5)) + 1)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # Device time of each kernel: each step's forward and backward queued
    # behind a device-side delay, so the events around them bracket the
    # kernels, not the host's launch latency (a separate pass: events inside
    # the timed loop would add host work to steps this short).
    fwd_t, bwd_t = [], []
    for _ in range(8):
        mk = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        torch.cuda._sleep(1_000_000)
        mk[0].record()
        y, _, _ = fused_cuda.fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=chunk, denominator_floor=1e-6)
        mk[1].record()
        torch.autograd.grad(y, leaves, gy)
        mk[2].record()
        torch.cuda.synchronize()
        fwd_t.append(mk[0].elapsed_time(mk[1]))
        bwd_t.append(mk[1].elapsed_time(mk[2]))
    fwd_ms = sorted(fwd_t)[4]
    bwd_ms = sorted(bwd_t)[4]
    fwd_b, bwd_b = algorithmic_bytes(d, m)
    if kqv_dtype is not None:
        # k, q, v (2D + M values) read at the narrow width in both passes and
        # their gradients written at it: 3 (2D + M) x (4 - width) bytes fewer.
        saved = 4 - torch.empty(0, dtype=kqv_dtype).element_size()
        fwd_b -= (2 * d + m) * saved
        bwd_b -= (2 * d + m) * 2 * saved
    out = {"B": b, "T": t, "H": h, "D": d, "M": m, "ms_per_step": ms, "tokens_per_s": b * t / (ms * 1e-3),
           "roofline_step_frac": (fwd_b + bwd_b) * b * h * t / (ms * 1e-3) / HBM_PEAK, "steps": steps,
           "forward_kernel_ms": fwd_ms, "backward_kernel_ms": bwd_ms,
           "forward_roofline_frac": fwd_b * b * h * t / (fwd_ms * 1e-3) / HBM_PEAK,
           "backward_roofline_frac": bwd_b * b * h * t / (bwd_ms * 1e-3) / HBM_PEAK}
    if kqv_dtype is not None:
        out["kqv_dtype"] = str(kqv_dtype).replace("torch.", "")
        out["bytes_per_token_head"] = fwd_b + bwd_b
    return out


class _NoopCore(torch.autograd.Function):
    """The fused function's autograd shape without its work: same inputs, outputs and saved tensors, no launch."""

    @staticmethod
    def forward(ctx, k, v, q, dec, p, r, m0, c0):
        n, t, d = k.shape
        m = v.shape[2]
        out = torch.empty(n, t, m, device=k.device)
        mf, cf = torch.empty_like(m0), torch.empty_like(c0)
        ctx.save_for_backward(k, v, q, dec, p, r, m0, c0, out, out)
        ctx.set_materialize_grads(False)
        return out, mf, cf

    @staticmethod
    def backward(ctx, gy, gm, gc):
        return tuple(torch.empty_like(x) for x in ctx.saved_tensors[:8])


def host_costs(b, t, h, d, m, chunk, device) -> dict:
    """Host wall time of one fwd+bwd call with the device kept busy (no waits inside): the fused function, and
    ``_NoopCore`` (torch's autograd machinery alone for the same inputs and outputs)."""
    from bayes_ssm import fused_cuda

    leaves, m0, c0, gy = make_workload(b, t, h, d, m, device, seed=1)
    leaves8 = [*leaves, m0.requires_grad_(True), c0.requires_grad_(True)]

    def fused():
        y, _, _ = fused_cuda.fused_diagonal_bayesian(*leaves8, chunk_length=chunk, denominator_floor=1e-6)
        torch.autograd.grad(y, leaves8, gy)

    def noop():
        y, _, _ = _NoopCore.apply(*leaves8)
        torch.autograd.grad(y, leaves8, gy)

    res = {}
    for name, fn in (("fused_host_ms", fused), ("autograd_noop_host_ms", noop)):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(41):
            torch.cuda._sleep(2_000_000)
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
            torch.cuda.synchronize()
        res[name] = sorted(ts)[20] * 1e3
    return res


def time_layer_graphed(b, t, h, d, m, chunk, steps, device) -> dict:
    """fwd+bwd of fused_diagonal_bayesian captured once in a HIP graph (torch.cuda.graph) and replayed.

    The same kernels on the same inputs as ``time_layer``, without the
    per-call host work (Python, torch's autograd engine, the launch calls):
    the rate at which the device runs the step.
    """
    from bayes_ssm import fused_cuda

    leaves, m0, c0, gy = make_workload(b, t, h, d, m, device, seed=1)

    def step():
        y, _, _ = fused_cuda.fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=chunk, denominator_floor=1e-6)
        return torch.autograd.grad(y, leaves, gy)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    per = _settle(graph.replay, 3)
    steps = max(steps, int(20e-3 / max(per, 1e-5)) + 1)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del graph
    fwd_b, bwd_b = algorithmic_bytes(d, m)
    return {"B": b, "T": t, "H": h, "D": d, "M": m, "ms_per_step": ms, "tokens_per_s": b * t / (ms * 1e-3),
            "roofline_step_frac": (fwd_b + bwd_b) * b * h * t / (ms * 1e-3) / HBM_PEAK, "steps": steps,
            "path": "forward + autograd.grad captured in one torch.cuda.graph, replayed"}


MIXER_FWD_BYTES = 2 * 22 + 4 * 8   # bf16 q, k, decay (4 each), v (8), noise (2) in; float32 read out
MIXER_BWD_BYTES = 2 * 22 + 4 * 8 + 2 * 22  # projections and read gradient in; bf16 projection gradients out


def time_mixer(b, t, h, steps, warmup, device, fused=True, gated=False) -> dict:
    """fwd+bwd of the Bayes mixer's layer core from its bf16 projections (train_6layer.py:627-710).

    fused: ``bayes_mixer_core`` (the producer-fused kernels).  Otherwise the
    reference's op chain on the same GPU: the float32 transforms and permutes
    (``mixer_layer_inputs``), ``bayesian_layer`` on the float32 layer kernels,
    and the readout permute.  The five projections are separate bf16 leaves.
    gated: up to the input of out_proj (:719-729): the readout's RMSNorm and
    SiLU gate as well (``bayes_mixer_readout``, or torch's rms_norm and silu
    on bf16 after the op chain); the gate and the norm weight are leaves too.
    """
    import bayes_ssm
    import torch.nn.functional as F
    from bayes_ssm.mixer import bayes_mixer_core, bayes_mixer_readout, mixer_layer_inputs

    gen = torch.Generator(device=device).manual_seed(3)
    shift = {3: 2.0, 4: 0.0}
    leaves = []
    for i, w in enumerate((4, 4, 8, 4, 2)):
        x = torch.randn(b, t, h * w, device=device, generator=gen) + shift.get(i, 0.0)
        if i == 4:
            x[..., 0::2] -= 3.0
        leaves.append(x.to(torch.bfloat16).requires_grad_(True))
    gy = torch.randn(b, t, h, 8, device=device, generator=gen)
    if gated:
        gate = torch.randn(b, t, h * 8, device=device, generator=gen).to(torch.bfloat16).requires_grad_(True)
        norm_w = torch.ones(8, device=device, dtype=torch.bfloat16, requires_grad=True)
        gy = gy.view(b, t, h * 8).to(torch.bfloat16)
        leaves = leaves + [gate, norm_w]

    def step():
        if fused and gated:
            out, _, _ = bayes_mixer_readout(*leaves[:5], gate, norm_w, heads=h)
        elif fused:
            out, _, _ = bayes_mixer_core(*leaves, heads=h)
        else:
            k, v, q, dec, p, r = mixer_layer_inputs(*leaves[:5], h)
            y, _, _ = bayes_ssm.bayesian_layer(k, v, q, transition_diagonals=dec, process_variances=p,
                                               observation_variances=r, chunk_length=64, optimized=True)
            out = y.view(b, h, t, 8).permute(0, 2, 1, 3)
            if gated:
                out = F.rms_norm(out.to(torch.bfloat16), (8,), norm_w, None)
                out = (out * F.silu(gate.view(b, t, h, 8))).reshape(b, t, h * 8)
        return torch.autograd.grad(out, leaves, gy)

    _settle(step, warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    out = {"B": b, "T": t, "H": h, "D": 4, "M": 8, "ms_per_step": ms, "tokens_per_s": b * t / (ms * 1e-3),
           "path": ("producer-fused kernels" if fused else "reference op chain + float32 layer kernels")
           + (", gated readout epilogue" if gated else "")}
    if fused and not gated:
        per = MIXER_FWD_BYTES + MIXER_BWD_BYTES
        out["bytes_per_token_head"] = per
        out["roofline_step_frac"] = per * b * h * t / (ms * 1e-3) / HBM_PEAK
    return out


BLOCK_FWD_BYTES = 2 * 30 + 2 * 8           # bf16 fused projection in (30 per head), bf16 gated readout out
BLOCK_BWD_BYTES = 2 * 30 + 2 * 8 + 2 * 30  # projection and readout gradient in; projection gradient out


def time_block(b, t, h, steps, warmup, device) -> dict:
    """fwd+bwd of config 4's Bayes block (``bayes_mixer_block``, train_6layer.py:583-729): the causal depthwise-4
    filter, the producer-fused layer core and the gated readout, from the fused bf16 projection to out_proj's
    input, with the gradients of the projection, the filter and norm weights and the aux bias."""
    from bayes_ssm.mixer import bayes_mixer_block

    gen = torch.Generator(device=device).manual_seed(4)
    state, width = 4 * h, 8 * h
    core, aux = 2 * state + width, state + 2 * h
    projected = torch.randn(b, t, core + aux + width, device=device, generator=gen)
    projected[..., core:core + state] -= 4.0
    projected[..., core + state:core + aux:2] -= 2.0
    leaves = [projected.to(torch.bfloat16).requires_grad_(True),
              (0.5 * torch.randn(core, 1, 4, device=device, generator=gen)).to(torch.bfloat16).requires_grad_(True),
              torch.ones(8, device=device, dtype=torch.bfloat16, requires_grad=True),
              torch.zeros(aux, device=device, dtype=torch.bfloat16, requires_grad=True)]
    gy = torch.randn(b, t, width, device=device, generator=gen).to(torch.bfloat16)

    def step():
        out, _, _ = bayes_mixer_block(leaves[0], leaves[1], leaves[2], heads=h, aux_bias=leaves[3])
        return torch.autograd.grad(out, leaves, gy)

    _settle(step, warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    per = BLOCK_FWD_BYTES + BLOCK_BWD_BYTES
    return {"B": b, "T": t, "H": h, "W": width, "D": 4, "M": 8, "ms_per_step": ms,
            "tokens_per_s": b * t / (ms * 1e-3), "bytes_per_token_head": per,
            "roofline_step_frac": per * b * h * t / (ms * 1e-3) / HBM_PEAK,
            "path": "causal depthwise-4 + producer-fused layer core + gated readout (HIP kernels)"}


def time_conv(b, t, c, steps, warmup, device, fused=True) -> dict:
    """fwd+bwd of CausalDepthwise4 on a bf16 [B, T, C] stream, as the mixer applies it (train_6layer.py:474-480).

    fused: the HIP kernels (``bayes_ssm.conv``); otherwise the reference's
    four shifted products in torch on the same GPU.  Algorithmic bytes per
    element: forward 2 in + 2 out, backward 2 + 2 in (x, grad) + 2 out.
    """
    from bayes_ssm.conv import CausalDepthwise4, _taps_formula

    gen = torch.Generator(device=device).manual_seed(5)
    value = torch.randn(b, t, c, device=device, generator=gen).to(torch.bfloat16).requires_grad_(True)
    m = CausalDepthwise4(c, dtype=torch.bfloat16, device=device)
    with torch.no_grad():
        m.weight.copy_(0.5 * torch.randn(c, 1, 4, device=device, generator=gen))
    gy = torch.randn(b, t, c, device=device, generator=gen).to(torch.bfloat16)

    def step():
        xv = value.transpose(1, 2)
        out = (m(xv) if fused else _taps_formula(xv, m.weight)).transpose(1, 2)
        return torch.autograd.grad(out, (value, m.weight), gy)

    _settle(step, warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    out = {"B": b, "T": t, "C": c, "ms_per_step": ms,
           "path": "HIP kernels" if fused else "reference shifted products in torch"}
    if fused:
        out["roofline_step_frac"] = 10 * b * t * c / (ms * 1e-3) / HBM_PEAK
    return out


def time_rotation(b, t, h, d, steps, warmup, device, fused=True) -> dict:
    """fwd+bwd of bayesian_layer with rotation dynamics (bayesian_layer.py:254-323) at one shape.

    fused: the HIP rotation kernels.  Otherwise the reference's rotation core
    run eagerly on the same GPU (the reference compiles it with Inductor,
    which this build does not use).  Algorithmic bytes per (sequence, token):
    forward k, q (D), v (8), radius, angle, process (D/2), observation in and
    y out; backward the inputs and gy in, their gradients out.
    """
    import bayes_ssm

    n, m = b * h, 8
    g = torch.Generator(device=device).manual_seed(4)
    k = (torch.randn(n, t, d, device=device, generator=g) / d ** 0.5).requires_grad_(True)
    v = torch.randn(n, t, m, device=device, generator=g).requires_grad_(True)
    q = torch.randn(n, t, d, device=device, generator=g).requires_grad_(True)
    rad = torch.exp(-torch.nn.functional.softplus(torch.randn(n, t, d // 2, device=device, generator=g) - 2.0))
    rad = rad.requires_grad_(True)
    ang = torch.randn(n, t, d // 2, device=device, generator=g).requires_grad_(True)
    p = (1e-4 + torch.nn.functional.softplus(torch.randn(n, t, d // 2, device=device, generator=g) - 3.0))
    r = (1e-4 + torch.nn.functional.softplus(torch.randn(n, t, device=device, generator=g))).requires_grad_(True)
    p = p.requires_grad_(True)
    gy = torch.randn(n, t, m, device=device, generator=g)
    leaves = (k, v, q, rad, ang, p, r)
    previous = os.environ.get("BAYES_SSM_DISABLE_FUSED_CUDA")
    if not fused:
        os.environ["BAYES_SSM_DISABLE_FUSED_CUDA"] = "1"
    try:
        def step():
            y, _, _ = bayes_ssm.bayesian_layer(k, v, q, rotation_radii=rad, rotation_angles=ang, process_variances=p,
                                               observation_variances=r, chunk_length=64, optimized=True)
            return torch.autograd.grad(y, leaves, gy)

        _settle(step, warmup)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
    finally:
        if previous is None:
            os.environ.pop("BAYES_SSM_DISABLE_FUSED_CUDA", None)
        else:
            os.environ["BAYES_SSM_DISABLE_FUSED_CUDA"] = previous
    ms = e0.elapsed_time(e1) / steps
    per = (2 * d + m + 3 * (d // 2) + 1) * 4
    fwd_b, bwd_b = per + m * 4, 2 * per + m * 4
    out = {"B": b, "T": t, "H": h, "D": d, "M": m, "ms_per_step": ms, "tokens_per_s": b * t / (ms * 1e-3),
           "path": "HIP rotation kernels" if fused else "reference rotation core, eager torch"}
    if fused:
        out["roofline_step_frac"] = (fwd_b + bwd_b) * n * t / (ms * 1e-3) / HBM_PEAK
    return out


def time_d64(b, t, h, steps, warmup, device, fused=True) -> dict:
    """fwd+bwd of bayesian_layer with D = M = 64 diagonal dynamics (persistent_bayes_chunked.cu's shape).

    fused: the HIP kernels (bssm_d64.hip) through the autograd boundary.
    Otherwise the reference's diagonal core run eagerly on the same GPU (the
    reference's non-fused path).  Keys and queries ~ N(0, 1/64); all six
    inputs require gradients.  The D = 64 step is bound by the VALU
    (about 20 thousand multiply-adds per token and sequence), not by HBM.
    """
    import bayes_ssm

    n, d = b * h, 64
    g = torch.Generator(device=device).manual_seed(5)
    k = (torch.randn(n, t, d, device=device, generator=g) / 8).requires_grad_(True)
    v = torch.randn(n, t, d, device=device, generator=g).requires_grad_(True)
    q = (torch.randn(n, t, d, device=device, generator=g) / 8).requires_grad_(True)
    dec = torch.sigmoid(torch.randn(n, t, d, device=device, generator=g) + 2.0).requires_grad_(True)
    p = torch.nn.functional.softplus(torch.randn(n, t, device=device, generator=g) - 3.0).requires_grad_(True)
    r = (1e-4 + torch.nn.functional.softplus(torch.randn(n, t, device=device, generator=g))).requires_grad_(True)
    gy = torch.randn(n, t, d, device=device, generator=g)
    leaves = (k, v, q, dec, p, r)
    previous = os.environ.get("BAYES_SSM_DISABLE_FUSED_CUDA")
    if not fused:
        os.environ["BAYES_SSM_DISABLE_FUSED_CUDA"] = "1"
    try:
        def step():
            y, _, _ = bayes_ssm.bayesian_layer(k, v, q, transition_diagonals=dec, process_variances=p,
                                               observation_variances=r, chunk_length=64, optimized=True)
            return torch.autograd.grad(y, leaves, gy)

        _settle(step, warmup)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
    finally:
        if previous is None:
            os.environ.pop("BAYES_SSM_DISABLE_FUSED_CUDA", None)
        else:
            os.environ["BAYES_SSM_DISABLE_FUSED_CUDA"] = previous
    ms = e0.elapsed_time(e1) / steps
    fwd_b, bwd_b = algorithmic_bytes(d, d)
    fwd_f, bwd_f = dense_flops(d, d)
    flops = n * t * (fwd_f + bwd_f) / (ms * 1e-3)
    return {"B": b, "T": t, "H": h, "D": d, "M": d, "sequences": n, "ms_per_step": ms,
            "tokens_per_s": b * t / (ms * 1e-3),
            # The HBM roofline of this shape is far from its bound; the vector ALUs bound it.
            "roofline_step_frac": n * t * (fwd_b + bwd_b) / (ms * 1e-3) / HBM_PEAK,
            "fp32_tflops": flops / 1e12, "fp32_roofline_frac": flops / FP32_PEAK,
            "path": "HIP D64 kernels" if fused else "reference diagonal core, eager torch"}


def _single_launch_us(launch, iters: int) -> float:
    """Median device time of one launch (microseconds): each launch and its two events are queued behind a
    device-side delay, so the events bracket the kernel(s) alone, not the host's launch rate."""
    times = []
    for _ in range(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(200_000)
        e0.record()
        launch()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3)
    return sorted(times)[len(times) // 2]


def time_scan(b, t, d, m, iters, device) -> dict:
    """Forward of associative_static_bayesian_cuda (one HIP kernel): mean microseconds per call."""
    from bayes_ssm.replay_ssm import associative_static_bayesian_cuda

    g = torch.Generator(device=device).manual_seed(0)
    k = torch.randn(b, t, d, device=device, generator=g) / d ** 0.5
    v = torch.randn(b, t, m, device=device, generator=g)
    q = torch.randn(b, t, d, device=device, generator=g)
    r = 1e-4 + torch.nn.functional.softplus(torch.randn(b, t, device=device, generator=g))
    for _ in range(5):
        associative_static_bayesian_cuda(k, v, q, observation_variances=r)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        associative_static_bayesian_cuda(k, v, q, observation_variances=r)
    e1.record()
    torch.cuda.synchronize()
    api_us = e0.elapsed_time(e1) / iters * 1e3
    # The kernel alone, through the C ABI (the API call above also validates
    # its inputs on the host, which synchronizes, as the reference does).
    from bayes_ssm import _hip

    m0 = torch.zeros(b, d, m, device=device)
    c0 = torch.eye(d, device=device).expand(b, d, d).contiguous()
    out, mT, cT = torch.empty(b, t, m, device=device), torch.empty(b, d, m, device=device), torch.empty_like(c0)
    P = _hip.ptr
    args = (P(k), P(v), P(q), P(r), P(m0), P(c0), P(out), P(mT), P(cT), b, t, d, m, _hip.stream_of(device))
    _hip.call("bssm_associative_static_scan", *args)
    torch.cuda.synchronize()
    kernel_us = _single_launch_us(lambda: _hip.call("bssm_associative_static_scan", *args), iters)
    # fwd+bwd through the API (HIP forward and HIP backward), all six inputs as leaves.
    leaves = [x.clone().requires_grad_(True) for x in (k, v, q, r, m0, c0)]
    gy = torch.randn(b, t, m, device=device, generator=g)

    def step():
        y, _, _ = associative_static_bayesian_cuda(leaves[0], leaves[1], leaves[2], observation_variances=leaves[3],
                                                   initial_mean=leaves[4], initial_covariance=leaves[5])
        return torch.autograd.grad(y, leaves, gy)

    for _ in range(5):
        step()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(iters):
        step()
    e1.record()
    torch.cuda.synchronize()
    step_us = e0.elapsed_time(e1) / iters * 1e3
    # The backward kernels alone through the C ABI.
    grads = [torch.empty_like(x) for x in (k, v, q, r, m0, c0)]
    ws = torch.empty(b * t * (d * d + d * m), device=device)
    bargs = (P(k), P(v), P(q), P(r), P(m0), P(c0), P(gy), None, None, P(ws), *map(P, grads), b, t, d, m,
             _hip.stream_of(device))
    _hip.call("bssm_associative_static_scan_backward", *bargs)
    torch.cuda.synchronize()
    bwd_us = _single_launch_us(lambda: _hip.call("bssm_associative_static_scan_backward", *bargs), iters)
    return {"B": b, "T": t, "D": d, "M": m, "api_us_per_call": api_us, "kernel_us_per_call": kernel_us,
            "api_fwd_bwd_us_per_step": step_us, "backward_kernels_us_per_call": bwd_us,
            "kernel_timing": "events around one launch queued behind a device-side delay (median of the calls)"}


def idle_probe(b, t, h, d, m, chunk, device) -> dict:
    """Per-step device times of the config-3 step right after an idle gap of 0, 1, 10 and 100 ms (the gap
    follows 60 back-to-back steps and a synchronize).  Shows the device's power-management transient: after
    an idle of 10 ms or more the following ~20 steps run up to 25 % slower, after 1 ms or less they do not."""
    from bayes_ssm import fused_cuda

    leaves, m0, c0, gy = make_workload(b, t, h, d, m, device)

    def step():
        y, _, _ = fused_cuda.fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=chunk, denominator_floor=1e-6)
        return torch.autograd.grad(y, leaves, gy)

    for _ in range(80):
        step()
    torch.cuda.synchronize()
    rows = {}
    for gap_ms in (0.0, 1.0, 10.0, 100.0):
        for _ in range(60):
            step()
        torch.cuda.synchronize()
        if gap_ms:
            time.sleep(gap_ms * 1e-3)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(41)]
        ev[0].record()
        for i in range(40):
            step()
            ev[i + 1].record()
        torch.cuda.synchronize()
        per = [ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(40)]
        rows[f"gap_{gap_ms:g}ms"] = {"first20_mean_us": sum(per[:20]) / 20, "last20_mean_us": sum(per[20:]) / 20,
                                     "per_step_us": [round(x, 1) for x in per]}
    return rows


def cpu_baseline(t: int, d: int, m: int, heads: int, budget_s: float) -> dict:
    """Time the CPU restatement of the reference CPU path on a bounded sample.

    ``bayesian_layer(..., optimized=False, chunk_length=64)`` is the
    transported-history chunk algorithm (oracle ``reference_layer``) with
    autograd backward, fp32, on all host cores.
    """
    from oracle import bssm_oracle as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    n = 256
    while True:
        k, v, q, dec, p, r, gy = O.make_inputs(n, t, d, m, seed=1, requires_grad=True)
        start = time.perf_counter()
        y, _, _ = O.reference_layer(k, v, q, dec, p, r, chunk=64)
        torch.autograd.grad(y, (k, v, q, dec, p, r), gy)
        elapsed = time.perf_counter() - start
        if elapsed * 2 > budget_s or n >= 16384:
            break
        n *= 2
    model_tokens = n * t / heads
    return {
        "value": model_tokens / elapsed,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n} of 16384 head-sequences x T={t} (D{d}M{m}), fwd+bwd of the oracle's restatement of "
                   f"bayesian_layer(optimized=False, chunk_length=64) with autograd, fp32, {threads} threads of "
                   f"{cpu_model()}, torch {torch.__version__}, {elapsed:.1f} s; sequences are independent, so "
                   f"tokens/s scales linearly to the full batch"),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--seq", type=int, default=512)
    ap.add_argument("--heads", type=int, default=64)
    ap.add_argument("--key-dim", type=int, default=4)
    ap.add_argument("--chunk", type=int, default=64)
    ap.add_argument("--kernel-iters", type=int, default=50,
                    help="launches of each kernel alone (event-timed, before the warmup steps)")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU-baseline work (0 = skip)")
    ap.add_argument("--idle-probe", action="store_true",
                    help="print per-step times of the config-3 step after idle gaps of 0-100 ms (power transient) "
                         "as its own JSON line, instead of the benchmark")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the secondary shapes (per-GPU DP shape, D1/D2/D8 variants, associative scan)")
    ap.add_argument("--secondary", choices=("mixer", "mixer-readout", "block", "conv4", "rotation", "d64",
                                            "kqv-bf16", "kqv-fp8"),
                    help="time only one secondary workload at the configured shape (the mixer's fused layer core, "
                         "with its readout epilogue, config 4's whole Bayes block, or the causal depthwise-4 filter "
                         "on the q/k/v stream, the rotation core, D = M = 64, or the layer with bf16 / float8 "
                         "k/v/q tensors), for "
                         "profiling its kernels; prints its own JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the layer shards over sequences with no exchange, "
              "so multi-GPU runs are not part of this build", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    from bayes_ssm import _hip, fused_cuda

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    b, t, h, d, m = args.batch, args.seq, args.heads, args.key_dim, 8
    if args.idle_probe:
        print(json.dumps({"workload": "idle_probe", **idle_probe(b, t, h, d, m, args.chunk, device)}), flush=True)
        return 0
    if args.secondary:
        if args.secondary == "conv4":
            row = time_conv(b, t, h * (2 * d + m), args.steps, args.warmup, device, fused=True)
        elif args.secondary == "rotation":
            row = time_rotation(b, t, h, d, args.steps, args.warmup, device, fused=True)
        elif args.secondary == "d64":
            row = time_d64(b, t, h, args.steps, args.warmup, device, fused=True)
        elif args.secondary == "block":
            row = time_block(b, t, h, args.steps, args.warmup, device)
        elif args.secondary.startswith("kqv-"):
            dt = torch.bfloat16 if args.secondary == "kqv-bf16" else torch.float8_e4m3fn
            row = time_layer(b, t, h, d, m, args.chunk, args.steps, args.warmup, device, kqv_dtype=dt)
        else:
            row = time_mixer(b, t, h, args.steps, args.warmup, device, fused=True,
                             gated=args.secondary == "mixer-readout")
        print(json.dumps({"workload": args.secondary, **row}), flush=True)
        return 0
    n = b * h
    leaves, m0, c0, gy = make_workload(b, t, h, d, m, device)

    def step():
        y, _, _ = fused_cuda.fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=args.chunk,
                                                     denominator_floor=1e-6)
        return torch.autograd.grad(y, leaves, gy)

    # 0. One call of the step as setup: its first-call host work (autograd's
    #    device threads, the ctypes bindings, the caching allocator's blocks)
    #    takes longer than 10 ms, and an idle device for 10 ms or more sends
    #    the next ~20 steps of this workload through a power-management dip
    #    (up to 25 % slower per step; per-step times in profiles/).  Done here,
    #    that idle precedes the ~30 ms of calibration work below instead of the
    #    warmup and timed steps.
    step()
    torch.cuda.synchronize()

    # 1. Streaming ceiling of this device: a plain 256 MiB device copy (64 Mi
    #    floats read + 64 Mi written), also the reference kernel for scaling
    #    the PMC byte counters.
    src = torch.randn(64 << 20, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * src.numel() * 4 / (e0.elapsed_time(e1) / 20 * 1e-3) / 1e9
    del src, dst

    # 2. Each kernel alone: --kernel-iters back-to-back launches of the
    #    forward, then of the backward, through the extension object, with
    #    events on the launch stream (torch's current stream).  These loops
    #    (about 30 ms of device work) run before the warmup steps.
    ext = fused_cuda._load_extension(d)
    interval = fused_cuda._checkpoint_interval(d, t, args.chunk)
    raw = [x.detach() for x in leaves]
    fwd_out = ext.forward_chunked(*raw, m0, c0, interval, 1e-6)
    bm, bc = fwd_out[3], fwd_out[4]
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    torch.cuda.synchronize()
    ev[0].record()
    for _ in range(args.kernel_iters):
        ext.forward_chunked(*raw, m0, c0, interval, 1e-6)
    ev[1].record()
    for _ in range(args.kernel_iters):
        ext.backward_chunked(*raw, m0, c0, bm, bc, gy, None, None, interval, 1e-6)
    ev[2].record()
    torch.cuda.synchronize()
    iso_fwd_ms = ev[0].elapsed_time(ev[1]) / args.kernel_iters
    iso_bwd_ms = ev[1].elapsed_time(ev[2]) / args.kernel_iters
    del fwd_out, bm, bc

    # 3. W warmup steps, then exactly K timed steps, with no other device work
    #    in between (an event recorded inside each step costs it 2-6 us).
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    stop.record()
    # 4. The same K steps again, queued right behind the timed ones (no idle
    #    device between them), with an event at each step's start, at the end
    #    of its forward (the forward kernel's launch is the only device work
    #    between the two) and at its end (the backward kernel), all on the
    #    launch stream: the in-step kernel times behind the roofline figures.
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        marks[i][0].record()
        y, _, _ = fused_cuda.fused_diagonal_bayesian(*leaves, m0, c0, chunk_length=args.chunk,
                                                     denominator_floor=1e-6)
        marks[i][1].record()
        torch.autograd.grad(y, leaves, gy)
        marks[i][2].record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(stop) / args.steps
    tokens_per_s = b * t / (ms_per_step * 1e-3)
    fwd_ms = sum(mk[0].elapsed_time(mk[1]) for mk in marks) / args.steps
    bwd_ms = sum(mk[1].elapsed_time(mk[2]) for mk in marks) / args.steps
    fwd_b, bwd_b = algorithmic_bytes(d, m)
    units = n * t
    bwd_gbs = bwd_b * units / (bwd_ms * 1e-3) / 1e9
    fwd_gbs = fwd_b * units / (fwd_ms * 1e-3) / 1e9
    step_frac = (fwd_b + bwd_b) * units / (ms_per_step * 1e-3) / HBM_PEAK

    # HBM bytes per backward launch from the committed PMC summary (FETCH_SIZE
    # and WRITE_SIZE, each scaled by the counter's reading on a 256 MiB copy).
    traffic = None
    traffic_file = ROOT / "profiles" / f"traffic_d{d}m{m}_b{b}t{t}h{h}.txt"
    if traffic_file.exists():
        for line in traffic_file.read_text().splitlines():
            if line.startswith("backward_bytes_per_launch ="):
                traffic = int(line.split("=")[1])

    fwd_kernel, bwd_kernel = dispatched_kernels(d, m, n, t, interval)
    result = {
        "metric": METRIC,
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": "bayes_layer_fwd_bwd_config3",
            "B": b, "T": t, "H": h, "D": d, "M": m, "sequences": n,
            "chunk_length": args.chunk, "checkpoint_interval": interval,
            "gradients": "k,v,q,decay,process,observation (full ABI)",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": bwd_kernel + ", checkpoint replay + reverse",
            "achieved": bwd_gbs,
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": bwd_gbs * 1e9 / HBM_PEAK,
            "traffic": traffic,
            "bytes_per_launch": bwd_b * units,
            "avg_launch_ms": bwd_ms,
            "timing": "events around the backward of each of K steps queued right behind the timed ones, on its launch stream",
            "isolated_launch_ms": iso_bwd_ms,
        },
        "roofline_forward": {"kernel": fwd_kernel, "achieved": fwd_gbs, "frac": fwd_gbs * 1e9 / HBM_PEAK,
                             "avg_launch_ms": fwd_ms, "bytes_per_launch": fwd_b * units,
                             "isolated_launch_ms": iso_fwd_ms},
        "roofline_step_frac": step_frac,
        "measured_copy_gbs": copy_gbs,
        "step_frac_of_measured_copy": (fwd_b + bwd_b) * units / (ms_per_step * 1e-3) / (copy_gbs * 1e9),
        "device": torch.cuda.get_device_name(device),
        "hip_library": str(_hip.LIB_PATH.relative_to(ROOT)),
    }
    if not args.no_extras:
        # Secondary shapes (not the metric): config 3 divided by 8 (one GPU's
        # share under 8-way data parallelism), the D2M8 / D8M8 variants of
        # config 3, config 2 (D1M8, B64), the mixer's layer core at config 3
        # (fused producer kernels, and the reference op chain beside it),
        # config 4's Bayes block (filter + layer core + gated readout), and
        # the associative-scan configs (forward, and fwd+bwd).
        extras = {"config3_bf16_kqv": time_layer(b, t, h, d, m, args.chunk, 30, 10, device,
                                                 kqv_dtype=torch.bfloat16),
                  "config3_fp8_kqv": time_layer(b, t, h, d, m, args.chunk, 30, 10, device,
                                                kqv_dtype=torch.float8_e4m3fn),
                  "dp8_share_d4m8": time_layer(b // 8, t, h, d, m, args.chunk, 30, 10, device)}
        for name, (eb, ed) in {"config3_d2m8": (b, 2), "config3_d8m8": (b, 8), "config2_d1m8": (64, 1)}.items():
            extras[name] = time_layer(eb, t, h, ed, m, args.chunk, 10, 3, device)
        # Config 2's step is short enough for host work to bound it: its host
        # costs, and the same step replayed from a HIP graph.
        extras["config2_d1m8"].update(host_costs(64, t, h, 1, m, args.chunk, device))
        extras["config2_d1m8_graphed"] = time_layer_graphed(64, t, h, 1, m, args.chunk, 10, device)
        extras["dp8_share_d4m8_graphed"] = time_layer_graphed(b // 8, t, h, d, m, args.chunk, 10, device)
        extras["mixer_core_config3_fused"] = time_mixer(b, t, h, 30, 10, device, fused=True)
        extras["mixer_core_config3_op_chain"] = time_mixer(b, t, h, 10, 3, device, fused=False)
        extras["mixer_readout_config3_fused"] = time_mixer(b, t, h, 30, 10, device, fused=True, gated=True)
        extras["mixer_readout_config3_op_chain"] = time_mixer(b, t, h, 10, 3, device, fused=False, gated=True)
        extras["block_config4_fused"] = time_block(b, t, h, 20, 5, device)
        qkv = h * (2 * d + m)  # channels of the mixer's fused q/k/v stream at this shape
        extras["conv4_config3_qkv"] = time_conv(b, t, qkv, 30, 10, device, fused=True)
        extras["conv4_config3_qkv_torch"] = time_conv(b, t, qkv, 10, 3, device, fused=False)
        extras["rotation_config3_d4m8"] = time_rotation(b, t, h, 4, 10, 3, device, fused=True)
        extras["rotation_config3_d4m8_eager"] = time_rotation(b // 32, t, h, 4, 2, 1, device, fused=False)
        # D = M = 64 at 8 heads (width 512): B = 32 (256 sequences) on the HIP
        # kernels, and the eager torch core at B = 4 beside it.
        extras["d64_b32t512h8"] = time_d64(32, t, 8, 3, 1, device, fused=True)
        extras["d64_b4t512h8_eager"] = time_d64(4, t, 8, 1, 1, device, fused=False)
        extras["assoc_scan_config0"] = time_scan(1, 16, 4, 4, 50, device)
        extras["assoc_scan_config1"] = time_scan(4, 64, 16, 16, 50, device)
        result["extras"] = extras
    if args.cpu_budget > 0:
        result["cpu_baseline"] = cpu_baseline(t, d, m, h, args.cpu_budget)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
