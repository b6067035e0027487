"""Exact fused Bayesian core on MI355X: the drop-in for the reference ``fused_cuda``.

Mirrors bayes_ssm/fused_cuda.py of the reference: ``_load_extension(key_dim)``
returns an object exposing the same per-key-dim method names and signatures as
the reference pybind modules (``forward_chunked``, ``backward_chunked``, ...;
export sets at persistent_bayes_chunked_d1m8.cu:673, _d2m8.cu:602,
_d4m8.cu:577, _d8.cu:653), ``_ChunkedBayesianFunction`` keeps the reference
autograd slot conventions (fused_cuda.py:58-322), and
``fused_diagonal_bayesian`` keeps the contract gate (fused_cuda.py:325-388).

Every method is a thin shim over the C ABI of ``libbssm_hip.so``: it checks the
tensors like the reference ``TORCH_CHECK``s, allocates the outputs with
``torch.empty`` on the inputs' device (the C ABI never allocates) and launches
on ``torch.cuda.current_stream()``.

Deliberate differences from the reference, all result-preserving:

* No JIT build: the library is prebuilt for gfx950.  A missing or stale
  library raises ``RuntimeError`` instead of silently returning ``None``, so a
  GPU run can never fall back to a slower path unnoticed.
  ``BAYES_SSM_DISABLE_FUSED_CUDA=1`` still disables the extension.
* Checkpoint interval: the autograd function checkpoints the belief every
  ``bssm_preferred_checkpoint(D)`` tokens (the on-chip replay length of the
  reverse kernel) rather than every ``chunk_length`` tokens.  The recurrence
  ignores chunking, so outputs and gradients are identical for every interval;
  ``BAYES_SSM_HIP_CHECKPOINT=chunk`` restores the caller's chunk length and an
  integer value forces a specific interval.
* D1 keeps its boundaries through the replay kernel by default; the reference
  saved-history ABI (forward_chunked_saved / backward_chunked_saved*) is still
  exported and is used when ``BAYES_SSM_D1_SAVED_HISTORY=1``.

Extension beyond the reference contract: ``fused_diagonal_bayesian`` also
accepts bfloat16 keys, values and queries, or float8 ones (float8_e4m3fn or
float8_e5m2; everything else float32).  For D = 4, M = 8 they are read as
such by the kernels (no float32 copies in HBM) and their gradients are
written in their dtype; results equal those of the float32 path on the
widened values, whose gradients autograd would round to that dtype the same
way.  Other shapes widen first and take the float32 path.
"""
from __future__ import annotations

import os
from typing import Optional

import torch
from torch import Tensor

from . import _hip

_SUPPORTED = ((1, 8), (2, 8), (4, 8), (8, 8), (64, 64))
_EXTENSIONS: dict[int, "_Extension"] = {}

# Method names of the reference extension module for each key_dim.
_EXPORTS = {
    1: ("forward_chunked", "forward_chunked_saved", "backward_chunked_saved_d1", "backward_chunked",
        "backward_chunked_lean", "backward_chunked_saved", "backward_chunked_saved_lean",
        "forward_chunked_fixed", "backward_chunked_lean_fixed", "backward_chunked_fixed"),
    2: ("forward_chunked", "backward_chunked", "backward_chunked_noinitial", "backward_chunked_lean",
        "forward_chunked_fixed", "backward_chunked_lean_fixed", "backward_chunked_fixed",
        "backward_chunked_noinitial_fixed"),
    4: ("forward_chunked", "backward_chunked", "backward_chunked_lean", "forward_chunked_fixed",
        "backward_chunked_lean_fixed", "backward_chunked_fixed"),
    8: ("forward_chunked", "backward_chunked", "backward_chunked_lean", "forward_chunked_fixed",
        "backward_chunked_lean_fixed", "backward_chunked_fixed"),
    # persistent_bayes_chunked.cu:436
    64: ("forward_chunked", "backward_chunked", "backward_chunked_lean", "forward_chunked_fixed",
         "backward_chunked_lean_fixed", "backward_chunked_fixed"),
}

# Value dimension of each key dimension's kernels.
_VALUE_DIM = {1: 8, 2: 8, 4: 8, 8: 8, 64: 64}


_ALL_METHODS = frozenset(name for names in _EXPORTS.values() for name in names)


def _check(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def _check_inputs(key_dim: int, tensors: tuple[Tensor, ...], names: tuple[str, ...]) -> None:
    for x, name in zip(tensors, names):
        _check(isinstance(x, Tensor), f"fused Bayesian {name} must be a tensor")
        _check(x.is_cuda, "fused Bayesian inputs must be CUDA tensors")
        _check(x.dtype == torch.float32, "fused Bayesian inputs must be float32")
        _check(x.is_contiguous(), "fused Bayesian inputs must be contiguous")
    k, v, q = tensors[:3]
    m = _VALUE_DIM[key_dim]
    _check(k.dim() == 3 and v.dim() == 3 and q.dim() == 3 and k.size(2) == key_dim and q.size(2) == key_dim
           and v.size(2) == m, f"fused Bayesian kernel expects [N,T,{key_dim}] keys/queries and [N,T,{m}] values")
    n, t = k.shape[:2]
    _check(tuple(v.shape[:2]) == (n, t) and tuple(q.shape[:2]) == (n, t), "keys/values/queries batch-time mismatch")
    _check(all(x.device == k.device for x in tensors), "fused Bayesian inputs must share one device")


def _launch_forward(d: int, m: int, name: str, fixed: bool, keys, values, queries, decay, process, observation,
                    mean0, cov0, chunks: int, floor: float, saved: bool = False) -> list:
    """Allocate the forward outputs and launch ``name`` on the current stream (arguments already checked)."""
    n, t = keys.shape[0], keys.shape[1]
    nb = -(-t // chunks)
    dev = keys.device
    f32 = torch.float32
    out = torch.empty((n, t, m), device=dev, dtype=f32)
    mf = torch.empty((n, d, m), device=dev, dtype=f32)
    cf = torch.empty((n, d, d), device=dev, dtype=f32)
    bm = torch.empty((n, nb + 1, d, m), device=dev, dtype=f32)
    bc = torch.empty((n, nb + 1, d, d), device=dev, dtype=f32)
    hist = ()
    if saved:
        hist = (torch.empty((n, t, d, m), device=dev, dtype=f32), torch.empty((n, t, d, d), device=dev, dtype=f32),
                torch.empty((n, t, d), device=dev, dtype=f32), torch.empty((n, t), device=dev, dtype=f32),
                torch.empty((n, t, m), device=dev, dtype=f32))
    _hip.launch(dev, name, d, m, keys.data_ptr(), values.data_ptr(), queries.data_ptr(),
                None if fixed else decay.data_ptr(), None if fixed else process.data_ptr(),
                None if fixed else observation.data_ptr(), mean0.data_ptr(), cov0.data_ptr(), out.data_ptr(),
                mf.data_ptr(), cf.data_ptr(), bm.data_ptr(), bc.data_ptr(), *[h.data_ptr() for h in hist],
                n, t, chunks, floor, _hip.stream_of(dev))
    return [out, mf, cf, bm, bc, *hist]


def _launch_backward(d: int, m: int, name: str, fixed: bool, outputs: int, keys, values, queries, decay, process,
                     observation, mean0, cov0, bm, bc, history, gy, gmf, gcf, chunks: int, floor: float) -> list:
    """Allocate ``outputs`` gradients (3, 6 or 8) and launch ``name`` (arguments already checked)."""
    n, t = keys.shape[0], keys.shape[1]
    dev = keys.device
    f32 = torch.float32
    grads = [torch.empty((n, t, d), device=dev, dtype=f32), torch.empty((n, t, m), device=dev, dtype=f32),
             torch.empty((n, t, d), device=dev, dtype=f32)]
    if outputs >= 6:
        grads += [torch.empty((n, t, d), device=dev, dtype=f32), torch.empty((n, t), device=dev, dtype=f32),
                  torch.empty((n, t), device=dev, dtype=f32)]
    if outputs == 8:
        grads += [torch.empty((n, d, m), device=dev, dtype=f32), torch.empty((n, d, d), device=dev, dtype=f32)]
    _hip.launch(dev, name, d, m, keys.data_ptr(), values.data_ptr(), queries.data_ptr(),
                None if fixed else decay.data_ptr(), None if fixed else process.data_ptr(),
                None if fixed else observation.data_ptr(), mean0.data_ptr(), cov0.data_ptr(), bm.data_ptr(),
                bc.data_ptr(), *[h.data_ptr() for h in history], gy.data_ptr(),
                None if gmf is None else gmf.data_ptr(), None if gcf is None else gcf.data_ptr(),
                *[g.data_ptr() for g in grads], n, t, chunks, floor, _hip.stream_of(dev))
    return grads


class _Extension:
    """Per-key-dim method table over the C ABI (replaces the pybind module)."""

    def __init__(self, key_dim: int) -> None:
        self.key_dim = key_dim
        self.value_dim = _VALUE_DIM[key_dim]
        self._exports = frozenset(_EXPORTS[key_dim])

    def __getattribute__(self, name: str):
        # Methods outside this key_dim's reference export set behave as absent,
        # so ``hasattr`` probes see the same module surface as the reference.
        if name in _ALL_METHODS and name not in object.__getattribute__(self, "_exports"):
            raise AttributeError(f"key_dim={object.__getattribute__(self, 'key_dim')} extension has no {name}")
        return object.__getattribute__(self, name)

    def __dir__(self):
        return sorted(self._exports)

    # -- helpers ---------------------------------------------------------
    def _sizes(self, keys: Tensor) -> tuple[int, int]:
        return int(keys.size(0)), int(keys.size(1))

    def _forward(self, name: str, fixed: bool, keys, values, queries, decay, process, observation, mean0, cov0,
                 chunks: int, floor: float, saved: bool = False, validate: bool = True):
        # validate=False: the caller (the autograd boundary behind
        # fused_diagonal_bayesian's contract check) has established the checks.
        if validate:
            tensors = (keys, values, queries) + (() if fixed else (decay, process, observation)) + (mean0, cov0)
            names = ("keys", "values", "queries") + (() if fixed else ("decay", "process", "observation")) + (
                "mean0", "cov0")
            _check_inputs(self.key_dim, tensors, names)
        _check(int(chunks) > 0, "fused Bayesian chunk length must be positive")
        return _launch_forward(self.key_dim, self.value_dim, name, fixed, keys, values, queries, decay, process,
                               observation, mean0, cov0, int(chunks), float(floor), saved)

    def _backward(self, name: str, fixed: bool, outputs: int, keys, values, queries, decay, process, observation,
                  mean0, cov0, bm, bc, history, gy, gmf, gcf, chunks: int, floor: float, validate: bool = True):
        if validate:
            n, t = self._sizes(keys)
            d, m = self.key_dim, self.value_dim
            tensors = (keys, values, queries) + (() if fixed else (decay, process, observation)) + (bm, bc, gy)
            names = ("keys", "values", "queries") + (() if fixed else ("decay", "process", "observation")) + (
                "boundary_mean", "boundary_covariance", "grad_output")
            _check_inputs(self.key_dim, tensors, names)
            for extra in (gmf, gcf, *history):
                if extra is not None:
                    _check(extra.is_cuda and extra.dtype == torch.float32 and extra.is_contiguous(),
                           "fused Bayesian backward inputs must be contiguous CUDA float32 tensors")
            _check(int(chunks) > 0, "fused Bayesian chunk length must be positive")
            nb = -(-t // int(chunks))
            _check(tuple(bm.shape) == (n, nb + 1, d, m) and tuple(bc.shape) == (n, nb + 1, d, d),
                   "boundary tensors do not match the chunk length")
            _check(tuple(gy.shape) == (n, t, m), "grad_output must be [N,T,M]")
        return _launch_backward(self.key_dim, self.value_dim, name, fixed, outputs, keys, values, queries, decay,
                                process, observation, mean0, cov0, bm, bc, history, gy, gmf, gcf, int(chunks),
                                float(floor))

    # -- reference method names ------------------------------------------
    def forward_chunked(self, keys, values, queries, decay, process, observation, mean0, cov0, chunks, floor):
        return self._forward("bssm_forward_chunked", False, keys, values, queries, decay, process, observation,
                             mean0, cov0, chunks, floor)

    def forward_chunked_fixed(self, keys, values, queries, decay, process, observation, mean0, cov0, chunks, floor):
        return self._forward("bssm_forward_chunked_fixed", True, keys, values, queries, decay, process, observation,
                             mean0, cov0, chunks, floor)

    def forward_chunked_saved(self, keys, values, queries, decay, process, observation, mean0, cov0, chunks, floor):
        self._require("forward_chunked_saved")
        _check(int(chunks) == int(keys.size(1)), "saved D1 history requires one full-sequence chunk")
        return self._forward("bssm_forward_chunked_saved", False, keys, values, queries, decay, process,
                             observation, mean0, cov0, chunks, floor, saved=True)

    def backward_chunked(self, keys, values, queries, decay, process, observation, mean0, cov0, bm, bc, gy, gmf,
                         gcf, chunks, floor):
        return self._backward("bssm_backward_chunked", False, 8, keys, values, queries, decay, process,
                              observation, mean0, cov0, bm, bc, (), gy, gmf, gcf, chunks, floor)

    def backward_chunked_lean(self, keys, values, queries, decay, process, observation, mean0, cov0, bm, bc, gy,
                              gmf, gcf, chunks, floor):
        return self._backward("bssm_backward_chunked_lean", False, 3, keys, values, queries, decay, process,
                              observation, mean0, cov0, bm, bc, (), gy, gmf, gcf, chunks, floor)

    def backward_chunked_noinitial(self, keys, values, queries, decay, process, observation, mean0, cov0, bm, bc,
                                   gy, gmf, gcf, chunks, floor):
        self._require("backward_chunked_noinitial")
        return self._backward("bssm_backward_chunked_noinitial", False, 6, keys, values, queries, decay, process,
                              observation, mean0, cov0, bm, bc, (), gy, gmf, gcf, chunks, floor)

    def backward_chunked_fixed(self, keys, values, queries, decay, process, observation, mean0, cov0, bm, bc, gy,
                               gmf, gcf, chunks, floor):
        return self._backward("bssm_backward_chunked_fixed", True, 8, keys, values, queries, decay, process,
                              observation, mean0, cov0, bm, bc, (), gy, gmf, gcf, chunks, floor)

    def backward_chunked_lean_fixed(self, keys, values, queries, decay, process, observation, mean0, cov0, bm, bc,
                                    gy, gmf, gcf, chunks, floor):
        return self._backward("bssm_backward_chunked_lean_fixed", True, 3, keys, values, queries, decay, process,
                              observation, mean0, cov0, bm, bc, (), gy, gmf, gcf, chunks, floor)

    def backward_chunked_noinitial_fixed(self, keys, values, queries, decay, process, observation, mean0, cov0, bm,
                                         bc, gy, gmf, gcf, chunks, floor):
        self._require("backward_chunked_noinitial_fixed")
        return self._backward("bssm_backward_chunked_noinitial_fixed", True, 6, keys, values, queries, decay,
                              process, observation, mean0, cov0, bm, bc, (), gy, gmf, gcf, chunks, floor)

    def backward_chunked_saved(self, keys, values, queries, decay, process, observation, mean0, cov0, bm, bc, mp, pp,
                               uh, bh, eh, gy, gmf, gcf, chunks, floor):
        self._require("backward_chunked_saved")
        return self._backward("bssm_backward_chunked_saved", False, 8, keys, values, queries, decay, process,
                              observation, mean0, cov0, bm, bc, (mp, pp, uh, bh, eh), gy, gmf, gcf, chunks, floor)

    def backward_chunked_saved_lean(self, keys, values, queries, decay, process, observation, mean0, cov0, bm, bc,
                                    mp, pp, uh, bh, eh, gy, gmf, gcf, chunks, floor):
        self._require("backward_chunked_saved_lean")
        return self._backward("bssm_backward_chunked_saved_lean", False, 3, keys, values, queries, decay, process,
                              observation, mean0, cov0, bm, bc, (mp, pp, uh, bh, eh), gy, gmf, gcf, chunks, floor)

    def backward_chunked_saved_d1(self, keys, values, queries, decay, process, observation, mean0, cov0, bm, bc, mp,
                                  pp, uh, bh, eh, gy, gmf, gcf, chunks, floor):
        # The reference's register-only D1 reverse returns the same eight
        # gradients as backward_chunked_saved (d1m8.cu:600-630).
        self._require("backward_chunked_saved_d1")
        return self._backward("bssm_backward_chunked_saved", False, 8, keys, values, queries, decay, process,
                              observation, mean0, cov0, bm, bc, (mp, pp, uh, bh, eh), gy, gmf, gcf, chunks, floor)

    def _require(self, name: str) -> None:
        # Reached only through an explicit unbound call; mirror the missing attribute.
        if name not in self._exports:
            raise AttributeError(f"key_dim={self.key_dim} extension has no {name}")


def _has(extension: Optional[_Extension], name: str) -> bool:
    return extension is not None and name in extension._exports


def _load_extension(key_dim: int) -> Optional[_Extension]:
    """Extension object for ``key_dim`` or ``None`` when unsupported/disabled.

    Raises ``RuntimeError`` when the prebuilt HIP library is missing or stale:
    on a GPU the fused path must never degrade silently.
    """
    if os.environ.get("BAYES_SSM_DISABLE_FUSED_CUDA", "0") == "1":
        return None
    if key_dim not in _EXPORTS:
        return None
    ext = _EXTENSIONS.get(key_dim)
    if ext is None:
        _hip.load()
        ext = _EXTENSIONS.setdefault(key_dim, _Extension(key_dim))
    return ext


def _checkpoint_interval(key_dim: int, t: int, chunk_length: int) -> int:
    mode = os.environ.get("BAYES_SSM_HIP_CHECKPOINT", "auto").strip().lower()
    if mode == "chunk":
        return max(1, int(chunk_length))
    if mode not in ("", "auto"):
        value = int(mode)
        if value <= 0:
            raise ValueError("BAYES_SSM_HIP_CHECKPOINT must be 'auto', 'chunk' or a positive integer")
        return value
    preferred = _hip.preferred_checkpoint(key_dim)
    return max(1, preferred if preferred > 0 else int(chunk_length))


class _ChunkedBayesianFunction(torch.autograd.Function):
    """Autograd boundary of the fused recurrence (slot conventions of fused_cuda.py:58-322)."""

    @staticmethod
    def forward(ctx, keys, values, queries, decay, process, observation, initial_mean, initial_covariance,
                chunk_length, denominator_floor, fixed_dynamics):
        n, t, d = keys.shape
        extension = _load_extension(d)
        if extension is None:
            raise RuntimeError("the fused Bayesian HIP extension is unavailable")
        floor = float(denominator_floor)
        fixed = bool(fixed_dynamics)
        use_saved_history = (
            d == 1 and not fixed and os.environ.get("BAYES_SSM_D1_SAVED_HISTORY", "0") == "1"
            and os.environ.get("BAYES_SSM_DISABLE_SAVED_HISTORY", "0") != "1"
        )
        if use_saved_history:
            interval = max(int(t), 1)
            (output, final_mean, final_covariance, boundary_mean, boundary_covariance, mp_history, pp_history,
             u_history, beta_history, e_history) = extension.forward_chunked_saved(
                keys, values, queries, decay, process, observation, initial_mean, initial_covariance, interval,
                floor)
            ctx.save_for_backward(keys, values, queries, decay, process, observation, initial_mean,
                                  initial_covariance, boundary_mean, boundary_covariance, mp_history, pp_history,
                                  u_history, beta_history, e_history)
        else:
            interval = _checkpoint_interval(d, t, chunk_length)
            output, final_mean, final_covariance, boundary_mean, boundary_covariance = _launch_forward(
                d, _VALUE_DIM[d], "bssm_forward_chunked_fixed" if fixed else "bssm_forward_chunked", fixed, keys,
                values, queries, decay, process, observation, initial_mean, initial_covariance, interval, floor)
            ctx.save_for_backward(keys, values, queries, decay, process, observation, initial_mean,
                                  initial_covariance, boundary_mean, boundary_covariance)
        need = ctx.needs_input_grad
        ctx.extension = extension
        ctx.use_saved_history = use_saved_history
        ctx.chunk_length = interval
        ctx.denominator_floor = floor
        ctx.fixed_dynamics = fixed
        ctx.need_dynamics_grad = need[3] or need[4] or need[5] or need[6] or need[7]
        ctx.need_initial_grad = need[6] or need[7]
        ctx.noinitial_backward = False
        ctx.set_materialize_grads(False)
        return output, final_mean, final_covariance

    @staticmethod
    def backward(ctx, grad_output, grad_mean, grad_covariance):
        saved = ctx.saved_tensors
        (keys, values, queries, decay, process, observation, initial_mean, initial_covariance, boundary_mean,
         boundary_covariance) = saved[:10]
        history = saved[10:]
        extension = ctx.extension
        lean = not ctx.need_dynamics_grad and grad_mean is None and grad_covariance is None
        d = keys.shape[2]
        m = _VALUE_DIM[d]
        if grad_output is None:
            grad_output = torch.zeros((keys.shape[0], keys.shape[1], m), device=keys.device, dtype=keys.dtype)
        elif not grad_output.is_contiguous():
            grad_output = grad_output.contiguous()
        # Null final-state gradients mean zero in the C ABI; no zero tensors needed.
        gm = None if grad_mean is None else grad_mean.contiguous()
        gc = None if grad_covariance is None else grad_covariance.contiguous()
        args_head = (keys, values, queries, decay, process, observation, initial_mean, initial_covariance,
                     boundary_mean, boundary_covariance)
        ctx.noinitial_backward = False
        if ctx.use_saved_history:
            if lean:
                backward = extension.backward_chunked_saved_lean
            elif _has(extension, "backward_chunked_saved_d1") and \
                    os.environ.get("BAYES_SSM_DISABLE_D1_SPECIALIZED", "0") != "1":
                backward = extension.backward_chunked_saved_d1
            else:
                backward = extension.backward_chunked_saved
            gradients = backward(*args_head, *history, grad_output, gm, gc, ctx.chunk_length, ctx.denominator_floor)
        else:
            # The reference's method choice (lean / noinitial / full), called
            # through the C names; the tensors are the forward's own, so the
            # argument checks of the public methods are not repeated.
            fixed = ctx.fixed_dynamics
            suffix = "_fixed" if fixed else ""
            if not lean and not ctx.need_initial_grad and _has(extension, "backward_chunked_noinitial" + suffix):
                name, outputs = "bssm_backward_chunked_noinitial" + suffix, 6
                ctx.noinitial_backward = True
            elif lean:
                name, outputs = "bssm_backward_chunked_lean" + suffix, 3
            else:
                name, outputs = "bssm_backward_chunked" + suffix, 8
            gradients = _launch_backward(d, m, name, fixed, outputs, *args_head, (), grad_output, gm, gc,
                                         ctx.chunk_length, ctx.denominator_floor)
        if lean:
            # 3 tensor gradients + 5 tensor and 3 scalar non-differentiable slots.
            return (*gradients, None, None, None, None, None, None, None, None)
        if ctx.noinitial_backward:
            # 6 tensor gradients + initial mean/covariance + 3 scalar slots.
            return (*gradients, None, None, None, None, None)
        # 8 tensor gradients + 3 scalar slots.
        return (*gradients, None, None, None)


# float8 encodings the D4M8 kernels read (C ABI format argument).
_FP8_FORMATS = {torch.float8_e4m3fn: 0, torch.float8_e5m2: 1}


def _narrow_call(keys: Tensor, direction: str) -> tuple[str, tuple[int, ...]]:
    """C ABI entry point and leading format argument for narrow keys/values/queries."""
    if keys.dtype == torch.bfloat16:
        return f"bssm_{direction}_chunked_bf16", ()
    return f"bssm_{direction}_chunked_fp8", (_FP8_FORMATS[keys.dtype],)


class _ChunkedBayesianBF16Function(torch.autograd.Function):
    """bfloat16 or float8 keys/values/queries read as such by the D4M8 kernels
    (C ABI ``bssm_*_chunked_bf16`` / ``bssm_*_chunked_fp8``).

    Outputs are float32; the gradients of keys, values and queries have
    their dtype (the float32 gradient rounded to nearest even, as autograd
    through a widening cast gives), the others float32.  Gradients are
    computed only for inputs that require them.
    """

    @staticmethod
    def forward(ctx, keys, values, queries, decay, process, observation, initial_mean, initial_covariance,
                denominator_floor, fixed_dynamics):
        n, t, d = keys.shape
        m = values.shape[-1]
        interval = _hip.preferred_checkpoint(d)
        nb = -(-t // interval)
        dev = keys.device
        out = torch.empty(n, t, m, device=dev, dtype=torch.float32)
        mean_t = torch.empty(n, d, m, device=dev, dtype=torch.float32)
        cov_t = torch.empty(n, d, d, device=dev, dtype=torch.float32)
        bmean = torch.empty(n, nb + 1, d, m, device=dev, dtype=torch.float32)
        bcov = torch.empty(n, nb + 1, d, d, device=dev, dtype=torch.float32)
        P = _hip.ptr
        with _hip.on_device(dev):
            name, fmt = _narrow_call(keys, "forward")
            _hip.call(name, d, m, int(bool(fixed_dynamics)), *fmt, P(keys), P(values), P(queries),
                      P(decay), P(process), P(observation), P(initial_mean), P(initial_covariance), P(out),
                      P(mean_t), P(cov_t), P(bmean), P(bcov), n, t, interval, float(denominator_floor),
                      _hip.stream_of(dev))
        ctx.save_for_backward(keys, values, queries, decay, process, observation, initial_mean, initial_covariance,
                              bmean, bcov)
        ctx.interval = interval
        ctx.denominator_floor = float(denominator_floor)
        ctx.fixed_dynamics = bool(fixed_dynamics)
        ctx.set_materialize_grads(False)
        return out, mean_t, cov_t

    @staticmethod
    def backward(ctx, grad_output, grad_mean, grad_covariance):
        keys, values, queries, decay, process, observation, mean0, cov0, bmean, bcov = ctx.saved_tensors
        n, t, d = keys.shape
        m = values.shape[-1]
        need = ctx.needs_input_grad
        if grad_output is None:
            grad_output = torch.zeros(n, t, m, device=keys.device, dtype=torch.float32)
        else:
            grad_output = grad_output.contiguous()
        gm = None if grad_mean is None else grad_mean.contiguous()
        gc = None if grad_covariance is None else grad_covariance.contiguous()
        gk, gv, gq = torch.empty_like(keys), torch.empty_like(values), torch.empty_like(queries)
        dyn = any(need[3:6])
        gd = torch.empty_like(decay) if dyn else None
        gp = torch.empty_like(process) if dyn else None
        gr = torch.empty_like(observation) if dyn else None
        gm0 = torch.empty_like(mean0) if need[6] else None
        gc0 = torch.empty_like(cov0) if need[7] else None
        P = _hip.ptr
        with _hip.on_device(keys.device):
            name, fmt = _narrow_call(keys, "backward")
            _hip.call(name, d, m, int(ctx.fixed_dynamics), *fmt, P(keys), P(values), P(queries),
                      P(decay), P(process), P(observation), P(mean0), P(cov0), P(bmean), P(bcov), P(grad_output),
                      P(gm), P(gc), P(gk), P(gv), P(gq), P(gd), P(gp), P(gr), P(gm0), P(gc0), n, t, ctx.interval,
                      ctx.denominator_floor, _hip.stream_of(keys.device))
        return (gk if need[0] else None, gv if need[1] else None, gq if need[2] else None,
                gd if need[3] else None, gp if need[4] else None, gr if need[5] else None, gm0, gc0, None, None)


def _bf16_kernels_apply(keys: Tensor, values: Tensor, queries: Tensor) -> bool:
    """The D4M8 kernels read these bfloat16 / float8 streams directly (else: widen, float32 path)."""
    n, t, d = keys.shape
    return ((d, values.shape[-1]) == (4, 8) and t > 0 and t % 4 == 0 and _hip.preferred_checkpoint(d) > 0
            and all(x.data_ptr() % 16 == 0 for x in (keys, values, queries)))


def fused_diagonal_bayesian(
    keys: Tensor,
    values: Tensor,
    queries: Tensor,
    decay: Tensor,
    process: Tensor,
    observation: Tensor,
    initial_mean: Tensor,
    initial_covariance: Tensor,
    *,
    chunk_length: int,
    denominator_floor: float,
    fixed_dynamics: bool = False,
) -> tuple[Tensor, Tensor, Tensor] | None:
    """Run the exact HIP core when its contract holds; ``None`` means "use the torch path".

    Contract (fused_cuda.py:346-371): CUDA device, 3-D fp32 tensors,
    (D, M) in {(1,8), (2,8), (4,8), (8,8), (64,64)}, decay [N,T,D], process and
    observation [N,T], initial mean [N,D,M] and covariance [N,D,D].
    Keys, values and queries may instead all be bfloat16, or all one float8
    encoding (see the module docstring).
    """
    if keys.device.type != "cuda":
        return None
    ks = keys.shape
    if len(ks) != 3 or values.ndim != 3 or queries.shape != ks:
        return None
    n, t, key_dim = ks
    value_dim = values.shape[2]
    f32 = torch.float32
    kdt = keys.dtype
    if kdt == f32:
        bf16 = False
        if values.dtype != f32 or queries.dtype != f32:
            return None
    else:
        bf16 = (kdt == torch.bfloat16 or kdt in _FP8_FORMATS) and values.dtype == kdt and queries.dtype == kdt
        if not bf16:
            return None
    if ((key_dim, value_dim) not in _SUPPORTED or values.shape[:2] != ks[:2]
            or decay.dtype != f32 or process.dtype != f32 or observation.dtype != f32
            or initial_mean.dtype != f32 or initial_covariance.dtype != f32):
        return None
    extension = _load_extension(key_dim)
    if extension is None:
        return None
    if (decay.shape != (n, t, key_dim) or process.shape != (n, t) or observation.shape != (n, t)
            or initial_mean.shape != (n, key_dim, value_dim)
            or initial_covariance.shape != (n, key_dim, key_dim)):
        return None
    dev = keys.device
    _check(values.device == dev and queries.device == dev and decay.device == dev and process.device == dev
           and observation.device == dev and initial_mean.device == dev and initial_covariance.device == dev,
           "fused Bayesian inputs must share one device")
    # .contiguous() as the reference (fused_cuda.py:376-383); the check first
    # skips a dispatcher round trip per tensor on the common contiguous case.
    keys, values, queries, decay, process, observation, initial_mean, initial_covariance = (
        x if x.is_contiguous() else x.contiguous()
        for x in (keys, values, queries, decay, process, observation, initial_mean, initial_covariance))
    if bf16:
        if _bf16_kernels_apply(keys, values, queries):
            return _ChunkedBayesianBF16Function.apply(
                keys, values, queries, decay, process, observation, initial_mean, initial_covariance,
                float(denominator_floor), bool(fixed_dynamics))
        keys, values, queries = keys.float(), values.float(), queries.float()
    return _ChunkedBayesianFunction.apply(
        keys, values, queries, decay, process, observation, initial_mean, initial_covariance,
        int(chunk_length), float(denominator_floor), bool(fixed_dynamics),
    )


class _ChunkedRotationFunction(torch.autograd.Function):
    """Rotation dynamics on the HIP kernels (C ABI ``bssm_*_chunked_rotation``).

    The reference runs its rotation core (bayesian_layer.py:254-323) through
    torch.compile; here one forward and one checkpoint-replay backward kernel
    replace it, with the same autograd results.
    """

    @staticmethod
    def forward(ctx, keys, values, queries, radii, angles, process, observation, initial_mean, initial_covariance,
                denominator_floor):
        n, t, d = keys.shape
        m = values.shape[-1]
        interval = int(_hip.load().bssm_rotation_checkpoint(d))
        nb = -(-t // interval)
        dev = keys.device
        out = torch.empty(n, t, m, device=dev, dtype=torch.float32)
        mean_t = torch.empty(n, d, m, device=dev, dtype=torch.float32)
        cov_t = torch.empty(n, d, d, device=dev, dtype=torch.float32)
        bmean = torch.empty(n, nb + 1, d, m, device=dev, dtype=torch.float32)
        bcov = torch.empty(n, nb + 1, d, d, device=dev, dtype=torch.float32)
        P = _hip.ptr
        with _hip.on_device(dev):
            _hip.call("bssm_forward_chunked_rotation", d, m, P(keys), P(values), P(queries), P(radii), P(angles),
                      P(process), P(observation), P(initial_mean), P(initial_covariance), P(out), P(mean_t),
                      P(cov_t), P(bmean), P(bcov), n, t, interval, float(denominator_floor), _hip.stream_of(dev))
        ctx.save_for_backward(keys, values, queries, radii, angles, process, observation, initial_mean,
                              initial_covariance, bmean, bcov)
        ctx.interval = interval
        ctx.denominator_floor = float(denominator_floor)
        ctx.set_materialize_grads(False)
        return out, mean_t, cov_t

    @staticmethod
    def backward(ctx, grad_output, grad_mean, grad_covariance):
        keys, values, queries, radii, angles, process, observation, mean0, cov0, bmean, bcov = ctx.saved_tensors
        n, t, d = keys.shape
        m = values.shape[-1]
        need = ctx.needs_input_grad
        grad_output = (torch.zeros(n, t, m, device=keys.device, dtype=torch.float32) if grad_output is None
                       else grad_output.contiguous())
        gm = None if grad_mean is None else grad_mean.contiguous()
        gc = None if grad_covariance is None else grad_covariance.contiguous()
        grads = [torch.empty_like(x) for x in (keys, values, queries, radii, angles, process, observation)]
        gm0 = torch.empty_like(mean0) if need[7] else None
        gc0 = torch.empty_like(cov0) if need[8] else None
        P = _hip.ptr
        with _hip.on_device(keys.device):
            _hip.call("bssm_backward_chunked_rotation", d, m, P(keys), P(values), P(queries), P(radii), P(angles),
                      P(process), P(observation), P(mean0), P(cov0), P(bmean), P(bcov), P(grad_output), P(gm),
                      P(gc), *map(P, grads), P(gm0), P(gc0), n, t, ctx.interval, ctx.denominator_floor,
                      _hip.stream_of(keys.device))
        return (*(g if need[i] else None for i, g in enumerate(grads)), gm0, gc0, None)


_ROTATION_SHAPES = ((2, 8), (4, 8), (8, 8))


def fused_rotation_bayesian(
    keys: Tensor,
    values: Tensor,
    queries: Tensor,
    radii: Tensor,
    angles: Tensor,
    process: Tensor,
    observation: Tensor,
    initial_mean: Tensor,
    initial_covariance: Tensor,
    *,
    denominator_floor: float,
) -> tuple[Tensor, Tensor, Tensor] | None:
    """Rotation-dynamics core on the HIP kernels; ``None`` means "use the torch path".

    Contract: CUDA float32 tensors, keys/queries [N,T,D] with (D, M) in
    {(2,8), (4,8), (8,8)}, values [N,T,M], radii/angles/process (per pair)
    [N,T,D/2], observation [N,T], initial mean [N,D,M] and covariance [N,D,D].
    """
    tensors = (keys, values, queries, radii, angles, process, observation, initial_mean, initial_covariance)
    if keys.device.type != "cuda" or keys.ndim != 3 or not all(x.dtype == torch.float32 for x in tensors):
        return None
    n, t, d = keys.shape
    m = values.shape[-1]
    if (d, m) not in _ROTATION_SHAPES or os.environ.get("BAYES_SSM_DISABLE_FUSED_CUDA", "0") == "1":
        return None
    expect = ((n, t, d), (n, t, m), (n, t, d), (n, t, d // 2), (n, t, d // 2), (n, t, d // 2), (n, t), (n, d, m),
              (n, d, d))
    if any(tuple(x.shape) != e for x, e in zip(tensors, expect)):
        return None
    _hip.load()
    return _ChunkedRotationFunction.apply(*(x.contiguous() for x in tensors), float(denominator_floor))


__all__ = ["fused_diagonal_bayesian", "fused_rotation_bayesian"]
