"""ctypes binding of the gfx950 HIP library ``libbssm_hip.so`` (C ABI in include/bssm.h).

The library is prebuilt in-tree by ``bayes-ssm_amd/build.py``; nothing is
compiled at import or first call (the reference JIT-compiles its ``.cu`` files
through ``torch.utils.cpp_extension.load``, bayes_ssm/fused_cuda.py:23-55).
PyTorch only supplies device memory and the current stream: every entry point
receives raw device pointers and the ``hipStream_t`` of
``torch.cuda.current_stream()``.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from pathlib import Path
from typing import Optional

import torch
from torch import Tensor

LIB_PATH = Path(__file__).with_name("libbssm_hip.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

# name -> argtypes (all return int status).  Order mirrors include/bssm.h.
_FWD = [_I, _I] + [_P] * 8 + [_P] * 5 + [_L, _L, _L, _F, _P]
_FWD_SAVED = [_I, _I] + [_P] * 8 + [_P] * 5 + [_P] * 5 + [_L, _L, _L, _F, _P]
_BWD_HEAD = [_I, _I] + [_P] * 10 + [_P] * 3
_BWD_FULL = _BWD_HEAD + [_P] * 8 + [_L, _L, _L, _F, _P]
_BWD_SIX = _BWD_HEAD + [_P] * 6 + [_L, _L, _L, _F, _P]
_BWD_LEAN = _BWD_HEAD + [_P] * 3 + [_L, _L, _L, _F, _P]
_BWD_SAVED_HEAD = [_I, _I] + [_P] * 10 + [_P] * 5 + [_P] * 3
_SIGNATURES = {
    "bssm_forward_chunked": _FWD,
    "bssm_forward_chunked_fixed": _FWD,
    "bssm_forward_chunked_saved": _FWD_SAVED,
    "bssm_backward_chunked": _BWD_FULL,
    "bssm_backward_chunked_lean": _BWD_LEAN,
    "bssm_backward_chunked_noinitial": _BWD_SIX,
    "bssm_backward_chunked_fixed": _BWD_FULL,
    "bssm_backward_chunked_lean_fixed": _BWD_LEAN,
    "bssm_backward_chunked_noinitial_fixed": _BWD_SIX,
    "bssm_backward_chunked_saved": _BWD_SAVED_HEAD + [_P] * 8 + [_L, _L, _L, _F, _P],
    "bssm_backward_chunked_saved_lean": _BWD_SAVED_HEAD + [_P] * 3 + [_L, _L, _L, _F, _P],
    "bssm_forward_chunked_bf16": [_I, _I, _I] + [_P] * 8 + [_P] * 5 + [_L, _L, _L, _F, _P],
    "bssm_backward_chunked_bf16": [_I, _I, _I] + [_P] * 10 + [_P] * 3 + [_P] * 8 + [_L, _L, _L, _F, _P],
    "bssm_forward_chunked_fp8": [_I, _I, _I, _I] + [_P] * 8 + [_P] * 5 + [_L, _L, _L, _F, _P],
    "bssm_backward_chunked_fp8": [_I, _I, _I, _I] + [_P] * 10 + [_P] * 3 + [_P] * 8 + [_L, _L, _L, _F, _P],
    "bssm_round_float8": [_I, _P, _P, _L],
    "bssm_value_stats_workspace": [_I, _P],
    "bssm_value_stats": [_I, _P, _P, _P, _P, _L, _P, _P],
    "bssm_associative_static_scan": [_P] * 9 + [_L, _L, _I, _I, _P],
    "bssm_associative_static_scan_backward": [_P] * 16 + [_L, _L, _I, _I, _P],
    "bssm_mixer_forward": [_P, _L] * 5 + [_P] * 7 + [_L, _L, _L, _L, _F, _P],
    "bssm_mixer_backward": [_P, _L] * 5 + [_P] * 7 + [_P] * 7 + [_L, _L, _L, _L, _F, _I, _P],
    "bssm_mixer_gated_forward": [_P, _L] * 6 + [_P, _F] + [_P] * 8 + [_L, _L, _L, _L, _F, _I, _P],
    "bssm_rotation_checkpoint": [_I],
    "bssm_small_batch_limit": [_I, _L],
    "bssm_forward_chunked_rotation": [_I, _I] + [_P] * 9 + [_P] * 5 + [_L, _L, _L, _F, _P],
    "bssm_backward_chunked_rotation": [_I, _I] + [_P] * 9 + [_P] * 5 + [_P] * 9 + [_L, _L, _L, _F, _P],
    "bssm_causal_conv4_forward": [_I, _P, _L, _P, _P, _L, _L, _L, _P],
    "bssm_causal_conv4_backward": [_I, _P, _L, _P, _P, _P, _P, _L, _L, _L, _P],
    "bssm_causal_conv4_backward_noalloc": [_I, _P, _L, _P, _P, _P, _P, _L, _L, _L, _P],
    "bssm_mixer_gated_backward": [_P, _L] * 6 + [_P, _F] + [_P] * 8 + [_P] * 9 + [_L, _L, _L, _L, _F, _I, _P],
    "bssm_mixer_block_forward": [_P, _L, _P, _P, _P, _F] + [_P] * 9 + [_L, _L, _L, _L, _F, _P],
    "bssm_mixer_block_backward": [_P, _L, _P, _P, _P, _P, _F] + [_P] * 10 + [_L] + [_P] * 6 + [_I]
                                 + [_P] * 2 + [_L, _L, _L, _L, _F, _P],
    "bssm_supported": [_I, _I],
    "bssm_preferred_checkpoint": [_I],
    "bssm_abi_version": [],
}
ABI_VERSION = 9

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[Exception] = None


class HipLibraryError(RuntimeError):
    """The HIP library is missing, stale or rejected a call."""


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise ``HipLibraryError`` if unusable."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if _load_error is not None:
            raise HipLibraryError(str(_load_error)) from _load_error
        try:
            path = os.environ.get("BSSM_HIP_LIBRARY", str(LIB_PATH))
            if not Path(path).exists():
                raise HipLibraryError(
                    f"{path} is missing; build it with `python bayes-ssm_amd/build.py`")
            lib = ctypes.CDLL(path)
            for name, argtypes in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int
            lib.bssm_value_stats_workspace.restype = ctypes.c_int64
            lib.bssm_small_batch_limit.restype = ctypes.c_int64
            lib.bssm_last_error.argtypes = []
            lib.bssm_last_error.restype = ctypes.c_char_p
            version = lib.bssm_abi_version()
            if version != ABI_VERSION:
                raise HipLibraryError(f"{path} has ABI {version}, expected {ABI_VERSION}; rebuild it")
        except Exception as exc:  # cache the failure, re-raise loudly every time
            _load_error = exc
            raise HipLibraryError(str(exc)) from exc
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except HipLibraryError:
        return False


def ptr(x: Optional[Tensor]) -> Optional[int]:
    return None if x is None else x.data_ptr()


def stream_of(device: torch.device) -> int:
    """The ``hipStream_t`` of torch's current stream on ``device``."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def on_device(device: torch.device):
    """Context that makes ``device`` current for a launch (a no-op when it already is)."""
    if device.index is None or device.index == torch._C._cuda_getDevice():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


_functions: dict = {}


def function(name: str):
    """The ctypes function object of entry point ``name`` (looked up once per process)."""
    fn = _functions.get(name)
    if fn is None:
        fn = _functions.setdefault(name, getattr(load(), name))
    return fn


def _raise(name: str, rc: int) -> None:
    msg = load().bssm_last_error().decode(errors="replace")
    raise RuntimeError(f"{name} failed (code {rc}): {msg}")


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise ``RuntimeError`` with the library message on failure."""
    rc = function(name)(*args)
    if rc != 0:
        _raise(name, rc)


def launch(device: torch.device, name: str, *args) -> None:
    """``call`` with ``device`` current; the common case (already current) enters no context."""
    index = device.index
    if index is None or index == torch._C._cuda_getDevice():
        rc = function(name)(*args)
    else:
        with torch.cuda.device(index):
            rc = function(name)(*args)
    if rc != 0:
        _raise(name, rc)


def supported(key_dim: int, value_dim: int) -> bool:
    return bool(load().bssm_supported(int(key_dim), int(value_dim)))


_preferred: dict[int, int] = {}


def preferred_checkpoint(key_dim: int) -> int:
    # A property of the built kernels: asked once per key dimension.
    key_dim = int(key_dim)
    value = _preferred.get(key_dim)
    if value is None:
        value = _preferred.setdefault(key_dim, int(load().bssm_preferred_checkpoint(key_dim)))
    return value
