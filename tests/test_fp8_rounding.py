"""float32 -> float8 rounding of the float8 gradients (C ABI ``bssm_round_float8``) against torch's conversion.

The kernels round the float32 gradients of float8 keys, values and queries
with the same template this host entry point runs; torch's ``.to(float8_*)``
is what autograd applies to the reference's float32 gradients of promoted
float8 inputs (bayesian_layer.py:823-827).  Checked bit for bit on every
bfloat16-representable float32 (all exponents, signs, NaN and infinities),
the exact ties around every float8 value, and random float32 values.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from bayes_ssm import _hip

FORMATS = {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}


def _round(fmt: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib = _hip.load()
    rc = lib.bssm_round_float8(fmt, x.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p), x.size)
    assert rc == 0, lib.bssm_last_error()
    return out


def _torch(fmt: int, x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(FORMATS[fmt]).view(torch.uint8).numpy()


def _ties(fmt: int) -> np.ndarray:
    """Every float8 value, the midpoints between neighbours and one float32 ulp either side of them."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(FORMATS[fmt]).float().numpy()
    vals = np.unique(np.abs(codes[np.isfinite(codes)]))
    mids = (vals[:-1].astype(np.float64) + vals[1:]) / 2
    top = vals[-1] + (vals[-1] - vals[-2]) / 2  # midpoint above the largest finite value
    mids = np.concatenate([mids, [top]]).astype(np.float32)
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0))])
    base = np.concatenate([vals, mids, near])
    return np.concatenate([base, -base])


@pytest.mark.parametrize("fmt", [0, 1])
def test_float8_rounding_matches_torch(fmt):
    every_bf16 = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    rng = np.random.default_rng(fmt)
    random = np.concatenate([rng.standard_normal(200_000).astype(np.float32) * s
                             for s in (1e-6, 1e-3, 1.0, 100.0, 1e4, 1e6)])
    for name, x in (("bf16 grid", every_bf16), ("ties", _ties(fmt)), ("random", random)):
        got, want = _round(fmt, x), _torch(fmt, x)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"{name}: {bad.size} mismatches, first x={x[bad[0]]!r} got {got[bad[0]]:#x} " \
                              f"want {want[bad[0]]:#x}"


def test_float8_rounding_rejects_bad_arguments():
    lib = _hip.load()
    assert lib.bssm_round_float8(2, None, None, 0) == 1
    assert lib.bssm_round_float8(0, None, None, 4) == 1
    assert lib.bssm_round_float8(0, None, None, 0) == 0
