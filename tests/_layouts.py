"""Forcing one wave layout of the D4M8 float32 kernels through the C ABI.

The library runs the row-per-sequence kernels (a 16-lane row per sequence) up
to its small-batch limits and the rotated-layout kernels (a quad per
sequence) above them; the bf16 and float8 entry points always use the
rotated layout.  Tests that compare those bit for bit with the float32
kernels, or that cover one layout on purpose, pick it here.
"""
from __future__ import annotations

import contextlib

BIG = 1 << 40
# Limits (forward row, backward row, forward two-wave, backward three-wave,
# rotation forward row) per layout.
LAYOUTS = {"row": (BIG, BIG, 0, 0, BIG), "split": (BIG, BIG, BIG, BIG, BIG), "quad": (0, 0, 0, 0, 0)}


@contextlib.contextmanager
def layout(name):
    """Force the D4 kernels of one layout, restoring the limits after."""
    from bayes_ssm import _hip

    lib = _hip.load()
    old = [lib.bssm_small_batch_limit(d, v) for d, v in enumerate(LAYOUTS[name])]
    try:
        yield
    finally:
        for d, v in enumerate(old):
            lib.bssm_small_batch_limit(d, v)
