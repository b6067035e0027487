"""C ABI of libbssm_hip.so — CPU only (loads the library, never launches a kernel)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "bssm.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bssm_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from bayes_ssm import _hip

    return _hip.load()


def test_library_exports_every_declared_symbol(lib):
    names = declared_symbols()
    assert len(names) >= 16
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/bssm.h but not exported"


def test_binding_signatures_cover_header():
    from bayes_ssm import _hip

    missing = [n for n in declared_symbols() if n not in _hip._SIGNATURES and n != "bssm_last_error"]
    assert not missing, missing


def test_abi_version_and_support(lib):
    from bayes_ssm import _hip

    assert lib.bssm_abi_version() == _hip.ABI_VERSION
    for d, m in ((1, 8), (2, 8), (4, 8), (8, 8), (64, 64)):
        assert lib.bssm_supported(d, m) == 1
        assert lib.bssm_preferred_checkpoint(d) > 0
    for d, m in ((3, 8), (4, 4), (64, 8), (8, 64), (16, 8)):
        assert lib.bssm_supported(d, m) == 0
    assert lib.bssm_preferred_checkpoint(3) == 0


def _fwd(lib, d=4, m=8, n=1, t=1, chunk=1, floor=1e-6, null=True):
    return lib.bssm_forward_chunked(d, m, *([None] * 13), n, t, chunk, ctypes.c_float(floor), None)


def test_argument_errors_are_reported(lib):
    assert _fwd(lib, d=3) == 2
    assert b"unsupported" in lib.bssm_last_error()
    assert _fwd(lib, chunk=0) == 1
    assert b"chunk" in lib.bssm_last_error()
    assert _fwd(lib, floor=0.0) == 1
    assert b"floor" in lib.bssm_last_error()
    assert _fwd(lib, n=-1) == 1
    assert _fwd(lib) == 1 and b"null" in lib.bssm_last_error()
    # Nothing to do: success without touching a device.
    assert _fwd(lib, n=0, t=5) == 0
    assert lib.bssm_last_error() == b""


def test_backward_requires_outputs(lib):
    rc = lib.bssm_backward_chunked(4, 8, *([None] * 21), 2, 3, 1, ctypes.c_float(1e-6), None)
    assert rc == 1 and b"required" in lib.bssm_last_error()
    rc = lib.bssm_forward_chunked_saved(1, 8, *([None] * 18), 2, 3, 2, ctypes.c_float(1e-6), None)
    assert rc == 1 and b"full-sequence" in lib.bssm_last_error()
    rc = lib.bssm_associative_static_scan(*([None] * 9), 1, 4, 40, 4, None)
    assert rc == 2


def test_python_wrapper_raises_runtime_error():
    from bayes_ssm import _hip

    with pytest.raises(RuntimeError, match="chunk must be positive"):
        _hip.call("bssm_forward_chunked", 4, 8, *([None] * 13), 1, 1, 0, 1e-6, None)


def test_extension_method_sets_match_reference():
    """Per-key-dim method names of the reference pybind modules."""
    from bayes_ssm import fused_cuda

    ext1 = fused_cuda._load_extension(1)
    ext2 = fused_cuda._load_extension(2)
    ext4 = fused_cuda._load_extension(4)
    for name in ("forward_chunked_saved", "backward_chunked_saved", "backward_chunked_saved_lean",
                 "backward_chunked_saved_d1"):
        assert hasattr(ext1, name) and not hasattr(ext4, name)
    for name in ("backward_chunked_noinitial", "backward_chunked_noinitial_fixed"):
        assert hasattr(ext2, name) and not hasattr(ext4, name) and not hasattr(ext1, name)
    ext64 = fused_cuda._load_extension(64)
    for ext in (ext1, ext2, ext4, fused_cuda._load_extension(8), ext64):
        for name in ("forward_chunked", "forward_chunked_fixed", "backward_chunked", "backward_chunked_lean",
                     "backward_chunked_fixed", "backward_chunked_lean_fixed"):
            assert hasattr(ext, name)
    # persistent_bayes_chunked.cu:436 exports no saved-history or no-initial variants.
    for name in ("forward_chunked_saved", "backward_chunked_saved", "backward_chunked_noinitial"):
        assert not hasattr(ext64, name)
    assert ext64.value_dim == 64
    assert fused_cuda._load_extension(3) is None
    assert fused_cuda._load_extension(16) is None


def test_disable_env(monkeypatch):
    from bayes_ssm import fused_cuda

    monkeypatch.setenv("BAYES_SSM_DISABLE_FUSED_CUDA", "1")
    assert fused_cuda._load_extension(4) is None


def test_contract_gate_returns_none_on_cpu():
    import torch

    from bayes_ssm.fused_cuda import fused_diagonal_bayesian

    k = torch.randn(2, 3, 4)
    out = fused_diagonal_bayesian(k, torch.randn(2, 3, 8), k, torch.ones(2, 3, 4), torch.zeros(2, 3),
                                  torch.ones(2, 3), torch.zeros(2, 4, 8), torch.eye(4).expand(2, 4, 4),
                                  chunk_length=2, denominator_floor=1e-6)
    assert out is None


def _mixer_fwd(lib, b=1, t=8, h=16, chunk=8, lds=(64, 64, 128, 64, 32), null=True, floor=1e-6):
    args = []
    for ld in lds:
        args += [None, ld]
    return lib.bssm_mixer_forward(*args, *([None] * 7), b, t, h, chunk, ctypes.c_float(floor), None)


def test_mixer_argument_errors_are_reported(lib):
    assert _mixer_fwd(lib, h=8) == 2 and b"heads" in lib.bssm_last_error()
    assert _mixer_fwd(lib, t=6) == 2
    assert _mixer_fwd(lib, t=0) == 2
    assert _mixer_fwd(lib, chunk=16) == 2
    assert _mixer_fwd(lib, floor=0.0) == 1
    assert _mixer_fwd(lib, b=-1) == 1
    assert _mixer_fwd(lib) == 1 and b"null" in lib.bssm_last_error()
    args = []
    for ld in (64, 64, 128, 64, 32):
        args += [None, ld]
    rc = lib.bssm_mixer_backward(*args, *([None] * 14), 1, 8, 16, 8, ctypes.c_float(1e-6), 0, None)
    assert rc == 1 and b"null" in lib.bssm_last_error()
    # Nothing to do: success without touching a device.
    assert _mixer_fwd(lib, b=0) == 0


def _block_fwd(lib, b=1, t=8, h=16, ld=480, chunk=8):
    return lib.bssm_mixer_block_forward(None, ld, None, None, None, ctypes.c_float(1e-6), *([None] * 9), b, t, h,
                                        chunk, ctypes.c_float(1e-6), None)


def test_block_argument_errors_are_reported(lib):
    assert _block_fwd(lib, h=0) == 1
    assert _block_fwd(lib, ld=472) == 1 and b"30 * heads" in lib.bssm_last_error()
    assert _block_fwd(lib, b=0, h=8, ld=240) == 2 and b"heads" in lib.bssm_last_error()
    assert _block_fwd(lib, b=0, t=6) == 2
    assert _block_fwd(lib) == 1 and b"required" in lib.bssm_last_error()
    assert _block_fwd(lib, b=0) == 0
    def block_bwd(ld_grad, b, aux_bias=None, grad_aux=None, apart=None):
        return lib.bssm_mixer_block_backward(None, 480, None, aux_bias, None, None, ctypes.c_float(1e-6),
                                             *([None] * 10), ld_grad, None, None, apart, None, None, grad_aux, 1,
                                             None, None, b, 8, 16, 8, ctypes.c_float(1e-6), None)

    assert block_bwd(480, 1) == 1 and b"required" in lib.bssm_last_error()
    assert block_bwd(472, 0) == 1 and b"grad_projected" in lib.bssm_last_error()
    # A misaligned bias, and a bias gradient without its partials workspace.
    assert block_bwd(480, 0, aux_bias=8) == 1 and b"aux_bias" in lib.bssm_last_error()
    assert _block_fwd(lib, b=0) == 0
    rc = lib.bssm_mixer_block_forward(None, 480, None, 8, None, ctypes.c_float(1e-6), *([None] * 9), 0, 8, 16, 8,
                                      ctypes.c_float(1e-6), None)
    assert rc == 1 and b"aux_bias" in lib.bssm_last_error()
    assert block_bwd(480, 0, grad_aux=16) == 1 and b"grad_aux_partials" in lib.bssm_last_error()


def test_conv_backward_checks_weight_and_partials_at_t0(lib):
    """With T = 0 the backward still reads the weight and writes the partials: both are required."""
    rc = lib.bssm_causal_conv4_backward(1, None, 8, None, None, None, None, 2, 0, 8, None)
    assert rc == 1 and b"grad_weight_partials" in lib.bssm_last_error()
    # No batch entries or channels: nothing to do, nothing required.
    assert lib.bssm_causal_conv4_backward(1, None, 8, None, None, None, None, 0, 0, 8, None) == 0


def test_conv_backward_noalloc_rejects_sizes_beyond_its_scratch(lib):
    """batch * channels above 524288 (2^21 scratch floats / 4 taps) is refused before any device work."""
    rc = lib.bssm_causal_conv4_backward_noalloc(1, None, 1024, None, None, None, None, 513, 0, 1024, None)
    assert rc == 1 and b"scratch" in lib.bssm_last_error()
    rc = lib.bssm_causal_conv4_backward_noalloc(1, None, 8, None, None, None, None, 4, 0, 8, None)
    assert rc == 1 and b"grad_weight" in lib.bssm_last_error()
    assert lib.bssm_causal_conv4_backward_noalloc(1, None, 8, None, None, None, None, 4, 0, 0, None) == 0


def test_small_batch_limits_read_set_restore(lib):
    """Forward and backward limits of the row-per-sequence D4 kernels: defaults, set, read, restore."""
    old = [lib.bssm_small_batch_limit(d, -1) for d in range(5)]
    assert old == [24576, 8192, 2048, 2048, 32768]
    try:
        assert lib.bssm_small_batch_limit(0, 7) == old[0]
        assert lib.bssm_small_batch_limit(0, -1) == 7
        assert lib.bssm_small_batch_limit(1, -1) == old[1], "directions are independent"
        assert lib.bssm_small_batch_limit(1, 0) == old[1]
        assert lib.bssm_small_batch_limit(1, -1) == 0
        assert lib.bssm_small_batch_limit(2, 3) == old[2] and lib.bssm_small_batch_limit(2, -1) == 3
        assert lib.bssm_small_batch_limit(3, 9) == old[3] and lib.bssm_small_batch_limit(3, -1) == 9
        assert lib.bssm_small_batch_limit(4, 11) == old[4] and lib.bssm_small_batch_limit(4, -1) == 11
    finally:
        for d in range(5):
            lib.bssm_small_batch_limit(d, old[d])
    assert lib.bssm_small_batch_limit(5, 5) == -1 and lib.bssm_small_batch_limit(-1, -1) == -1
    assert [lib.bssm_small_batch_limit(d, -1) for d in range(5)] == old
