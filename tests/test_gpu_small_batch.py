"""D4M8 float32 kernels in both wave layouts: the row-per-sequence kernels
(a 16-lane row per sequence, used up to the small-batch limits) and the
rotated-layout kernels (a quad per sequence), each forced through the C ABI's
``bssm_small_batch_limit`` and checked against the float64 oracle.

The library picks the layout from the sequence count, so at the parity
tests' sizes the other files see the row kernels; here both layouts run the
same cases.  Tolerance (north star): 1e-5 relative, 1e-4 absolute; checkpoint
indexing and chunk invariance bit-exact.
"""
from __future__ import annotations

import contextlib

import pytest
import torch

from oracle import bssm_oracle as O
from tests.test_gpu_floor import NAMES, _check, _floor_case, _run_abi
from tests._layouts import LAYOUTS, layout
from tests.test_gpu_parity import ABIS, _case, _fixed_dynamics, _oracle_forward, close

pytestmark = pytest.mark.gpu

def _ext():
    from bayes_ssm import fused_cuda

    e = fused_cuda._load_extension(4)
    assert e is not None
    return e


def _forward(ext, dev, fixed, chunk, floor=1e-6):
    fn = ext.forward_chunked_fixed if fixed else ext.forward_chunked
    return fn(dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], chunk, floor)


def _backward(ext, name, fixed, nout, dev, bm, bc, chunk, final_grads, floor=1e-6):
    gmf = dev["gmf"] if final_grads else None
    gcf = dev["gcf"] if final_grads else None
    args = (dev["k"], dev["v"], dev["q"], dev["d"], dev["p"], dev["r"], dev["m0"], dev["c0"], bm, bc, dev["gy"], gmf,
            gcf, chunk, floor)
    if hasattr(ext, name):
        return getattr(ext, name)(*args)
    return ext._backward("bssm_" + name, fixed, nout, *args[:8], bm, bc, (), dev["gy"], gmf, gcf, chunk, floor)


# Both layouts need T a multiple of 4 (other T take the generic kernels).
# T = 4, 20 and 52: partial last tiles (the row backward needs T a multiple of
# 16, so there the backward keeps the rotated layout); N = 37, 6 and 1 leave
# idle rows in the last wave.
@pytest.mark.parametrize("name", list(LAYOUTS))
@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("chunk", [1, 8, 13])
@pytest.mark.parametrize("n,t", [(37, 16), (37, 20), (37, 52), (1, 64), (6, 4)])
def test_layout_forward_matches_oracle(cuda_device, name, fixed, chunk, n, t):
    print(f"layout {name} forward fixed={fixed} chunk={chunk} n={n} t={t}", flush=True)
    cpu, dev = _case(n, t, 4, seed=11 * chunk + t, device=cuda_device)
    with layout(name):
        y, mT, cT, bm, bc = _forward(_ext(), dev, fixed, chunk)
        torch.cuda.synchronize()
    ref = _fixed_dynamics(cpu) if fixed else cpu
    ey, em, ec = _oracle_forward(ref, False)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    f64 = {k: x.double() for k, x in ref.items()}
    ebm, ebc = O.checkpoints(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                             chunk, 1e-6)
    close(bm, ebm, "bmean")
    close(bc, ebc, "bcov")
    nb = -(-t // chunk)
    assert torch.equal(bm[:, nb].cpu(), mT.cpu()) and torch.equal(bc[:, nb].cpu(), cT.cpu())
    assert torch.equal(bm[:, 0].cpu(), dev["m0"].cpu())


@pytest.mark.parametrize("name", list(LAYOUTS))
@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
@pytest.mark.parametrize("final_grads", [False, True])
@pytest.mark.parametrize("n,t", [(37, 16), (37, 48), (5, 64), (37, 52)])
def test_layout_backward_matches_oracle(cuda_device, name, abi, final_grads, n, t):
    abi_name, fixed, nout = abi
    print(f"layout {name} backward {abi_name} final_grads={final_grads} n={n} t={t}", flush=True)
    cpu, dev = _case(n, t, 4, seed=3 * t + n, device=cuda_device)
    ext = _ext()
    with layout(name):
        _, _, _, bm, bc = _forward(ext, dev, fixed, 8)
        grads = _backward(ext, abi_name, fixed, nout, dev, bm, bc, 8, final_grads)
        torch.cuda.synchronize()
    assert len(grads) == nout
    ref = _fixed_dynamics(cpu) if fixed else cpu
    f64 = {k: x.double() for k, x in ref.items()}
    _, _, _, eg = O.diagonal_grads(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"], f64["c0"],
                                   f64["gy"], f64["gmf"] if final_grads else None,
                                   f64["gcf"] if final_grads else None)
    for i in range(nout):
        if fixed and NAMES[i] in ("gd", "gp", "gr"):
            assert torch.count_nonzero(grads[i]) == 0, f"{NAMES[i]} must be zero for fixed dynamics"
            continue
        close(grads[i], eg[i], NAMES[i])


@pytest.mark.parametrize("name", list(LAYOUTS))
@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
def test_layout_floor_active(cuda_device, name, abi):
    """The innovation floor on a share of the tokens, and the strict gate at tokens exactly at it."""
    abi_name, fixed, nout = abi
    print(f"layout {name} floor {abi_name}", flush=True)
    cpu, dev, floor = _floor_case(29, 64, 4, seed=41, device=cuda_device, fixed=fixed)
    with layout(name):
        outs, grads = _run_abi(_ext(), abi_name, fixed, nout, dev, 8, floor)
    _check(cpu, fixed, floor, outs, grads, nout)


@pytest.mark.parametrize("name", ["row", "split"])
@pytest.mark.parametrize("fixed", [False, True])
def test_row_layout_chunk_invariance_and_symmetry(cuda_device, name, fixed):
    """Row forward (one or two waves): outputs bitwise identical for every chunk, checkpoint c = state before
    token c * chunk, and the covariance bitwise symmetric."""
    print(f"{name} chunk invariance fixed={fixed}", flush=True)
    _, dev = _case(9, 80, 4, seed=5, device=cuda_device)
    ext = _ext()
    with layout(name):
        runs = {c: _forward(ext, dev, fixed, c) for c in (1, 4, 8, 16, 80, 200)}
        torch.cuda.synchronize()
    for c, out in runs.items():
        for a, b in zip(out[:3], runs[8][:3]):
            assert torch.equal(a, b), f"chunk {c} changes the recurrence"
    for c in (4, 8, 16, 80):
        assert torch.equal(runs[c][3], runs[1][3][:, ::c]), f"bmean layout chunk {c}"
        assert torch.equal(runs[c][4], runs[1][4][:, ::c]), f"bcov layout chunk {c}"
    cT, bc = runs[8][2], runs[1][4]
    assert torch.equal(cT, cT.transpose(-1, -2))
    assert torch.equal(bc, bc.transpose(-1, -2))


@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("chunk", [1, 8, 13])
# N = 1029 and 1028: above 1024 sequences two groups of 4 share a workgroup (the last workgroup's second group
# holds one sequence, or none).
@pytest.mark.parametrize("n,t", [(1, 16), (7, 20), (37, 52), (9, 64), (6, 4), (33, 512), (1029, 20), (1028, 16)])
def test_two_wave_forward_is_bitwise_the_one_wave_forward(cuda_device, fixed, chunk, n, t):
    """The covariance / mean split over two waves performs the one-wave kernel's operations in its order."""
    print(f"two-wave forward n={n} t={t} chunk={chunk} fixed={fixed}", flush=True)
    _, dev = _case(n, t, 4, seed=n + t + chunk, device=cuda_device)
    ext = _ext()
    outs = {}
    for name in ("row", "split"):
        with layout(name):
            outs[name] = [x.clone() for x in _forward(ext, dev, fixed, chunk)]
            torch.cuda.synchronize()
    for lab, a, b in zip(("y", "mean_T", "cov_T", "bmean", "bcov"), outs["row"], outs["split"]):
        assert torch.equal(a, b), lab


@pytest.mark.parametrize("abi", ABIS, ids=[a[0] for a in ABIS])
@pytest.mark.parametrize("final_grads", [False, True])
@pytest.mark.parametrize("n,t", [(1, 16), (7, 32), (37, 48), (9, 64), (33, 512), (1029, 32), (1028, 16)])
def test_three_wave_backward_is_bitwise_the_one_wave_backward(cuda_device, abi, final_grads, n, t):
    """The covariance replay / covariance reverse / mean split over three waves performs the one-wave
    kernel's operations in its order."""
    abi_name, fixed, nout = abi
    print(f"three-wave backward {abi_name} final_grads={final_grads} n={n} t={t}", flush=True)
    _, dev = _case(n, t, 4, seed=5 * n + t, device=cuda_device)
    ext = _ext()
    outs = {}
    for name in ("row", "split"):
        with layout(name):
            _, _, _, bm, bc = _forward(ext, dev, fixed, 8)
            outs[name] = [g.clone() for g in _backward(ext, abi_name, fixed, nout, dev, bm, bc, 8, final_grads)]
            torch.cuda.synchronize()
    for lab, a, b in zip(NAMES, outs["row"], outs["split"]):
        assert torch.equal(a, b), lab


NARROW = {"bf16": (torch.bfloat16, None), "e4m3": (torch.float8_e4m3fn, 0), "e5m2": (torch.float8_e5m2, 1)}


@pytest.mark.parametrize("fmt", list(NARROW))
@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("n,t,chunk", [(37, 52, 8), (5, 64, 13), (9, 16, 1), (2, 4, 8), (1029, 16, 8)])
def test_row_forward_narrow_inputs_equal_float32(cuda_device, fmt, fixed, n, t, chunk):
    """The two-wave row forward with bf16 / float8 keys, values and queries (widened on chip, exactly) gives bit
    for bit the row forward on the widened float32 values; bf16 / float8 streams take it at these sizes by
    default."""
    from bayes_ssm import _hip

    name = "split"
    print(f"narrow row forward {fmt} fixed={fixed} n={n} t={t} chunk={chunk}", flush=True)
    dtype, code = NARROW[fmt]
    _, dev = _case(n, t, 4, seed=7 * n + t, device=cuda_device)
    for x in "kvq":
        dev[x + "h"] = dev[x].to(dtype).contiguous()
        dev[x] = dev[x + "h"].float().contiguous()
    P = _hip.ptr
    with layout(name):
        ref = _forward(_ext(), dev, fixed, chunk)
        out = [torch.empty_like(x) for x in ref]
        head = ("bssm_forward_chunked_bf16", 4, 8, int(fixed)) if code is None else \
            ("bssm_forward_chunked_fp8", 4, 8, int(fixed), code)
        _hip.call(*head, P(dev["kh"]), P(dev["vh"]), P(dev["qh"]), P(dev["d"]), P(dev["p"]), P(dev["r"]),
                  P(dev["m0"]), P(dev["c0"]), *[P(x) for x in out], n, t, chunk, 1e-6, _hip.stream_of(cuda_device))
        torch.cuda.synchronize()
    for lab, a, b in zip(("y", "mean_T", "cov_T", "bmean", "bcov"), out, ref):
        assert torch.equal(a, b), lab


@pytest.mark.parametrize("fmt", list(NARROW))
@pytest.mark.parametrize("fixed,dyn", [(False, True), (False, False), (True, False)])
@pytest.mark.parametrize("n,t", [(37, 48), (5, 16), (9, 64), (1029, 16)])
def test_row_backward_narrow_inputs_equal_float32(cuda_device, fmt, fixed, dyn, n, t):
    """The three-wave row backward with bf16 / float8 keys, values and queries: gk, gv, gq are the float32 row
    backward's gradients on the widened values rounded as torch rounds them (.to(dtype)); every other gradient
    is bit for bit the float32 one."""
    from bayes_ssm import _hip

    print(f"narrow row backward {fmt} fixed={fixed} dyn={dyn} n={n} t={t}", flush=True)
    dtype, code = NARROW[fmt]
    _, dev = _case(n, t, 4, seed=3 * n + t, device=cuda_device)
    for x in "kvq":
        dev[x + "h"] = dev[x].to(dtype).contiguous()
        dev[x] = dev[x + "h"].float().contiguous()
    P = _hip.ptr
    ext = _ext()
    with layout("split"):
        _, _, _, bm, bc = _forward(ext, dev, fixed, 8)
        name = "backward_chunked" + ("" if dyn or fixed else "_lean") + ("_fixed" if fixed else "")
        nout = 8 if (dyn or fixed) else 3
        ref = _backward(ext, name, fixed, nout, dev, bm, bc, 8, True)
        gk, gv, gq = (torch.empty_like(dev[x + "h"]) for x in "kvq")
        gd, gp, gr = ((torch.empty_like(dev[x]) for x in "dpr") if nout == 8 else (None, None, None))
        gm0, gc0 = torch.empty_like(dev["m0"]), torch.empty_like(dev["c0"])
        head = ("bssm_backward_chunked_bf16", 4, 8, int(fixed)) if code is None else \
            ("bssm_backward_chunked_fp8", 4, 8, int(fixed), code)
        _hip.call(*head, P(dev["kh"]), P(dev["vh"]), P(dev["qh"]), P(dev["d"]), P(dev["p"]), P(dev["r"]),
                  P(dev["m0"]), P(dev["c0"]), P(bm), P(bc), P(dev["gy"]), P(dev["gmf"]), P(dev["gcf"]),
                  P(gk), P(gv), P(gq), P(gd), P(gp), P(gr), P(gm0), P(gc0), n, t, 8, 1e-6,
                  _hip.stream_of(cuda_device))
        torch.cuda.synchronize()
    for lab, a, b in (("gk", gk, ref[0]), ("gv", gv, ref[1]), ("gq", gq, ref[2])):
        assert a.dtype == dtype
        assert torch.equal(a.view(torch.uint8) if a.element_size() == 1 else a, b.to(dtype).view(torch.uint8)
                           if a.element_size() == 1 else b.to(dtype)), lab
    if nout == 8:
        for lab, a, b in zip(("gd", "gp", "gr", "gm0", "gc0"), (gd, gp, gr, gm0, gc0), ref[3:]):
            assert torch.equal(a, b), lab


def test_layouts_at_many_sequences(cuda_device):
    """4099 sequences (a partial last wave): both layouts match the oracle on every output and gradient, and
    the default limits route this size to the row kernels (whose results differ from the rotated ones in the
    last bits)."""
    print("layouts n=4099 t=64", flush=True)
    cpu, dev = _case(4099, 64, 4, seed=9, device=cuda_device)
    ext = _ext()
    res = {}
    for name in ("row", "quad", None):
        with (layout(name) if name else contextlib.nullcontext()):
            y, mT, cT, bm, bc = _forward(ext, dev, False, 8)
            grads = _backward(ext, "backward_chunked", False, 8, dev, bm, bc, 8, True)
            torch.cuda.synchronize()
        res[name] = [y, mT, cT, *grads]
    f64 = {k: x.double() for k, x in cpu.items()}
    ey, em, ec, eg = O.diagonal_grads(f64["k"], f64["v"], f64["q"], f64["d"], f64["p"], f64["r"], f64["m0"],
                                      f64["c0"], f64["gy"], f64["gmf"], f64["gcf"])
    labels = ["y", "mean_T", "cov_T"] + NAMES
    for name in ("row", "quad"):
        for lab, a, e in zip(labels, res[name], [ey, em, ec, *eg]):
            close(a, e, f"{name} {lab}")
    for lab, a, b in zip(labels, res[None], res["row"]):
        assert torch.equal(a, b), f"default dispatch at N = 4099 is not the row layout ({lab})"
    assert not torch.equal(res["row"][0], res["quad"][0])
