"""The public API around the hot path on the CPU: ReplaySSM, BayesianLayer and bayesian_layer's branches.

Each case is checked against the float64 oracle (oracle/bssm_oracle.py):
``run_dense`` for dense transitions and process covariances, ``run_diagonal``
for diagonal ones, ``associative_static`` for the static scan; gradients by
autograd through the oracle.  Reference: bayes_ssm/replay_ssm.py:34-145,
bayes_ssm/bayesian_layer.py:735-1085, :1185-1274.  Tolerance (north star):
1e-5 relative, 1e-4 absolute.
"""
from __future__ import annotations

import math

import pytest
import torch

import bayes_ssm
from bayes_ssm import BayesianLayer, ReplaySSM, bayesian_layer
from oracle import bssm_oracle as O

RTOL, ATOL = 1e-5, 1e-4


def close(actual, expected, name="", rtol=RTOL, atol=ATOL):
    torch.testing.assert_close(actual.detach().double(), expected.detach().double(), rtol=rtol, atol=atol,
                               msg=lambda m: f"{name}: {m}")


def _inputs(batch, t, d, m, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(*batch, t, d, generator=g) / d ** 0.5
    v = torch.randn(*batch, t, m, generator=g)
    q = torch.randn(*batch, t, d, generator=g)
    return k, v, q


def _dense_transitions(batch, t, d, seed):
    g = torch.Generator().manual_seed(seed)
    a = 0.9 * torch.eye(d) + 0.1 * torch.randn(*batch, t, d, d, generator=g) / d ** 0.5
    return a


def _oracle_dense(k, v, q, A, Q, r, m0, c0, floor=1e-6):
    return O.run_dense(*(x.double() for x in (k, v, q, A, Q, r, m0, c0)), floor)


# ------------------------------------------------------------------ ReplaySSM
def test_replay_ssm_forward_matches_oracle_and_defaults():
    """ReplaySSM (replay_ssm.py:34-115): q = 0.05, r = 0.2, P0 = I, chunk 64 by default; A = I when not given."""
    layer = ReplaySSM(4, 3)
    assert layer.chunk_length == 64 and layer.denominator_floor == 1e-6
    assert float(layer.process_variance) == pytest.approx(0.05)
    assert float(layer.observation_variance) == pytest.approx(0.2)
    torch.testing.assert_close(layer.initial_covariance, torch.eye(4))
    k, v, q = _inputs((2,), 70, 4, 3, seed=1)
    with torch.no_grad():
        y, mT, cT = layer(k, v, q)
    t = k.shape[-2]
    A = torch.eye(4).expand(2, t, 4, 4)
    Q = 0.05 * torch.eye(4).expand(2, t, 4, 4)
    r = torch.full((2, t), 0.2)
    ey, em, ec = _oracle_dense(k, v, q, A, Q, r, torch.zeros(2, 4, 3), torch.eye(4).expand(2, 4, 4))
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")


def test_replay_ssm_backward_through_replay_matches_oracle(monkeypatch):
    """With grad, every chunk goes through the replay autograd boundary (bayesian_layer.py:616-667)."""
    import importlib

    bl = importlib.import_module("bayes_ssm.bayesian_layer")
    calls = []
    orig = bl._ReplayChunk.apply
    monkeypatch.setattr(bl._ReplayChunk, "apply", staticmethod(lambda *a: calls.append(1) or orig(*a)))
    layer = ReplaySSM(3, 2, chunk_length=16)
    k, v, q = _inputs((2,), 40, 3, 2, seed=2)
    dec = 0.6 + 0.39 * torch.rand(2, 40, 3, generator=torch.Generator().manual_seed(3))
    leaves = [x.clone().requires_grad_(True) for x in (k, v, q, dec)]
    y, mT, cT = layer(*leaves[:3], transition_diagonals=leaves[3])
    gy = torch.randn_like(y)
    (y * gy).sum().backward()
    assert len(calls) == 3, "three chunks of 16, 16 and 8 tokens replay"
    el = [x.double().clone().requires_grad_(True) for x in (k, v, q, dec)]
    A = torch.diag_embed(el[3])
    Q = 0.05 * torch.eye(3, dtype=torch.float64).expand(2, 40, 3, 3)
    ey, _, _ = O.run_dense(el[0], el[1], el[2], A, Q, torch.full((2, 40), 0.2, dtype=torch.float64),
                           torch.zeros(2, 3, 2, dtype=torch.float64), torch.eye(3, dtype=torch.float64).expand(2, 3, 3),
                           1e-6)
    (ey * gy.double()).sum().backward()
    close(y, ey, "y")
    for name, a, e in zip(("k", "v", "q", "decay"), leaves, el):
        close(a.grad, e.grad, "grad " + name)


def test_replay_ssm_associative_scan_cpu_and_static_guard():
    layer = ReplaySSM(4, 4, process_variance=0.0, observation_variance=0.3, initial_covariance=2.0)
    k, v, q = _inputs((3,), 20, 4, 4, seed=4)
    y, mT, cT = layer.associative_scan(k, v, q)
    r = torch.full((3, 20), 0.3, dtype=torch.float64)
    c0 = 2.0 * torch.eye(4, dtype=torch.float64).expand(3, 4, 4)
    ey, em, ec = O.associative_static(k.double(), v.double(), q.double(), r, None, c0)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    # The same scan equals the dense recurrence with A = I, Q = 0.
    with torch.no_grad():
        dy, _, _ = layer(k, v, q)
    close(dy, ey, "dense recurrence")
    with pytest.raises(ValueError, match="process_variance=0"):
        ReplaySSM(4, 4).associative_scan(k, v, q)


@pytest.mark.parametrize("kwargs, message", [
    (dict(key_dim=0, value_dim=2), "key_dim"),
    (dict(key_dim=2, value_dim=True), "value_dim"),
    (dict(key_dim=2, value_dim=2, chunk_length=0), "chunk_length"),
    (dict(key_dim=2, value_dim=2, process_variance=float("nan")), "finite"),
    (dict(key_dim=2, value_dim=2, observation_variance=0.0), "positive"),
    (dict(key_dim=2, value_dim=2, denominator_floor=0.0), "denominator_floor"),
])
def test_replay_ssm_constructor_errors(kwargs, message):
    with pytest.raises(ValueError, match=message):
        ReplaySSM(**kwargs)


# -------------------------------------------------------------- BayesianLayer
def test_bayesian_layer_module_dense_transitions_and_learned_noise():
    """BayesianLayer (bayesian_layer.py:1185-1274): P0 = 3 I, q = r = 0.05, softplus noise parameters."""
    torch.manual_seed(0)
    layer = BayesianLayer(3, 2, learn_noise=True)
    assert float(layer.process_variance.detach()) == pytest.approx(0.05, rel=1e-6)
    assert float(layer.observation_variance.detach()) == pytest.approx(0.05, rel=1e-6)
    assert float(layer.initial_covariance) == 3.0
    k, v, q = _inputs((2,), 25, 3, 2, seed=5)
    A = _dense_transitions((2,), 25, 3, seed=6)
    y, mT, cT = layer(k, v, q, transitions=A, chunk_length=10)
    gy = torch.randn_like(y)
    (y * gy).sum().backward()

    raw_p = torch.tensor(math.log(math.expm1(0.05)), dtype=torch.float64, requires_grad=True)
    raw_r = torch.tensor(math.log(math.expm1(0.05)), dtype=torch.float64, requires_grad=True)
    qv = torch.nn.functional.softplus(raw_p)
    rv = torch.nn.functional.softplus(raw_r)
    Q = qv * torch.eye(3, dtype=torch.float64).expand(2, 25, 3, 3)
    r = rv.expand(2, 25)
    ey, em, ec = O.run_dense(k.double(), v.double(), q.double(), A.double(), Q, r,
                             torch.zeros(2, 3, 2, dtype=torch.float64),
                             3.0 * torch.eye(3, dtype=torch.float64).expand(2, 3, 3), 1e-6)
    (ey * gy.double()).sum().backward()
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    close(layer._process_raw.grad, raw_p.grad, "grad process raw")
    close(layer._observation_raw.grad, raw_r.grad, "grad observation raw")


def test_bayesian_layer_module_zero_process_and_errors():
    layer = BayesianLayer(2, 2, process_variance=0.0)
    assert float(layer.process_variance) == 0.0
    with pytest.raises(ValueError, match="key_dim"):
        layer(torch.zeros(1, 3, 3), torch.zeros(1, 3, 2), torch.zeros(1, 3, 3))
    with pytest.raises(ValueError, match="positive"):
        BayesianLayer(2, 2, observation_variance=0.0)
    with pytest.raises(ValueError, match="learn_noise"):
        BayesianLayer(2, 2, process_variance=0.0, learn_noise=True)


# ------------------------------------------------ bayesian_layer's branches
@pytest.mark.parametrize("optimized", [False, True])
def test_dense_transitions_and_process_covariances(optimized):
    """transitions= and process_covariances= (dense dynamics) against run_dense, both dispatch modes."""
    k, v, q = _inputs((2,), 30, 3, 2, seed=7)
    A = _dense_transitions((2,), 30, 3, seed=8)
    g = torch.Generator().manual_seed(9)
    b = 0.3 * torch.randn(2, 30, 3, 3, generator=g)
    Qc = b @ b.transpose(-1, -2) + 0.01 * torch.eye(3)
    r = 0.2 + torch.rand(2, 30, generator=g)
    leaves = [x.clone().requires_grad_(True) for x in (k, v, q, A, Qc, r)]
    y, mT, cT = bayesian_layer(*leaves[:3], transitions=leaves[3], process_covariances=leaves[4],
                               observation_variances=leaves[5], chunk_length=8, optimized=optimized)
    gy = torch.randn_like(y)
    (y * gy).sum().backward()
    el = [x.double().clone().requires_grad_(True) for x in (k, v, q, A, Qc, r)]
    m0 = torch.zeros(2, 3, 2, dtype=torch.float64)
    c0 = torch.eye(3, dtype=torch.float64).expand(2, 3, 3)
    if optimized:  # the per-token dense core (bayesian_layer.py:184-204)
        ey, em, ec = O.run_dense(*el, m0, c0, 1e-6)
    else:  # the transported-history chunks (:670-732), which symmetrise the prediction
        ey, em, ec = O.run_chunked(*el, m0, c0, 8, 1e-6)
    (ey * gy.double()).sum().backward()
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")
    for name, a, e in zip(("k", "v", "q", "A", "Q", "r"), leaves, el):
        close(a.grad, e.grad, "grad " + name)


def test_replay_flag_matches_plain_autograd():
    """replay_ssm=True gives the same values and gradients as the taped chunk loop."""
    k, v, q = _inputs((3,), 33, 2, 4, seed=10)
    dec = 0.5 + 0.49 * torch.rand(3, 33, 2, generator=torch.Generator().manual_seed(11))
    outs = []
    for replay in (False, True):
        leaves = [x.clone().requires_grad_(True) for x in (k, v, q, dec)]
        y, mT, cT = bayesian_layer(*leaves[:3], transition_diagonals=leaves[3], process_variances=0.1,
                                   observation_variances=0.5, chunk_length=7, optimized=True, replay_ssm=replay)
        (y.sum() + mT.square().sum() + cT.sum()).backward()
        outs.append((y, mT, cT, [x.grad for x in leaves]))
    for a, b in zip(outs[0][:3], outs[1][:3]):
        close(a, b, "value", rtol=1e-6, atol=1e-6)
    for a, b in zip(outs[0][3], outs[1][3]):
        close(a, b, "grad", rtol=1e-5, atol=1e-5)


def test_scalar_noise_and_broadcast_initial_state():
    """Scalar process/observation noise expand to [N, T] (bayesian_layer.py:74-92); a [D, M] mean broadcasts."""
    k, v, q = _inputs((4,), 12, 2, 3, seed=12)
    dec = torch.full((4, 12, 2), 0.9)
    m0 = torch.randn(2, 3, generator=torch.Generator().manual_seed(13))
    y, mT, cT = bayesian_layer(k, v, q, transition_diagonals=dec, process_variances=0.07,
                               observation_variances=torch.tensor(0.4), initial_mean=m0, optimized=True)
    ey, em, ec = O.run_diagonal(k.double(), v.double(), q.double(), dec.double(),
                                torch.full((4, 12), 0.07, dtype=torch.float64),
                                torch.full((4, 12), 0.4, dtype=torch.float64), m0.double().expand(4, 2, 3),
                                torch.eye(2, dtype=torch.float64).expand(4, 2, 2), 1e-6)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")


def test_low_precision_inputs_are_promoted():
    """fp16 / bf16 inputs are promoted to float32 (bayesian_layer.py:823-827)."""
    k, v, q = _inputs((2,), 10, 2, 2, seed=14)
    dec = torch.full((2, 10, 2), 0.95)
    for dt in (torch.float16, torch.bfloat16):
        y, mT, cT = bayesian_layer(k.to(dt), v.to(dt), q.to(dt), transition_diagonals=dec, optimized=True)
        assert y.dtype == torch.float32 and mT.dtype == torch.float32
        ey, _, _ = O.run_diagonal(*(x.to(dt).double() for x in (k, v, q)), dec.double(),
                                  torch.zeros(2, 10, dtype=torch.float64), torch.ones(2, 10, dtype=torch.float64),
                                  torch.zeros(2, 2, 2, dtype=torch.float64),
                                  torch.eye(2, dtype=torch.float64).expand(2, 2, 2), 1e-6)
        close(y, ey, f"y {dt}")


def test_optimized_false_is_the_transported_history_path():
    """optimized=False runs the chunk algorithm of bayesian_layer.py:670-732 (oracle run_chunked)."""
    k, v, q = _inputs((2,), 21, 3, 2, seed=15)
    dec = 0.7 + 0.29 * torch.rand(2, 21, 3, generator=torch.Generator().manual_seed(16))
    y, mT, cT = bayesian_layer(k, v, q, transition_diagonals=dec, process_variances=0.05,
                               observation_variances=0.3, chunk_length=5, optimized=False)
    A, Q = O.diagonal_as_dense(dec.double(), torch.full((2, 21), 0.05, dtype=torch.float64))
    ey, em, ec = O.run_chunked(k.double(), v.double(), q.double(), A, Q, torch.full((2, 21), 0.3,
                               dtype=torch.float64), torch.zeros(2, 3, 2, dtype=torch.float64),
                               torch.eye(3, dtype=torch.float64).expand(2, 3, 3), 5, 1e-6)
    close(y, ey, "y")
    close(mT, em, "mean_T")
    close(cT, ec, "cov_T")


def _valid():
    k, v, q = _inputs((2,), 5, 2, 3, seed=17)
    return k, v, q


@pytest.mark.parametrize("mutate, exc, message", [
    (lambda a: a.update(keys=a["keys"][:, :4]), ValueError, "batch and time"),
    (lambda a: a.update(values=a["values"][:, :4]), ValueError, "same sequence length"),
    (lambda a: a.update(keys=a["keys"].long()), TypeError, "floating-point"),
    (lambda a: a.update(transitions=torch.eye(2).expand(2, 5, 2, 2),
                        transition_diagonals=torch.ones(2, 5, 2)), ValueError, "not both"),
    (lambda a: a.update(rotation_radii=torch.ones(2, 5, 1)), ValueError, "together"),
    (lambda a: a.update(transition_diagonals=torch.ones(2, 4, 2)), ValueError, "transition_diagonals"),
    (lambda a: a.update(process_variances=-0.1), ValueError, "nonnegative"),
    (lambda a: a.update(observation_variances=0.0), ValueError, "strictly positive"),
    (lambda a: a.update(observation_variances=torch.ones(2, 4)), ValueError, "observation_variances"),
    (lambda a: a.update(initial_covariance=torch.tensor([[1.0, 2.0], [0.0, 1.0]])), ValueError, "symmetric"),
    (lambda a: a.update(initial_covariance=-torch.eye(2)), ValueError, "positive semidefinite"),
    (lambda a: a.update(initial_mean=torch.zeros(2, 2)), ValueError, "initial_mean"),
    (lambda a: a.update(denominator_floor=0.0), ValueError, "denominator_floor"),
    (lambda a: a.update(chunk_length=0), ValueError, "chunk_length"),
    (lambda a: a.update(keys=a["keys"].clone().index_fill_(1, torch.tensor([2]), float("nan"))), ValueError,
     "finite"),
    (lambda a: a.update(process_variances=0.1, process_covariances=torch.eye(2).expand(2, 5, 2, 2)), ValueError,
     "not both"),
    (lambda a: a.update(replay_ssm=1), TypeError, "replay_ssm"),
])
def test_validation_errors(mutate, exc, message):
    """The reference's argument checks (bayesian_layer.py:798-985) raise the same exception types."""
    k, v, q = _valid()
    args = dict(keys=k, values=v, queries=q)
    mutate(args)
    keys, values, queries = args.pop("keys"), args.pop("values"), args.pop("queries")
    with pytest.raises(exc, match=message):
        bayesian_layer(keys, values, queries, **args)


def _nan_at(x, i=2):
    return x.clone().index_fill_(1, torch.tensor([i]), float("nan"))


@pytest.mark.parametrize("mutate, message", [
    # A value error registered before a shape/type error is raised first, as the reference checks in turn.
    (lambda a: a.update(keys=_nan_at(a["keys"]), rotation_radii=torch.ones(2, 5, 1)), "keys must contain only"),
    (lambda a: a.update(queries=_nan_at(a["queries"]), replay_ssm=1), "queries must contain only"),
    # Shape errors before any failing value check keep their place.
    (lambda a: a.update(observation_variances=0.0, chunk_length=0), "strictly positive"),
    (lambda a: a.update(rotation_radii=torch.ones(2, 5, 1), observation_variances=0.0), "together"),
    # Among value checks the first registered wins.
    (lambda a: a.update(values=_nan_at(a["values"]), observation_variances=0.0), "values must contain only"),
    (lambda a: a.update(process_variances=-0.1, observation_variances=0.0), "nonnegative"),
    (lambda a: a.update(observation_variances=float("inf")), "observation_variances must contain only"),
    (lambda a: a.update(transition_diagonals=_nan_at(torch.ones(2, 5, 2))), "transition_diagonals must contain"),
    (lambda a: a.update(initial_mean=torch.full((2, 3), float("nan")), observation_variances=0.0),
     "strictly positive"),
    (lambda a: a.update(process_variances=-0.1, initial_covariance=-torch.eye(2)), "nonnegative"),
])
def test_deferred_value_checks_keep_the_reference_order(mutate, message):
    """Finite/sign checks are read back together; errors still come in the reference's order."""
    k, v, q = _valid()
    args = dict(keys=k, values=v, queries=q)
    mutate(args)
    keys, values, queries = args.pop("keys"), args.pop("values"), args.pop("queries")
    with pytest.raises((ValueError, TypeError), match=message):
        bayesian_layer(keys, values, queries, **args)


def test_empty_time_axis_returns_the_prior():
    k, v, q = (x[:, :0] for x in _valid())
    y, mT, cT = bayesian_layer(k, v, q)
    assert y.shape == (2, 0, 3)
    torch.testing.assert_close(mT, torch.zeros(2, 2, 3))
    torch.testing.assert_close(cT, torch.eye(2).expand(2, 2, 2))


def test_public_names():
    assert sorted(bayes_ssm.__all__) == sorted([
        "BayesianLayer", "bayesian_layer", "make_diagonal_dynamics", "make_rotation_dynamics",
        "make_rotation_process_covariances", "ReplaySSM", "associative_static_bayesian",
        "associative_static_bayesian_cuda"])
    with pytest.raises(ValueError, match="CUDA"):
        bayes_ssm.associative_static_bayesian_cuda(*_valid())


def test_scan_checks_compare_the_floor_in_the_tensor_dtype():
    """associative_static_bayesian: r equal to the floor passes in float32 and float64 (the reference's
    ``r2 < floor`` compares in the tensor's dtype); below it, or non-finite, fails; a NaN initial mean fails
    before a bad floor."""
    from bayes_ssm import associative_static_bayesian

    k, v, q = _valid()
    for dtype in (torch.float32, torch.float64):
        kk, vv, qq = (x.to(dtype) for x in (k, v, q))
        associative_static_bayesian(kk, vv, qq, observation_variances=torch.full((2, 5), 1e-6, dtype=dtype),
                                    denominator_floor=1e-6)
        with pytest.raises(ValueError, match="greater than or equal"):
            associative_static_bayesian(kk, vv, qq, observation_variances=torch.full((2, 5), 9e-7, dtype=dtype),
                                        denominator_floor=1e-6)
        with pytest.raises(ValueError, match="greater than or equal"):
            associative_static_bayesian(kk, vv, qq, observation_variances=float("nan"))
    with pytest.raises(ValueError, match="initial_mean must contain only finite"):
        associative_static_bayesian(k, v, q, initial_mean=torch.full((2, 3), float("nan")), denominator_floor=0.0)
