"""MI355X-native exact dense-covariance Bayesian sequence layers.

Same public API as the reference ``bayes_ssm`` package (bayes_ssm/__init__.py:2-20):
the recurrence API, the modules, the dynamics helpers and the associative
static scan.  On CUDA (ROCm) devices the eligible diagonal-dynamics calls run
on prebuilt gfx950 HIP kernels (``bayes_ssm.fused_cuda``).
"""
from .bayesian_layer import (
    BayesianLayer,
    bayesian_layer,
    make_diagonal_dynamics,
    make_rotation_dynamics,
    make_rotation_process_covariances,
)
from .replay_ssm import (
    ReplaySSM,
    associative_static_bayesian,
    associative_static_bayesian_cuda,
)

__all__ = [
    "BayesianLayer", "bayesian_layer", "make_diagonal_dynamics",
    "make_rotation_dynamics", "make_rotation_process_covariances",
    "ReplaySSM", "associative_static_bayesian",
    "associative_static_bayesian_cuda",
]
