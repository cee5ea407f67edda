"""rl_triton for AMD MI355X (gfx950): drop-in return-estimation ops on hand-written HIP kernels.

Same public surface as simonsays1980/rl-triton v0.1.3 (src/rl_triton/__init__.py:1-17),
plus compute_gae_normalized (GAE, returns and batch-normalised advantages in one fused call;
the reference lists it on its ROADMAP.md:75-81 but does not have it).
"""
__version__ = "0.1.3"

from rl_triton.ops.gae import compute_gae
from rl_triton.ops.gae_norm import compute_gae_normalized
from rl_triton.ops.retrace import compute_retrace
from rl_triton.ops.prefix_sum import compute_episodic_prefix_sum
from rl_triton.ops.returns import compute_discounted_returns, compute_eligibility_traces, compute_lambda_returns
from rl_triton.ops.vtrace import compute_vtrace

__all__ = [
    "compute_discounted_returns",
    "compute_eligibility_traces",
    "compute_episodic_prefix_sum",
    "compute_gae",
    "compute_gae_normalized",
    "compute_lambda_returns",
    "compute_retrace",
    "compute_vtrace",
]
