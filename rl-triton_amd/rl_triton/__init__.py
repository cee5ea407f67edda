"""rl_triton for AMD MI355X (gfx950): drop-in return-estimation ops on hand-written HIP kernels.

Same public surface as simonsays1980/rl-triton v0.1.3 (src/rl_triton/__init__.py:1-17).
Beyond it, items the reference lists on its ROADMAP.md but does not have:
  * compute_gae_normalized: GAE, returns and batch-normalised advantages (ROADMAP.md:75-81);
  * bfloat16 I/O: every op also takes bfloat16 tensors (all float tensors of a call alike)
    and returns bfloat16, computing in float32 (ROADMAP.md:82-99);
  * skipped steps: compute_gae(..., mask=...) and compute_gae_normalized(..., mask=...) pass
    the recurrence through steps with mask == 0, as verl does for observation tokens
    (ROADMAP.md:131-140).
Where the docstrings of rl_triton.ops say float32, bfloat16 throughout is accepted too.
"""
__version__ = "0.1.3"

from rl_triton import _native
from rl_triton.ops import gae as _gae
from rl_triton.ops import gae_norm as _gae_norm
from rl_triton.ops import prefix_sum as _prefix_sum
from rl_triton.ops import retrace as _retrace
from rl_triton.ops import returns as _returns
from rl_triton.ops import vtrace as _vtrace

# The public functions: the Python implementations in rl_triton.ops, each behind the C++
# fast path that launches well-formed calls without a Python frame (_native.public_entry).
compute_gae = _native.public_entry(_gae.compute_gae, "gae")
compute_gae_normalized = _native.public_entry(_gae_norm.compute_gae_normalized, "gae_normalized")
compute_retrace = _native.public_entry(_retrace.compute_retrace, "retrace")
compute_episodic_prefix_sum = _native.public_entry(_prefix_sum.compute_episodic_prefix_sum, "prefix_sum")
compute_discounted_returns = _native.public_entry(_returns.compute_discounted_returns, "discounted_returns")
compute_eligibility_traces = _native.public_entry(_returns.compute_eligibility_traces, "eligibility_traces")
compute_lambda_returns = _native.public_entry(_returns.compute_lambda_returns, "lambda_returns")
compute_vtrace = _native.public_entry(_vtrace.compute_vtrace, "vtrace")

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
