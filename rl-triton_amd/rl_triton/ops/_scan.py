"""
Internal scan dispatch shared by the estimators (drop-in for src/rl_triton/ops/_scan.py).

Two directions of the same linear recurrence:

Backward (right-to-left): A[t] = u[t] + v[t] * A[t+1],  A[T] = bootstrap
Forward  (left-to-right): e[t] = u[t] + v[t] * e[t-1],  e[-1] = seed

Both run on the gfx950 affine-scan kernel (librl_triton_amd.so, rlk_affine_scan),
which handles every sequence length: rows up to one workgroup tile are scanned
whole, longer rows are split into tiles chained by a decoupled look-back.  The
reference's flat/chunked split (_FLAT_MAX_SEQ_LEN, _CHUNK_SIZE) is kept as
importable constants only.
"""
import os
import warnings

import torch

from rl_triton import _native

# Set RL_TRITON_PERF_WARNINGS=1 to be warned about implicit copies of
# non-contiguous inputs (read at import, as in ops/_scan.py:27).
_PERF_WARNINGS = os.environ.get("RL_TRITON_PERF_WARNINGS", "0") == "1"


# Set RL_TRITON_CORRECTNESS_WARNINGS=1 to enable the expensive input assertions
# (read per call, as in ops/_scan.py:30-31).
def _CORRECTNESS_WARNINGS() -> bool:
    return os.environ.get("RL_TRITON_CORRECTNESS_WARNINGS", "0") == "1"


def _float_io(t, lead) -> bool:
    """The dtype rule of every op: float32 as in the reference, or else bfloat16 for every
    float tensor of the call (the dtype of `lead`, the call's first [num_envs, seq_len]
    tensor).  bfloat16 calls compute in float32 and return bfloat16, rounded as torch's
    float -> bfloat16 conversion rounds."""
    return t.dtype == lead.dtype and lead.dtype in (torch.float32, torch.bfloat16)


def _perf_warn(msg: str) -> None:
    if _PERF_WARNINGS:
        warnings.warn(msg, stacklevel=3)


def _correctness_warn(msg: str) -> None:
    if _CORRECTNESS_WARNINGS():
        warnings.warn(msg, stacklevel=3)


# The reference's Triton limit for one-block scans (ops/_scan.py:46-49).  Kept for import
# compatibility and for the assertions the reference makes against it; the HIP kernels
# have no such limit.
_FLAT_MAX_SEQ_LEN = 131072
_CHUNK_SIZE = 1024


def _run_scan(
    u: torch.Tensor,
    v: torch.Tensor,
    bootstrap: torch.Tensor | None = None,
) -> torch.Tensor:
    """
    Backward linear scan: A[t] = u[t] + v[t] * A[t+1], A[T] = bootstrap.

    Same contract as ops/_scan.py:69-144.  Non-contiguous inputs are copied.

    Args:
        u:         Additive term [num_envs, seq_len], float32, GPU.
        v:         Multiplicative decay [num_envs, seq_len], float32, GPU.
        bootstrap: Boundary value A[T] per environment, [num_envs], float32.
                   Defaults to zeros.

    Returns:
        out: A[t], shape [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.affine_scan(u, v, bootstrap, _native.BACKWARD)
        if res is not None:
            return res

    if not u.is_contiguous():
        _perf_warn("u is not contiguous; a copy will be made. Call .contiguous() before the hot loop to avoid this overhead.")
    if not v.is_contiguous():
        _perf_warn("v is not contiguous; a copy will be made. Call .contiguous() before the hot loop to avoid this overhead.")

    if _CORRECTNESS_WARNINGS():
        assert u.shape == v.shape,      "u and v must have the same shape"
        assert u.is_cuda and v.is_cuda, "u and v must be on CUDA"
        assert _float_io(u, u), f"u: expected float32 (or bfloat16 throughout), got {u.dtype}"
        assert _float_io(v, u), f"v: expected float32 (or bfloat16 throughout), got {v.dtype}"
        if bootstrap is not None:
            assert bootstrap.shape == (u.shape[0],), \
                f"bootstrap must have shape [{u.shape[0]}], got {bootstrap.shape}"
            assert bootstrap.is_cuda, "bootstrap must be on CUDA"

    u = u.contiguous()
    v = v.contiguous()
    if bootstrap is not None:
        bootstrap = bootstrap.contiguous()
    out = torch.empty_like(u)
    return _native.affine_scan(u, v, bootstrap, out, _native.BACKWARD)


def _run_scan_forward(
    u: torch.Tensor,
    v: torch.Tensor,
    seed: torch.Tensor | None = None,
) -> torch.Tensor:
    """
    Forward linear scan: e[t] = u[t] + v[t] * e[t-1], e[-1] = seed.

    Same contract as ops/_scan.py:147-213, except that sequences longer than
    _FLAT_MAX_SEQ_LEN are scanned instead of rejected.

    Args:
        u:    Additive term [num_envs, seq_len], float32, GPU.
        v:    Multiplicative decay [num_envs, seq_len], float32, GPU.
        seed: Initial carry e[-1] per environment, [num_envs], float32.  Defaults to zeros.

    Returns:
        out: e[t], shape [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.affine_scan(u, v, seed, _native.FORWARD)
        if res is not None:
            return res

    if not u.is_contiguous():
        _perf_warn("u is not contiguous; a copy will be made. Call .contiguous() before the hot loop to avoid this overhead.")
    if not v.is_contiguous():
        _perf_warn("v is not contiguous; a copy will be made. Call .contiguous() before the hot loop to avoid this overhead.")

    if _CORRECTNESS_WARNINGS():
        assert u.shape == v.shape,      "u and v must have the same shape"
        assert u.is_cuda and v.is_cuda, "u and v must be on CUDA"
        assert _float_io(u, u), f"u: expected float32 (or bfloat16 throughout), got {u.dtype}"
        assert _float_io(v, u), f"v: expected float32 (or bfloat16 throughout), got {v.dtype}"
        if seed is not None:
            assert seed.shape == (u.shape[0],), \
                f"seed must have shape [{u.shape[0]}], got {seed.shape}"
            assert seed.is_cuda, "seed must be on CUDA"

    u = u.contiguous()
    v = v.contiguous()
    if seed is not None:
        seed = seed.contiguous()
    out = torch.empty_like(u)
    return _native.affine_scan(u, v, seed, out, _native.FORWARD)
