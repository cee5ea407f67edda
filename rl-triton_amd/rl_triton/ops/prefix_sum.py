import torch

from rl_triton import _native
from rl_triton.ops._scan import _FLAT_MAX_SEQ_LEN, _CORRECTNESS_WARNINGS, _float_io  # noqa: F401


def compute_episodic_prefix_sum(
    inputs: torch.Tensor,
    dones: torch.Tensor,
    seed_values: torch.Tensor | None = None,
    boundary: str = "ends_at",
) -> torch.Tensor:
    """
    Cumulative sum that resets at episode/segment boundaries (forward scan on gfx950).

    Drop-in for src/rl_triton/ops/prefix_sum.py:23-111:

    - "ends_at" (default): done[t] = 1 means the segment ENDS at t, the reset lands at t+1:
        C[t] = x[t] + (1 - done[t-1])·C[t-1],  C[-1] = seed,  done[-1] := 0
    - "starts_at": done[t] = 1 means the segment STARTS at t, the reset lands at t:
        C[t] = x[t] + (1 - done[t])·C[t-1],    C[-1] = seed

    Input checks run only with RL_TRITON_CORRECTNESS_WARNINGS=1, as in the reference
    (the GPU binding still refuses malformed tensors).  Deliberate divergence: the
    reference rejects seq_len > 131072 (ops/prefix_sum.py:83-86); here every length
    is scanned (look-back path).

    Returns:
        prefix_sums: C[t], [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None and (boundary == "ends_at" or boundary == "starts_at"):
        res = fast.prefix_sum(inputs, dones, seed_values, boundary == "ends_at")
        if res is not None:
            return res

    num_envs, seq_len = inputs.shape

    if _CORRECTNESS_WARNINGS():
        assert inputs.is_cuda and dones.is_cuda, "inputs and dones must be on CUDA"
        assert _float_io(inputs, inputs), f"inputs: expected float32 (or bfloat16 throughout), got {inputs.dtype}"
        assert _float_io(dones, inputs),  f"dones: expected float32 (or bfloat16 throughout), got {dones.dtype}"
        assert inputs.shape == dones.shape,   "inputs and dones must have the same shape"
        if seed_values is not None:
            assert seed_values.shape == (num_envs,), \
                f"seed_values must have shape [{num_envs}], got {seed_values.shape}"
            assert seed_values.is_cuda, "seed_values must be on CUDA"
        assert boundary in ("ends_at", "starts_at"), \
            f"boundary must be 'ends_at' or 'starts_at', got {boundary!r}"
    if boundary not in ("ends_at", "starts_at"):
        raise ValueError(f"boundary must be 'ends_at' or 'starts_at', got {boundary!r}")

    inputs = inputs.contiguous()
    dones  = dones.contiguous()
    if seed_values is not None:
        seed_values = seed_values.contiguous()

    out = torch.empty_like(inputs)
    return _native.prefix_sum(inputs, dones, seed_values, out, boundary == "ends_at")
