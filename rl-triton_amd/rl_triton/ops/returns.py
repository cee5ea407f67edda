import torch

from rl_triton import _native
from rl_triton.ops._scan import _FLAT_MAX_SEQ_LEN, _CORRECTNESS_WARNINGS, _float_io  # noqa: F401


def compute_lambda_returns(
    rewards: torch.Tensor,
    next_values: torch.Tensor,
    terminateds: torch.Tensor,
    truncateds: torch.Tensor | None = None,
    gamma: float = 0.99,
    lambda_: float = 0.95,
    bootstrap_values: torch.Tensor | None = None,
) -> torch.Tensor:
    """
    TD(λ) targets (λ-returns) by a backward affine scan on gfx950.

    Drop-in for src/rl_triton/ops/returns.py:33-152:

    - G[t] = r[t] + γ·(1-done[t])·[(1-λ)·V(s_{t+1}) + λ·G[t+1]] + γ·truncated[t]·bootstrap[t]
    - done[t] = min(terminated[t] + truncated[t], 1) (terminated when truncateds is None)
    - G[T] = bootstrap_values[:, -1] (0 without bootstrap_values)

    `next_values` is V(s_{t+1}) as supplied by the caller (zero it at truncated steps).
    λ = 0 gives one-step TD targets, λ = 1 discounted returns.

    Returns:
        lambda_returns: G[t], [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.lambda_returns(rewards, next_values, terminateds, truncateds, gamma, lambda_, bootstrap_values)
        if res is not None:
            return res

    num_envs, seq_len = rewards.shape
    has_truncations   = truncateds is not None

    # Cheap structural checks -- always-on (ops/returns.py:81-95).
    for name, t in [("rewards", rewards), ("next_values", next_values), ("terminateds", terminateds)]:
        assert t.is_cuda,                f"{name} must be on CUDA"
        assert _float_io(t, rewards), f"{name}: expected float32 (or bfloat16 throughout), got {t.dtype}"
        assert t.shape == rewards.shape, f"{name} shape {t.shape} != rewards shape {rewards.shape}"
    if has_truncations:
        assert truncateds.is_cuda,                "truncateds must be on CUDA"
        assert _float_io(truncateds, rewards), "truncateds: expected float32 (or bfloat16 throughout)"
        assert truncateds.shape == rewards.shape, \
            f"truncateds shape {truncateds.shape} != rewards shape {rewards.shape}"
    if bootstrap_values is not None:
        assert bootstrap_values.is_cuda,                "bootstrap_values must be on CUDA"
        assert _float_io(bootstrap_values, rewards), "bootstrap_values: expected float32 (or bfloat16 throughout)"
        assert bootstrap_values.shape == rewards.shape, \
            f"bootstrap_values shape {bootstrap_values.shape} != rewards shape {rewards.shape}"

    # Expensive tensor scans -- correctness-warning path only.
    if _CORRECTNESS_WARNINGS():
        if has_truncations:
            assert not (terminateds.bool() & truncateds.bool()).any(), \
                "terminated and truncated are mutually exclusive: a step cannot be both"

    rewards     = rewards.contiguous()
    next_values = next_values.contiguous()
    terminateds = terminateds.contiguous()
    if has_truncations:
        truncateds = truncateds.contiguous()
    if bootstrap_values is not None:
        bootstrap_values = bootstrap_values.contiguous()

    out = torch.empty_like(rewards)
    return _native.lambda_returns(rewards, next_values, terminateds, truncateds, bootstrap_values,
                                  out, gamma, lambda_)


def compute_discounted_returns(
    rewards: torch.Tensor,
    terminateds: torch.Tensor,
    truncateds: torch.Tensor | None = None,
    gamma: float = 0.99,
    bootstrap_values: torch.Tensor | None = None,
) -> torch.Tensor:
    """
    Discounted returns (reward-to-go) by a backward affine scan on gfx950.

    Drop-in for src/rl_triton/ops/returns.py:155-263:

    - G[t] = r[t] + γ·(1-done[t])·G[t+1] + γ·truncated[t]·bootstrap[t]
    - done[t] = min(terminated[t] + truncated[t], 1) (terminated when truncateds is None)
    - G[T] = bootstrap_values[:, -1] (0 without bootstrap_values)

    Returns:
        returns: G[t], [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.discounted_returns(rewards, terminateds, truncateds, gamma, bootstrap_values)
        if res is not None:
            return res

    num_envs, seq_len = rewards.shape
    has_truncations   = truncateds is not None

    # Cheap structural checks -- always-on (ops/returns.py:194-208).
    for name, t in [("rewards", rewards), ("terminateds", terminateds)]:
        assert t.is_cuda,                f"{name} must be on CUDA"
        assert _float_io(t, rewards), f"{name}: expected float32 (or bfloat16 throughout), got {t.dtype}"
        assert t.shape == rewards.shape, f"{name} shape {t.shape} != rewards shape {rewards.shape}"
    if has_truncations:
        assert truncateds.is_cuda,                "truncateds must be on CUDA"
        assert _float_io(truncateds, rewards), "truncateds: expected float32 (or bfloat16 throughout)"
        assert truncateds.shape == rewards.shape, \
            f"truncateds shape {truncateds.shape} != rewards shape {rewards.shape}"
    if bootstrap_values is not None:
        assert bootstrap_values.is_cuda,                "bootstrap_values must be on CUDA"
        assert _float_io(bootstrap_values, rewards), "bootstrap_values: expected float32 (or bfloat16 throughout)"
        assert bootstrap_values.shape == rewards.shape, \
            f"bootstrap_values shape {bootstrap_values.shape} != rewards shape {rewards.shape}"

    # Expensive tensor scans -- correctness-warning path only.
    if _CORRECTNESS_WARNINGS():
        if has_truncations:
            assert not (terminateds.bool() & truncateds.bool()).any(), \
                "terminated and truncated are mutually exclusive: a step cannot be both"

    rewards     = rewards.contiguous()
    terminateds = terminateds.contiguous()
    if has_truncations:
        truncateds = truncateds.contiguous()
    if bootstrap_values is not None:
        bootstrap_values = bootstrap_values.contiguous()

    out = torch.empty_like(rewards)
    return _native.discounted_returns(rewards, terminateds, truncateds, bootstrap_values, out, gamma)


def compute_eligibility_traces(
    gradients: torch.Tensor,
    dones: torch.Tensor,
    gamma: float,
    lambda_: float,
    seed_values: torch.Tensor | None = None,
) -> torch.Tensor:
    """
    Accumulating eligibility traces by a forward affine scan on gfx950.

    Drop-in for src/rl_triton/ops/returns.py:266-347:

    - z[t] = g[t] + γ·λ·(1 - done[t-1])·z[t-1],  z[-1] = seed,  done[-1] := 0

    `done[t] = 1` means the episode ends AT t (the same convention as compute_gae);
    the carry into t is cut when the PRECEDING step ended an episode.  Pass the raw
    flags, unshifted.  Deliberate divergence: the reference rejects seq_len > 131072
    (ops/returns.py:319-322); here every length is scanned (look-back path).

    Returns:
        traces: z[t], [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.eligibility_traces(gradients, dones, gamma, lambda_, seed_values)
        if res is not None:
            return res

    num_envs, seq_len = gradients.shape

    # Cheap structural checks -- always-on (ops/returns.py:309-317).
    assert gradients.is_cuda and dones.is_cuda, "gradients and dones must be on CUDA"
    assert _float_io(gradients, gradients), f"gradients: expected float32 (or bfloat16 throughout), got {gradients.dtype}"
    assert _float_io(dones, gradients),     f"dones: expected float32 (or bfloat16 throughout), got {dones.dtype}"
    assert gradients.shape == dones.shape,   "gradients and dones must have the same shape"
    if seed_values is not None:
        assert seed_values.shape == (num_envs,), \
            f"seed_values must have shape [{num_envs}], got {seed_values.shape}"
        assert seed_values.is_cuda, "seed_values must be on CUDA"

    gradients = gradients.contiguous()
    dones     = dones.contiguous()
    if seed_values is not None:
        seed_values = seed_values.contiguous()

    out = torch.empty_like(gradients)
    return _native.eligibility_traces(gradients, dones, seed_values, out, gamma, lambda_)
