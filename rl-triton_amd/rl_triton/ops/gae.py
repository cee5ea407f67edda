import torch

from rl_triton import _native
from rl_triton.ops._scan import _CORRECTNESS_WARNINGS, _float_io


def _check_gae_args(rewards, values, terminateds, truncateds, bootstrap_values, last_value,
                    mask=None):
    """The reference's compute_gae checks (ops/gae.py:106-145), in its order and with its
    messages: always-on structural checks, then the expensive ones under
    RL_TRITON_CORRECTNESS_WARNINGS=1.  `mask` (an extension) gets the same structural
    checks as truncateds."""
    num_envs, seq_len = rewards.shape
    has_truncations   = truncateds is not None

    # Cheap structural checks -- always-on (ops/gae.py:106-129).
    for name, t in [("rewards", rewards), ("values", values), ("terminateds", terminateds)]:
        assert t.is_cuda,                f"{name} must be on CUDA"
        assert _float_io(t, rewards), f"{name}: expected float32 (or bfloat16 throughout), got {t.dtype}"
        assert t.shape == rewards.shape, f"{name} shape {t.shape} != rewards shape {rewards.shape}"
    if has_truncations:
        assert truncateds.is_cuda,                "truncateds must be on CUDA"
        assert _float_io(truncateds, rewards), "truncateds: expected float32 (or bfloat16 throughout)"
        assert truncateds.shape == rewards.shape, \
            f"truncateds shape {truncateds.shape} != rewards shape {rewards.shape}"
    if mask is not None:
        assert mask.is_cuda,                "mask must be on CUDA"
        assert _float_io(mask, rewards),    "mask: expected float32 (or bfloat16 throughout)"
        assert mask.shape == rewards.shape, f"mask shape {mask.shape} != rewards shape {rewards.shape}"
    if last_value is not None:
        assert bootstrap_values is None, \
            "pass either last_value (shape [num_envs], convenience for the " \
            "window boundary) or bootstrap_values (shape [num_envs, seq_len], " \
            "full per-step control), not both."
        assert last_value.shape == (num_envs,), \
            f"last_value must have shape [{num_envs}], got {last_value.shape}"
        assert not has_truncations, \
            "last_value cannot be combined with truncateds; use bootstrap_values instead."
    if bootstrap_values is not None:
        assert bootstrap_values.is_cuda,                "bootstrap_values must be on CUDA"
        assert _float_io(bootstrap_values, rewards), "bootstrap_values: expected float32 (or bfloat16 throughout)"
        assert bootstrap_values.shape == rewards.shape, \
            f"bootstrap_values shape {bootstrap_values.shape} != rewards shape {rewards.shape}"

    # Expensive tensor scans -- correctness-warning path only (ops/gae.py:132-145).
    if _CORRECTNESS_WARNINGS():
        if has_truncations:
            assert not (terminateds.bool() & truncateds.bool()).any(), \
                "terminated and truncated are mutually exclusive: a step cannot be both"
        if has_truncations and bootstrap_values is not None:
            interior = torch.ones_like(truncateds, dtype=torch.bool)
            interior[:, -1] = False
            stray = (bootstrap_values != 0) & (truncateds == 0) & interior
            assert not stray.any(), (
                "bootstrap_values must be zero at non-truncated interior steps. "
                "Nonzero entries there double-count via the additive v_next trick "
                "and corrupt delta. Populate bootstrap_values only at truncated "
                "steps and at the final column (window boundary)."
            )



def compute_gae(
    rewards: torch.Tensor,
    values: torch.Tensor,
    terminateds: torch.Tensor,
    truncateds: torch.Tensor | None = None,
    gamma: float = 0.99,
    lambda_: float = 0.95,
    bootstrap_values: torch.Tensor | None = None,
    last_value: torch.Tensor | None = None,
    *,
    mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """
    Generalized Advantage Estimation by a backward affine scan on gfx950.

    Drop-in for src/rl_triton/ops/gae.py:34-215 (same arguments, checks and result):

    - A[t] = δ[t] + β[t] * A[t+1],  A[T] = 0
    - δ[t] = r[t] + γ·(1-terminated[t])·v_next[t] - V(s_t)
    - β[t] = γ·λ·(1-done[t]),  done[t] = min(terminated[t] + truncated[t], 1)
      (done = terminated when truncateds is None)
    - v_next[t] = bootstrap_values[t] at t = T-1 and at truncated steps,
      values[t+1] elsewhere

    `last_value` ([num_envs]) is the continuation value V(s_T) for the window
    boundary; `bootstrap_values` ([num_envs, seq_len]) gives it per step (truncated
    steps and t = T-1, zero elsewhere).  They are mutually exclusive, and
    `last_value` cannot be combined with `truncateds`.  The bootstrap enters δ only;
    the scan carry A[T] is always 0.

    One kernel launch for every seq_len (rows longer than one workgroup tile use the
    look-back path); truncation and bootstrap are folded into (δ, β) in-kernel.

    `mask` (keyword-only; an extension listed in the reference's ROADMAP.md:131-140, in
    the manner of verl's compute_gae_advantage_return with its response_mask): steps with
    mask == 0 are skipped.  A skipped step passes the recurrence through (β = 1, δ = 0)
    and returns the advantage of the next kept step (0 if none); the value a kept step
    bootstraps from is that of the nearest kept step after it, so credit crosses skipped
    spans (observation tokens of multi-turn rollouts).  Kept steps follow the rules
    above; with every step kept the result is the unmasked one.

    Args:
        rewards:          [num_envs, seq_len], float32, GPU.
        values:           V(s_t), [num_envs, seq_len], float32, GPU.
        terminateds:      1.0 where the episode terminated, [num_envs, seq_len], float32.
        truncateds:       1.0 where the episode was truncated, same shape, or None.
        gamma:            Discount factor (default 0.99).
        lambda_:          GAE λ (default 0.95).
        bootstrap_values: V(s_{t+1}^true) per step, [num_envs, seq_len], or None.
        last_value:       V(s_T) per environment, [num_envs], or None.
        mask:             1.0 for steps that take part, 0.0 for skipped ones, same shape,
                          or None (every step takes part).

    Returns:
        advantages: A[t], shape [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.gae(rewards, values, terminateds, truncateds, gamma, lambda_, bootstrap_values,
                       last_value, mask)
        if res is not None:
            return res

    has_truncations = truncateds is not None
    _check_gae_args(rewards, values, terminateds, truncateds, bootstrap_values, last_value, mask)

    rewards     = rewards.contiguous()
    values      = values.contiguous()
    terminateds = terminateds.contiguous()
    if has_truncations:
        truncateds = truncateds.contiguous()
    if last_value is not None:
        bootstrap = last_value.contiguous()
    elif bootstrap_values is not None:
        bootstrap = bootstrap_values.contiguous()
    else:
        bootstrap = None

    out = torch.empty_like(rewards)
    if mask is not None:
        return _native.gae_masked(rewards, values, terminateds, truncateds, bootstrap,
                                  mask.contiguous(), out, gamma, lambda_)
    return _native.gae(rewards, values, terminateds, truncateds, bootstrap, out, gamma, lambda_)
