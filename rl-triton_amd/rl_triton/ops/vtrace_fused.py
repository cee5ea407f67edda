import torch

from rl_triton import _native
from rl_triton.ops._scan import _FLAT_MAX_SEQ_LEN, _CORRECTNESS_WARNINGS, _float_io


def compute_vtrace_fused(
    log_pi_target: torch.Tensor,
    log_pi_behavior: torch.Tensor,
    values: torch.Tensor,
    rewards: torch.Tensor,
    terminateds: torch.Tensor,
    truncateds: torch.Tensor | None = None,
    gamma: float = 0.99,
    rho_bar: float = 1.0,
    c_bar: float = 1.0,
    bootstrap_values: torch.Tensor | None = None,
    last_value: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """
    V-trace targets and advantages in one gfx950 kernel launch.

    Drop-in for src/rl_triton/ops/vtrace_fused.py:23-220: same arguments, always-on
    checks and the same `seq_len <= 131072` assertion (use compute_vtrace above it).

    - ρ[t] = min(ρ̄, exp(logπ_target - logπ_behavior)),  c[t] = min(c̄, same ratio)
    - Δ[t] = ρ[t]·(r[t] + γ·v_next[t]·(1-terminated[t]) - V(s_t)) + γ·c[t]·(1-done[t])·Δ[t+1],
      Δ[T] = 0
    - targets vs[t] = Δ[t] + V(s_t)
    - advantages A[t] = ρ[t]·(r[t] + γ·vs_next[t]·(1-terminated[t]) - V(s_t))

    Without truncateds: v_next / vs_next are values[t+1] / vs[t+1], and the
    bootstrap (last_value, or bootstrap_values[:, -1]) at t = T-1.  With truncateds:
    v_next = values[t+1]·[t < T-1 and not truncated] + bootstrap_values[t] (likewise
    vs_next), done = min(terminated + truncated, 1).  The kernel keeps vs[t+1] in
    registers instead of round-tripping the targets through memory.

    Returns:
        vtrace_targets:    [num_envs, seq_len], float32.
        vtrace_advantages: [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.vtrace(log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds, gamma, rho_bar, c_bar, bootstrap_values, last_value)
        if res is not None:
            return res

    num_envs, seq_len = rewards.shape
    has_truncations   = truncateds is not None

    # Cheap structural checks -- always-on (ops/vtrace_fused.py:96-125).
    for name, t in [
        ("log_pi_target",   log_pi_target),
        ("log_pi_behavior", log_pi_behavior),
        ("values",          values),
        ("rewards",         rewards),
        ("terminateds",     terminateds),
    ]:
        assert t.is_cuda,                f"{name} must be on CUDA"
        assert _float_io(t, rewards), f"{name}: expected float32 (or bfloat16 throughout), got {t.dtype}"
        assert t.shape == rewards.shape, f"{name} shape {t.shape} != rewards shape {rewards.shape}"
    if has_truncations:
        assert truncateds.is_cuda,                "truncateds must be on CUDA"
        assert _float_io(truncateds, rewards), "truncateds: expected float32 (or bfloat16 throughout)"
        assert truncateds.shape == rewards.shape, \
            f"truncateds shape {truncateds.shape} != rewards shape {rewards.shape}"
    if last_value is not None:
        assert bootstrap_values is None, \
            "pass either last_value (shape [num_envs], convenience for the " \
            "window boundary) or bootstrap_values (shape [num_envs, seq_len], " \
            "full per-step control), not both."
        assert last_value.shape == (num_envs,), \
            f"last_value must have shape [{num_envs}], got {last_value.shape}"
        assert last_value.is_cuda,                "last_value must be on CUDA"
        assert _float_io(last_value, rewards), "last_value: expected float32 (or bfloat16 throughout)"
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

    assert seq_len <= _FLAT_MAX_SEQ_LEN, (
        f"seq_len={seq_len} exceeds the flat kernel limit {_FLAT_MAX_SEQ_LEN}. "
        "Use compute_vtrace for longer sequences (it auto-dispatches to chunked)."
    )
    return _vtrace_launch(log_pi_target, log_pi_behavior, values, rewards, terminateds,
                          truncateds, gamma, rho_bar, c_bar, bootstrap_values, last_value)


def _vtrace_launch(log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds,
                   gamma, rho_bar, c_bar, bootstrap_values, last_value):
    """Make inputs contiguous, allocate both outputs, launch rlk_vtrace (any seq_len)."""
    log_pi_target   = log_pi_target.contiguous()
    log_pi_behavior = log_pi_behavior.contiguous()
    values          = values.contiguous()
    rewards         = rewards.contiguous()
    terminateds     = terminateds.contiguous()
    if truncateds is not None:
        truncateds = truncateds.contiguous()
    if last_value is not None:
        bootstrap = last_value.contiguous()
    elif bootstrap_values is not None:
        bootstrap = bootstrap_values.contiguous()
    else:
        bootstrap = None

    vtrace_targets    = torch.empty_like(rewards)
    vtrace_advantages = torch.empty_like(rewards)
    return _native.vtrace(log_pi_target, log_pi_behavior, values, rewards, terminateds,
                          truncateds, bootstrap, vtrace_targets, vtrace_advantages,
                          gamma, rho_bar, c_bar)
