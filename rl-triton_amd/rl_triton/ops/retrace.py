import torch

from rl_triton import _native
from rl_triton.ops._scan import _CORRECTNESS_WARNINGS, _float_io
from rl_triton.ops.retrace_fused import _retrace_launch, compute_retrace_fused

# The reference routes seq_len > 2048 away from its fused Triton kernel because of
# register spills at long rows (ops/retrace.py:6-49).  The HIP kernel keeps a fixed
# number of steps per thread at every length, so one kernel serves all seq_len; the
# constant stays importable.
_TRITON_SEQ_LEN_CEILING = 2048


def compute_retrace(
    action_probs_target: torch.Tensor,
    action_probs_behavior: torch.Tensor,
    q_values: torch.Tensor,
    next_q_values_all: torch.Tensor,
    actions: torch.Tensor,
    rewards: torch.Tensor,
    terminateds: torch.Tensor,
    truncateds: torch.Tensor,
    gamma: float,
    lambda_: float = 1.0,
    c_bar: float = 1.0,
    rho_bar: float = 1.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """
    Retrace(λ) Q-value targets and advantages (Munos et al. 2016).

    Drop-in for src/rl_triton/ops/retrace.py:52-196:

    - Δ[t] = δ[t] + γ·c[t+1]·(1-done[t])·Δ[t+1],  Δ[T] = 0,  c[T] = 0
    - δ[t] = r[t] + γ·E_π[Q(s_{t+1},·)]·(1-terminated[t]) - Q(s_t,a_t)
    - c[t] = λ·min(c̄, π(a_t|s_t)/μ(a_t|s_t)),  ρ[t] = min(ρ̄, same ratio)
    - done[t] = min(terminated[t] + truncated[t], 1)
    - Q_ret[t] = Q(s_t,a_t) + Δ[t]
    - A[t] = ρ[t]·(r[t] + γ·Q_ret[t+1]·(1-terminated[t]) - Q(s_t,a_t)),  Q_ret[T] = 0

    Discrete actions; `actions` is int64.  One kernel launch for every seq_len.

    Returns:
        retrace_targets: Q_ret[t], [num_envs, seq_len], float32.
        advantages:      A[t],     [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.retrace(action_probs_target, action_probs_behavior, q_values, next_q_values_all, actions, rewards, terminateds, truncateds, gamma, lambda_, c_bar, rho_bar)
        if res is not None:
            return res

    # Cheap structural checks -- always-on (ops/retrace.py:116-141).
    for name, t in [
        ("action_probs_behavior", action_probs_behavior),
        ("q_values",              q_values),
        ("rewards",               rewards),
        ("terminateds",           terminateds),
        ("truncateds",            truncateds),
    ]:
        assert t.is_cuda,                 f"{name} must be on CUDA"
        assert _float_io(t, rewards),  f"{name}: expected float32 (or bfloat16 throughout), got {t.dtype}"
        assert t.shape == rewards.shape,  f"{name} shape {t.shape} != rewards shape {rewards.shape}"

    assert action_probs_target.is_cuda,                "action_probs_target must be on CUDA"
    assert _float_io(action_probs_target, rewards), "action_probs_target: expected float32 (or bfloat16 throughout)"
    assert action_probs_target.shape[:2] == rewards.shape, (
        f"action_probs_target shape {action_probs_target.shape} incompatible with rewards {rewards.shape}"
    )
    assert next_q_values_all.is_cuda,                "next_q_values_all must be on CUDA"
    assert _float_io(next_q_values_all, rewards), "next_q_values_all: expected float32 (or bfloat16 throughout)"
    assert next_q_values_all.shape == action_probs_target.shape, (
        f"next_q_values_all {next_q_values_all.shape} != action_probs_target {action_probs_target.shape}"
    )
    assert actions.is_cuda,              "actions must be on CUDA"
    assert actions.dtype == torch.int64, f"actions: expected int64, got {actions.dtype}"
    assert actions.shape == rewards.shape, \
        f"actions shape {actions.shape} != rewards shape {rewards.shape}"

    # Expensive tensor scan -- correctness-warning path only.
    if _CORRECTNESS_WARNINGS():
        assert not (terminateds.bool() & truncateds.bool()).any(), \
            "terminated and truncated are mutually exclusive: a step cannot be both"

    num_envs, seq_len = rewards.shape
    if seq_len <= _TRITON_SEQ_LEN_CEILING:
        return compute_retrace_fused(
            action_probs_target, action_probs_behavior,
            q_values, next_q_values_all, actions,
            rewards, truncateds, terminateds,
            gamma=gamma, lambda_=lambda_, c_bar=c_bar, rho_bar=rho_bar,
        )
    return _retrace_launch(action_probs_target, action_probs_behavior, q_values,
                           next_q_values_all, actions, rewards, terminateds, truncateds,
                           gamma, lambda_, c_bar, rho_bar)
