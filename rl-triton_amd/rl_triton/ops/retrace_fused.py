import torch

from rl_triton import _native

_FLAT_MAX_SEQ_LEN = 131072


def compute_retrace_fused(
    action_probs_target: torch.Tensor,
    action_probs_behavior: torch.Tensor,
    q_values: torch.Tensor,
    next_q_values_all: torch.Tensor,
    actions: torch.Tensor,
    rewards: torch.Tensor,
    truncateds: torch.Tensor,
    terminated: torch.Tensor,
    gamma: float,
    lambda_: float = 1.0,
    c_bar: float = 1.0,
    rho_bar: float = 1.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """
    Retrace(λ) targets and advantages in one gfx950 kernel launch.

    Drop-in for src/rl_triton/ops/retrace_fused.py:26-118 -- note the argument order
    (rewards, truncateds, terminated) differs from compute_retrace.  Computes
    E_π[Q(s_{t+1},·)], π(a_t|s_t), the clipped ratios, the backward scan, Q_ret and the
    advantages in registers; c[t+1] and Q_ret[t+1] come from the neighbouring step in
    registers, so no [E, T] scratch buffer is allocated.

    Args (all GPU, contiguous after this call copies them):
        action_probs_target: [num_envs, seq_len, num_actions], float32.
        action_probs_behavior, q_values, rewards, truncateds, terminated:
                             [num_envs, seq_len], float32.
        next_q_values_all:   [num_envs, seq_len, num_actions], float32.
        actions:             [num_envs, seq_len], int64.

    Returns:
        retrace_targets: Q_ret[t], [num_envs, seq_len], float32.
        advantages:      A[t],     [num_envs, seq_len], float32.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.retrace(action_probs_target, action_probs_behavior, q_values, next_q_values_all, actions, rewards, terminated, truncateds, gamma, lambda_, c_bar, rho_bar)
        if res is not None:
            return res

    num_envs, seq_len = rewards.shape

    assert seq_len <= _FLAT_MAX_SEQ_LEN, (
        f"seq_len={seq_len} exceeds flat kernel limit {_FLAT_MAX_SEQ_LEN}."
    )
    return _retrace_launch(action_probs_target, action_probs_behavior, q_values,
                           next_q_values_all, actions, rewards, terminated, truncateds,
                           gamma, lambda_, c_bar, rho_bar)


def _retrace_launch(action_probs_target, action_probs_behavior, q_values, next_q_values_all,
                    actions, rewards, terminateds, truncateds, gamma, lambda_, c_bar, rho_bar):
    out        = torch.empty_like(rewards, memory_format=torch.contiguous_format)
    advantages = torch.empty_like(rewards, memory_format=torch.contiguous_format)
    return _native.retrace(
        action_probs_target.contiguous(), action_probs_behavior.contiguous(),
        q_values.contiguous(), next_q_values_all.contiguous(), actions.contiguous(),
        rewards.contiguous(), terminateds.contiguous(),
        truncateds.contiguous() if truncateds is not None else None,
        out, advantages, gamma, lambda_, c_bar, rho_bar)
