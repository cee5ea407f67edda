"""float32 PyTorch-on-CPU restatement of the reference's sequential loops.

TEST INFRASTRUCTURE ONLY: used by ``tests/`` as a second, float32 checker
next to the float64 C oracle, and by ``bench.py``'s ``cpu_baseline`` leg as
the timed CPU baseline.  The rl_triton package never imports it.

These are the loops the reference times as its CPU column: one vectorised
step over all environments per time step, in float32 on CPU tensors.  They
restate

* ``reference_gae`` / ``_ref_gae_trunc``  -- tests/test_gae.py:34-60,
  tests/bench_release.py:128-156
* ``numpy_vtrace_cpu`` / ``reference_vtrace`` -- tests/bench_release.py:296-320,
  tests/test_vtrace.py:56-101
* ``reference_retrace`` -- tests/test_retrace.py:19-60
* ``reference_lambda_returns`` / ``_ref_lambda_sequential``,
  ``reference_discounted_returns`` / ``_ref_discounted_sequential``,
  ``reference_eligibility_traces`` -- tests/test_returns.py:19-57,362-384,449-510
* ``reference_episodic_prefix_sum`` -- tests/test_prefix_sum.py:18-56

keeping the reference's operation order, so their float32 roundings are the
ones the reference's own loops produce.
"""
from __future__ import annotations

import torch


def gae_loop(rewards, values, terminateds, truncateds=None, gamma=0.99, lambda_=0.95,
             bootstrap_values=None, last_value=None):
    """GAE by a backward loop over time, vectorised over environments.

    ``last_value`` ([E]) or ``bootstrap_values`` ([E, T]) supply the
    continuation value at t = T-1 and, with ``truncateds``, at truncated steps.
    """
    n_env, n_t = rewards.shape
    boot = bootstrap_values
    if boot is None:
        boot = torch.zeros_like(rewards)
        if last_value is not None:
            boot[:, -1] = last_value
    shifted = torch.zeros_like(values)
    shifted[:, :-1] = values[:, 1:]
    out = torch.empty_like(rewards)
    carry = torch.zeros(n_env, dtype=rewards.dtype)
    for t in range(n_t - 1, -1, -1):
        if t == n_t - 1:
            v_next = boot[:, t]
        elif truncateds is not None:
            v_next = torch.where(truncateds[:, t].bool(), boot[:, t], shifted[:, t])
        else:
            v_next = shifted[:, t]
        if truncateds is not None:
            done = (terminateds[:, t] + truncateds[:, t]).clamp(max=1.0)
        else:
            done = terminateds[:, t]
        delta = rewards[:, t] + gamma * (1.0 - terminateds[:, t]) * v_next - values[:, t]
        carry = delta + gamma * lambda_ * (1.0 - done) * carry
        out[:, t] = carry
    return out


def vtrace_loop(log_pi_target, log_pi_behavior, values, rewards, terminateds,
                gamma=0.99, rho_bar=1.0, c_bar=1.0, last_value=None):
    """V-trace (no truncations) by a backward loop over time."""
    n_env, n_t = rewards.shape
    shifted = torch.zeros_like(values)
    shifted[:, :-1] = values[:, 1:]
    if last_value is not None:
        shifted[:, -1] = last_value
    ratio = torch.exp(log_pi_target - log_pi_behavior)
    rho = torch.clamp(ratio, max=rho_bar)
    c = torch.clamp(ratio, max=c_bar)
    disc = gamma * (1.0 - terminateds)
    deltas = rho * (rewards + disc * shifted - values)
    acc = torch.empty_like(rewards)
    carry = torch.zeros(n_env, dtype=rewards.dtype)
    for t in range(n_t - 1, -1, -1):
        carry = deltas[:, t] + disc[:, t] * c[:, t] * carry
        acc[:, t] = carry
    targets = acc + values
    nxt_t = torch.empty_like(targets)
    nxt_t[:, :-1] = targets[:, 1:]
    nxt_t[:, -1] = shifted[:, -1]
    adv = rho * (rewards + disc * nxt_t - values)
    return targets, adv


def retrace_loop(action_probs_target, action_probs_behavior, q_values, next_q_values_all, actions,
                 rewards, terminateds, truncateds, gamma, lambda_=1.0, c_bar=1.0, rho_bar=1.0):
    """Retrace(lambda) by a backward loop over time: reference_retrace,
    tests/test_retrace.py:19-60."""
    n_env, n_t = rewards.shape
    dones = (terminateds + truncateds).clamp(max=1.0)
    expected_next_q = (action_probs_target * next_q_values_all).sum(dim=-1)
    deltas = rewards + gamma * expected_next_q * (1.0 - terminateds) - q_values
    pi_a = action_probs_target.gather(-1, actions.unsqueeze(-1)).squeeze(-1)
    c = lambda_ * torch.clamp(pi_a / action_probs_behavior, max=c_bar)
    rho = torch.clamp(pi_a / action_probs_behavior, max=rho_bar)
    q_deltas = torch.zeros_like(rewards)
    carry = torch.zeros(n_env, dtype=rewards.dtype)
    for t in range(n_t - 1, -1, -1):
        c_next = c[:, t + 1] if t + 1 < n_t else torch.zeros(n_env, dtype=rewards.dtype)
        decay = gamma * c_next * (1.0 - dones[:, t])
        carry = deltas[:, t] + decay * carry
        q_deltas[:, t] = carry
    targets = q_deltas + q_values
    next_q_ret = torch.zeros_like(targets)
    next_q_ret[:, :-1] = targets[:, 1:]
    return targets, rho * (rewards + gamma * next_q_ret * (1.0 - terminateds) - q_values)


def lambda_returns_loop(rewards, next_values, terminateds, truncateds=None, gamma=0.99,
                        lambda_=0.95, bootstrap_values=None):
    """TD(lambda) returns by a backward loop: reference_lambda_returns,
    tests/test_returns.py:19-38, and with truncations _ref_lambda_sequential, :449-485."""
    n_env, n_t = rewards.shape
    out = torch.zeros_like(rewards)
    carry = torch.zeros(n_env, dtype=rewards.dtype)
    if bootstrap_values is not None:
        carry = bootstrap_values[:, -1].clone()
    for t in range(n_t - 1, -1, -1):
        if truncateds is None:
            not_done = 1.0 - terminateds[:, t]
            carry = (rewards[:, t] + gamma * (1.0 - lambda_) * not_done * next_values[:, t]
                     + gamma * lambda_ * not_done * carry)
        else:
            not_done = 1.0 - (terminateds[:, t] + truncateds[:, t]).clamp(max=1.0)
            u = (rewards[:, t] + gamma * (1.0 - lambda_) * not_done * next_values[:, t]
                 + gamma * truncateds[:, t] * bootstrap_values[:, t])
            carry = u + gamma * lambda_ * not_done * carry
        out[:, t] = carry
    return out


def discounted_returns_loop(rewards, terminateds, truncateds=None, gamma=0.99,
                            bootstrap_values=None):
    """Discounted returns by a backward loop: reference_discounted_returns,
    tests/test_returns.py:41-57, and with truncations _ref_discounted_sequential, :488-510."""
    n_env, n_t = rewards.shape
    out = torch.zeros_like(rewards)
    carry = torch.zeros(n_env, dtype=rewards.dtype)
    if bootstrap_values is not None:
        carry = bootstrap_values[:, -1].clone()
    for t in range(n_t - 1, -1, -1):
        if truncateds is None:
            carry = rewards[:, t] + gamma * (1.0 - terminateds[:, t]) * carry
        else:
            not_done = 1.0 - (terminateds[:, t] + truncateds[:, t]).clamp(max=1.0)
            carry = (rewards[:, t] + gamma * not_done * carry
                     + gamma * truncateds[:, t] * bootstrap_values[:, t])
        out[:, t] = carry
    return out


def eligibility_traces_loop(gradients, dones, gamma, lambda_, seed_values=None):
    """Eligibility traces by a forward loop: reference_eligibility_traces,
    tests/test_returns.py:362-384."""
    n_env, n_t = gradients.shape
    out = torch.zeros_like(gradients)
    carry = torch.zeros(n_env, dtype=gradients.dtype)
    if seed_values is not None:
        carry = seed_values.clone()
    prev_done = torch.zeros(n_env, dtype=gradients.dtype)
    for t in range(n_t):
        carry = gradients[:, t] + gamma * lambda_ * (1.0 - prev_done) * carry
        out[:, t] = carry
        prev_done = dones[:, t]
    return out


def prefix_sum_loop(inputs, dones, seed_values=None, boundary="ends_at"):
    """The episodic prefix sum by a forward loop: reference_episodic_prefix_sum,
    tests/test_prefix_sum.py:18-56."""
    n_env, n_t = inputs.shape
    out = torch.zeros_like(inputs)
    carry = torch.zeros(n_env, dtype=inputs.dtype)
    if seed_values is not None:
        carry = seed_values.clone()
    prev_done = torch.zeros(n_env, dtype=inputs.dtype)
    for t in range(n_t):
        gate = prev_done if boundary == "ends_at" else dones[:, t]
        carry = inputs[:, t] + (1.0 - gate) * carry
        out[:, t] = carry
        prev_done = dones[:, t]
    return out
