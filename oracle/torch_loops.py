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
