"""GAE with returns and batch-normalised advantages, fused on gfx950.

Not in the reference's API: it is the first item of the reference's ROADMAP.md:75-81
("Fused GAE + advantage normalisation"), built on the same scan.  The composition it
replaces is what a PPO loop writes after compute_gae:

    adv = compute_gae(...)
    returns = adv + values
    adv = (adv - adv.mean()) / (adv.std() + eps)

Here the scan writes the raw advantages, the returns and per-workgroup float64 partial sums
in one pass; a second launch turns the advantages into (A - mean) / (std + eps) in place
(std unbiased, as Tensor.std()).  The statistics are reduced in a fixed order, so results
are bit-reproducible run to run.
"""
import torch

from rl_triton import _native
from rl_triton.ops.gae import _check_gae_args


def compute_gae_normalized(
    rewards: torch.Tensor,
    values: torch.Tensor,
    terminateds: torch.Tensor,
    truncateds: torch.Tensor | None = None,
    gamma: float = 0.99,
    lambda_: float = 0.95,
    bootstrap_values: torch.Tensor | None = None,
    last_value: torch.Tensor | None = None,
    eps: float = 1e-8,
    *,
    mask: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """
    Normalised GAE advantages and returns.

    Arguments, checks and the advantage recurrence are those of compute_gae (the same
    AssertionErrors, in the same order).

    `mask` (keyword-only): A is compute_gae(..., mask=mask) and mean and std are taken over
    the kept steps (mask != 0) only, then applied to every step -- the masked whitening verl
    applies after compute_gae_advantage_return (with its response_mask).

    Returns:
        advantages: (A - mean(A)) / (std(A) + eps), A = compute_gae(...), mean and std over
                    all num_envs * seq_len elements (the kept ones with a mask),
                    [num_envs, seq_len], the inputs' dtype.
        returns:    A + values, [num_envs, seq_len], the inputs' dtype.
    """
    # fast path: a well-formed call goes straight to the C ABI (rl_triton._rlk_torch)
    fast = _native.fast
    if fast is not None:
        res = fast.gae_normalized(rewards, values, terminateds, truncateds, gamma, lambda_,
                                  bootstrap_values, last_value, eps, mask)
        if res is not None:
            return res

    _check_gae_args(rewards, values, terminateds, truncateds, bootstrap_values, last_value, mask)
    rewards = rewards.contiguous()
    values = values.contiguous()
    terminateds = terminateds.contiguous()
    if truncateds is not None:
        truncateds = truncateds.contiguous()
    if last_value is not None:
        bootstrap = last_value.contiguous()
    elif bootstrap_values is not None:
        bootstrap = bootstrap_values.contiguous()
    else:
        bootstrap = None
    advantages = torch.empty_like(rewards)
    returns = torch.empty_like(rewards)
    return _native.gae_normalized(rewards, values, terminateds, truncateds, bootstrap, advantages,
                                  returns, gamma, lambda_, eps,
                                  None if mask is None else mask.contiguous())
