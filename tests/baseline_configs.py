"""The BASELINE.json configurations as seeded input factories.

Shared by the full-size parity tests (tests/test_gpu_parity.py) and bench.py's
per-configuration kernel timings, so both see the same distributions:

  C1  GAE [64, 512]: r, v ~ N(0,1), terminateds = 0, last_value ~ N(0,1)
  C2  GAE [4096, 128]: r, v ~ N(0,1), terminateds ~ Bern(0.01), truncateds ~ Bern(0.005)
      (exclusive with terminateds), bootstrap_values ~ N(0,1) at truncations and t = T-1
  C3  V-trace [4096, 128]: log_pi_target ~ N(0, 0.5^2), log_pi_behavior = 0, r, v ~ N(0,1),
      last_value ~ N(0,1), terminateds ~ Bern(0.01), rho_bar = c_bar = 1
  C4  Retrace(lambda) and TD(lambda) [4096, 128] and [256, 2048]: A = 2 actions,
      actions = 0, pi = [p, 1-p] with p ~ U(0.05, 1), mu ~ U(0.05, 1), both next-Q columns
      = expected_q_next ~ N(0,1) (so E_pi[Q'] = expected_q_next), q ~ N(0,1), r ~ N(0,1),
      terminateds ~ Bern(0.01), truncateds = 0, lambda = 0.95;  TD(lambda) takes
      next_values = expected_q_next
  C5  episodic prefix sum (ends_at) and eligibility traces (gamma*lambda = 0.9405) on
      [8, 1048576], discounted returns and V-trace on [16, 131072]: x ~ N(0,1),
      done ~ Bern(1e-4), gamma = 0.99; V-trace log-ratios ~ N(0, 0.5^2), last_value ~ N(0,1)

gamma = 0.99 throughout.  BYTES is each configuration's algorithmic bytes per element:
the compulsory reads of every per-step input plus the writes of every output (per-row
values ignored).
"""
from __future__ import annotations

import math

import torch

# name -> (op, num_envs, seq_len, algorithmic bytes per element)
CONFIGS = {
    "C1_gae_64x512": ("gae", 64, 512, 16),
    "C2_gae_4096x128": ("gae", 4096, 128, 24),
    "C3_vtrace_4096x128": ("vtrace", 4096, 128, 28),
    "C4_retrace_4096x128": ("retrace", 4096, 128, 52),
    "C4_retrace_256x2048": ("retrace", 256, 2048, 52),
    "C4_lambda_returns_4096x128": ("lambda_returns", 4096, 128, 16),
    "C4_lambda_returns_256x2048": ("lambda_returns", 256, 2048, 16),
    "C5_prefix_sum_8x1048576": ("prefix_sum", 8, 1 << 20, 12),
    "C5_eligibility_traces_8x1048576": ("eligibility_traces", 8, 1 << 20, 12),
    "C5_discounted_returns_16x131072": ("discounted_returns", 16, 131072, 12),
    "C5_vtrace_16x131072": ("vtrace", 16, 131072, 28),
}

# BASELINE's north-star targets (fraction of 8 TB/s) where it states one
TARGETS = {"C2_gae_4096x128": 0.60, "C3_vtrace_4096x128": 0.60,
           "C5_prefix_sum_8x1048576": 0.50, "C5_eligibility_traces_8x1048576": 0.50,
           "C5_discounted_returns_16x131072": 0.50, "C5_vtrace_16x131072": 0.50}


def make(name: str, seed: int = 0, device="cpu", shape=None):
    """Inputs (dict of float32 / int64 tensors on `device`) and keyword params of `name`.
    With device="cpu" the draw is a seeded CPU generator (the parity sets); on a GPU the
    same distributions come from a seeded device generator (the bench's rotating sets).
    shape=(E, T) draws the same distributions at another shape."""
    op, E, T, _ = CONFIGS[name]
    if shape is not None:
        E, T = shape
    g = torch.Generator(device=device).manual_seed(seed)
    kw = {"generator": g, "device": device}
    rn = lambda *s: torch.randn(*s, **kw)           # noqa: E731
    ru = lambda *s: torch.rand(*s, **kw)            # noqa: E731
    bern = lambda p: (ru(E, T) < p).float()         # noqa: E731
    if name.startswith("C1"):
        inp = dict(rewards=rn(E, T), values=rn(E, T), terminateds=torch.zeros(E, T, device=device),
                   last_value=rn(E))
        return inp, {"gamma": 0.99, "lambda_": 0.95}
    if name.startswith("C2"):
        term = bern(0.01)
        trunc = bern(0.005) * (1.0 - term)
        boot = torch.where(trunc.bool(), rn(E, T), torch.zeros(E, T, device=device))
        boot[:, -1] = rn(E)
        inp = dict(rewards=rn(E, T), values=rn(E, T), terminateds=term, truncateds=trunc,
                   bootstrap_values=boot)
        return inp, {"gamma": 0.99, "lambda_": 0.95}
    if op == "vtrace":
        p_done = 0.01 if name.startswith("C3") else 1e-4
        inp = dict(log_pi_target=0.5 * rn(E, T), log_pi_behavior=torch.zeros(E, T, device=device),
                   values=rn(E, T), rewards=rn(E, T), terminateds=bern(p_done), last_value=rn(E))
        return inp, {"gamma": 0.99, "rho_bar": 1.0, "c_bar": 1.0}
    if op == "retrace":
        p = 0.05 + 0.95 * ru(E, T)
        eq = rn(E, T)
        inp = dict(action_probs_target=torch.stack((p, 1.0 - p), dim=-1).contiguous(),
                   action_probs_behavior=0.05 + 0.95 * ru(E, T),
                   q_values=rn(E, T),
                   next_q_values_all=torch.stack((eq, eq), dim=-1).contiguous(),
                   actions=torch.zeros(E, T, dtype=torch.int64, device=device),
                   rewards=rn(E, T), terminateds=bern(0.01),
                   truncateds=torch.zeros(E, T, device=device))
        return inp, {"gamma": 0.99, "lambda_": 0.95, "c_bar": 1.0, "rho_bar": 1.0}
    if op == "lambda_returns":
        inp = dict(rewards=rn(E, T), next_values=rn(E, T), terminateds=bern(0.01))
        return inp, {"gamma": 0.99, "lambda_": 0.95}
    if op == "discounted_returns":
        inp = dict(rewards=rn(E, T), terminateds=bern(1e-4))
        return inp, {"gamma": 0.99}
    if op == "eligibility_traces":
        inp = dict(gradients=rn(E, T), dones=bern(1e-4))
        return inp, {"gamma": 0.99, "lambda_": 0.95}
    if op == "prefix_sum":
        inp = dict(inputs=rn(E, T), dones=bern(1e-4))
        return inp, {"boundary": "ends_at"}
    raise KeyError(name)


def make_exact(name: str, seed: int = 0, device="cpu"):
    """Configuration `name` at its full shape and done/truncation distributions, with inputs
    on which float32 arithmetic is exact in any order: integer rewards, values and
    bootstraps in [-3, 3], unit discounts (gamma = lambda = 1), V-trace log-ratios >= 0 with
    rho_bar = 0.5 and c_bar = 1 (so rho = 0.5 and c = 1 at every step: the two clips
    differ), Retrace with pi = [0.25, 0.75], mu = 0.125 (ratios 2 and 6, clipped to
    c = 1, rho = 0.5).  Every partial result is then a multiple of 1/8 below 2^21 in
    magnitude, so a correct kernel equals the float64 oracle bit for bit whatever its
    association order, and any error in indexing, done gating or carry passing shows as a
    difference."""
    op, E, T, _ = CONFIGS[name]
    inp, params = make(name, seed=seed, device=device)
    g = torch.Generator(device=device).manual_seed(seed + 7)
    ri = lambda *s: torch.randint(-3, 4, s, generator=g, device=device).float()  # noqa: E731
    for k in ("rewards", "values", "gradients", "inputs", "q_values"):
        if k in inp:
            inp[k] = ri(E, T)
    if "last_value" in inp:
        inp["last_value"] = ri(E)
    if "bootstrap_values" in inp:
        inp["bootstrap_values"] = torch.where(inp["bootstrap_values"] != 0, ri(E, T),
                                              torch.zeros(E, T, device=device))
        inp["bootstrap_values"][:, -1] = ri(E)
    if "next_values" in inp:
        inp["next_values"] = ri(E, T)
    params = {k: (1.0 if k in ("gamma", "lambda_") else v) for k, v in params.items()}
    if op == "vtrace":
        lpb = torch.randn(E, T, generator=g, device=device)
        inp["log_pi_behavior"] = lpb
        inp["log_pi_target"] = lpb + torch.rand(E, T, generator=g, device=device)
        params.update(rho_bar=0.5, c_bar=1.0)
    if op == "retrace":
        p = torch.tensor([0.25, 0.75], device=device)
        inp["action_probs_target"] = p.expand(E, T, 2).contiguous()
        inp["action_probs_behavior"] = torch.full((E, T), 0.125, device=device)
        inp["next_q_values_all"] = torch.stack((ri(E, T), ri(E, T)), dim=-1).contiguous()
        inp["actions"] = torch.randint(0, 2, (E, T), generator=g, device=device)
        params.update(c_bar=1.0, rho_bar=0.5)
    return inp, params


def as_dtype(inp: dict, dtype) -> dict:
    """The float inputs of a configuration as `dtype` (int64 actions unchanged)."""
    return {k: (v.to(dtype) if v is not None and v.is_floating_point() else v)
            for k, v in inp.items()}


def bytes_per_elem(name: str, dtype=torch.float32) -> int:
    """Algorithmic bytes per element with float arrays of `dtype` (Retrace's int64 actions
    are 8 bytes either way)."""
    bpe = CONFIGS[name][3]
    ints = 8 if CONFIGS[name][0] == "retrace" else 0
    return ints + (bpe - ints) * torch.finfo(dtype).bits // 32


def span_mask(n_env: int, n_t: int, g: torch.Generator, mean_span: float = 12.0):
    """A multi-turn mask for compute_gae(..., mask=...): alternating kept (response) and
    skipped (observation) spans of geometric lengths with mean `mean_span`, each row
    starting with either; float32 [n_env, n_t] on the CPU, drawn from `g`."""
    p = 1.0 / mean_span
    n_spans = int(2 * n_t / mean_span) + 64
    u = torch.rand(n_env, n_spans, generator=g).clamp_min(1e-12)
    ends = torch.cumsum(1 + torch.floor(torch.log(u) / math.log(1.0 - p)).long(), dim=1)
    t = torch.arange(n_t).expand(n_env, n_t).contiguous()
    span = torch.searchsorted(ends, t, right=True)
    first_kept = (torch.rand(n_env, 1, generator=g) < 0.5).long()
    return ((span + first_kept) % 2 == 1).float()


def call(name: str, inp: dict, params: dict):
    """One public-API call of configuration `name` on device tensors; returns a tuple."""
    import rl_triton
    op = CONFIGS[name][0]
    if op == "gae":
        return (rl_triton.compute_gae(inp["rewards"], inp["values"], inp["terminateds"],
                                      inp.get("truncateds"),
                                      bootstrap_values=inp.get("bootstrap_values"),
                                      last_value=inp.get("last_value"), **params),)
    if op == "vtrace":
        return rl_triton.compute_vtrace(inp["log_pi_target"], inp["log_pi_behavior"], inp["values"],
                                        inp["rewards"], inp["terminateds"],
                                        last_value=inp["last_value"], **params)
    if op == "retrace":
        return rl_triton.compute_retrace(inp["action_probs_target"], inp["action_probs_behavior"],
                                         inp["q_values"], inp["next_q_values_all"], inp["actions"],
                                         inp["rewards"], inp["terminateds"], inp["truncateds"],
                                         **params)
    if op == "lambda_returns":
        return (rl_triton.compute_lambda_returns(inp["rewards"], inp["next_values"],
                                                 inp["terminateds"], **params),)
    if op == "discounted_returns":
        return (rl_triton.compute_discounted_returns(inp["rewards"], inp["terminateds"], **params),)
    if op == "eligibility_traces":
        return (rl_triton.compute_eligibility_traces(inp["gradients"], inp["dones"], **params),)
    if op == "prefix_sum":
        return (rl_triton.compute_episodic_prefix_sum(inp["inputs"], inp["dones"], **params),)
    raise KeyError(name)


def set_bytes(name: str) -> int:
    """Bytes of one input set plus its outputs (what one call touches)."""
    _, E, T, bpe = CONFIGS[name]
    return E * T * bpe


def horizon_atol(name: str, expected, dones=None) -> float:
    """The long-scan tolerance: 1e-5 * sqrt(L_eff / 128) * max(1, max|expected|), with
    L_eff = 1 / (1 - decay) for decaying scans and the longest done-free run for the
    prefix sum (decay 1)."""
    import numpy as np
    op = CONFIGS[name][0]
    scale = max(1.0, float(np.max(np.abs(expected))))
    if op == "prefix_sum":
        l_eff = 1
        for row in np.asarray(dones) > 0:
            idx = np.flatnonzero(np.concatenate(([True], row, [True])))
            l_eff = max(l_eff, int(np.max(np.diff(idx))))
    elif op == "discounted_returns":
        l_eff = 1.0 / (1.0 - 0.99)
    else:
        l_eff = 1.0 / (1.0 - 0.99 * 0.95)
    return 1e-5 * math.sqrt(max(l_eff, 128) / 128.0) * scale
