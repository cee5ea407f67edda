"""Shared test helpers: golden fixtures, seeded input factories, op adapters.

Inputs are drawn on the CPU from seeded generators (CPU and GPU RNG streams differ)
and copied to the device, so the GPU path and the oracle see identical bits.
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

from baseline_configs import span_mask  # noqa: F401  (re-exported for the tests)
from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "known_answers.json")


def golden_cases(op=None):
    with open(GOLDEN) as f:
        cases = json.load(f)["cases"]
    return [c for c in cases if op is None or c["op"] == op]


# ---------------------------------------------------------------------------------------
# op adapters: the same case dict drives the oracle (NumPy) and the rl_triton API (torch)
# ---------------------------------------------------------------------------------------
OUTPUTS = {
    "gae": ("advantages",), "vtrace": ("targets", "advantages"),
    "retrace": ("targets", "advantages"), "lambda_returns": ("returns",),
    "discounted_returns": ("returns",), "eligibility_traces": ("traces",),
    "prefix_sum": ("prefix_sums",), "backward_scan": ("out",), "forward_scan": ("out",),
    "gae_normalized": ("advantages", "returns"), "gae_masked": ("advantages",),
    "gae_normalized_masked": ("advantages", "returns"),
}


def normalized_from_oracle(adv, values, eps, mask=None):
    """The float64 composition compute_gae_normalized fuses: returns = A + values and
    (A - mean) / (std + eps), std unbiased -- numpy's ddof=1, torch's Tensor.std().  With a
    mask, mean and std are over the kept steps (mask != 0) and applied to every step."""
    a = np.asarray(adv, dtype=np.float64)
    ret = a + np.asarray(values, dtype=np.float64)
    kept = a if mask is None else a[np.asarray(mask) != 0]
    mean = kept.mean() if kept.size else np.nan
    std = kept.std(ddof=1) if kept.size > 1 else np.nan
    return (a - mean) / (std + eps), ret


def run_oracle(op, inp, params):
    g = lambda k: inp.get(k)  # noqa: E731
    if op == "gae":
        boot = g("last_value") if g("last_value") is not None else g("bootstrap_values")
        return (orc.gae(g("rewards"), g("values"), g("terminateds"), g("truncateds"),
                        bootstrap=boot, **params),)
    if op == "gae_masked":
        boot = g("last_value") if g("last_value") is not None else g("bootstrap_values")
        return (orc.gae_masked(g("rewards"), g("values"), g("terminateds"), g("mask"),
                               g("truncateds"), bootstrap=boot, **params),)
    if op == "gae_normalized_masked":
        boot = g("last_value") if g("last_value") is not None else g("bootstrap_values")
        p = dict(params)
        eps = p.pop("eps", 1e-8)
        adv = orc.gae_masked(g("rewards"), g("values"), g("terminateds"), g("mask"),
                             g("truncateds"), bootstrap=boot, **p)
        return normalized_from_oracle(adv, g("values"), eps, g("mask"))
    if op == "gae_normalized":
        boot = g("last_value") if g("last_value") is not None else g("bootstrap_values")
        p = dict(params)
        eps = p.pop("eps", 1e-8)
        adv = orc.gae(g("rewards"), g("values"), g("terminateds"), g("truncateds"), bootstrap=boot, **p)
        return normalized_from_oracle(adv, g("values"), eps)
    if op == "vtrace":
        boot = g("last_value") if g("last_value") is not None else g("bootstrap_values")
        return orc.vtrace(g("log_pi_target"), g("log_pi_behavior"), g("values"), g("rewards"),
                          g("terminateds"), g("truncateds"), bootstrap=boot, **params)
    if op == "retrace":
        p = dict(params)
        return orc.retrace(g("action_probs_target"), g("action_probs_behavior"), g("q_values"),
                           g("next_q_values_all"), g("actions"), g("rewards"), g("terminateds"),
                           g("truncateds"), **p)
    if op == "lambda_returns":
        return (orc.lambda_returns(g("rewards"), g("next_values"), g("terminateds"),
                                   g("truncateds"), bootstrap=g("bootstrap_values"), **params),)
    if op == "discounted_returns":
        return (orc.discounted_returns(g("rewards"), g("terminateds"), g("truncateds"),
                                       bootstrap=g("bootstrap_values"), **params),)
    if op == "eligibility_traces":
        return (orc.eligibility_traces(g("gradients"), g("dones"), params["gamma"],
                                       params["lambda_"], g("seed_values")),)
    if op == "prefix_sum":
        return (orc.episodic_prefix_sum(g("inputs"), g("dones"), g("seed_values"),
                                        params.get("boundary", "ends_at")),)
    if op == "backward_scan":
        return (orc.backward_scan(g("u"), g("v"), g("bootstrap")),)
    if op == "forward_scan":
        return (orc.forward_scan(g("u"), g("v"), g("seed")),)
    raise KeyError(op)


def _placed(t, offset):
    """`t` as a contiguous view that starts `offset` elements into a larger buffer, so its
    data pointer is only element-aligned (offset 1: not 16-byte aligned)."""
    if not offset:
        return t
    buf = torch.empty(t.numel() + offset, dtype=t.dtype, device=t.device)
    buf[offset:].copy_(t.reshape(-1))
    return buf[offset:].view(t.shape)


def to_device(inp, device, dtype=torch.float32, offset=0):
    """Float inputs as `dtype` (float32 or bfloat16, rounded to nearest even), int64 actions;
    offset > 0 places every array that many elements into a larger buffer."""
    out = {}
    for k, v in inp.items():
        if v is None:
            out[k] = None
        elif k == "actions":
            out[k] = _placed(torch.as_tensor(np.asarray(v, dtype=np.int64)).to(device), offset)
        else:
            out[k] = _placed(torch.as_tensor(np.asarray(v, dtype=np.float32)).to(dtype).to(device), offset)
    return out


def run_api(op, inp, params, device, dtype=torch.float32, offset=0):
    import rl_triton
    from rl_triton.ops._scan import _run_scan, _run_scan_forward
    d = to_device(inp, device, dtype, offset)
    g = lambda k: d.get(k)  # noqa: E731
    if op == "gae":
        return (rl_triton.compute_gae(g("rewards"), g("values"), g("terminateds"), g("truncateds"),
                                      bootstrap_values=g("bootstrap_values"),
                                      last_value=g("last_value"), **params),)
    if op == "gae_masked":
        return (rl_triton.compute_gae(g("rewards"), g("values"), g("terminateds"), g("truncateds"),
                                      bootstrap_values=g("bootstrap_values"),
                                      last_value=g("last_value"), mask=g("mask"), **params),)
    if op == "gae_normalized_masked":
        return rl_triton.compute_gae_normalized(g("rewards"), g("values"), g("terminateds"),
                                                g("truncateds"),
                                                bootstrap_values=g("bootstrap_values"),
                                                last_value=g("last_value"), mask=g("mask"),
                                                **params)
    if op == "gae_normalized":
        return rl_triton.compute_gae_normalized(g("rewards"), g("values"), g("terminateds"),
                                                g("truncateds"),
                                                bootstrap_values=g("bootstrap_values"),
                                                last_value=g("last_value"), **params)
    if op == "vtrace":
        return rl_triton.compute_vtrace(g("log_pi_target"), g("log_pi_behavior"), g("values"),
                                        g("rewards"), g("terminateds"), g("truncateds"),
                                        bootstrap_values=g("bootstrap_values"),
                                        last_value=g("last_value"), **params)
    if op == "retrace":
        tr = g("truncateds") if g("truncateds") is not None else torch.zeros_like(g("rewards"))
        return rl_triton.compute_retrace(g("action_probs_target"), g("action_probs_behavior"),
                                         g("q_values"), g("next_q_values_all"), g("actions"),
                                         g("rewards"), g("terminateds"), tr, **params)
    if op == "lambda_returns":
        return (rl_triton.compute_lambda_returns(g("rewards"), g("next_values"), g("terminateds"),
                                                 g("truncateds"),
                                                 bootstrap_values=g("bootstrap_values"), **params),)
    if op == "discounted_returns":
        return (rl_triton.compute_discounted_returns(g("rewards"), g("terminateds"),
                                                     g("truncateds"),
                                                     bootstrap_values=g("bootstrap_values"),
                                                     **params),)
    if op == "eligibility_traces":
        return (rl_triton.compute_eligibility_traces(g("gradients"), g("dones"), params["gamma"],
                                                     params["lambda_"],
                                                     seed_values=g("seed_values")),)
    if op == "prefix_sum":
        return (rl_triton.compute_episodic_prefix_sum(g("inputs"), g("dones"),
                                                      seed_values=g("seed_values"),
                                                      boundary=params.get("boundary", "ends_at")),)
    if op == "backward_scan":
        return (_run_scan(g("u"), g("v"), g("bootstrap")),)
    if op == "forward_scan":
        return (_run_scan_forward(g("u"), g("v"), g("seed")),)
    raise KeyError(op)


# ---------------------------------------------------------------------------------------
# seeded input factories (distributions of the reference's tests and BASELINE configs)
# ---------------------------------------------------------------------------------------
def _gen(seed):
    return torch.Generator().manual_seed(seed)


def make_inputs(op, n_env, n_t, seed=0, p_term=0.05, p_trunc=0.0, boot="none", n_act=4,
                p_done=None):
    """Inputs for `op` as float32/int64 NumPy arrays (CPU), plus default params."""
    g = _gen(seed)
    rn = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    ru = lambda *s: torch.rand(*s, generator=g)   # noqa: E731
    shape = (n_env, n_t)
    term = (ru(*shape) < p_term).float()
    trunc = None
    if p_trunc > 0:
        trunc = (ru(*shape) < p_trunc).float() * (1.0 - term)
    inp = {}
    if op in ("gae", "gae_normalized", "gae_masked", "gae_normalized_masked", "vtrace",
              "lambda_returns", "discounted_returns"):
        if boot == "row":
            inp["last_value"] = rn(n_env)
        elif boot == "full":
            bv = torch.zeros(shape)
            if trunc is not None:
                bv = torch.where(trunc.bool(), rn(*shape), bv)
            bv[:, -1] = rn(n_env)
            inp["bootstrap_values"] = bv
    if op in ("gae", "gae_normalized", "gae_masked", "gae_normalized_masked"):
        inp.update(rewards=rn(*shape), values=rn(*shape), terminateds=term, truncateds=trunc)
        params = {"gamma": 0.99, "lambda_": 0.95}
        if op in ("gae_masked", "gae_normalized_masked"):
            inp["mask"] = span_mask(n_env, n_t, g)
    elif op == "vtrace":
        inp.update(log_pi_target=-ru(*shape), log_pi_behavior=-ru(*shape), values=rn(*shape),
                   rewards=rn(*shape), terminateds=term, truncateds=trunc)
        params = {"gamma": 0.99, "rho_bar": 1.0, "c_bar": 1.0}
    elif op == "retrace":
        inp.update(action_probs_target=torch.softmax(rn(n_env, n_t, n_act), dim=-1),
                   action_probs_behavior=ru(*shape) * 0.8 + 0.1, q_values=rn(*shape),
                   next_q_values_all=rn(n_env, n_t, n_act),
                   actions=torch.randint(0, n_act, shape, generator=g),
                   rewards=rn(*shape), terminateds=term,
                   truncateds=trunc if trunc is not None else torch.zeros(shape))
        params = {"gamma": 0.99, "lambda_": 0.95}
    elif op == "lambda_returns":
        inp.update(rewards=rn(*shape), next_values=rn(*shape), terminateds=term, truncateds=trunc)
        params = {"gamma": 0.99, "lambda_": 0.95}
    elif op == "discounted_returns":
        inp.update(rewards=rn(*shape), terminateds=term, truncateds=trunc)
        params = {"gamma": 0.99}
    elif op == "eligibility_traces":
        pd = p_term if p_done is None else p_done
        inp.update(gradients=rn(*shape), dones=(ru(*shape) < pd).float())
        if boot == "row":
            inp["seed_values"] = rn(n_env)
        params = {"gamma": 0.99, "lambda_": 0.95}
    elif op == "prefix_sum":
        pd = p_term if p_done is None else p_done
        inp.update(inputs=rn(*shape), dones=(ru(*shape) < pd).float())
        if boot == "row":
            inp["seed_values"] = rn(n_env)
        params = {"boundary": "ends_at"}
    elif op in ("backward_scan", "forward_scan"):
        inp.update(u=rn(*shape), v=ru(*shape) * 0.99)
        if boot == "row":
            inp["bootstrap" if op == "backward_scan" else "seed"] = ru(n_env) * 2.0
        params = {}
    else:
        raise KeyError(op)
    out = {}
    for k, v in inp.items():
        if v is None:
            out[k] = None
        elif k == "actions":
            out[k] = v.numpy().astype(np.int64)
        else:
            out[k] = v.numpy().astype(np.float32)
    return out, params


def suite_atol(op, inp, expected, seq_len):
    """The suite's absolute tolerance against the float64 oracle for one output: 1e-5 for
    rows of up to 2048 steps; for longer rows (the look-back path)
    1e-5 * sqrt(L_eff / 128) * max(1, max|expected|), with L_eff = 1 / (1 - decay) for
    decaying scans (gamma = 0.99, lambda = 0.95) and the longest done-free run for the
    prefix sum."""
    import math
    if seq_len <= 2048:
        return 1e-5
    scale = max(1.0, float(np.max(np.abs(expected))))
    if op == "prefix_sum":
        l_eff = 1
        for row in np.asarray(inp["dones"]) > 0:
            idx = np.flatnonzero(np.concatenate(([True], row, [True])))
            l_eff = max(l_eff, int(np.max(np.diff(idx))))
    elif op in ("discounted_returns", "backward_scan", "forward_scan"):
        l_eff = 1.0 / (1.0 - 0.99)
    else:
        l_eff = 1.0 / (1.0 - 0.99 * 0.95)
    return 1e-5 * math.sqrt(max(l_eff, 128) / 128.0) * scale


def max_abs_err(actual, expected):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(a - e))) if a.size else 0.0


def assert_close(actual, expected, rtol, atol, what=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    if a.size == 0:
        return
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    err = np.abs(a - e)
    bound = atol + rtol * np.abs(e)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} elements out of tolerance "
                             f"(rtol={rtol}, atol={atol}); max abs err {err.max():.3e}; "
                             f"worst at {i}: got {a[i]!r}, expected {e[i]!r}")
