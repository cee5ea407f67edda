"""Write tests/golden/known_answers.json.

Two kinds of fixture:

1. The reference's own known-answer tests: hand-computed inputs and expected outputs
   written inline in simonsays1980/rl-triton v0.1.3 tests/*.py.  They are transcribed
   here as data (each case cites its test); nothing from the reference is imported.
2. Interior-truncation fixtures on the reference's shared layout (N=2, T=12,
   truncations at (0,3), (0,7), (1,5), bootstraps 2.5 / 1.8 / 0.9, window boundary
   3.2 -- tests/test_gae.py:457-492, tests/test_vtrace.py:487-570,
   tests/test_returns.py:513-583).  Their inputs come from a seeded NumPy generator
   and their expected outputs from the pure-Python float64 loops below, written from
   the estimators' definitions independently of oracle/rlk_oracle.c.

Run:  python tests/golden/make_known_answers.py
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")


def case(name, op, source, inputs, params, expected):
    return {"name": name, "op": op, "source": source, "inputs": inputs, "params": params,
            "expected": expected}


Z = lambda n, t: [[0.0] * t for _ in range(n)]  # noqa: E731
O = lambda n, t: [[1.0] * t for _ in range(n)]  # noqa: E731


def reference_known_answers():
    c = []
    # ---------------- GAE: tests/test_gae.py ----------------
    c.append(case("gae_single_env", "gae", "tests/test_gae.py:126-140",
                  {"rewards": [[1, 2, 3]], "values": Z(1, 3), "terminateds": Z(1, 3)},
                  {"gamma": 1.0, "lambda_": 1.0}, {"advantages": [[6, 5, 3]]}))
    c.append(case("gae_delta", "gae", "tests/test_gae.py:143-160",
                  {"rewards": [[1, 2, 3]], "values": O(1, 3), "terminateds": Z(1, 3)},
                  {"gamma": 1.0, "lambda_": 1.0}, {"advantages": [[5, 4, 2]]}))
    c.append(case("gae_gamma", "gae", "tests/test_gae.py:163-176",
                  {"rewards": [[1, 2]], "values": Z(1, 2), "terminateds": Z(1, 2)},
                  {"gamma": 0.9, "lambda_": 1.0}, {"advantages": [[2.8, 2.0]]}))
    c.append(case("gae_lambda0", "gae", "tests/test_gae.py:179-188",
                  {"rewards": [[1, 2, 3]], "values": Z(1, 3), "terminateds": Z(1, 3)},
                  {"gamma": 1.0, "lambda_": 0.0}, {"advantages": [[1, 2, 3]]}))
    c.append(case("gae_last_value", "gae", "tests/test_gae.py:191-211",
                  {"rewards": [[1, 2, 3]], "values": Z(1, 3), "terminateds": Z(1, 3),
                   "last_value": [2.0]},
                  {"gamma": 1.0, "lambda_": 1.0}, {"advantages": [[8, 7, 5]]}))
    c.append(case("gae_mixed_termination", "gae", "tests/test_gae.py:214-233",
                  {"rewards": [[1, 2], [1, 2]], "values": Z(2, 2), "terminateds": Z(2, 2),
                   "last_value": [0.0, 5.0]},
                  {"gamma": 1.0, "lambda_": 1.0}, {"advantages": [[3, 2], [8, 7]]}))
    c.append(case("gae_episode_boundary", "gae", "tests/test_gae.py:236-250",
                  {"rewards": [[1, 2, 3]], "values": Z(1, 3), "terminateds": [[0, 1, 0]]},
                  {"gamma": 1.0, "lambda_": 1.0}, {"advantages": [[3, 2, 3]]}))
    c.append(case("gae_batch", "gae", "tests/test_gae.py:253-264",
                  {"rewards": [[1, 2], [3, 4]], "values": Z(2, 2), "terminateds": Z(2, 2)},
                  {"gamma": 1.0, "lambda_": 1.0}, {"advantages": [[3, 2], [7, 4]]}))
    # ---------------- V-trace: tests/test_vtrace.py ----------------
    c.append(case("vtrace_single_env", "vtrace", "tests/test_vtrace.py:178-197",
                  {"log_pi_target": Z(1, 2), "log_pi_behavior": Z(1, 2), "values": Z(1, 2),
                   "rewards": O(1, 2), "terminateds": Z(1, 2)},
                  {"gamma": 1.0, "rho_bar": 100.0, "c_bar": 100.0},
                  {"targets": [[2, 1]], "advantages": [[2, 1]]}))
    c.append(case("vtrace_last_value", "vtrace", "tests/test_vtrace.py:200-226",
                  {"log_pi_target": Z(1, 2), "log_pi_behavior": Z(1, 2), "values": Z(1, 2),
                   "rewards": O(1, 2), "terminateds": Z(1, 2), "last_value": [0.5]},
                  {"gamma": 1.0, "rho_bar": 100.0, "c_bar": 100.0},
                  {"targets": [[2.5, 1.5]], "advantages": [[2.5, 1.5]]}))
    c.append(case("vtrace_done", "vtrace", "tests/test_vtrace.py:229-251",
                  {"log_pi_target": Z(1, 2), "log_pi_behavior": Z(1, 2), "values": Z(1, 2),
                   "rewards": O(1, 2), "terminateds": [[1, 0]]},
                  {"gamma": 1.0, "rho_bar": 100.0, "c_bar": 100.0}, {"targets": [[1, 1]]}))
    c.append(case("vtrace_clipping", "vtrace", "tests/test_vtrace.py:254-270",
                  {"log_pi_target": Z(1, 2), "log_pi_behavior": [[math.log(2.0)] * 2],
                   "values": Z(1, 2), "rewards": O(1, 2), "terminateds": Z(1, 2)},
                  {"gamma": 1.0, "rho_bar": 1.0, "c_bar": 1.0}, {"targets": [[0.75, 0.5]]}))
    # ---------------- lambda-returns: tests/test_returns.py ----------------
    c.append(case("lambda_returns_lambda0", "lambda_returns", "tests/test_returns.py:182-193",
                  {"rewards": [[1, 2]], "next_values": [[3, 4]], "terminateds": Z(1, 2)},
                  {"gamma": 1.0, "lambda_": 0.0}, {"returns": [[4, 6]]}))
    c.append(case("lambda_returns_lambda1", "lambda_returns", "tests/test_returns.py:196-205",
                  {"rewards": [[1, 2]], "next_values": [[99, 99]], "terminateds": Z(1, 2)},
                  {"gamma": 1.0, "lambda_": 1.0}, {"returns": [[3, 2]]}))
    c.append(case("lambda_returns_intermediate", "lambda_returns", "tests/test_returns.py:208-225",
                  {"rewards": [[1, 2]], "next_values": [[3, 4]], "terminateds": Z(1, 2)},
                  {"gamma": 1.0, "lambda_": 0.5}, {"returns": [[4.5, 4.0]]}))
    c.append(case("lambda_returns_done", "lambda_returns", "tests/test_returns.py:228-238",
                  {"rewards": [[1, 2]], "next_values": [[3, 4]], "terminateds": [[1, 0]]},
                  {"gamma": 1.0, "lambda_": 0.5}, {"returns": [[1, 4]]}))
    c.append(case("lambda_returns_bootstrap", "lambda_returns", "tests/test_returns.py:241-250",
                  {"rewards": [[1, 2]], "next_values": [[99, 99]], "terminateds": Z(1, 2),
                   "bootstrap_values": [[0, 5]]},
                  {"gamma": 1.0, "lambda_": 1.0}, {"returns": [[8, 7]]}))
    # ---------------- eligibility traces ----------------
    c.append(case("elig_basic", "eligibility_traces", "tests/test_returns.py:301-310",
                  {"gradients": [[1, 2, 3]], "dones": Z(1, 3)},
                  {"gamma": 1.0, "lambda_": 1.0}, {"traces": [[1, 3, 6]]}))
    c.append(case("elig_decay", "eligibility_traces", "tests/test_returns.py:313-320",
                  {"gradients": [[1, 2]], "dones": Z(1, 2)},
                  {"gamma": 1.0, "lambda_": 0.5}, {"traces": [[1, 2.5]]}))
    c.append(case("elig_done", "eligibility_traces", "tests/test_returns.py:323-333",
                  {"gradients": [[1, 2, 3]], "dones": [[0, 1, 0]]},
                  {"gamma": 1.0, "lambda_": 0.9}, {"traces": [[1, 2.9, 3.0]]}))
    c.append(case("elig_seed", "eligibility_traces", "tests/test_returns.py:336-345",
                  {"gradients": [[1, 2]], "dones": Z(1, 2), "seed_values": [2.0]},
                  {"gamma": 1.0, "lambda_": 1.0}, {"traces": [[3, 5]]}))
    c.append(case("elig_lambda0", "eligibility_traces", "tests/test_returns.py:348-355",
                  {"gradients": [[1, 2, 3]], "dones": Z(1, 3)},
                  {"gamma": 0.99, "lambda_": 0.0}, {"traces": [[1, 2, 3]]}))
    # ---------------- discounted returns ----------------
    c.append(case("discounted_basic", "discounted_returns", "tests/test_returns.py:418-424",
                  {"rewards": [[1, 2]], "terminateds": Z(1, 2)},
                  {"gamma": 0.9}, {"returns": [[2.8, 2.0]]}))
    c.append(case("discounted_done", "discounted_returns", "tests/test_returns.py:427-433",
                  {"rewards": [[1, 2]], "terminateds": [[1, 0]]},
                  {"gamma": 0.9}, {"returns": [[1, 2]]}))
    # ---------------- Retrace: tests/test_retrace.py ----------------
    def rt(q_next, probs_b, term, trunc, T):
        return {"action_probs_target": [[[1.0]] * T], "action_probs_behavior": [probs_b],
                "q_values": Z(1, T), "next_q_values_all": [[[x] for x in q_next]],
                "actions": [[0] * T], "rewards": O(1, T), "terminateds": [term],
                "truncateds": [trunc]}
    c.append(case("retrace_single_env", "retrace", "tests/test_retrace.py:146-165",
                  rt([2.0, 3.0], [1.0, 1.0], [0, 0], [0, 0], 2), {"gamma": 1.0},
                  {"targets": [[7, 4]], "advantages": [[5, 1]]}))
    c.append(case("retrace_done", "retrace", "tests/test_retrace.py:168-183",
                  rt([2.0, 3.0], [1.0, 1.0], [1, 0], [0, 0], 2), {"gamma": 1.0},
                  {"targets": [[1, 4]], "advantages": [[1, 1]]}))
    c.append(case("retrace_clipping", "retrace", "tests/test_retrace.py:186-201",
                  rt([0.5, 0.5], [0.5, 0.5], [0, 0], [0, 0], 2), {"gamma": 1.0},
                  {"targets": [[3.0, 1.5]]}))
    c.append(case("retrace_terminal_no_bootstrap", "retrace", "tests/test_retrace.py:208-222",
                  rt([5.0], [1.0], [1], [0], 1), {"gamma": 1.0}, {"targets": [[1.0]]}))
    c.append(case("retrace_truncated_keeps_bootstrap", "retrace", "tests/test_retrace.py:225-239",
                  rt([5.0], [1.0], [0], [1], 1), {"gamma": 1.0}, {"targets": [[6.0]]}))
    c.append(case("retrace_truncated_c_boundary", "retrace", "tests/test_retrace.py:242-258",
                  rt([5.0, 5.0], [1.0, 1.0], [0, 0], [0, 1], 2), {"gamma": 1.0},
                  {"targets": [[12.0, 6.0]]}))
    # ---------------- prefix sum: tests/test_prefix_sum.py ----------------
    for b in ("ends_at", "starts_at"):
        c.append(case(f"prefix_no_reset_{b}", "prefix_sum", "tests/test_prefix_sum.py:63-78",
                      {"inputs": [[1, 2, 3]], "dones": Z(1, 3)}, {"boundary": b},
                      {"prefix_sums": [[1, 3, 6]]}))
        c.append(case(f"prefix_all_resets_{b}", "prefix_sum", "tests/test_prefix_sum.py:141-153",
                      {"inputs": [[1, 2, 3]], "dones": O(1, 3)}, {"boundary": b},
                      {"prefix_sums": [[1, 2, 3]]}))
        c.append(case(f"prefix_seed_{b}", "prefix_sum", "tests/test_prefix_sum.py:156-173",
                      {"inputs": [[1, 2]], "dones": Z(1, 2), "seed_values": [10.0]},
                      {"boundary": b}, {"prefix_sums": [[11, 13]]}))
    c.append(case("prefix_reset_at_start_starts_at", "prefix_sum", "tests/test_prefix_sum.py:81-93",
                  {"inputs": [[5, 2, 3]], "dones": [[1, 0, 0]]}, {"boundary": "starts_at"},
                  {"prefix_sums": [[5, 7, 10]]}))
    c.append(case("prefix_reset_at_start_ends_at", "prefix_sum", "tests/test_prefix_sum.py:96-108",
                  {"inputs": [[5, 2, 3]], "dones": [[1, 0, 0]]}, {"boundary": "ends_at"},
                  {"prefix_sums": [[5, 2, 5]]}))
    c.append(case("prefix_mid_reset_starts_at", "prefix_sum", "tests/test_prefix_sum.py:111-123",
                  {"inputs": [[1, 2, 3, 4]], "dones": [[0, 0, 1, 0]]}, {"boundary": "starts_at"},
                  {"prefix_sums": [[1, 3, 3, 7]]}))
    c.append(case("prefix_mid_reset_ends_at", "prefix_sum", "tests/test_prefix_sum.py:126-138",
                  {"inputs": [[1, 2, 3, 4]], "dones": [[0, 0, 1, 0]]}, {"boundary": "ends_at"},
                  {"prefix_sums": [[1, 3, 6, 4]]}))
    c.append(case("prefix_seed_cancelled_starts_at", "prefix_sum", "tests/test_prefix_sum.py:176-188",
                  {"inputs": [[1, 2]], "dones": [[1, 0]], "seed_values": [10.0]},
                  {"boundary": "starts_at"}, {"prefix_sums": [[1, 3]]}))
    c.append(case("prefix_seed_cancelled_ends_at", "prefix_sum", "tests/test_prefix_sum.py:191-205",
                  {"inputs": [[1, 2]], "dones": [[1, 0]], "seed_values": [10.0]},
                  {"boundary": "ends_at"}, {"prefix_sums": [[11, 2]]}))
    c.append(case("prefix_batch_starts_at", "prefix_sum", "tests/test_prefix_sum.py:208-218",
                  {"inputs": [[1, 2, 3], [4, 2, 3]], "dones": [[0, 0, 0], [0, 1, 0]]},
                  {"boundary": "starts_at"}, {"prefix_sums": [[1, 3, 6], [4, 2, 5]]}))
    c.append(case("prefix_batch_ends_at", "prefix_sum", "tests/test_prefix_sum.py:221-231",
                  {"inputs": [[1, 2, 3], [4, 2, 3]], "dones": [[0, 0, 0], [0, 1, 0]]},
                  {"boundary": "ends_at"}, {"prefix_sums": [[1, 3, 6], [4, 6, 3]]}))
    return c


# ---------------------------------------------------------------------------------------
# Interior-truncation fixtures: expected values from element-by-element float64 loops.
# ---------------------------------------------------------------------------------------
N, T = 2, 12
TRUNC_AT = [(0, 3), (0, 7), (1, 5)]
BOOT_AT = {(0, 3): 2.5, (0, 7): 1.8, (0, 11): 3.2, (1, 5): 0.9}


def _f32(x):
    return float(np.float32(x))


def _layout():
    trunc = [[0.0] * T for _ in range(N)]
    for n, t in TRUNC_AT:
        trunc[n][t] = 1.0
    boot = [[0.0] * T for _ in range(N)]
    for (n, t), b in BOOT_AT.items():
        boot[n][t] = b
    return trunc, boot


def _rand(rng, lo=0.0, hi=1.0):
    return [[_f32(x) for x in row] for row in rng.uniform(lo, hi, size=(N, T))]


def brute_gae(r, v, term, trunc, boot, gamma, lam):
    out = [[0.0] * T for _ in range(N)]
    for n in range(N):
        acc = 0.0
        for t in reversed(range(T)):
            if t == T - 1 or trunc[n][t] == 1.0:
                nxt = boot[n][t]
            else:
                nxt = v[n][t + 1]
            delta = r[n][t] + gamma * (1.0 - term[n][t]) * nxt - v[n][t]
            cut = min(term[n][t] + trunc[n][t], 1.0)
            acc = delta + gamma * lam * (1.0 - cut) * acc
            out[n][t] = acc
    return out


def brute_vtrace(lpt, lpb, v, r, term, trunc, boot, gamma, rho_bar, c_bar):
    tg = [[0.0] * T for _ in range(N)]
    adv = [[0.0] * T for _ in range(N)]
    for n in range(N):
        acc = 0.0
        for t in reversed(range(T)):
            ratio = math.exp(lpt[n][t] - lpb[n][t])
            nxt = (v[n][t + 1] if (t < T - 1 and trunc[n][t] == 0.0) else 0.0) + boot[n][t]
            delta = min(ratio, rho_bar) * (r[n][t] + gamma * nxt * (1.0 - term[n][t]) - v[n][t])
            cut = min(term[n][t] + trunc[n][t], 1.0)
            acc = delta + gamma * min(ratio, c_bar) * (1.0 - cut) * acc
            tg[n][t] = acc + v[n][t]
        for t in range(T):
            ratio = math.exp(lpt[n][t] - lpb[n][t])
            nxt = (tg[n][t + 1] if (t < T - 1 and trunc[n][t] == 0.0) else 0.0) + boot[n][t]
            adv[n][t] = min(ratio, rho_bar) * (r[n][t] + gamma * nxt * (1.0 - term[n][t]) - v[n][t])
    return tg, adv


def brute_retrace(pi, mu, q, nq, act, r, term, trunc, gamma, lam, c_bar, rho_bar):
    """Retrace(lambda) from its definition (tests/test_retrace.py:19-60 states the same):
    E_pi[Q'] = sum over actions of pi * Q';  pi(a_t) = the target probability of the action
    taken;  c = lambda * min(c_bar, pi(a_t)/mu),  rho = min(rho_bar, pi(a_t)/mu);
    Q_ret[t] = q + (r + gamma*E_pi[Q']*(1-term) - q) + gamma*c[t+1]*(1-done)*(Q_ret[t+1] - q[t+1]),
    with c[T] = 0, and adv = rho*(r + gamma*Q_ret[t+1]*(1-term) - q), Q_ret[T] = 0."""
    A = len(pi[0][0])
    tg = [[0.0] * T for _ in range(N)]
    adv = [[0.0] * T for _ in range(N)]
    for n in range(N):
        c = [0.0] * (T + 1)
        rho = [0.0] * T
        enq = [0.0] * T
        for t in range(T):
            enq[t] = sum(pi[n][t][a] * nq[n][t][a] for a in range(A))
            ratio = pi[n][t][act[n][t]] / mu[n][t]
            c[t] = lam * min(c_bar, ratio)
            rho[t] = min(rho_bar, ratio)
        acc = 0.0
        for t in reversed(range(T)):
            cut = min(term[n][t] + trunc[n][t], 1.0)
            acc = (r[n][t] + gamma * enq[t] * (1.0 - term[n][t]) - q[n][t]
                   + gamma * c[t + 1] * (1.0 - cut) * acc)
            tg[n][t] = acc + q[n][t]
        for t in range(T):
            nxt = tg[n][t + 1] if t + 1 < T else 0.0
            adv[n][t] = rho[t] * (r[n][t] + gamma * nxt * (1.0 - term[n][t]) - q[n][t])
    return tg, adv


def brute_lambda(r, nv, term, trunc, boot, gamma, lam):
    out = [[0.0] * T for _ in range(N)]
    for n in range(N):
        g = boot[n][T - 1]
        for t in reversed(range(T)):
            keep = 1.0 - min(term[n][t] + trunc[n][t], 1.0)
            g = (r[n][t] + gamma * keep * ((1.0 - lam) * nv[n][t] + lam * g)
                 + gamma * trunc[n][t] * boot[n][t])
            out[n][t] = g
    return out


def brute_discounted(r, term, trunc, boot, gamma):
    out = [[0.0] * T for _ in range(N)]
    for n in range(N):
        g = boot[n][T - 1]
        for t in reversed(range(T)):
            keep = 1.0 - min(term[n][t] + trunc[n][t], 1.0)
            g = r[n][t] + gamma * keep * g + gamma * trunc[n][t] * boot[n][t]
            out[n][t] = g
    return out


def truncation_fixtures():
    rng = np.random.default_rng(20260805)
    trunc, boot = _layout()
    zeros = [[0.0] * T for _ in range(N)]
    g, lam = 0.99, 0.95
    c = []
    r, v = _rand(rng), _rand(rng)
    c.append(case("gae_two_interior_truncations", "gae", "tests/test_gae.py:457-492 (layout)",
                  {"rewards": r, "values": v, "terminateds": zeros, "truncateds": trunc,
                   "bootstrap_values": boot},
                  {"gamma": g, "lambda_": lam},
                  {"advantages": brute_gae(r, v, zeros, trunc, boot, g, lam)}))
    lpt, lpb = _rand(rng, -1.0, 0.0), _rand(rng, -1.0, 0.0)
    v, r = _rand(rng), _rand(rng)
    tg, adv = brute_vtrace(lpt, lpb, v, r, zeros, trunc, boot, g, 1.0, 1.0)
    c.append(case("vtrace_two_interior_truncations", "vtrace", "tests/test_vtrace.py:487-570 (layout)",
                  {"log_pi_target": lpt, "log_pi_behavior": lpb, "values": v, "rewards": r,
                   "terminateds": zeros, "truncateds": trunc, "bootstrap_values": boot},
                  {"gamma": g, "rho_bar": 1.0, "c_bar": 1.0}, {"targets": tg, "advantages": adv}))
    r, nv = _rand(rng), _rand(rng)
    c.append(case("lambda_returns_two_interior_truncations", "lambda_returns",
                  "tests/test_returns.py:513-549 (layout)",
                  {"rewards": r, "next_values": nv, "terminateds": zeros, "truncateds": trunc,
                   "bootstrap_values": boot},
                  {"gamma": g, "lambda_": lam},
                  {"returns": brute_lambda(r, nv, zeros, trunc, boot, g, lam)}))
    r = _rand(rng)
    c.append(case("discounted_two_interior_truncations", "discounted_returns",
                  "tests/test_returns.py:552-583 (layout)",
                  {"rewards": r, "terminateds": zeros, "truncateds": trunc, "bootstrap_values": boot},
                  {"gamma": g}, {"returns": brute_discounted(r, zeros, trunc, boot, g)}))
    # GAE lambda=1 with an interior truncation is the Monte-Carlo advantage
    # (tests/test_gae.py:377-411): G restarts from the truncation bootstrap.
    r, v = _rand(rng, -1, 1), _rand(rng, -1, 1)
    tr1 = [[1.0 if t == 2 else 0.0 for t in range(T)] for _ in range(N)]
    b1 = [[0.0] * T for _ in range(N)]
    for n in range(N):
        b1[n][2] = _f32(rng.normal())
        b1[n][T - 1] = _f32(rng.normal())
    mc = [[0.0] * T for _ in range(N)]
    for n in range(N):
        gg = b1[n][T - 1]
        for t in reversed(range(T)):
            gg = r[n][t] + 0.95 * (b1[n][t] if t == 2 else gg)
            mc[n][t] = gg - v[n][t]
    c.append(case("gae_lambda1_mc_interior_truncation", "gae", "tests/test_gae.py:377-411 (identity)",
                  {"rewards": r, "values": v, "terminateds": zeros, "truncateds": tr1,
                   "bootstrap_values": b1},
                  {"gamma": 0.95, "lambda_": 1.0}, {"advantages": mc}))
    c.extend(clip_split_fixtures(rng))
    return c


def clip_split_fixtures(rng):
    """V-trace with rho_bar != c_bar, and Retrace with several actions: the clips the
    reference applies separately (kernels/vtrace_fused.py:104-106, ops/retrace.py:178-182)
    and the action reduction and gather over the [E, T, A] layout.  Ratios are spread over
    [e^-1, e] so that many fall between, and beyond, the two clip levels."""
    trunc, boot = _layout()
    zeros = [[0.0] * T for _ in range(N)]
    term = [[0.0] * T for _ in range(N)]
    term[0][9] = term[1][2] = 1.0
    g = 0.99
    c = []
    for rho_bar, c_bar in ((0.8, 0.9), (1.3, 0.6)):
        lpt, lpb = _rand(rng, -1.0, 0.0), _rand(rng, -1.0, 0.0)
        v, r = _rand(rng), _rand(rng, -1.0, 1.0)
        tg, adv = brute_vtrace(lpt, lpb, v, r, term, trunc, boot, g, rho_bar, c_bar)
        c.append(case(f"vtrace_rho{rho_bar}_c{c_bar}_interior_truncations", "vtrace",
                      "kernels/vtrace_fused.py:104-106 (separate clips), tests/test_vtrace.py:487-570 (layout)",
                      {"log_pi_target": lpt, "log_pi_behavior": lpb, "values": v, "rewards": r,
                       "terminateds": term, "truncateds": trunc, "bootstrap_values": boot},
                      {"gamma": g, "rho_bar": rho_bar, "c_bar": c_bar},
                      {"targets": tg, "advantages": adv}))
        # no truncations, last_value only (the window boundary value alone)
        lv = [_f32(x) for x in rng.normal(size=N)]
        boot_last = [[0.0] * (T - 1) + [lv[n]] for n in range(N)]
        tg, adv = brute_vtrace(lpt, lpb, v, r, term, zeros, boot_last, g, rho_bar, c_bar)
        c.append(case(f"vtrace_rho{rho_bar}_c{c_bar}_last_value", "vtrace",
                      "kernels/vtrace_fused.py:104-106 (separate clips)",
                      {"log_pi_target": lpt, "log_pi_behavior": lpb, "values": v, "rewards": r,
                       "terminateds": term, "last_value": lv},
                      {"gamma": g, "rho_bar": rho_bar, "c_bar": c_bar},
                      {"targets": tg, "advantages": adv}))
    for A in (3, 5):
        logits = rng.normal(size=(N, T, A))
        p = np.exp(logits) / np.exp(logits).sum(-1, keepdims=True)
        pi = [[[_f32(x) for x in p[n, t]] for t in range(T)] for n in range(N)]
        nq = [[[_f32(x) for x in rng.normal(size=A)] for _ in range(T)] for _ in range(N)]
        mu = _rand(rng, 0.1, 0.9)
        q, r = _rand(rng, -1.0, 1.0), _rand(rng, -1.0, 1.0)
        act = [[int(a) for a in rng.integers(0, A, size=T)] for _ in range(N)]
        tg, adv = brute_retrace(pi, mu, q, nq, act, r, term, trunc, g, 0.9, 0.9, 0.8)
        c.append(case(f"retrace_A{A}_clipped", "retrace",
                      "ops/retrace.py:178-182 (action reduction, gather), tests/test_retrace.py:19-60",
                      {"action_probs_target": pi, "action_probs_behavior": mu, "q_values": q,
                       "next_q_values_all": nq, "actions": act, "rewards": r, "terminateds": term,
                       "truncateds": trunc},
                      {"gamma": g, "lambda_": 0.9, "c_bar": 0.9, "rho_bar": 0.8},
                      {"targets": tg, "advantages": adv}))
    return c


def main():
    cases = reference_known_answers() + truncation_fixtures()
    for cs in cases:  # normalise ints to floats except Retrace actions
        for k, val in cs["inputs"].items():
            if k != "actions":
                cs["inputs"][k] = np.asarray(val, dtype=np.float64).tolist()
        for k, val in cs["expected"].items():
            cs["expected"][k] = np.asarray(val, dtype=np.float64).tolist()
    with open(OUT, "w") as f:
        json.dump({"generator": "tests/golden/make_known_answers.py", "cases": cases}, f, indent=1)
    print(f"wrote {len(cases)} cases to {OUT}")


if __name__ == "__main__":
    main()
