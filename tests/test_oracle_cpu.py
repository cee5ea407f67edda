"""Pins the CPU oracle (oracle/rlk_oracle.c) before it is trusted as the GPU checker.

1. the reference's own known answers and the interior-truncation fixtures
   (tests/golden/known_answers.json);
2. identities the mathematics fixes, independent of any implementation;
3. library routines the recurrences reduce to (cumsum, geometric convolution);
4. brute force of the affine recurrence through its explicit product formula;
5. the float32 torch-loop restatement of the reference loops (oracle/torch_loops.py);
6. for V-trace's separate rho/c clips and Retrace's action reduction and gather: IMPALA's
   explicit sum, the uniform on-policy and greedy-target cases of Retrace, and NumPy's
   einsum / take_along_axis over the [E, T, A] layout.
A planted mistake (sign, shift of done by one step, dropped bootstrap; rho/c clips swapped,
a wrong action stride or gather) fails at least one of these -- see
test_checks_catch_planted_mistakes and test_clip_and_action_pins_catch_planted_mistakes.
"""
import numpy as np
import pytest
import torch

from _common import OUTPUTS, assert_close, golden_cases, make_inputs, run_oracle
from oracle import oracle as orc
from oracle import torch_loops


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c["name"])
def test_oracle_known_answers(case):
    got = run_oracle(case["op"], case["inputs"], case["params"])
    for name, g in zip(OUTPUTS[case["op"]], got):
        if name in case["expected"]:
            assert_close(g, case["expected"][name], 1e-6, 1e-6, f"{case['name']}:{name}")


def _rng(seed):
    return np.random.default_rng(seed)


def test_gae_lambda1_is_monte_carlo_advantage():
    """λ=1 ⇒ A = G − V with a nonzero window bootstrap (tests/test_gae.py:339-374)."""
    r = _rng(0)
    E, T, g = 16, 37, 0.97
    rew, val = r.normal(size=(E, T)).astype(np.float32), r.normal(size=(E, T)).astype(np.float32)
    lv = r.normal(size=E).astype(np.float32)
    G = np.zeros((E, T))
    acc = lv.astype(np.float64)
    for t in reversed(range(T)):
        acc = rew[:, t] + g * acc
        G[:, t] = acc
    adv = orc.gae(rew, val, np.zeros((E, T), np.float32), None, g, 1.0, bootstrap=lv)
    assert_close(adv, G - val, 1e-12, 1e-12, "MC identity")


def test_gae_lambda0_is_td_error():
    rew, val, term = (make_inputs("gae", 8, 64, seed=1)[0][k] for k in ("rewards", "values", "terminateds"))
    nv = np.zeros_like(val)
    nv[:, :-1] = val[:, 1:]
    rew64, val64, term64, nv64 = (a.astype(np.float64) for a in (rew, val, term, nv))
    td = rew64 + 0.99 * (1.0 - term64) * nv64 - val64
    assert_close(orc.gae(rew, val, term, None, 0.99, 0.0), td, 1e-12, 1e-12, "λ=0")


def test_vtrace_on_policy_targets_are_returns():
    """ρ = c = 1 ⇒ vs = G (tests/test_vtrace.py:354-387)."""
    r = _rng(3)
    E, T, g = 16, 41, 0.98
    lp = r.normal(size=(E, T)).astype(np.float32)
    val, rew = r.normal(size=(E, T)).astype(np.float32), r.normal(size=(E, T)).astype(np.float32)
    lv = r.normal(size=E).astype(np.float32)
    G = np.zeros((E, T))
    acc = lv.astype(np.float64)
    for t in reversed(range(T)):
        acc = rew[:, t] + g * acc
        G[:, t] = acc
    tg, adv = orc.vtrace(lp, lp, val, rew, np.zeros((E, T), np.float32), None, g, 100.0, 100.0,
                         bootstrap=lv)
    assert_close(tg, G, 1e-11, 1e-11, "vs = G")
    assert_close(adv, G - val, 1e-11, 1e-11, "adv = G - V")


def test_lambda1_returns_equal_discounted_and_lambda0_is_one_step():
    inp, _ = make_inputs("lambda_returns", 32, 200, seed=4, boot="full")
    a = orc.lambda_returns(inp["rewards"], inp["next_values"], inp["terminateds"], None, 0.99, 1.0,
                           bootstrap=inp["bootstrap_values"])
    b = orc.discounted_returns(inp["rewards"], inp["terminateds"], None, 0.99,
                               bootstrap=inp["bootstrap_values"])
    assert_close(a, b, 1e-12, 1e-12, "λ=1")
    z = orc.lambda_returns(inp["rewards"], inp["next_values"], inp["terminateds"], None, 0.99, 0.0)
    r64, te64, nv64 = (inp[k].astype(np.float64) for k in ("rewards", "terminateds", "next_values"))
    one = r64 + 0.99 * (1.0 - te64) * nv64
    assert_close(z, one, 1e-12, 1e-12, "λ=0")


def test_discounted_no_dones_is_geometric_convolution():
    """G = M r with M[t, k] = γ^(k-t) for k >= t: a dense matrix product."""
    r = _rng(5).normal(size=(6, 50)).astype(np.float32)
    g = 0.9
    t = np.arange(50)
    M = np.where(t[None, :] >= t[:, None], g ** (t[None, :] - t[:, None]).astype(np.float64), 0.0)
    assert_close(orc.discounted_returns(r, np.zeros_like(r), None, g), r.astype(np.float64) @ M.T,
                 1e-11, 1e-11, "geometric")


@pytest.mark.parametrize("boundary", ["ends_at", "starts_at"])
def test_prefix_sum_library_cases(boundary):
    x = _rng(6).normal(size=(4, 300)).astype(np.float32)
    zeros, ones = np.zeros_like(x), np.ones_like(x)
    assert_close(orc.episodic_prefix_sum(x, zeros, boundary=boundary),
                 np.cumsum(x.astype(np.float64), axis=1), 1e-10, 1e-10, "cumsum")
    assert_close(orc.episodic_prefix_sum(x, ones, boundary=boundary), x, 0, 0, "all dones")


def test_prefix_sum_segments_against_split_cumsum():
    """ends_at: a reset after every flagged step -- the cumsum of each segment."""
    r = _rng(7)
    x = r.normal(size=(3, 500)).astype(np.float32)
    d = (r.random(size=(3, 500)) < 0.03).astype(np.float32)
    exp = np.zeros(x.shape)
    for n in range(3):
        start = 0
        for t in range(500):
            if d[n, t] or t == 499:
                exp[n, start:t + 1] = np.cumsum(x[n, start:t + 1].astype(np.float64))
                start = t + 1
    assert_close(orc.episodic_prefix_sum(x, d), exp, 1e-10, 1e-10, "segments")
    # starts_at on the same flags shifted one step earlier gives the same result
    d_start = np.zeros_like(d)
    d_start[:, 1:] = d[:, :-1]
    assert_close(orc.episodic_prefix_sum(x, d_start, boundary="starts_at"), exp, 1e-10, 1e-10, "starts_at")


def test_eligibility_traces_unit_decay_is_cumsum():
    x = _rng(8).normal(size=(2, 100)).astype(np.float32)
    assert_close(orc.eligibility_traces(x, np.zeros_like(x), 1.0, 1.0),
                 np.cumsum(x.astype(np.float64), axis=1), 1e-10, 1e-10, "γλ=1")


@pytest.mark.parametrize("direction", ["backward", "forward"])
def test_affine_scan_product_formula(direction):
    """x[t] = Σ_k (Π v) u[k] + (Π v) carry, evaluated term by term (no recurrence)."""
    r = _rng(9)
    E, T = 3, 25
    u = r.normal(size=(E, T)).astype(np.float32)
    v = r.uniform(0, 1, size=(E, T)).astype(np.float32)
    c = r.normal(size=E).astype(np.float32)
    exp = np.zeros((E, T))
    u64, v64 = u.astype(np.float64), v.astype(np.float64)
    for n in range(E):
        for t in range(T):
            ks = range(t, T) if direction == "backward" else range(t, -1, -1)
            s, p = 0.0, 1.0
            for k in ks:
                s += p * u64[n, k]
                p *= v64[n, k]
            exp[n, t] = s + p * c[n]
    got = orc.backward_scan(u, v, c) if direction == "backward" else orc.forward_scan(u, v, c)
    assert_close(got, exp, 1e-12, 1e-12, direction)
    zero = orc.backward_scan(u, np.zeros_like(v)) if direction == "backward" else orc.forward_scan(u, np.zeros_like(v))
    assert_close(zero, u, 0, 0, "decay 0")


def test_retrace_on_policy_single_action_is_n_step_td():
    """A = 1, π = μ = 1, λ = 1: Q_ret[t] = Σ_{k>=t} γ^(k-t) δ_k + q_t with
    δ_k = r_k + γ Q'_k − q_k, the trace cut after the last step (c[T] = 0 ends it)."""
    r = _rng(10)
    E, T, g = 2, 30, 0.9
    q = r.normal(size=(E, T)).astype(np.float32)
    nq = r.normal(size=(E, T, 1)).astype(np.float32)
    rew = r.normal(size=(E, T)).astype(np.float32)
    z = np.zeros((E, T), np.float32)
    tg, _ = orc.retrace(np.ones((E, T, 1), np.float32), np.ones((E, T), np.float32), q, nq,
                        np.zeros((E, T), np.int64), rew, z, z, g, 1.0, 1.0, 1.0)
    delta = rew.astype(np.float64) + g * nq[..., 0].astype(np.float64) - q.astype(np.float64)
    exp = np.zeros((E, T))
    for t in range(T):
        exp[:, t] = sum(g ** (k - t) * delta[:, k] for k in range(t, T)) + q[:, t].astype(np.float64)
    assert_close(tg, exp, 1e-11, 1e-11, "n-step")


def test_torch_loops_match_oracle():
    inp, _ = make_inputs("gae", 256, 128, seed=0, p_term=0.01, p_trunc=0.005, boot="full")
    t = {k: torch.from_numpy(v) for k, v in inp.items() if v is not None}
    got = torch_loops.gae_loop(t["rewards"], t["values"], t["terminateds"], t["truncateds"], 0.99, 0.95,
                               bootstrap_values=t["bootstrap_values"]).numpy()
    exp = orc.gae(inp["rewards"], inp["values"], inp["terminateds"], inp["truncateds"], 0.99, 0.95,
                  bootstrap=inp["bootstrap_values"])
    assert_close(got, exp, 1e-5, 1e-5, "gae loop")
    inp, _ = make_inputs("vtrace", 256, 128, seed=1, p_term=0.01, boot="row")
    t = {k: torch.from_numpy(v) for k, v in inp.items() if v is not None}
    tg, ad = torch_loops.vtrace_loop(t["log_pi_target"], t["log_pi_behavior"], t["values"],
                                     t["rewards"], t["terminateds"], 0.99, 1.0, 1.0,
                                     last_value=t["last_value"])
    etg, ead = orc.vtrace(inp["log_pi_target"], inp["log_pi_behavior"], inp["values"], inp["rewards"],
                          inp["terminateds"], None, 0.99, 1.0, 1.0, bootstrap=inp["last_value"])
    assert_close(tg.numpy(), etg, 1e-5, 1e-5, "vtrace targets loop")
    assert_close(ad.numpy(), ead, 1e-5, 1e-5, "vtrace adv loop")


def test_checks_catch_planted_mistakes():
    """Plausible mistakes planted in a Python copy of the GAE recurrence are caught by the
    known answers used above (so those checks have teeth)."""
    cases = {c["name"]: c for c in golden_cases("gae")}

    def gae_variant(inp, params, mistake):
        r, v, te = (np.asarray(inp[k], np.float64) for k in ("rewards", "values", "terminateds"))
        lv = np.asarray(inp.get("last_value") or np.zeros(r.shape[0]), np.float64)
        g, lam = params["gamma"], params["lambda_"]
        E, T = r.shape
        out = np.zeros((E, T))
        for n in range(E):
            acc = lv[n] if mistake == "carry_seeded_with_bootstrap" else 0.0
            for t in reversed(range(T)):
                nxt = lv[n] if t == T - 1 else v[n, t + 1]
                if mistake == "dropped_bootstrap" and t == T - 1:
                    nxt = 0.0
                gate = te[n, t - 1] if (mistake == "done_shifted" and t > 0) else te[n, t]
                sign = -1.0 if mistake == "sign" else 1.0
                delta = r[n, t] + g * (1 - te[n, t]) * nxt + sign * -v[n, t]
                acc = delta + g * lam * (1 - gate) * acc
                out[n, t] = acc
        return out

    names = ["gae_single_env", "gae_delta", "gae_last_value", "gae_episode_boundary",
             "gae_mixed_termination"]
    for mistake in ("sign", "done_shifted", "dropped_bootstrap", "carry_seeded_with_bootstrap"):
        caught = False
        for nm in names:
            c = cases[nm]
            got = gae_variant(c["inputs"], c["params"], mistake)
            if not np.allclose(got, c["expected"]["advantages"], atol=1e-6):
                caught = True
        assert caught, f"planted mistake {mistake!r} not caught by the known answers"
    for nm in names:  # and the unplanted copy passes them all
        c = cases[nm]
        assert np.allclose(gae_variant(c["inputs"], c["params"], None), c["expected"]["advantages"])


# ---------------------------------------------------------------------------------------
# masked GAE (steps with mask == 0 pass A and the next value through; the reference's
# ROADMAP.md:131-140 item, restating verl's compute_gae_advantage_return).  No reference
# implementation or fixture exists, so it is pinned by what the semantics fix:
#   * every step kept == compute_gae's oracle, bit for bit;
#   * dropping the skipped steps and running plain GAE on what is left gives the kept
#     steps' advantages, and each skipped step carries the next kept step's (0 if none);
#   * a hand-worked example of verl's loop.
# ---------------------------------------------------------------------------------------
def _masked_case(seed, E, T, p_keep, boot, trunc):
    inp, _ = make_inputs("gae", E, T, seed=seed, p_term=0.05, p_trunc=0.05 if trunc else 0.0,
                         boot=boot)
    mask = (_rng(seed + 100).random((E, T)) < p_keep).astype(np.float32)
    bootstrap = inp.get("last_value") if boot == "row" else inp.get("bootstrap_values")
    return inp, mask, bootstrap


@pytest.mark.parametrize("boot", ["none", "row", "full"])
@pytest.mark.parametrize("trunc", [False, True])
def test_masked_gae_all_kept_is_gae(boot, trunc):
    if boot == "row" and trunc:
        pytest.skip("last_value cannot be combined with truncateds")
    inp, _, bootstrap = _masked_case(1, 9, 77, 1.0, boot, trunc)
    ones = np.ones_like(inp["rewards"])
    got = orc.gae_masked(inp["rewards"], inp["values"], inp["terminateds"], ones,
                         inp["truncateds"], 0.99, 0.95, bootstrap=bootstrap)
    ref = orc.gae(inp["rewards"], inp["values"], inp["terminateds"], inp["truncateds"], 0.99,
                  0.95, bootstrap=bootstrap)
    assert np.array_equal(got, ref)


def _compressed_reference(inp, mask, bootstrap, boot, gamma, lam):
    """Plain GAE (the pinned orc.gae) on each row's kept steps only, spread back: a kept
    step gets its compressed advantage, a skipped one the next kept step's (0 if none)."""
    r, v, te = (inp[k] for k in ("rewards", "values", "terminateds"))
    tr = inp["truncateds"]
    E, T = r.shape
    out = np.zeros((E, T))
    for n in range(E):
        keep = np.flatnonzero(mask[n] != 0)
        if keep.size == 0:
            continue
        sub = lambda a: a[n, keep][None, :]  # noqa: E731
        b = None
        if boot == "row":
            b = bootstrap[n:n + 1]
        elif boot == "full":
            # the window boundary value boot(T-1) follows the last kept step, unless that
            # step is truncated and bootstraps from its own column
            b = sub(bootstrap).copy()
            last = keep[-1]
            if tr is None or tr[n, last] != 1.0:
                b[0, -1] = bootstrap[n, T - 1]
        a = orc.gae(sub(r), sub(v), sub(te), None if tr is None else sub(tr), gamma, lam,
                    bootstrap=b)[0]
        nxt = 0.0
        j = keep.size - 1
        for t in range(T - 1, -1, -1):
            if j >= 0 and keep[j] == t:
                nxt = a[j]
                j -= 1
            out[n, t] = nxt
    return out


@pytest.mark.parametrize("boot", ["none", "row", "full"])
@pytest.mark.parametrize("trunc", [False, True])
@pytest.mark.parametrize("p_keep", [0.0, 0.3, 0.8])
def test_masked_gae_equals_gae_on_kept_steps(boot, trunc, p_keep):
    if boot == "row" and trunc:
        pytest.skip("last_value cannot be combined with truncateds")
    inp, mask, bootstrap = _masked_case(2, 7, 61, p_keep, boot, trunc)
    mask[0, :] = 0.0          # a row with nothing kept
    mask[1, -5:] = 0.0        # a skipped tail: the boundary value crosses it
    got = orc.gae_masked(inp["rewards"], inp["values"], inp["terminateds"], mask,
                         inp["truncateds"], 0.97, 0.9, bootstrap=bootstrap)
    ref = _compressed_reference(inp, mask, bootstrap, boot, 0.97, 0.9)
    assert_close(got, ref, 1e-12, 1e-12, f"boot={boot} trunc={trunc} p_keep={p_keep}")


def test_masked_gae_hand_worked():
    """verl's loop by hand, gamma = lambda = 0.5, mask [1, 0, 0, 1, 0], no bootstrap:
    t=4 skipped: A=0, nv=0;  t=3: delta = 2 + 0.5*0 - 0.25 = 1.75, A = 1.75, nv = 0.25;
    t=2, t=1 skipped: A = 1.75;  t=0: delta = 1 + 0.5*0.25 - 0.5 = 0.625,
    A = 0.625 + 0.25*1.75 = 1.0625."""
    r = np.array([[1.0, 7.0, 7.0, 2.0, 7.0]], np.float32)
    v = np.array([[0.5, 9.0, 9.0, 0.25, 9.0]], np.float32)
    mask = np.array([[1.0, 0.0, 0.0, 1.0, 0.0]], np.float32)
    got = orc.gae_masked(r, v, np.zeros_like(r), mask, None, 0.5, 0.5)
    assert np.array_equal(got, [[1.0625, 1.75, 1.75, 1.75, 0.0]])
    # a planted mistake -- the skipped steps' own values as the next value (plain GAE on
    # the unmasked row, then masked) -- misses the hand-worked answer
    plain = orc.gae(r, v, np.zeros_like(r), None, 0.5, 0.5)
    assert not np.allclose(plain[0, 0], 1.0625)


# ---------------------------------------------------------------------------------------
# V-trace with rho_bar != c_bar and Retrace with several actions.  The reference clips rho
# and c separately (kernels/vtrace_fused.py:104-106) and reduces Retrace's [E, T, A] inputs
# by an expectation over actions and a gather of the taken action (ops/retrace.py:178-182).
# Besides the golden fixtures (independent brute-force loops, tests/golden), each is pinned
# by a closed form evaluated term by term, with no recurrence:
#   * V-trace: the explicit sum of Espeholt et al. 2018 (IMPALA), eq. (1):
#       v_s = V(x_s) + sum_{t>=s} (prod_{i=s}^{t-1} gamma_i c_i) rho_t delta_t
#     with gamma_i = gamma*(1 - done_i); c_bar = 0 leaves the one-step target
#     V + rho*delta, rho_bar = 0 leaves V and zero advantages;
#   * Retrace: the on-policy uniform case of tests/test_retrace.py:343-361 (pi = mu = 1/A,
#     lambda = 1: n-step expected-SARSA TD, E_pi[Q'] = the mean over actions), and a greedy
#     (one-hot) target, Watkins' case: pi(a_t) = [a_t == greedy_t], so an off-greedy action
#     cuts the trace and has a zero advantage, and E_pi[Q'] = Q'[t, greedy_t].
# A planted mistake -- rho and c clips swapped, a wrong action stride, a gather of the
# wrong step's action, c[t] in place of c[t+1], SARSA in place of expected SARSA, ... --
# fails at least one of them (test_clip_and_action_pins_catch_planted_mistakes).
# ---------------------------------------------------------------------------------------
def _vtrace_case(seed, rho_bar, c_bar, E=6, T=40):
    r = _rng(seed)
    lpt = r.uniform(-1.0, 0.0, size=(E, T)).astype(np.float32)
    lpb = r.uniform(-1.0, 0.0, size=(E, T)).astype(np.float32)
    val = r.normal(size=(E, T)).astype(np.float32)
    rew = r.normal(size=(E, T)).astype(np.float32)
    term = (r.random((E, T)) < 0.08).astype(np.float32)
    lv = r.normal(size=E).astype(np.float32)
    inp = {"log_pi_target": lpt, "log_pi_behavior": lpb, "values": val, "rewards": rew,
           "terminateds": term, "last_value": lv}
    return inp, {"gamma": 0.97, "rho_bar": rho_bar, "c_bar": c_bar}


def _impala_closed_form(inp, p):
    """V-trace targets and policy-gradient advantages by IMPALA's eq. (1), term by term."""
    lpt, lpb, v, r, te = (inp[k].astype(np.float64) for k in
                          ("log_pi_target", "log_pi_behavior", "values", "rewards", "terminateds"))
    lv = inp["last_value"].astype(np.float64)
    E, T = r.shape
    g = p["gamma"]
    ratio = np.exp(lpt - lpb)
    rho, c = np.minimum(p["rho_bar"], ratio), np.minimum(p["c_bar"], ratio)
    v_next = np.concatenate([v[:, 1:], lv[:, None]], axis=1)
    gam = g * (1.0 - te)
    delta = rho * (r + gam * v_next - v)
    vs = np.zeros((E, T))
    for s in range(T):
        acc, prod = 0.0, np.ones(E)
        for t in range(s, T):
            acc = acc + prod * delta[:, t]
            prod = prod * gam[:, t] * c[:, t]
        vs[:, s] = v[:, s] + acc
    vs_next = np.concatenate([vs[:, 1:], lv[:, None]], axis=1)
    adv = rho * (r + gam * vs_next - v)
    return vs, adv


@pytest.mark.parametrize("rho_bar,c_bar", [(0.8, 0.9), (1.3, 0.6), (2.0, 2.0)])
def test_vtrace_separate_clips_explicit_sum(rho_bar, c_bar):
    inp, p = _vtrace_case(20, rho_bar, c_bar)
    tg, adv = run_oracle("vtrace", inp, p)
    etg, eadv = _impala_closed_form(inp, p)
    assert_close(tg, etg, 1e-12, 1e-12, "vs")
    assert_close(adv, eadv, 1e-12, 1e-12, "adv")


def test_vtrace_zero_clips():
    """c_bar = 0: no trace, vs = V + rho*delta; rho_bar = 0: vs = V, advantages 0."""
    inp, p = _vtrace_case(21, 0.8, 0.0)
    tg, adv = run_oracle("vtrace", inp, p)
    lpt, lpb, v, r, te = (inp[k].astype(np.float64) for k in
                          ("log_pi_target", "log_pi_behavior", "values", "rewards", "terminateds"))
    v_next = np.concatenate([v[:, 1:], inp["last_value"].astype(np.float64)[:, None]], axis=1)
    rho = np.minimum(0.8, np.exp(lpt - lpb))
    assert_close(tg, v + rho * (r + 0.97 * (1 - te) * v_next - v), 1e-12, 1e-12, "c_bar=0")
    tg, adv = run_oracle("vtrace", inp, dict(p, rho_bar=0.0, c_bar=1.0))
    assert_close(tg, v, 0, 0, "rho_bar=0 targets")
    assert np.array_equal(adv, np.zeros_like(adv))


def _retrace_uniform_case(seed, A=4, E=5, T=33):
    """tests/test_retrace.py:343-361: pi = mu = 1/A, lambda = 1, clips far above 1."""
    r = _rng(seed)
    inp = {"action_probs_target": np.full((E, T, A), 1.0 / A, np.float32),
           "action_probs_behavior": np.full((E, T), 1.0 / A, np.float32),
           "q_values": r.normal(size=(E, T)).astype(np.float32),
           "next_q_values_all": r.normal(size=(E, T, A)).astype(np.float32),
           "actions": r.integers(0, A, size=(E, T)).astype(np.int64),
           "rewards": r.normal(size=(E, T)).astype(np.float32),
           "terminateds": np.zeros((E, T), np.float32),
           "truncateds": np.zeros((E, T), np.float32)}
    return inp, {"gamma": 0.99, "lambda_": 1.0, "c_bar": 1e6, "rho_bar": 1e6}


def _retrace_uniform_expected(inp, p):
    q, r = inp["q_values"].astype(np.float64), inp["rewards"].astype(np.float64)
    mean_q = inp["next_q_values_all"].astype(np.float64).mean(axis=-1)
    g = p["gamma"]
    delta = r + g * mean_q - q
    E, T = q.shape
    tg = np.zeros((E, T))
    for t in range(T):
        tg[:, t] = q[:, t] + sum(g ** (k - t) * delta[:, k] for k in range(t, T))
    nxt = np.concatenate([tg[:, 1:], np.zeros((E, 1))], axis=1)
    return tg, r + g * nxt - q


def _retrace_greedy_case(seed, A=3, E=5, T=37):
    r = _rng(seed)
    greedy = r.integers(0, A, size=(E, T))
    pi = np.zeros((E, T, A), np.float32)
    np.put_along_axis(pi, greedy[..., None], 1.0, axis=-1)
    term = (r.random((E, T)) < 0.06).astype(np.float32)
    trunc = ((r.random((E, T)) < 0.06) * (1 - term)).astype(np.float32)
    inp = {"action_probs_target": pi,
           "action_probs_behavior": r.uniform(0.2, 1.0, size=(E, T)).astype(np.float32),
           "q_values": r.normal(size=(E, T)).astype(np.float32),
           "next_q_values_all": r.normal(size=(E, T, A)).astype(np.float32),
           # the behaviour picks the greedy action about two times in three
           "actions": np.where(r.random((E, T)) < 0.67, greedy,
                               r.integers(0, A, size=(E, T))).astype(np.int64),
           "rewards": r.normal(size=(E, T)).astype(np.float32),
           "terminateds": term, "truncateds": trunc}
    return inp, {"gamma": 0.95, "lambda_": 0.9, "c_bar": 2.0, "rho_bar": 1.2}, greedy


def _retrace_greedy_expected(inp, p, greedy):
    """Watkins' case: D[t] = sum_{k>=t} (prod_{i=t}^{k-1} gamma*c[i+1]*(1-done_i)) delta_k,
    delta_k = r + gamma*Q'[k, greedy_k]*(1-term) - q, c = lambda*min(c_bar, [a == greedy]/mu)."""
    q, r, mu, te, tr = (inp[k].astype(np.float64) for k in
                        ("q_values", "rewards", "action_probs_behavior", "terminateds", "truncateds"))
    nq = inp["next_q_values_all"].astype(np.float64)
    on = (inp["actions"] == greedy).astype(np.float64)
    g, lam = p["gamma"], p["lambda_"]
    E, T = q.shape
    qg = np.take_along_axis(nq, greedy[..., None], axis=-1)[..., 0]
    delta = r + g * qg * (1.0 - te) - q
    c = lam * np.minimum(p["c_bar"], on / mu)
    keep = 1.0 - np.minimum(te + tr, 1.0)
    tg = np.zeros((E, T))
    for t in range(T):
        acc, prod = 0.0, np.ones(E)
        for k in range(t, T):
            acc = acc + prod * delta[:, k]
            prod = prod * (g * c[:, k + 1] * keep[:, k] if k + 1 < T else 0.0)
        tg[:, t] = q[:, t] + acc
    nxt = np.concatenate([tg[:, 1:], np.zeros((E, 1))], axis=1)
    adv = on * np.minimum(p["rho_bar"], 1.0 / mu) * (r + g * nxt * (1.0 - te) - q)
    return tg, adv


def test_retrace_uniform_on_policy_is_expected_sarsa_td():
    inp, p = _retrace_uniform_case(30)
    tg, adv = run_oracle("retrace", inp, p)
    etg, eadv = _retrace_uniform_expected(inp, p)
    assert_close(tg, etg, 1e-11, 1e-11, "targets")
    assert_close(adv, eadv, 1e-11, 1e-11, "advantages")


def test_retrace_greedy_target_cuts_traces():
    inp, p, greedy = _retrace_greedy_case(31)
    tg, adv = run_oracle("retrace", inp, p)
    etg, eadv = _retrace_greedy_expected(inp, p, greedy)
    assert_close(tg, etg, 1e-12, 1e-12, "targets")
    assert_close(adv, eadv, 1e-12, 1e-12, "advantages")
    off = inp["actions"] != greedy
    assert off.any() and np.array_equal(adv[off], np.zeros(int(off.sum())))


@pytest.mark.parametrize("A", [2, 4, 7])
def test_retrace_matches_numpy_reduction_and_gather(A):
    """E_pi[Q'] by einsum and pi(a_t) by take_along_axis -- NumPy's own reduction and gather
    over the [E, T, A] layout -- fed through a float64 backward scan, at clipped ratios."""
    inp, p = make_inputs("retrace", 7, 45, seed=32, n_act=A, p_trunc=0.05)
    p = dict(p, c_bar=0.9, rho_bar=0.8)
    tg, adv = run_oracle("retrace", inp, p)
    pi, nq = inp["action_probs_target"].astype(np.float64), inp["next_q_values_all"].astype(np.float64)
    mu, q, r, te, tr = (inp[k].astype(np.float64) for k in
                        ("action_probs_behavior", "q_values", "rewards", "terminateds", "truncateds"))
    enq = np.einsum("eta,eta->et", pi, nq)
    pa = np.take_along_axis(pi, inp["actions"][..., None], axis=-1)[..., 0]
    c = p["lambda_"] * np.minimum(p["c_bar"], pa / mu)
    rho = np.minimum(p["rho_bar"], pa / mu)
    u = r + p["gamma"] * enq * (1.0 - te) - q
    c_next = np.concatenate([c[:, 1:], np.zeros((c.shape[0], 1))], axis=1)
    v = p["gamma"] * c_next * (1.0 - np.minimum(te + tr, 1.0))
    d = np.zeros_like(u)
    acc = np.zeros(u.shape[0])
    for t in range(u.shape[1] - 1, -1, -1):
        acc = u[:, t] + v[:, t] * acc
        d[:, t] = acc
    etg = d + q
    nxt = np.concatenate([etg[:, 1:], np.zeros((q.shape[0], 1))], axis=1)
    assert_close(tg, etg, 1e-12, 1e-12, "targets")
    assert_close(adv, rho * (r + p["gamma"] * nxt * (1.0 - te) - q), 1e-12, 1e-12, "advantages")


def _vtrace_variant(inp, p, mistake=None):
    """A float64 copy of the V-trace recurrence in which a mistake can be planted."""
    lpt, lpb, v, r, te = (np.asarray(inp[k], np.float64) for k in
                          ("log_pi_target", "log_pi_behavior", "values", "rewards", "terminateds"))
    E, T = r.shape
    tr = np.asarray(inp["truncateds"], np.float64) if inp.get("truncateds") is not None else np.zeros((E, T))
    if inp.get("bootstrap_values") is not None:
        boot = np.asarray(inp["bootstrap_values"], np.float64)
    else:
        boot = np.zeros((E, T))
        if inp.get("last_value") is not None:
            boot[:, -1] = np.asarray(inp["last_value"], np.float64)
    g = p["gamma"]
    ratio = np.exp(lpt - lpb)
    rb, cb = (p["c_bar"], p["rho_bar"]) if mistake == "clip_swap" else (p["rho_bar"], p["c_bar"])
    rho, c = np.minimum(rb, ratio), np.minimum(cb, ratio)
    if mistake == "c_shifted":
        c = np.concatenate([c[:, 1:], np.zeros((E, 1))], axis=1)
    if mistake == "rho_missing":
        rho_d = np.ones_like(rho)
    else:
        rho_d = rho
    done = np.minimum(te + tr, 1.0)

    def nxt_of(x):
        raw = np.concatenate([x[:, 1:], np.zeros((E, 1))], axis=1)
        return np.where(tr == 0.0, raw, 0.0) + boot

    delta = rho_d * (r + g * nxt_of(v) * (1.0 - te) - v)
    d = np.zeros((E, T))
    acc = np.zeros(E)
    for t in range(T - 1, -1, -1):
        acc = delta[:, t] + g * c[:, t] * (1.0 - done[:, t]) * acc
        d[:, t] = acc
    vs = d + v
    nv = nxt_of(v) if mistake == "adv_uses_values" else nxt_of(vs)
    return vs, rho * (r + g * nv * (1.0 - te) - v)


def _retrace_variant(inp, p, mistake=None):
    """A float64 copy of the Retrace recurrence in which a mistake can be planted."""
    pi, nq = (np.asarray(inp[k], np.float64) for k in ("action_probs_target", "next_q_values_all"))
    mu, q, r, te, tr = (np.asarray(inp[k], np.float64) for k in
                        ("action_probs_behavior", "q_values", "rewards", "terminateds", "truncateds"))
    act = np.asarray(inp["actions"], np.int64)
    E, T, A = pi.shape
    g, lam = p["gamma"], p.get("lambda_", 1.0)
    c_bar, rho_bar = p.get("c_bar", 1.0), p.get("rho_bar", 1.0)
    if mistake == "action_stride":  # the flat buffer read as [E, A, T]
        pi = pi.reshape(E, A, T).transpose(0, 2, 1)
        nq = nq.reshape(E, A, T).transpose(0, 2, 1)
    if mistake == "next_step_action":
        act = np.concatenate([act[:, 1:], act[:, -1:]], axis=1)
    enq = (pi * nq).sum(-1)
    if mistake == "sarsa":
        enq = np.take_along_axis(nq, act[..., None], axis=-1)[..., 0]
    pa = np.take_along_axis(pi, act[..., None], axis=-1)[..., 0]
    if mistake == "clip_swap":
        c_bar, rho_bar = rho_bar, c_bar
    c = lam * np.minimum(c_bar, pa / mu)
    rho = np.minimum(rho_bar, pa / mu) * (lam if mistake == "lambda_on_rho" else 1.0)
    c_next = c if mistake == "c_unshifted" else np.concatenate([c[:, 1:], np.zeros((E, 1))], axis=1)
    done = np.minimum(te + tr, 1.0)
    u = r + g * enq * (1.0 - te) - q
    d = np.zeros((E, T))
    acc = np.zeros(E)
    for t in range(T - 1, -1, -1):
        acc = u[:, t] + g * c_next[:, t] * (1.0 - done[:, t]) * acc
        d[:, t] = acc
    tg = d + q
    nxt = np.concatenate([tg[:, 1:], np.zeros((E, 1))], axis=1)
    return tg, rho * (r + g * nxt * (1.0 - te) - q)


def _clip_and_action_pins():
    """(op, inputs, params, expected outputs) of every pin above, golden fixtures included."""
    pins = []
    for c in golden_cases("vtrace") + golden_cases("retrace"):
        exp = tuple(np.asarray(c["expected"].get(n), np.float64) if n in c["expected"] else None
                    for n in OUTPUTS[c["op"]])
        inp = {k: (np.asarray(v, np.int64) if k == "actions" else np.asarray(v, np.float32))
               for k, v in c["inputs"].items()}
        pins.append((c["op"], inp, c["params"], exp))
    for rb, cb in [(0.8, 0.9), (1.3, 0.6)]:
        inp, p = _vtrace_case(20, rb, cb)
        pins.append(("vtrace", inp, p, _impala_closed_form(inp, p)))
    inp, p = _retrace_uniform_case(30)
    pins.append(("retrace", inp, p, _retrace_uniform_expected(inp, p)))
    inp, p, greedy = _retrace_greedy_case(31)
    pins.append(("retrace", inp, p, _retrace_greedy_expected(inp, p, greedy)))
    return pins


def _fails_a_pin(op, impl, pins):
    for pop, inp, p, exp in pins:
        if pop != op:
            continue
        for got, want in zip(impl(inp, p), exp):
            if want is not None and not np.allclose(got, want, rtol=1e-6, atol=1e-6):
                return True
    return False


def test_clip_and_action_pins_catch_planted_mistakes():
    pins = _clip_and_action_pins()
    assert not _fails_a_pin("vtrace", _vtrace_variant, pins)   # the unplanted copies pass
    assert not _fails_a_pin("retrace", _retrace_variant, pins)
    for mistake in ("clip_swap", "c_shifted", "rho_missing", "adv_uses_values"):
        assert _fails_a_pin("vtrace", lambda i, p, m=mistake: _vtrace_variant(i, p, m), pins), mistake
    for mistake in ("action_stride", "next_step_action", "sarsa", "clip_swap", "lambda_on_rho",
                    "c_unshifted"):
        assert _fails_a_pin("retrace", lambda i, p, m=mistake: _retrace_variant(i, p, m), pins), mistake
    # and the clip swap is caught by the rho_bar != c_bar pins alone, the action stride by
    # the multi-action ones alone: the single-action, equal-clip pins would miss both
    is_split = lambda x: x[0] == "vtrace" and x[2]["rho_bar"] != x[2]["c_bar"]  # noqa: E731
    is_multi = lambda x: x[0] == "retrace" and x[1]["action_probs_target"].shape[-1] > 1  # noqa: E731
    split = [x for x in pins if is_split(x)]
    multi = [x for x in pins if is_multi(x)]
    same = [x for x in pins if not is_split(x) and not is_multi(x)]
    assert _fails_a_pin("vtrace", lambda i, p: _vtrace_variant(i, p, "clip_swap"), split)
    assert not _fails_a_pin("vtrace", lambda i, p: _vtrace_variant(i, p, "clip_swap"), same)
    assert _fails_a_pin("retrace", lambda i, p: _retrace_variant(i, p, "action_stride"), multi)
    assert not _fails_a_pin("retrace", lambda i, p: _retrace_variant(i, p, "action_stride"), same)


# ---------------------------------------------------------------------------------------
# the reference's float32 loops: the C restatement (oracle.loop32, fast enough for the
# full-size configurations) equals the torch restatement (oracle/torch_loops.py) bit for
# bit -- same operations, same order, same float32 roundings -- except through exp
# (V-trace: the C library's expf against torch's, which may differ in the last place)
# ---------------------------------------------------------------------------------------
def _torch_loop(op, inp, params):
    t = {k: torch.from_numpy(np.asarray(v)) for k, v in inp.items() if v is not None}
    g = t.get
    if op == "gae":
        return (torch_loops.gae_loop(g("rewards"), g("values"), g("terminateds"), g("truncateds"),
                                     params["gamma"], params["lambda_"],
                                     bootstrap_values=g("bootstrap_values"),
                                     last_value=g("last_value")),)
    if op == "vtrace":
        return torch_loops.vtrace_loop(g("log_pi_target"), g("log_pi_behavior"), g("values"),
                                       g("rewards"), g("terminateds"), params["gamma"],
                                       params["rho_bar"], params["c_bar"], last_value=g("last_value"))
    if op == "retrace":
        return torch_loops.retrace_loop(g("action_probs_target"), g("action_probs_behavior"),
                                        g("q_values"), g("next_q_values_all"), g("actions"),
                                        g("rewards"), g("terminateds"), g("truncateds"), **params)
    if op == "lambda_returns":
        return (torch_loops.lambda_returns_loop(g("rewards"), g("next_values"), g("terminateds"),
                                                g("truncateds"), params["gamma"], params["lambda_"],
                                                bootstrap_values=g("bootstrap_values")),)
    if op == "discounted_returns":
        return (torch_loops.discounted_returns_loop(g("rewards"), g("terminateds"), g("truncateds"),
                                                    params["gamma"],
                                                    bootstrap_values=g("bootstrap_values")),)
    if op == "eligibility_traces":
        return (torch_loops.eligibility_traces_loop(g("gradients"), g("dones"), params["gamma"],
                                                    params["lambda_"], g("seed_values")),)
    if op == "prefix_sum":
        return (torch_loops.prefix_sum_loop(g("inputs"), g("dones"), g("seed_values"),
                                            params.get("boundary", "ends_at")),)
    raise KeyError(op)


LOOP_CASES = [
    ("gae", dict(p_term=0.05, boot="row")), ("gae", dict(p_term=0.05, p_trunc=0.05, boot="full")),
    ("vtrace", dict(p_term=0.05, boot="row")), ("retrace", dict(n_act=2)),
    ("retrace", dict(n_act=3, p_trunc=0.05)),
    ("lambda_returns", dict(boot="full")), ("lambda_returns", dict(p_trunc=0.05, boot="full")),
    ("discounted_returns", dict()), ("discounted_returns", dict(p_trunc=0.05, boot="full")),
    ("eligibility_traces", dict(boot="row")), ("prefix_sum", dict(boot="row")),
]


@pytest.mark.parametrize("op,kw", LOOP_CASES, ids=lambda v: v if isinstance(v, str) else
                         "-".join(f"{k}{w}" for k, w in v.items()))
def test_float32_loops_c_equals_torch(op, kw):
    inp, params = make_inputs(op, 16, 300, seed=60, **kw)
    if op == "vtrace":
        params = dict(params, rho_bar=0.8, c_bar=0.9)
    if op == "retrace":
        params = dict(params, c_bar=0.9, rho_bar=0.8)
    want = _torch_loop(op, inp, params)
    got = orc.loop32(op, inp, params)
    for g, w in zip(got, want):
        assert g.dtype == np.float32
        if op == "vtrace":
            np.testing.assert_allclose(g, w.numpy(), rtol=2e-6, atol=2e-6)
        else:
            assert np.array_equal(g, w.numpy()), f"{op}: {np.max(np.abs(g - w.numpy()))}"
    if op == "prefix_sum":
        p2 = {"boundary": "starts_at"}
        assert np.array_equal(orc.loop32(op, inp, p2)[0], _torch_loop(op, inp, p2)[0].numpy())


# ---------------------------------------------------------------------------------------
# the float32 loops themselves, pinned: against the reference's known answers (every golden
# case whose call the reference's float32 loop takes) and against the float64 oracle on a
# seeded medium shape.  A mistake shared by the C and torch restatements (which the test
# above cannot see) fails here, so a gate of "no further from float64 than the float32
# loop" cannot pass for want of a correct loop.
# ---------------------------------------------------------------------------------------
def _loop32_takes(case):
    """The reference's float32 V-trace loop takes last_value only (no truncations and no
    per-step bootstrap values); every other golden case has a float32 loop."""
    inp = case["inputs"]
    if case["op"] == "vtrace":
        return inp.get("truncateds") is None and inp.get("bootstrap_values") is None
    return True


def _golden_arrays(case):
    inp = {}
    for k, v in case["inputs"].items():
        if v is None:
            inp[k] = None
        elif k == "actions":
            inp[k] = np.asarray(v, dtype=np.int64)
        else:
            inp[k] = np.asarray(v, dtype=np.float32)
    return inp


LOOP_GOLDEN = [c for c in golden_cases() if _loop32_takes(c)]


def test_float32_loops_cover_every_op():
    ops = {c["op"] for c in LOOP_GOLDEN}
    assert ops == {"gae", "vtrace", "retrace", "lambda_returns", "discounted_returns",
                   "eligibility_traces", "prefix_sum"}, ops


@pytest.mark.parametrize("case", LOOP_GOLDEN, ids=lambda c: c["name"])
def test_float32_loops_known_answers(case):
    """Both float32 restatements of the reference's loops give the reference's own known
    answers (float32 arithmetic: rtol = atol = 1e-5)."""
    inp = _golden_arrays(case)
    params = dict(case["params"])
    c_out = orc.loop32(case["op"], inp, params)
    t_out = _torch_loop(case["op"], inp, params)
    for name, c, t in zip(OUTPUTS[case["op"]], c_out, t_out):
        if name not in case["expected"]:
            continue
        want = np.asarray(case["expected"][name], dtype=np.float64)
        assert_close(c, want, 1e-5, 1e-5, f"{case['name']}:{name} (C float32 loop)")
        assert_close(t.numpy(), want, 1e-5, 1e-5, f"{case['name']}:{name} (torch float32 loop)")


LOOP_F64_CASES = LOOP_CASES + [
    ("retrace", dict(n_act=4, p_term=0.02)), ("eligibility_traces", dict()),
    ("prefix_sum", dict(p_done=0.01)),
]


@pytest.mark.parametrize("op,kw", LOOP_F64_CASES, ids=lambda v: v if isinstance(v, str) else
                         "-".join(f"{k}{w}" for k, w in v.items()))
def test_float32_loops_near_float64(op, kw):
    """Each float32 loop against the float64 oracle on a seeded [32, 512] case, at float32
    tolerance: 1e-5 of the output scale (the magnitude of a discounted sum grows with the
    horizon; a prefix sum's with the episode length)."""
    inp, params = make_inputs(op, 32, 512, seed=61, **kw)
    if op == "vtrace":
        params = dict(params, rho_bar=0.8, c_bar=0.9)
    if op == "retrace":
        params = dict(params, c_bar=0.9, rho_bar=0.8)
    want = run_oracle(op, inp, params)
    got = orc.loop32(op, inp, params)
    for name, g, w in zip(OUTPUTS[op], got, want):
        scale = max(1.0, float(np.max(np.abs(w))))
        err = float(np.max(np.abs(g.astype(np.float64) - w)))
        assert err <= 1e-5 * scale, f"{op}:{name}: max abs err {err} (scale {scale})"
