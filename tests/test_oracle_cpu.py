"""Pins the CPU oracle (oracle/rlk_oracle.c) before it is trusted as the GPU checker.

1. the reference's own known answers and the interior-truncation fixtures
   (tests/golden/known_answers.json);
2. identities the mathematics fixes, independent of any implementation;
3. library routines the recurrences reduce to (cumsum, geometric convolution);
4. brute force of the affine recurrence through its explicit product formula;
5. the float32 torch-loop restatement of the reference loops (oracle/torch_loops.py).
A planted mistake (sign, shift of done by one step, dropped bootstrap) fails at least one
of these -- see test_checks_catch_planted_mistakes.
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
