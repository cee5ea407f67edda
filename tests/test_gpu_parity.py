"""GPU parity: the HIP kernels (through the rl_triton API and its C ABI) against the
float64 CPU oracle and the reference's known answers.

Tolerances (stated per test):
  * known answers: rtol = atol = 1e-5 (the reference's own bar for them);
  * seq_len <= 2048: rtol = atol = 1e-5 against the float64 oracle (discounted returns:
    atol = 1e-5 * max(1, max|expected|), see _check), and no further from it than 2x the
    reference's float32 sequential loop on the same inputs (oracle.loop32, the reference's
    torch loops restated in C) plus 1e-6;
  * long rows (look-back path): atol = 1e-5 * sqrt(L_eff / 128) * max(1, max|ref|), rtol = 1e-5,
    L_eff = 1/(1 - decay) for discounted scans, the longest done-free run for prefix sums,
    and the same 2x-the-float32-loop bound;
  * the BASELINE configurations at full size: all of the above, and also on inputs where
    float32 arithmetic is exact in any order (integer data, unit discounts), where the
    result must equal the oracle bit for bit.
Done/reset indices are exact by construction of the fixtures (known answers, the
all-dones identity and the exact-arithmetic cases).
"""
import math

import numpy as np
import pytest
import torch

import baseline_configs
from _common import OUTPUTS, assert_close, golden_cases, make_inputs, max_abs_err, run_api, run_oracle
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (1, 7), (4, 128), (32, 333), (128, 1024), (256, 2048)]
OPS = ["gae", "vtrace", "retrace", "lambda_returns", "discounted_returns", "eligibility_traces",
       "prefix_sum", "backward_scan", "forward_scan"]


def loop_gate(op, inp, params, got, exp, what, floor=1e-6):
    """The north star's bar: the GPU result is no further from float64 than the reference's
    float32 sequential loop on the same inputs (here within a factor 2, plus `floor` for
    results the loop happens to get exact).  Returns {output: (gpu error, loop error)}."""
    if not orc.has_loop32(op, inp):
        return {}
    loop = orc.loop32(op, inp, params)
    errs = {}
    for name, g, e, lp in zip(OUTPUTS[op], got, exp, loop):
        err, err_loop = max_abs_err(g, e), max_abs_err(lp, e)
        errs[name] = (err, err_loop)
        assert err <= 2.0 * err_loop + floor, (f"{what}:{name}: max abs err {err:.3e} vs float64, "
                                               f"float32 loop {err_loop:.3e}")
    return errs


def _check(op, inp, params, device, rtol, atol, what):
    """rtol and atol as given (1e-5 at rows of up to 2048 steps), except for discounted
    returns and rows longer than 2048 steps, where atol is scaled by max(1, max|expected|):
    an element near zero in a row of large values (undamped discounted returns over 2048
    steps reach ~25) is a difference of large terms, so its float32 rounding error is
    relative to them (e.g. 1.9e-5 at an element of 0.0095 in discounted returns
    [256, 2048]; the reference's own float32 loop reaches 0.75 of the plain tolerance
    there).  The float32-loop gate bounds every result tightly."""
    got = run_api(op, inp, params, device)
    exp = run_oracle(op, inp, params)
    torch.cuda.synchronize()
    got = [g.cpu().numpy() for g in got]
    T = int(np.asarray(got[0]).shape[-1]) if got and np.asarray(got[0]).ndim else 0
    for name, g, e in zip(OUTPUTS[op], got, exp):
        scaled = op == "discounted_returns" or T > 2048
        scale = max(1.0, float(np.max(np.abs(e)))) if (e.size and scaled) else 1.0
        assert_close(g, e, rtol, atol * scale, f"{what}:{name}")
    loop_gate(op, inp, params, got, exp, what)
    return got, exp


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c["name"])
def test_known_answers(case, device):
    got = run_api(case["op"], case["inputs"], case["params"], device)
    names = OUTPUTS[case["op"]]
    for name, g in zip(names, got):
        if name in case["expected"]:
            assert_close(g.cpu().numpy(), case["expected"][name], 1e-5, 1e-5,
                         f"{case['name']}:{name} ({case['source']})")


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_parity_shapes(op, shape, device):
    inp, params = make_inputs(op, *shape, seed=42)
    _check(op, inp, params, device, 1e-5, 1e-5, f"{op}{shape}")


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", [(3, 32), (5, 33), (7, 61), (9, 64), (6, 65), (3, 127), (2, 128),
                                   (4, 129), (3, 256), (2, 257), (8200, 64), (4100, 128),
                                   (2050, 256)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_parity_scan_width_instances(op, shape, device):
    """Row lengths on both sides of each change of short-row kernel instance: up to 32 steps
    the scan width comes from the launch; 33-64, 65-128 and 129-2048 steps run instances
    with the width fixed at compile time (16, 32, 64), aligned (T % 4 == 0) or not, in
    256-thread workgroups (few rows) and 512-thread ones (the larger E, ragged last
    workgroup)."""
    inp, params = make_inputs(op, *shape, seed=77)
    _check(op, inp, params, device, 1e-5, 1e-5, f"{op}{shape}")


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", [(5, 1028), (3, 1500), (40, 2044), (300, 2048), (2, 1027)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_parity_rows_of_1025_to_2048_steps(op, shape, device):
    """Aligned rows of 1025..2048 steps run one row per 256-thread workgroup with two
    wave-strided segments per thread (all ops but V-trace and Retrace), padding segments and
    padding waves included; element-aligned rows (1027 steps) keep one segment per thread."""
    inp, params = make_inputs(op, *shape, seed=91)
    _check(op, inp, params, device, 1e-5, 1e-5, f"{op}{shape}")


def _sweep_cases(n=40, seed=2024):
    """Seeded random (op, E, T, bootstrap, truncation) cases, T up to 2300 so that every
    short-row instance and the first long-row tiles are reached."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        op = OPS[i % len(OPS)]
        T = int(rng.choice([rng.integers(1, 70), rng.integers(70, 600), rng.integers(600, 2300)]))
        E = int(rng.integers(1, 300 if T < 600 else 40))
        boot = str(rng.choice(["none", "row", "full"])) if op in (
            "gae", "vtrace", "lambda_returns", "discounted_returns") else "row"
        if op in ("lambda_returns", "discounted_returns") and boot == "row":
            boot = "full"
        trunc = float(rng.choice([0.0, 0.05])) if op in (
            "gae", "vtrace", "lambda_returns", "discounted_returns") else 0.0
        if op == "gae" and boot == "row":
            trunc = 0.0
        cases.append((op, E, T, boot, trunc, 1000 + i))
    return cases


@pytest.mark.parametrize("case", _sweep_cases(), ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}-{c[3]}-{c[4]}")
def test_parity_random_shapes(case, device):
    """A seeded sweep of random shapes, bootstrap modes and truncation rates for every op."""
    op, E, T, boot, trunc, seed = case
    inp, params = make_inputs(op, E, T, seed=seed, p_trunc=trunc, boot=boot)
    rtol, atol = 1e-5, 1e-5
    if T > 2048:
        atol = 1e-5 * math.sqrt(max(1.0 / (1.0 - 0.99), 128) / 128.0)
        if op == "prefix_sum":
            atol = 1e-5 * math.sqrt(max(float(T), 128) / 128.0)
    _check(op, inp, params, device, rtol, atol, f"{op}[{E},{T}] boot={boot} trunc={trunc}")


def _wide_cases(n=120, seed=77):
    """Seeded cases over every op: rows of 1 to 300000 steps (short, multi-wave and
    look-back paths), tensors placed 0-2 elements off alignment (the element-aligned paths),
    done rates from 1e-4 to 0.3 for the forward scans, and each op's bootstrap and
    truncation modes."""
    ops = ["gae", "gae_masked", "vtrace", "retrace", "lambda_returns", "discounted_returns",
           "eligibility_traces", "prefix_sum", "backward_scan", "forward_scan"]
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        op = ops[i % len(ops)]
        band = int(rng.integers(0, 4))
        T = int([rng.integers(1, 9), rng.integers(9, 129), rng.integers(129, 2049),
                 math.exp(rng.uniform(math.log(2049), math.log(300000)))][band])
        E = int(max(1, min(rng.integers(1, 5000), 1_500_000 // T)))
        returns = op in ("lambda_returns", "discounted_returns")
        boot = str(rng.choice(["none", "row", "full"])) if returns or op in ("gae", "gae_masked", "vtrace") else "row"
        if returns and boot == "row":
            boot = "full"
        trunc = float(rng.choice([0.0, 0.03])) if returns or op in ("gae", "gae_masked", "vtrace") else 0.0
        if op in ("gae", "gae_masked") and boot == "row":
            trunc = 0.0
        p_done = float(rng.choice([1e-4, 1e-2, 0.3]))
        cases.append((op, E, T, boot, trunc, p_done, int(rng.choice([0, 0, 0, 1, 2])), 5000 + i))
    return cases


@pytest.mark.parametrize("case", _wide_cases(), ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}-{c[3]}-{c[4]}-off{c[6]}")
def test_parity_random_lengths_and_offsets(case, device):
    """The seeded wide sweep against the float64 oracle at the suite's tolerances, with the
    absolute tolerance of the undamped prefix sum scaled by max(1, max|expected|) at every
    length, as discounted returns' is (its values grow with the done-free run); the float32
    loop gate holds each result to the reference loop's own error.  Every third case also
    runs in bfloat16, bit-identical to the float32 result rounded."""
    from _common import suite_atol
    from rl_triton import _native
    op, E, T, boot, trunc, p_done, offset, seed = case
    kw = {"p_done": p_done} if op in ("prefix_sum", "eligibility_traces") else {}
    inp, params = make_inputs(op, E, T, seed=seed, p_trunc=trunc, boot=boot, **kw)
    what = f"{op}[{E},{T}] boot={boot} trunc={trunc} offset={offset}"
    got = [g.cpu().numpy() for g in run_api(op, inp, params, device, offset=offset)]
    exp = run_oracle(op, inp, params)
    for name, g, e in zip(OUTPUTS[op], got, exp):
        atol = suite_atol(op, inp, e, T) if e.size else 1e-5
        if T <= 2048 and op in ("discounted_returns", "prefix_sum") and e.size:
            atol = 1e-5 * max(1.0, float(np.max(np.abs(e))))
        assert_close(g, e, 1e-5, atol, f"{what}:{name}")
    loop_gate(op, inp, params, got, exp, what)
    assert not _native.workspace_error(device)
    if seed % 3 == 0:
        rounded = {k: (v if v is None or k == "actions" else
                       torch.as_tensor(v).to(torch.bfloat16).float().numpy()) for k, v in inp.items()}
        got_b = run_api(op, rounded, params, device, dtype=torch.bfloat16, offset=offset)
        ref = run_api(op, rounded, params, device, dtype=torch.float32, offset=offset)
        for g, r in zip(got_b, ref):
            assert torch.equal(g.view(torch.int16), r.to(torch.bfloat16).view(torch.int16)), what


@pytest.mark.parametrize("op", ["gae", "vtrace", "lambda_returns", "discounted_returns"])
@pytest.mark.parametrize("boot", ["none", "row", "full"])
@pytest.mark.parametrize("trunc", [0.0, 0.05])
@pytest.mark.parametrize("shape", [(8, 64), (33, 257), (16, 2048)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_parity_truncation_bootstrap(op, boot, trunc, shape, device):
    if op == "gae" and boot == "row" and trunc > 0:
        pytest.skip("last_value cannot be combined with truncateds (reference contract)")
    if op in ("lambda_returns", "discounted_returns") and boot == "row":
        pytest.skip("the returns API takes bootstrap_values only")
    inp, params = make_inputs(op, *shape, seed=7, p_trunc=trunc, boot=boot)
    _check(op, inp, params, device, 1e-5, 1e-5, f"{op}{shape} boot={boot} trunc={trunc}")


@pytest.mark.parametrize("n_act", [1, 2, 3, 4, 6, 8])
@pytest.mark.parametrize("shape", [(4, 128), (32, 333), (16, 4096)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_retrace_action_counts(n_act, shape, device):
    inp, params = make_inputs("retrace", *shape, seed=3, n_act=n_act, p_trunc=0.02)
    params = dict(params, c_bar=0.9, rho_bar=0.8)
    _check("retrace", inp, params, device, 1e-5, 1e-5, f"retrace A={n_act}{shape}")


@pytest.mark.parametrize("n_act", [1, 2, 3, 4])
@pytest.mark.parametrize("trunc", [0.0, 0.02])
@pytest.mark.parametrize("shape", [(4100, 128), (4097, 100), (8192, 68)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_retrace_paired_rows(n_act, trunc, shape, device):
    """float32 Retrace on aligned rows of 65..128 steps in a grid of at least one 512-thread
    workgroup per compute unit runs two row groups per thread (256-thread workgroups); the
    last workgroup's second group is partly or wholly past the last row."""
    inp, params = make_inputs("retrace", *shape, seed=5, n_act=n_act, p_trunc=trunc)
    params = dict(params, c_bar=0.9, rho_bar=0.8)
    _check("retrace", inp, params, device, 1e-5, 1e-5, f"retrace A={n_act}{shape} trunc={trunc}")


@pytest.mark.parametrize("boundary", ["ends_at", "starts_at"])
@pytest.mark.parametrize("seed_row", [False, True])
@pytest.mark.parametrize("shape", [(64, 512), (5, 3001), (2, 20000)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_prefix_sum_boundaries(boundary, seed_row, shape, device):
    inp, params = make_inputs("prefix_sum", *shape, seed=11, boot="row" if seed_row else "none")
    params = {"boundary": boundary}
    _check("prefix_sum", inp, params, device, 1e-5, 1e-4, f"prefix {boundary}{shape}")


@pytest.mark.parametrize("op", ["eligibility_traces", "prefix_sum", "forward_scan"])
@pytest.mark.parametrize("shape", [(3, 1100), (2, 1537), (5, 2047)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_forward_scans_with_padding_waves(op, shape, device):
    """Rows whose last wave starts beyond seq_len (a padding wave): its neighbour-step read
    stays inside the row, and results match the oracle."""
    inp, params = make_inputs(op, *shape, seed=13, boot="row")
    if op == "prefix_sum":
        params = {"boundary": "ends_at"}
    _check(op, inp, params, device, 1e-5, 1e-5, f"{op}{shape}")


# ---------------------------------------------------------------------------------------
# long rows: the decoupled look-back path
# ---------------------------------------------------------------------------------------
def _longest_run(d):
    best = 0
    for row in np.asarray(d) > 0:
        idx = np.flatnonzero(np.concatenate(([True], row, [True])))
        best = max(best, int(np.max(np.diff(idx))))
    return best


def _long_atol(op, inp, exp, decay=0.99 * 0.95):
    scale = max(1.0, float(np.max(np.abs(exp))))
    if op == "prefix_sum":
        l_eff = _longest_run(inp["dones"])
    elif op in ("discounted_returns",):
        l_eff = 1.0 / (1.0 - 0.99)
    else:
        l_eff = 1.0 / (1.0 - decay)
    return 1e-5 * math.sqrt(max(l_eff, 128) / 128.0) * scale


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", [(3, 2049), (2, 5000), (1, 65536), (2, 131073)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_parity_long_rows(op, shape, device):
    kw = {"p_done": 1e-3} if op in ("prefix_sum", "eligibility_traces") else {}
    inp, params = make_inputs(op, *shape, seed=5, p_trunc=0.01 if op in ("gae", "vtrace") else 0.0,
                              boot="full" if op in ("gae", "vtrace") else "none", **kw)
    got = [g.cpu().numpy() for g in run_api(op, inp, params, device)]
    exp = run_oracle(op, inp, params)
    for name, g, e in zip(OUTPUTS[op], got, exp):
        atol = _long_atol(op, inp, e)
        assert_close(g, e, 1e-5, atol, f"{op}{shape}:{name}")
    loop_gate(op, inp, params, got, exp, f"{op}{shape}")


@pytest.mark.parametrize("name", list(baseline_configs.CONFIGS))
def test_baseline_configs_full_size(name, device):
    """Every BASELINE.json configuration at its full size and distributions, against the
    float64 oracle.  seq_len <= 2048: rtol = atol = 1e-5; longer rows (look-back path): the
    horizon-scaled atol of baseline_configs.horizon_atol.  Everywhere: no further from
    float64 than 2x the reference's float32 sequential loop (+1e-7).  Also asserts that no
    look-back wait gave up."""
    from rl_triton import _native
    op, E, T, _ = baseline_configs.CONFIGS[name]
    inp, params = baseline_configs.make(name, seed=0)
    print(f"[case] {name} [{E},{T}]", flush=True)
    got = baseline_configs.call(name, {k: v.to(device) for k, v in inp.items()}, params)
    np_inp = {k: v.numpy() for k, v in inp.items()}
    exp = run_oracle(op, np_inp, params)
    torch.cuda.synchronize()
    assert not _native.workspace_error(device)
    got = [g.cpu().numpy() for g in got]
    for out_name, g, e in zip(OUTPUTS[op], got, exp):
        atol = 1e-5 if T <= 2048 else baseline_configs.horizon_atol(name, e, inp.get("dones"))
        assert_close(g, e, 1e-5, atol, f"{name}:{out_name}")
    errs = loop_gate(op, np_inp, params, got, exp, name, floor=1e-7)
    for out_name, (err, err_loop) in errs.items():
        print(f"{name}:{out_name} max abs err {err:.3e} vs float64 (float32 loop: {err_loop:.3e})")
    assert set(errs) == set(OUTPUTS[op])


@pytest.mark.parametrize("name", list(baseline_configs.CONFIGS))
def test_baseline_configs_exact_arithmetic(name, device):
    """Every BASELINE configuration at its full shape and done/truncation pattern, on inputs
    where float32 arithmetic is exact in any order (baseline_configs.make_exact: integer
    data, unit discounts, V-trace with rho = 0.5 and c = 1, Retrace with two actions of
    probability 1/4 and 3/4): every output equals the float64 oracle bit for bit.  At these
    sizes that pins every done reset, truncation, bootstrap and tile-to-tile carry exactly,
    which no rounding tolerance can."""
    from rl_triton import _native
    op, E, T, _ = baseline_configs.CONFIGS[name]
    inp, params = baseline_configs.make_exact(name, seed=1)
    print(f"[case] {name} exact [{E},{T}]", flush=True)
    got = baseline_configs.call(name, {k: v.to(device) for k, v in inp.items()}, params)
    exp = run_oracle(op, {k: v.numpy() for k, v in inp.items()}, params)
    torch.cuda.synchronize()
    assert not _native.workspace_error(device)
    for out_name, g, e in zip(OUTPUTS[op], got, exp):
        g = g.cpu().numpy().astype(np.float64)
        bad = int(np.count_nonzero(g != e))
        assert bad == 0, f"{name}:{out_name}: {bad} elements differ, max {np.max(np.abs(g - e))}"


@pytest.mark.parametrize("rho_bar,c_bar", [(0.8, 0.9), (1.3, 0.6)])
@pytest.mark.parametrize("shape,kw", [
    ((4, 128), {}), ((33, 257), {"p_trunc": 0.03, "boot": "full"}),
    ((4096, 128), {"config": "C3_vtrace_4096x128"}), ((3, 5000), {"p_trunc": 0.01, "boot": "full"}),
    ((2, 131073), {}), ((16, 131072), {"config": "C5_vtrace_16x131072"})],
    ids=lambda v: f"{v[0]}x{v[1]}" if isinstance(v, tuple) else (v.get("config") or "-".join(v) or "plain"))
def test_vtrace_separate_clips(rho_bar, c_bar, shape, kw, device):
    """V-trace with rho_bar != c_bar (the reference clips them separately,
    kernels/vtrace_fused.py:104-106): short rows, the C3 and C5 configurations (their
    distributions: log-ratios ~ N(0, 0.5^2), so ratios fall on both sides of both clips)
    and look-back rows, against the float64 oracle and the float32 loop."""
    kw = dict(kw)
    config = kw.pop("config", None)
    if config:
        tin, params = baseline_configs.make(config, seed=3)
        inp = {k: v.numpy() for k, v in tin.items()}
    else:
        inp, params = make_inputs("vtrace", *shape, seed=23, **kw)
        inp.setdefault("last_value", None)
        if "boot" not in kw:
            inp["last_value"] = np.random.default_rng(5).normal(size=shape[0]).astype(np.float32)
    params = dict(params, rho_bar=rho_bar, c_bar=c_bar)
    print(f"[case] vtrace{shape} rho_bar={rho_bar} c_bar={c_bar}", flush=True)
    got = [g.cpu().numpy() for g in run_api("vtrace", inp, params, device)]
    exp = run_oracle("vtrace", inp, params)
    for name, g, e in zip(OUTPUTS["vtrace"], got, exp):
        atol = 1e-5 if shape[1] <= 2048 else _long_atol("vtrace", inp, e)
        assert_close(g, e, 1e-5, atol, f"vtrace{shape} rho_bar={rho_bar} c_bar={c_bar}:{name}")
    loop_gate("vtrace", inp, params, got, exp, f"vtrace{shape}")


def test_lookback_deterministic_and_clean(device):
    """Repeated look-back calls give bit-identical results and no wait ever gives up."""
    from rl_triton import _native
    inp, params = make_inputs("prefix_sum", 4, 300000, seed=9, p_done=1e-4)
    first = run_api("prefix_sum", inp, params, device)[0].cpu()
    for _ in range(3):
        again = run_api("prefix_sum", inp, params, device)[0].cpu()
        assert torch.equal(first, again)
    torch.cuda.synchronize()
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", [(4096, 128), (256, 2048), (16, 131072)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_repeat_runs_bit_identical(op, shape, device):
    """The reference's assert_deterministic (tests/bench_utils.py:308-329): repeated calls on
    the same inputs give the same bits, short rows and look-back rows alike."""
    from rl_triton import _native
    inp, params = make_inputs(op, *shape, seed=5)
    first = [t.clone() for t in run_api(op, inp, params, device)]
    for _ in range(2):
        again = run_api(op, inp, params, device)
        for a, b in zip(first, again):
            assert torch.equal(a, b), f"{op}{shape}: repeat differs"
    assert not _native.workspace_error(device)


# ---------------------------------------------------------------------------------------
# API behaviour on the GPU
# ---------------------------------------------------------------------------------------
def test_non_contiguous_inputs(device):
    import rl_triton
    g = torch.Generator().manual_seed(4)
    base = torch.randn(64, 512, 2, generator=g)
    r = base[..., 0]
    v = torch.randn(64, 512, 2, generator=g)[..., 0]
    d = (torch.rand(64, 512, 2, generator=g) < 0.05).float()[..., 0]
    exp = run_oracle("gae", {"rewards": r.contiguous().numpy(), "values": v.contiguous().numpy(),
                             "terminateds": d.contiguous().numpy()},
                     {"gamma": 0.99, "lambda_": 0.95})[0]
    got = rl_triton.compute_gae(r.to(device), v.to(device), d.to(device))
    assert_close(got.cpu().numpy(), exp, 1e-5, 1e-5, "gae non-contiguous")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("op", ["gae", "vtrace", "retrace", "lambda_returns", "discounted_returns",
                                "eligibility_traces", "prefix_sum", "backward_scan"])
@pytest.mark.parametrize("shape", [(64, 128), (3, 1024), (2, 8192)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_misaligned_inputs(op, shape, dtype, device):
    """Inputs that are contiguous but start one element into their buffer (not 16-byte
    aligned) take the element-wise load path (the 16-byte path needs every array on a
    four-element boundary, rlk_capi.hip quad_aligned).  Its results equal the aligned
    call's bit for bit: both paths fold the same four-step segments in the same order."""
    inp, params = make_inputs(op, *shape, seed=17, p_trunc=0.02 if op in ("gae", "vtrace") else 0.0,
                              boot="full" if op in ("gae", "lambda_returns") else "none")
    ref = run_api(op, inp, params, device, dtype)
    got = run_api(op, inp, params, device, dtype, offset=1)
    torch.cuda.synchronize()
    for name, g, r in zip(OUTPUTS[op], got, ref):
        assert torch.equal(g, r), f"{op}{shape} {dtype}: {name} differs between aligned and offset inputs"
    if dtype is torch.float32:
        exp = run_oracle(op, inp, params)
        for name, g, e in zip(OUTPUTS[op], got, exp):
            scale = max(1.0, float(np.max(np.abs(e))))
            assert_close(g.cpu().numpy(), e, 1e-5, 1e-4 * scale, f"{op}{shape} offset:{name}")


@pytest.mark.parametrize("shape", [(0, 16), (4, 0), (0, 0)])
def test_empty_inputs(shape, device):
    import rl_triton
    z = torch.zeros(shape, device=device)
    assert rl_triton.compute_gae(z, z, z).shape == shape
    t, a = rl_triton.compute_vtrace(z, z, z, z, z)
    assert t.shape == shape and a.shape == shape
    assert rl_triton.compute_episodic_prefix_sum(z, z).shape == shape


def test_all_dones_identity(device):
    import rl_triton
    g = torch.Generator().manual_seed(2)
    x = torch.randn(16, 256, generator=g).to(device)
    ones = torch.ones_like(x)
    for b in ("ends_at", "starts_at"):
        torch.testing.assert_close(rl_triton.compute_episodic_prefix_sum(x, ones, boundary=b), x,
                                   atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(rl_triton.compute_discounted_returns(x, ones, gamma=0.9), x,
                               atol=1e-6, rtol=1e-6)


def test_last_value_equals_bootstrap_column(device):
    """last_value == bootstrap_values[:, -1] (tests/test_gae.py:539-556, test_vtrace.py:619-640)."""
    import rl_triton
    inp, _ = make_inputs("gae", 8, 64, seed=7)
    d = {k: torch.as_tensor(v).to(device) for k, v in inp.items() if v is not None}
    lv = torch.rand(8, generator=torch.Generator().manual_seed(1)).to(device)
    bv = torch.zeros(8, 64, device=device)
    bv[:, -1] = lv
    a = rl_triton.compute_gae(d["rewards"], d["values"], d["terminateds"], last_value=lv)
    b = rl_triton.compute_gae(d["rewards"], d["values"], d["terminateds"], bootstrap_values=bv)
    assert torch.equal(a, b)


def test_last_value_and_bootstrap_values_are_exclusive(device):
    """tests/test_gae.py:526-536, tests/test_vtrace.py:604-616."""
    import rl_triton
    r = torch.rand(4, 16, device=device)
    z = torch.zeros(4, 16, device=device)
    lv = torch.rand(4, device=device)
    with pytest.raises(AssertionError, match="not both"):
        rl_triton.compute_gae(r, r, z, bootstrap_values=z, last_value=lv)
    with pytest.raises(AssertionError, match="not both"):
        rl_triton.compute_vtrace(r, r, r, r, z, bootstrap_values=z, last_value=lv)
    with pytest.raises(AssertionError, match="cannot be combined with truncateds"):
        rl_triton.compute_gae(r, r, z, z, last_value=lv)


def test_vtrace_fused_rejects_long(device):
    from rl_triton.ops.vtrace_fused import compute_vtrace_fused
    z = torch.zeros(1, 131073, device=device)
    with pytest.raises(AssertionError, match="131072"):
        compute_vtrace_fused(z, z, z, z, z)


def test_max_abs_error_report(device):
    """Headline configurations at full size: max abs error vs float64, bounded by 1e-4 and by
    twice the error of the reference's float32 sequential loop on the same inputs."""
    from oracle import torch_loops
    for op, shape, kw in [("gae", (4096, 128), {"p_term": 0.01, "p_trunc": 0.005, "boot": "full"}),
                          ("vtrace", (4096, 128), {"p_term": 0.01, "boot": "row"})]:
        inp, params = make_inputs(op, *shape, seed=0, **kw)
        got = run_api(op, inp, params, device)
        exp = run_oracle(op, inp, params)
        t = {k: torch.from_numpy(v) for k, v in inp.items() if v is not None}
        if op == "gae":
            loop = (torch_loops.gae_loop(t["rewards"], t["values"], t["terminateds"], t["truncateds"],
                                         0.99, 0.95, bootstrap_values=t["bootstrap_values"]),)
        else:
            loop = torch_loops.vtrace_loop(t["log_pi_target"], t["log_pi_behavior"], t["values"],
                                           t["rewards"], t["terminateds"], 0.99, 1.0, 1.0,
                                           last_value=t["last_value"])
        for name, g, e, lp in zip(OUTPUTS[op], got, exp, loop):
            err = max_abs_err(g.cpu().numpy(), e)
            err_loop = max_abs_err(lp.numpy(), e)
            print(f"{op}{shape} {name}: max abs err vs float64 = {err:.3e} "
                  f"(float32 sequential loop: {err_loop:.3e})")
            assert err < 1e-4
            assert err <= 2.0 * err_loop + 1e-7


# ---------------------------------------------------------------------------------------
# the tensor-level fast path (rl_triton._rlk_torch) against the general Python path
# ---------------------------------------------------------------------------------------
FAST_OPS = ["gae", "gae_masked", "gae_normalized", "gae_normalized_masked", "vtrace", "retrace",
            "lambda_returns", "discounted_returns", "eligibility_traces", "prefix_sum",
            "backward_scan", "forward_scan"]


@pytest.mark.parametrize("op", FAST_OPS)
@pytest.mark.parametrize("shape", [(1, 1), (33, 257), (4096, 128), (16, 2048), (3, 5000),
                                   (2, 131073)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_fast_path_matches_python_path(op, shape, device, monkeypatch):
    """With RL_TRITON_CORRECTNESS_WARNINGS unset a well-formed call takes the C++ fast path
    (the public functions are its entries); with it set, the Python path.  Both launch the
    same kernel with the same arguments, so the results are bit-identical -- also for long
    rows, where each path uses a look-back workspace of its own (the look-back gives the
    same bits whatever the timing)."""
    from rl_triton import _native
    assert _native.fast is not None, "rl_triton._rlk_torch is not built"
    boot = ("full" if op in ("gae", "gae_masked", "gae_normalized", "gae_normalized_masked",
                             "vtrace", "lambda_returns", "discounted_returns")
            else "row")
    inp, params = make_inputs(op, *shape, seed=21, p_trunc=0.02 if op != "retrace" else 0.0,
                              boot=boot)
    before = _native.fast.launched()
    slow = run_api(op, inp, params, device)
    assert _native.fast.launched() == before, "the flag should keep calls off the fast path"
    monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
    fast = run_api(op, inp, params, device)
    assert _native.fast.launched() == before + 1, "the call did not take the fast path"
    for s, f in zip(slow, fast):  # bit-identical (nan where both are: one-element batch std)
        torch.testing.assert_close(s, f, rtol=0, atol=0, equal_nan=True)
    assert not _native.workspace_error(device)


def test_public_functions_keep_the_python_contract(device, monkeypatch):
    """The public functions bind arguments like their Python implementations: keywords in any
    order, defaults, and every malformed call (unknown keyword, missing argument, bad
    boundary) raising the Python implementation's error."""
    import inspect

    import rl_triton
    from rl_triton.ops import gae as gae_mod
    monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
    assert inspect.signature(rl_triton.compute_gae) == inspect.signature(gae_mod.compute_gae)
    assert rl_triton.compute_gae.__doc__ == gae_mod.compute_gae.__doc__
    inp, params = make_inputs("gae", 16, 64, seed=3, boot="row")
    r, v, te, lv = (torch.as_tensor(inp[k]).to(device) for k in ("rewards", "values",
                                                                 "terminateds", "last_value"))
    a = rl_triton.compute_gae(r, v, te, None, 0.99, 0.95, None, lv)
    b = rl_triton.compute_gae(r, v, te, last_value=lv, lambda_=0.95, gamma=0.99)
    c = gae_mod.compute_gae(r, v, te, last_value=lv)
    assert torch.equal(a, b) and torch.equal(a, c)
    with pytest.raises(TypeError, match="unexpected keyword"):
        rl_triton.compute_gae(r, v, te, lamda=0.9)
    with pytest.raises(TypeError, match="multiple values"):
        rl_triton.compute_gae(r, v, te, None, gamma=0.9, truncateds=None)
    with pytest.raises(TypeError, match="missing"):
        rl_triton.compute_eligibility_traces(r, te)
    with pytest.raises(ValueError, match="boundary"):
        rl_triton.compute_episodic_prefix_sum(r, te, boundary="middle")
    with pytest.raises(AssertionError, match="not both"):
        rl_triton.compute_gae(r, v, te, bootstrap_values=r, last_value=lv)


def test_fast_path_declines_what_it_cannot_take(device, monkeypatch):
    """Non-contiguous inputs, the correctness flag, and long rows inside a graph capture go
    to the Python path (which gives a captured call a workspace of its own)."""
    from rl_triton import _native
    f = _native.fast
    x = torch.zeros(8, 64, device=device)
    assert f.gae(x, x, x, None, 0.99, 0.95, None, None, None) is None  # flag set by the fixture
    monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
    assert f.gae(x, x, x, None, 0.99, 0.95, None, None, None) is not None
    assert f.gae(x.t(), x.t(), x.t(), None, 0.99, 0.95, None, None, None) is None
    long = torch.zeros(2, 4096, device=device)
    assert f.gae(long, long, long, None, 0.99, 0.95, None, None, None) is not None
    assert f.gae(x, x, x, None, 0.99, 0.95, x, torch.zeros(8, device=device), None) is None
    assert f.gae(x, x, x.double(), None, 0.99, 0.95, None, None, None) is None
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert f.gae(long, long, long, None, 0.99, 0.95, None, None, None) is None
        assert f.gae(x, x, x, None, 0.99, 0.95, None, None, None) is not None
    g.replay()
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------------------
# compute_gae_normalized: GAE + returns + batch-normalised advantages (the reference's
# ROADMAP.md:75-81 item; no reference implementation, so the oracle is the float64 GAE
# oracle composed with the textbook formulas, tests/_common.normalized_from_oracle)
# ---------------------------------------------------------------------------------------
def _check_normalized(inp, params, device, what, long_rows=False):
    got = run_api("gae_normalized", inp, params, device)
    adv_exp, ret_exp = run_oracle("gae_normalized", inp, params)
    torch.cuda.synchronize()
    raw = run_oracle("gae", inp, {k: v for k, v in params.items() if k != "eps"})[0]
    std = float(np.std(raw, ddof=1))
    scale = max(1.0, float(np.max(np.abs(ret_exp))))
    if long_rows:
        base = _long_atol("gae", inp, raw)
    else:
        base = 1e-5 * max(1.0, float(np.max(np.abs(raw))))
    # returns carry A's error; normalised advantages carry it divided by std
    assert_close(got[1].cpu().numpy(), ret_exp, 1e-5, base + 1e-6 * scale, f"{what}:returns")
    assert_close(got[0].cpu().numpy(), adv_exp, 1e-5, base / min(std, 1.0) + 1e-6,
                 f"{what}:advantages")
    return got


@pytest.mark.parametrize("boot", ["none", "row", "full"])
@pytest.mark.parametrize("trunc", [0.0, 0.05])
@pytest.mark.parametrize("shape", [(2, 3), (4, 128), (33, 257), (16, 2048), (3, 5000), (2, 40000),
                                   (64, 40000), (512, 2500)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_gae_normalized_parity(boot, trunc, shape, device):
    if boot == "row" and trunc > 0:
        pytest.skip("last_value cannot be combined with truncateds (reference contract)")
    inp, params = make_inputs("gae_normalized", *shape, seed=17, p_trunc=trunc, boot=boot)
    params = dict(params, eps=1e-8)
    _check_normalized(inp, params, device, f"gae_normalized{shape} boot={boot} trunc={trunc}",
                      long_rows=shape[1] > 2048)


def test_gae_normalized_full_size_and_repeatable(device):
    """BASELINE C2 at full size: against the float64 composition; the advantages come out
    with mean 0 and std 1 (to float32 rounding); repeated calls are bit-identical."""
    import baseline_configs
    inp, params = baseline_configs.make("C2_gae_4096x128", seed=0)
    np_inp = {k: v.numpy() for k, v in inp.items()}
    got = _check_normalized(np_inp, dict(params, eps=1e-8), device, "C2 normalized")
    a = got[0].double()
    assert abs(float(a.mean())) < 1e-6 and abs(float(a.std()) - 1.0) < 1e-5
    again = run_api("gae_normalized", np_inp, dict(params, eps=1e-8), device)
    assert torch.equal(got[0], again[0]) and torch.equal(got[1], again[1])


@pytest.mark.filterwarnings("ignore:std\\(\\):UserWarning")
def test_gae_normalized_single_element_is_nan_like_torch(device):
    """The unbiased std of one element is nan in torch (which warns about it, as expected
    here); so are the normalised advantages."""
    import rl_triton
    x = torch.ones(1, 1, device=device)
    adv, ret = rl_triton.compute_gae_normalized(x, x, torch.zeros_like(x))
    ref = rl_triton.compute_gae(x, x, torch.zeros_like(x))
    assert torch.isnan(adv).all() and torch.isnan((ref - ref.mean()) / (ref.std() + 1e-8)).all()
    torch.testing.assert_close(ret, ref + x)


def _normalized_cases(n=40, seed=91):
    """Seeded compute_gae_normalized calls, masked and not: rows of 1 to 200000 steps (short,
    multi-wave and look-back paths; up to 9000 rows, so from one scan workgroup to several
    thousand partials), each bootstrap mode, with and without truncation."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        band = int(rng.integers(0, 3))
        T = int([rng.integers(1, 129), rng.integers(129, 2049),
                 math.exp(rng.uniform(math.log(2049), math.log(200000)))][band])
        E = int(max(1, min(rng.integers(1, 9000), 1_500_000 // T)))
        boot = str(rng.choice(["none", "row", "full"]))
        trunc = 0.0 if boot == "row" else float(rng.choice([0.0, 0.03]))
        cases.append((("gae_normalized", "gae_normalized_masked")[i % 2], E, T, boot, trunc, 9100 + i))
    return cases


@pytest.mark.parametrize("case", _normalized_cases(), ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}-{c[3]}-{c[4]}")
def test_gae_normalized_random_shapes(case, device):
    """Seeded shapes against the float64 composition (statistics over the kept steps when
    masked).  Every third case also runs in bfloat16: the returns are the float32 result
    rounded, bit for bit; the advantages, normalised from the rounded raw advantages, agree
    with the float32 path's to bfloat16 precision."""
    op, E, T, boot, trunc, seed = case
    inp, params = make_inputs(op, E, T, seed=seed, p_trunc=trunc, boot=boot)
    params = dict(params, eps=1e-8)
    what = f"{op}[{E},{T}] boot={boot} trunc={trunc}"
    print(f"[normalized-random] {what}", flush=True)
    adv, ret = run_api(op, inp, params, device)
    adv_exp, ret_exp = run_oracle(op, inp, params)
    raw_op = "gae_masked" if op == "gae_normalized_masked" else "gae"
    raw = run_oracle(raw_op, inp, {k: v for k, v in params.items() if k != "eps"})[0]
    kept = raw if op == "gae_normalized" else raw[np.asarray(inp["mask"]) != 0]
    base = _long_atol("gae", inp, raw)
    scale = max(1.0, float(np.max(np.abs(ret_exp))))
    assert_close(ret.cpu().numpy(), ret_exp, 1e-5, base + 1e-6 * scale, f"{what}:returns")
    if kept.size >= 2:
        std = float(np.std(kept, ddof=1))
        assert_close(adv.cpu().numpy(), adv_exp, 1e-5, base / min(std, 1.0) + 1e-6,
                     f"{what}:advantages")
    if seed % 3 == 0:
        bf = torch.bfloat16
        rounded = {k: (v if v is None else torch.as_tensor(v).to(bf).float().numpy())
                   for k, v in inp.items()}
        ab, rb = run_api(op, rounded, params, device, dtype=bf)
        af, rf = run_api(op, rounded, params, device, dtype=torch.float32)
        assert torch.equal(rb.view(torch.int16), rf.to(bf).view(torch.int16)), f"{what}: bf16 returns"
        if kept.size >= 2:
            torch.testing.assert_close(ab.float(), af, rtol=2.0 ** -7, atol=2.0 ** -7 * math.sqrt(2),
                                       msg=f"{what}: bf16 advantages")
