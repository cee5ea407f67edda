"""bfloat16 I/O (the reference's ROADMAP.md:82-99 item; the reference itself accepts float32
only, so there is no reference output to match).

What pins it:
  * bit identity: every op on bfloat16 tensors returns exactly the float32 op's result on
    the same (widened) inputs, rounded by torch's float -> bfloat16 conversion.  The float32
    path is pinned against the oracle by test_gpu_parity.py, so this carries that parity
    over.  Both launch paths (the C++ fast path and the Python path), short rows, padding
    waves, scalar (seq_len % 4 != 0) and vector loads, and the look-back path are covered.
  * precision drift: against the float64 oracle on the unrounded float32 inputs, the
    bfloat16-I/O error stays within the bound of input and output rounding propagated
    through the recurrence, 2^-8 * (max|expected| + L_eff * max|input|), with L_eff the
    effective horizon (1/(1 - decay); the longest done-free run for the prefix sum).
  * compute_gae_normalized: returns bit-identical as above; normalised advantages within
    one bfloat16 rounding of normalising the rounded advantages (the second launch reads
    the stored bfloat16 advantages, so those values are rounded twice).
"""
import math

import numpy as np
import pytest
import torch

from _common import OUTPUTS, make_inputs, run_api, run_oracle

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
OPS = ["gae", "gae_masked", "vtrace", "retrace", "lambda_returns", "discounted_returns",
       "eligibility_traces", "prefix_sum", "backward_scan", "forward_scan"]
SHAPES = [(1, 1), (1, 7), (5, 64), (9, 61), (6, 127), (33, 257), (4096, 128), (16, 2048), (3, 1100),
          (2, 5001), (3, 5000), (2, 40000)]


def _inputs(op, shape, seed):
    boot = ("full" if op in ("gae", "gae_masked", "vtrace", "lambda_returns", "discounted_returns")
            else "row")
    kw = {"p_done": 1e-3} if op in ("prefix_sum", "eligibility_traces") else {}
    return make_inputs(op, *shape, seed=seed, p_trunc=0.02 if op != "retrace" else 0.0,
                       boot=boot, **kw)


def _bf16_values(inp):
    """The inputs rounded to bfloat16 and widened back (exact), as float32 arrays."""
    out = {}
    for k, v in inp.items():
        if v is None or k == "actions":
            out[k] = v
        else:
            out[k] = torch.as_tensor(v).to(BF16).float().numpy()
    return out


def _bits(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("path", ["python", "fast"])
@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_bf16_is_float32_result_rounded(op, shape, path, device, monkeypatch):
    if path == "fast":
        monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
    inp, params = _inputs(op, shape, seed=31)
    inp = _bf16_values(inp)
    got = run_api(op, inp, params, device, dtype=BF16)
    ref = run_api(op, inp, params, device, dtype=torch.float32)
    for name, g, r in zip(OUTPUTS[op], got, ref):
        assert g.dtype == BF16, f"{op}:{name} returned {g.dtype}"
        want = r.to(BF16)
        same = _bits(g) == _bits(want)
        if not bool(same.all()):
            i = int((~same).flatten().nonzero()[0])
            raise AssertionError(f"{op}{shape}:{name}: {int((~same).sum())} elements differ; "
                                 f"first at flat index {i}: got {g.flatten()[i].item()!r}, "
                                 f"float32 result {r.flatten()[i].item()!r}")


@pytest.mark.parametrize("op", ["discounted_returns", "prefix_sum", "vtrace", "gae"])
@pytest.mark.parametrize("shape", [(6, 128), (3, 61), (2, 5000)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_bf16_rounding_of_non_finite_and_tiny_results(op, shape, device):
    """bfloat16 outputs round as torch's conversion on the GPU does (`Tensor.to`), for
    results that are NaN of either sign (0x7fc0), infinite, float32 denormals or halfway
    cases: NaN, infinities, denormal and halfway-valued inputs are planted in the rows (the
    bfloat16 twins convert on gfx950's v_cvt_pk_bf16_f32 and map NaN to 0x7fc0 afterwards).
    torch's vectorised CPU conversion writes NaN as 0xffff instead, so the CPU is not the
    reference here."""
    inp, params = _inputs(op, shape, seed=5)
    inp = _bf16_values(inp)
    key = {"discounted_returns": "rewards", "prefix_sum": "inputs", "vtrace": "rewards",
           "gae": "rewards"}[op]
    x = np.array(inp[key], dtype=np.float32)
    E, T = x.shape
    rng = np.random.default_rng(9)
    specials = np.array([np.nan, -np.nan, np.inf, -np.inf, 1e-39, -3e-40, 1e-45,
                         np.float32(1.0 + 2.0 ** -8), -np.float32(3.0 * 2.0 ** -9)], dtype=np.float32)
    neg_nan = np.frombuffer(np.uint32(0xFFC00001).tobytes(), dtype=np.float32)[0]
    specials = np.concatenate([specials, [neg_nan]]).astype(np.float32)
    for e in range(E):
        cols = rng.choice(T, size=min(T, len(specials)), replace=False)
        x[e, cols] = specials[:len(cols)]
    inp[key] = torch.as_tensor(x).to(BF16).float().numpy()
    got = run_api(op, inp, params, device, dtype=BF16)
    ref = run_api(op, inp, params, device, dtype=torch.float32)
    for name, g, r in zip(OUTPUTS[op], got, ref):
        want = r.to(BF16)
        same = _bits(g) == _bits(want)
        assert bool(same.all()), (f"{op}{shape}:{name}: {int((~same).sum())} elements differ; first "
                                  f"got {hex(int(_bits(g).flatten()[(~same).flatten()][0]) & 0xffff)} "
                                  f"want {hex(int(_bits(want).flatten()[(~same).flatten()][0]) & 0xffff)}")
        nan_bits = (_bits(g)[torch.isnan(g)].int() & 0xffff).unique().tolist()
        assert nan_bits in ([], [0x7fc0]), f"{op}:{name}: NaN written as {[hex(b) for b in nan_bits]}"
    assert any(bool(torch.isnan(g).any()) for g in got), "no NaN result: the NaN path was not exercised"


def _longest_run(d):
    best = 0
    for row in np.asarray(d) > 0:
        idx = np.flatnonzero(np.concatenate(([True], row, [True])))
        best = max(best, int(np.max(np.diff(idx))))
    return best


def drift_bound(op, inp, exp):
    """2^-8 * (max|expected| + L_eff * max|input|): each input's bfloat16 rounding (relative
    2^-9) reaches an output through weights whose sum is at most L_eff, and the output's own
    rounding adds 2^-9 relative."""
    if op == "prefix_sum":
        l_eff = _longest_run(inp["dones"])
    elif op == "gae_masked":
        # skipped steps do not decay: the horizon in steps grows by the skipped share
        l_eff = 1.0 / (1.0 - 0.99 * 0.95) / max(float(np.mean(inp["mask"])), 1e-3)
    elif op == "discounted_returns":
        l_eff = 1.0 / (1.0 - 0.99)
    elif op in ("backward_scan", "forward_scan"):
        l_eff = 1.0 / (1.0 - 0.99)
    else:
        l_eff = 1.0 / (1.0 - 0.99 * 0.95)
    vin = max(float(np.max(np.abs(v))) for k, v in inp.items()
              if v is not None and k != "actions" and np.size(v))
    return 2.0 ** -8 * (float(np.max(np.abs(exp))) + l_eff * vin)


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", [(64, 128), (16, 2048), (2, 131072)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_bf16_drift_against_float64(op, shape, device):
    inp, params = _inputs(op, shape, seed=7)
    got = run_api(op, inp, params, device, dtype=BF16)
    exp = run_oracle(op, inp, params)
    for name, g, e in zip(OUTPUTS[op], got, exp):
        err = float(np.max(np.abs(g.float().cpu().numpy().astype(np.float64) - e)))
        bound = drift_bound(op, inp, e)
        assert err <= bound, f"{op}{shape}:{name}: max abs err {err:.3e} > bound {bound:.3e}"


@pytest.mark.parametrize("shape", [(2, 3), (33, 257), (4096, 128), (3, 5000), (8193, 300)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_bf16_gae_normalized(shape, device):
    # [8193, 300]: 2049 workgroups' partials, summed by a tree level before the normalisation
    inp, params = make_inputs("gae_normalized", *shape, seed=9, p_trunc=0.02, boot="full")
    inp = _bf16_values(inp)
    params = dict(params, eps=1e-8)
    adv, ret = run_api("gae_normalized", inp, params, device, dtype=BF16)
    a32, r32 = run_api("gae_normalized", inp, params, device, dtype=torch.float32)
    raw = run_api("gae", inp, {k: v for k, v in params.items() if k != "eps"}, device)[0]
    assert adv.dtype == BF16 and ret.dtype == BF16
    assert torch.equal(_bits(ret), _bits(r32.to(BF16)))
    # normalise the rounded advantages with the float32 path's statistics
    a = raw.double()
    mean, std = float(a.mean()), float(a.std())
    want = ((raw.to(BF16).double() - mean) / (std + 1e-8))
    err = (adv.double() - want).abs()
    assert bool((err <= want.abs() * 2.0 ** -8 + 1e-6).all()), f"max err {float(err.max()):.3e}"
    # and the float32 path's normalised advantages to within bfloat16 precision
    torch.testing.assert_close(adv.float(), a32, rtol=2.0 ** -7, atol=2.0 ** -7 * max(1.0, math.sqrt(2)))


def test_bf16_mixed_dtypes_are_rejected(device, monkeypatch):
    """All float tensors of a call share one dtype; a mix raises before any launch, on both
    launch paths (the fast path declines and the Python path raises)."""
    import rl_triton
    x = torch.zeros(4, 8, device=device)
    b = x.to(BF16)
    for flag in ("1", None):
        if flag is None:
            monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
        with pytest.raises(AssertionError, match="expected float32"):
            rl_triton.compute_gae(b, x, x)
        with pytest.raises(AssertionError, match="expected float32"):
            rl_triton.compute_discounted_returns(x, b)
        with pytest.raises(AssertionError, match="expected float32"):
            rl_triton.compute_gae(x.double(), x.double(), x.double())


# ---------------------------------------------------------------------------------------
# Precision drift (the study the reference's ROADMAP.md:82-99 names as the prerequisite of
# bfloat16 support).  Per (op, seq_len), on seeded float32 inputs of 2^20 elements (2^23 at
# a million steps), each error is max |x - exact| / max |exact|, exact = the float64 oracle
# on the float32 inputs:
#   f32 I/O        the float32 kernels;
#   bf16 I/O       the bfloat16 kernels (inputs rounded to bfloat16, outputs bfloat16);
#   quantisation   the float64 oracle on the bfloat16-rounded inputs, its result rounded
#                  to bfloat16: what any bfloat16-I/O implementation loses.
# The bfloat16 kernels must sit at the quantisation floor (float32 accumulation adds
# nothing visible), whatever the length; each case prints its row of the table.
# ---------------------------------------------------------------------------------------
DRIFT_OPS = ["gae", "vtrace", "retrace", "lambda_returns", "discounted_returns",
             "eligibility_traces", "prefix_sum"]
DRIFT_CASES = [(op, T) for op in DRIFT_OPS for T in (128, 2048, 131072)] + \
              [("eligibility_traces", 1 << 20), ("prefix_sum", 1 << 20)]


def _rel(x, exact):
    scale = float(np.max(np.abs(exact))) or 1.0
    return float(np.max(np.abs(np.asarray(x, dtype=np.float64) - exact))) / scale


@pytest.mark.parametrize("op,T", DRIFT_CASES, ids=lambda v: str(v))
def test_bf16_drift_at_the_quantisation_floor(op, T, device):
    E = max(1, (1 << (23 if T == 1 << 20 else 20)) // T)
    kw = {"p_done": 1e-4} if op in ("prefix_sum", "eligibility_traces") else {}
    boot = "full" if op in ("gae", "vtrace", "lambda_returns", "discounted_returns") else "none"
    inp, params = make_inputs(op, E, T, seed=3, p_term=0.01,
                              p_trunc=0.005 if op != "retrace" else 0.0, boot=boot, **kw)
    print(f"[case] bf16 drift {op} [{E},{T}]", flush=True)
    exact = run_oracle(op, inp, params)
    f32 = run_api(op, inp, params, device)
    b16 = run_api(op, inp, params, device, dtype=BF16)
    quant = run_oracle(op, _bf16_values(inp), params)
    for name, e, a, b, q in zip(OUTPUTS[op], exact, f32, b16, quant):
        floor = _rel(torch.as_tensor(np.asarray(q, np.float32)).to(BF16).float().numpy(), e)
        err_b, err_f = _rel(b.float().cpu().numpy(), e), _rel(a.cpu().numpy(), e)
        print(f"| {op} | {name} | {E} x {T} | {err_f:.1e} | {err_b:.1e} | {floor:.1e} | "
              f"{err_b / floor:.2f} | {float(np.max(np.abs(e))):.3g} |")
        assert err_b <= 1.25 * floor + 1e-6, f"{op} T={T} {name}: bf16 {err_b:.2e}, floor {floor:.2e}"
        assert err_f < 1e-5


# bfloat16 long rows at every long-row tile shape (1024 x 8, 512 x 4, 1024 x 2, the
# few-row and many-row placements), with arrays 16-byte aligned and 8 bytes off that: the
# float32 result rounded, bit for bit.
LONG_BF16 = [("prefix_sum", (8, 1048576)), ("eligibility_traces", (8, 1048576)),
          ("discounted_returns", (16, 131072)), ("vtrace", (16, 131072)), ("gae", (16, 131072)),
          ("lambda_returns", (16, 131072)), ("gae_masked", (16, 131072)),
          ("backward_scan", (3, 65536)), ("forward_scan", (3, 65536)), ("gae", (64, 40000)),
          ("vtrace", (200, 10000)), ("prefix_sum", (64, 40000)), ("discounted_returns", (3, 500000))]


@pytest.mark.parametrize("offset", [0, 4], ids=["aligned16", "aligned8"])
@pytest.mark.parametrize("op,shape", LONG_BF16, ids=lambda v: v if isinstance(v, str) else f"{v[0]}x{v[1]}")
def test_bf16_long_rows_are_float32_result_rounded(op, shape, offset, device):
    inp, params = _inputs(op, shape, seed=37)
    inp = _bf16_values(inp)
    got = run_api(op, inp, params, device, dtype=BF16, offset=offset)
    ref = run_api(op, inp, params, device, dtype=torch.float32)
    for name, g, r in zip(OUTPUTS[op], got, ref):
        same = _bits(g) == _bits(r.to(BF16))
        assert bool(same.all()), f"{op}{shape} offset {offset}:{name}: {int((~same).sum())} elements differ"
