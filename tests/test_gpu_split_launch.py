"""Calls larger than one HIP launch.  HIP launches at most 2^32 - 1 work-items per grid
dimension, so a call whose launch would need more (over 4194303 workgroups of up to 1024
threads) runs as calls over consecutive row ranges on the same stream (rlk_capi.hip
launch, rows_per_launch).  The rows repeat a 4096-row pattern k times, so every repetition
must equal the result for the pattern; the split falls inside a repetition.

* Short rows, [4096 * 65537, 3] (4194368 workgroups, split 268434944 + 4608 rows):
  * the episodic prefix sum with per-row seeds, against the float64 oracle on the pattern;
  * the normalised GAE, whose statistics partials continue across the two launches: the
    oracle's raw advantages for the pattern normalised with the call's mean (the
    pattern's) and its std (unbiased over all rows, not the pattern's own).
* Every other op at [4096 * 65537, 3] (split alike), its arrays advanced by whole rows in
  each launch: [E, T], [E, T, A] (Retrace) and per-row ones (bootstrap, seed), against the
  float64 oracle on the pattern.
* Long rows, [4096 * 1025, 2049] in bfloat16 (one 32768-step tile per row, 4198400
  workgroups of 1024 threads, split 4193792 + 4608 rows; T odd, so phased access): the
  episodic prefix sum with seeds, bit-identical in every repetition to the float32
  kernels' result for the pattern rounded (rows at the same element placement), which is
  itself checked against the float64 oracle.
"""
import numpy as np
import pytest
import torch

from _common import OUTPUTS, assert_close, make_inputs, run_oracle, suite_atol

pytestmark = pytest.mark.gpu

P = 4096


@pytest.fixture
def big_memory(device):
    def need(gib):
        free, _ = torch.cuda.mem_get_info(device)
        if free < gib * 2 ** 30:
            pytest.skip(f"needs {gib} GiB of free device memory, {free / 2 ** 30:.0f} GiB free")
    yield need
    torch.cuda.empty_cache()


def _rep(a, k, device, dtype=torch.float32):
    t = torch.as_tensor(a).to(device=device, dtype=dtype)
    return t.repeat(k, 1) if t.dim() == 2 else t.repeat(k)


def _worst(got, exp, k, rtol, atol):
    """Largest excess of |got - exp| over atol + rtol*|exp|, over the k repetitions of exp
    (float64 [P, T] on the device) in got ([k*P, T])."""
    rows = got.view(k, *exp.shape)
    worst = -1.0
    step = max(1, (1 << 26) // exp.numel())
    for c in range(0, k, step):
        d = (rows[c:c + step].double() - exp).abs() - (atol + rtol * exp.abs())
        worst = max(worst, float(d.max()))
    return worst


def test_prefix_sum_short_rows_over_two_launches(device, big_memory):
    import rl_triton
    k, T = 65537, 3
    big_memory(16)
    print(f"[split] prefix_sum [{P * k},{T}]", flush=True)
    pat, params = make_inputs("prefix_sum", P, T, seed=1, boot="row", p_done=0.3)
    exp = torch.as_tensor(run_oracle("prefix_sum", pat, params)[0], dtype=torch.float64,
                          device=device)
    out = rl_triton.compute_episodic_prefix_sum(_rep(pat["inputs"], k, device),
                                                _rep(pat["dones"], k, device),
                                                _rep(pat["seed_values"], k, device))
    torch.cuda.synchronize()
    assert _worst(out, exp, k, 1e-5, 1e-5) <= 0.0


def test_normalized_gae_short_rows_over_two_launches(device, big_memory):
    import rl_triton
    from rl_triton import _native
    k, T = 65537, 3
    E = P * k
    # one partial per workgroup of both launches (4194296 + 72), then the tree's levels
    assert _native.load().rlk_gae_normalized_partials_bytes(E, T) == (4194368 + 2049 + 2) * 24
    big_memory(28)
    print(f"[split] gae_normalized [{E},{T}]", flush=True)
    pat, params = make_inputs("gae_normalized", P, T, seed=2, boot="row", p_term=0.2)
    raw = np.asarray(run_oracle("gae", pat, params)[0], dtype=np.float64)
    mean = raw.mean()
    std = np.sqrt(((raw - mean) ** 2).sum() * k / (E * T - 1))
    adv_exp = torch.as_tensor((raw - mean) / (std + 1e-8), device=device)
    ret_exp = torch.as_tensor(raw + np.asarray(pat["values"], dtype=np.float64), device=device)
    adv, ret = rl_triton.compute_gae_normalized(_rep(pat["rewards"], k, device),
                                                _rep(pat["values"], k, device),
                                                _rep(pat["terminateds"], k, device),
                                                last_value=_rep(pat["last_value"], k, device),
                                                eps=1e-8, **params)
    torch.cuda.synchronize()
    assert _worst(ret, ret_exp, k, 1e-5, 1e-5) <= 0.0
    assert _worst(adv, adv_exp, k, 1e-5, 2e-5) <= 0.0


def test_prefix_sum_long_rows_over_two_launches_bf16(device, big_memory):
    import rl_triton
    k, T = 1025, 2049
    big_memory(64)
    print(f"[split] prefix_sum bf16 [{P * k},{T}]", flush=True)
    pat, params = make_inputs("prefix_sum", P, T, seed=3, boot="row", p_done=1e-3)
    pat = {n: torch.as_tensor(v).to(torch.bfloat16).float().numpy() for n, v in pat.items()
           if v is not None}
    f32 = rl_triton.compute_episodic_prefix_sum(*(torch.as_tensor(pat[n]).to(device)
                                                  for n in ("inputs", "dones", "seed_values")))
    e64 = run_oracle("prefix_sum", pat, params)[0]
    assert_close(f32.cpu().numpy(), e64, 1e-5, suite_atol("prefix_sum", pat, e64, T),
                 "prefix_sum pattern, float32")
    want = f32.to(torch.bfloat16).view(torch.int16)
    del f32
    out = rl_triton.compute_episodic_prefix_sum(
        *(_rep(pat[n], k, device, torch.bfloat16) for n in ("inputs", "dones", "seed_values")))
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    rows = out.view(torch.int16).view(k, P, T)
    for c in range(0, k, 8):
        same = rows[c:c + 8] == want
        assert bool(same.all()), f"repetitions {c}..{c + 7}: {int((~same).sum())} elements differ"


@pytest.mark.parametrize("op", ["gae", "gae_masked", "vtrace", "retrace", "lambda_returns",
                                "discounted_returns", "eligibility_traces", "backward_scan",
                                "forward_scan"])
def test_every_op_short_rows_over_two_launches(op, device, big_memory):
    from test_gpu_graph import _call, _inputs
    k, T = 65537, 3
    pat, params = _inputs(op, (P, T), seed=11)
    exp = run_oracle(op, pat, params)
    per_rep = sum(np.asarray(v).nbytes for v in pat.values() if v is not None)
    per_rep += sum(np.asarray(e, np.float32).nbytes for e in exp)
    big_memory(int(per_rep * k * 1.2 / 2 ** 30) + 4)
    print(f"[split] {op} [{P * k},{T}]", flush=True)
    big = {}
    for name, v in pat.items():
        t = None if v is None else torch.as_tensor(v).to(device)
        big[name] = None if t is None else t.repeat(k, *([1] * (t.dim() - 1)))
    outs = _call(op, big, params)
    torch.cuda.synchronize()
    del big
    base_op = "gae" if op == "gae_masked" else op
    for name, o, e in zip(OUTPUTS[op], outs, exp):
        e64 = torch.as_tensor(np.asarray(e, np.float64), device=device)
        worst = _worst(o, e64, k, 1e-5, suite_atol(base_op, pat, e, T))
        assert worst <= 0.0, f"{op}:{name}: beyond the tolerance by {worst}"
