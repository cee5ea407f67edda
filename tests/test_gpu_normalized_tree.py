"""compute_gae_normalized when its first launch has more workgroups than the normalising
kernel reads partials from directly (2048): the per-workgroup (count, sum, sum of squares)
triples are first summed by one or more tree levels of 2048 triples each
(rlk_capi.hip normalized_launch, rlk_engine.hpp reduce_partials_kernel).

* Against the float64 oracle at the boundary: [8192, 300] has 2048 workgroups (read
  directly), [8193, 300] 2049 (one level, whose second workgroup holds one triple), and
  [65536, 128] 4096; masked and not.
* At [2^31 + 12288, 1]: 8388656 workgroups, two levels (4097 triples, then 3).  The rows
  repeat a 4096-row pattern k = 524291 times, so the call's mean is the pattern's and its
  sum of squared deviations k times the pattern's: every repetition must match the
  oracle's raw advantages for the pattern normalised with those (std unbiased over all
  k * 4096 elements, which is not the pattern's own unbiased std).
"""
import numpy as np
import pytest
import torch

from _common import assert_close, make_inputs, run_api, run_oracle

pytestmark = pytest.mark.gpu


def _triples(lib, E, T):
    return lib.rlk_gae_normalized_partials_bytes(E, T) // 24


@pytest.mark.parametrize("op,E,T,direct", [("gae_normalized", 8192, 300, 2048),
                                           ("gae_normalized", 8193, 300, 2049),
                                           ("gae_normalized", 65536, 128, 4096),
                                           ("gae_normalized_masked", 8193, 300, 2049)],
                         ids=lambda v: str(v))
def test_partials_tree_matches_oracle(op, E, T, direct, device):
    from rl_triton import _native
    print(f"[normalized-tree] {op} [{E},{T}]", flush=True)
    # the first launch's workgroups, then one triple per 2048 for each level above 2048
    levels = [direct]
    while levels[-1] > 2048:
        levels.append(-(-levels[-1] // 2048))
    assert _triples(_native.load(), E, T) == sum(levels)
    inp, params = make_inputs(op, E, T, seed=E + T, p_trunc=0.02, boot="full")
    params = dict(params, eps=1e-8)
    adv, ret = run_api(op, inp, params, device)
    adv_exp, ret_exp = run_oracle(op, inp, params)
    raw_op = "gae_masked" if op == "gae_normalized_masked" else "gae"
    raw = run_oracle(raw_op, inp, {k: v for k, v in params.items() if k != "eps"})[0]
    kept = raw if op == "gae_normalized" else raw[np.asarray(inp["mask"]) != 0]
    std = float(np.std(kept, ddof=1))
    base = 1e-5 * max(1.0, float(np.max(np.abs(raw))))
    scale = max(1.0, float(np.max(np.abs(ret_exp))))
    assert_close(ret.cpu().numpy(), ret_exp, 1e-5, base + 1e-6 * scale, f"{op}[{E},{T}]:returns")
    assert_close(adv.cpu().numpy(), adv_exp, 1e-5, base / min(std, 1.0) + 1e-6,
                 f"{op}[{E},{T}]:advantages")


def test_two_tree_levels_on_repeated_rows(device):
    import rl_triton
    from rl_triton import _native
    P, k = 4096, 524291
    E = P * k
    assert E > 2 ** 31 and _triples(_native.load(), E, 1) == 8388656 + 4097 + 3
    free, _ = torch.cuda.mem_get_info(device)
    if free < 64 * 2 ** 30:
        pytest.skip(f"needs ~50 GiB of device memory, {free / 2 ** 30:.0f} GiB free")
    print(f"[normalized-tree] gae_normalized [{E},1] two levels", flush=True)
    pat, params = make_inputs("gae_normalized", P, 1, seed=3, boot="row")
    params = dict(params, eps=1e-8)
    raw = run_oracle("gae", pat, {k_: v for k_, v in params.items() if k_ != "eps"})[0]
    raw = np.asarray(raw, dtype=np.float64)
    mean = raw.mean()
    std = np.sqrt(((raw - mean) ** 2).sum() * k / (E - 1))
    adv_exp = (raw - mean) / (std + params["eps"])
    ret_exp = raw + np.asarray(pat["values"], dtype=np.float64)
    big = {name: torch.as_tensor(pat[name]).to(device).repeat(k, 1)
           for name in ("rewards", "values", "terminateds")}
    last = torch.as_tensor(pat["last_value"]).to(device).repeat(k)
    adv, ret = rl_triton.compute_gae_normalized(big["rewards"], big["values"], big["terminateds"],
                                                last_value=last, **params)
    torch.cuda.synchronize()
    del big, last
    exp_a = torch.as_tensor(adv_exp, dtype=torch.float64, device=device).view(1, P)
    exp_r = torch.as_tensor(ret_exp, dtype=torch.float64, device=device).view(1, P)
    for got, exp, what in ((adv, exp_a, "advantages"), (ret, exp_r, "returns")):
        rows = got.view(k, P)
        worst = 0.0
        for c in range(0, k, 16384):
            d = (rows[c:c + 16384].double() - exp).abs() - (2e-5 + 1e-5 * exp.abs())
            worst = max(worst, float(d.max()))
        assert worst <= 0.0, f"{what}: a repetition differs from the pattern's oracle result by {worst} beyond the tolerance"
