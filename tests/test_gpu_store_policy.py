"""Output stores: each launch stores its outputs non-temporally or write-through, chosen by
the call's shape and storage type (rlk_capi.hip store_write_through), and both store the
same bits.  With the policy forced each way (rlk_debug_store_policy), every kernel built
with both policies -- short rows of one wave and of several, the normalised GAE's scan,
the long rows of the chain kernel, aligned and phased -- must give bit-identical outputs,
and the default must match them.  The write-through store is inline assembly that carries
its own wait states (on gfx950 a vector write to the data registers of a store wider than
8 bytes too soon after it changes what is stored), so this compares it with the
compiler's own stores on every op that has both.  Against the float64 oracle as well.
"""
import pytest
import torch

from _common import OUTPUTS, assert_close, make_inputs, run_api, run_oracle, suite_atol

pytestmark = pytest.mark.gpu

CASES = [("gae", 64, 512), ("gae", 4096, 128), ("gae", 300, 1000), ("gae_masked", 16, 2048),
         ("vtrace", 1024, 512), ("retrace", 16, 2048), ("lambda_returns", 64, 1000),
         ("gae_normalized", 64, 512), ("discounted_returns", 16, 131072),
         ("prefix_sum", 8, 65536), ("eligibility_traces", 4, 40001), ("gae", 16, 131071),
         ("backward_scan", 8, 20000), ("forward_scan", 3, 9999)]


def _lib():
    from rl_triton import _native
    return _native.load()


@pytest.mark.parametrize("op,E,T", CASES, ids=lambda v: str(v))
def test_store_policies_store_the_same_bits(op, E, T, device):
    lib = _lib()
    print(f"[store-policy] {op} [{E},{T}]", flush=True)
    boot = "full" if op in ("gae", "gae_masked", "gae_normalized", "vtrace", "lambda_returns",
                            "discounted_returns") else "row"
    inp, params = make_inputs(op, E, T, seed=E + T, p_trunc=0.0 if op == "retrace" else 0.01,
                              boot=boot)
    got = {}
    try:
        for policy in (0, 1, -1):
            assert lib.rlk_debug_store_policy(policy) == 0
            got[policy] = [g.clone() for g in run_api(op, inp, params, device)]
            torch.cuda.synchronize()
    finally:
        lib.rlk_debug_store_policy(-1)
    for name, nt, wt, auto in zip(OUTPUTS[op], got[0], got[1], got[-1]):
        assert torch.equal(nt, wt), f"{op}[{E},{T}]:{name}: write-through differs from non-temporal"
        assert torch.equal(nt, auto), f"{op}[{E},{T}]:{name}: the default differs from a forced policy"
    exp = run_oracle(op, inp, params)
    for name, g, e in zip(OUTPUTS[op], got[-1], exp):
        assert_close(g.cpu().numpy(), e, 1e-5, suite_atol(op, inp, e, T), f"{op}[{E},{T}]:{name}")


def test_store_policy_rejects_other_values(device):
    lib = _lib()
    assert lib.rlk_debug_store_policy(2) == -1
    assert lib.rlk_debug_store_policy(-2) == -1
    assert lib.rlk_debug_store_policy(-1) == 0
