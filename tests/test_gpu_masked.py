"""GAE with skipped steps (compute_gae(..., mask=...), the reference's ROADMAP.md:131-140
"verl-style" masking) on the GPU against the float64 oracle (oracle.gae_masked, pinned in
test_oracle_cpu.py by the all-kept identity, the kept-steps compression identity and a
hand-worked example).

Masks are multi-turn span patterns (alternating kept/skipped spans, mean length 12), plus
all-kept, all-skipped, skipped heads and tails.  Tolerances as in test_gpu_parity.py:
seq_len <= 2048: rtol = atol = 1e-5; longer rows (look-back path): rtol = 1e-5,
atol = 1e-5 * sqrt(L_eff / 128) * max(1, max|expected|), L_eff = 1/(1 - gamma*lambda).
"""
import math

import numpy as np
import pytest
import torch

from _common import assert_close, make_inputs, run_api, run_oracle

pytestmark = pytest.mark.gpu

SHORT = [(1, 1), (1, 7), (4, 128), (33, 257), (128, 1024), (3, 1100), (16, 2048)]
LONG = [(3, 2049), (2, 5000), (1, 65536), (2, 131073)]


def _check(inp, params, device, what):
    got = run_api("gae_masked", inp, params, device)[0]
    exp = run_oracle("gae_masked", inp, params)[0]
    T = exp.shape[1] if exp.ndim == 2 else 1
    atol = 1e-5
    if T > 2048:
        scale = max(1.0, float(np.max(np.abs(exp)))) if exp.size else 1.0
        atol *= scale * math.sqrt(max(1.0 / (1.0 - 0.99 * 0.95), 128) / 128.0)
    assert_close(got.cpu().numpy(), exp, 1e-5, atol, what)
    return got


@pytest.mark.parametrize("boot", ["none", "row", "full"])
@pytest.mark.parametrize("trunc", [0.0, 0.03])
@pytest.mark.parametrize("shape", SHORT + LONG, ids=lambda s: f"{s[0]}x{s[1]}")
def test_masked_gae_parity(shape, boot, trunc, device):
    if boot == "row" and trunc > 0:
        pytest.skip("last_value cannot be combined with truncateds (reference contract)")
    inp, params = make_inputs("gae_masked", *shape, seed=11, p_trunc=trunc, boot=boot)
    _check(inp, params, device, f"gae_masked{shape} boot={boot} trunc={trunc}")


@pytest.mark.parametrize("shape", [(64, 128), (8, 2048), (5, 10000)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_masked_gae_edge_masks(shape, device):
    """Rows with nothing kept (all zero), everything kept, a skipped head and a skipped
    tail (the boundary value crosses it), and single kept steps."""
    E, T = shape
    inp, params = make_inputs("gae_masked", E, T, seed=12, boot="full", p_trunc=0.02)
    mask = inp["mask"]
    mask[0, :] = 0.0
    mask[1, :] = 1.0
    mask[2, : T // 3] = 0.0
    mask[3 % E, -T // 3:] = 0.0
    if E > 4:
        mask[4, :] = 0.0
        mask[4, T // 2] = 1.0
    got = _check(inp, params, device, f"edge masks {shape}")
    assert float(got[0].abs().max()) == 0.0


@pytest.mark.parametrize("shape", [(4096, 128), (16, 2048), (2, 40000)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_all_kept_mask_matches_compute_gae(shape, device):
    """With every step kept the masked kernel computes compute_gae (to float32 rounding:
    the next value enters through the scan instead of the neighbour step)."""
    inp, params = make_inputs("gae", *shape, seed=13, boot="full", p_trunc=0.02)
    plain = run_api("gae", inp, params, device)[0]
    inp["mask"] = np.ones_like(inp["rewards"])
    masked = run_api("gae_masked", inp, params, device)[0]
    scale = max(1.0, float(plain.abs().max()))
    torch.testing.assert_close(masked, plain, rtol=1e-5, atol=1e-5 * scale)


def test_masked_gae_rejects_bad_mask(device):
    import rl_triton
    x = torch.zeros(4, 8, device=device)
    with pytest.raises(AssertionError, match="mask shape"):
        rl_triton.compute_gae(x, x, x, mask=torch.zeros(4, 7, device=device))
    with pytest.raises(AssertionError, match="mask must be on CUDA"):
        rl_triton.compute_gae(x, x, x, mask=torch.zeros(4, 8))
    with pytest.raises(AssertionError, match="mask: expected float32"):
        rl_triton.compute_gae(x, x, x, mask=torch.zeros(4, 8, device=device, dtype=torch.float64))


def test_masked_gae_repeatable(device):
    inp, params = make_inputs("gae_masked", 4, 70000, seed=14, boot="row")
    a = run_api("gae_masked", inp, params, device)[0]
    b = run_api("gae_masked", inp, params, device)[0]
    assert torch.equal(a, b)


# ---------------------------------------------------------------------------------------
# compute_gae_normalized(..., mask=...): statistics over the kept steps (verl's masked
# whitening), against the float64 composition of the masked GAE oracle
# (tests/_common.normalized_from_oracle with the mask)
# ---------------------------------------------------------------------------------------
def _check_normalized_masked(inp, params, device, what):
    got = run_api("gae_normalized_masked", inp, params, device)
    adv_exp, ret_exp = run_oracle("gae_normalized_masked", inp, params)
    raw = run_oracle("gae_masked", inp, {k: v for k, v in params.items() if k != "eps"})[0]
    kept = raw[np.asarray(inp["mask"]) != 0]
    std = float(np.std(kept, ddof=1))
    T = raw.shape[1]
    base = 1e-5 * max(1.0, float(np.max(np.abs(raw))))
    if T > 2048:
        base *= math.sqrt(max(1.0 / (1.0 - 0.99 * 0.95), 128) / 128.0)
    scale = max(1.0, float(np.max(np.abs(ret_exp))))
    assert_close(got[1].cpu().numpy(), ret_exp, 1e-5, base + 1e-6 * scale, f"{what}:returns")
    assert_close(got[0].cpu().numpy(), adv_exp, 1e-5, base / min(std, 1.0) + 1e-6,
                 f"{what}:advantages")
    return got


@pytest.mark.parametrize("boot", ["none", "row", "full"])
@pytest.mark.parametrize("shape", [(4, 128), (33, 257), (16, 2048), (3, 5000), (2, 40000)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_masked_gae_normalized_parity(shape, boot, device):
    trunc = 0.0 if boot == "row" else 0.03
    inp, params = make_inputs("gae_normalized_masked", *shape, seed=15, p_trunc=trunc, boot=boot)
    params = dict(params, eps=1e-8)
    _check_normalized_masked(inp, params, device, f"normalized masked {shape} boot={boot}")


def test_masked_gae_normalized_statistics_are_over_kept_steps(device):
    """C2 shape with a span mask: the kept steps come out with mean 0 and std 1, the skipped
    ones are normalised with the same statistics; an all-ones mask reproduces the unmasked
    call."""
    inp, params = make_inputs("gae_normalized_masked", 4096, 128, seed=16, p_trunc=0.005,
                              boot="full")
    params = dict(params, eps=1e-8)
    adv, ret = _check_normalized_masked(inp, params, device, "C2 masked normalized")
    kept = torch.as_tensor(inp["mask"], device=device) != 0
    a = adv.double()[kept]
    assert abs(float(a.mean())) < 1e-6 and abs(float(a.std()) - 1.0) < 1e-5
    ones = dict(inp, mask=np.ones_like(inp["mask"]))
    m_adv, m_ret = run_api("gae_normalized_masked", ones, params, device)
    u_adv, u_ret = run_api("gae_normalized", {k: v for k, v in inp.items() if k != "mask"},
                           params, device)
    scale = max(1.0, float(u_ret.abs().max()))
    torch.testing.assert_close(m_ret, u_ret, rtol=1e-5, atol=1e-5 * scale)
    torch.testing.assert_close(m_adv, u_adv, rtol=1e-5, atol=1e-5 * scale)
