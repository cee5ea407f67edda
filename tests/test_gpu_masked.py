"""GAE with skipped steps (compute_gae(..., mask=...), the reference's ROADMAP.md:131-140
"verl-style" masking) on the GPU against the float64 oracle (oracle.gae_masked, pinned in
test_oracle_cpu.py by the all-kept identity, the kept-steps compression identity and a
hand-worked example).

Masks are multi-turn span patterns (alternating kept/skipped spans, mean length 12), plus
all-kept, all-skipped, skipped heads and tails.  Tolerances as in test_gpu_parity.py:
seq_len <= 2048: rtol = 1e-5, atol = 1e-5 * max(1, max|expected|); longer rows (look-back
path): atol = 1e-5 * sqrt(L_eff / 128) * max(1, max|expected|), L_eff = 1/(1 - gamma*lambda).
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
    scale = max(1.0, float(np.max(np.abs(exp)))) if exp.size else 1.0
    T = exp.shape[1] if exp.ndim == 2 else 1
    atol = 1e-5 * scale
    if T > 2048:
        atol *= math.sqrt(max(1.0 / (1.0 - 0.99 * 0.95), 128) / 128.0)
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
