"""Long rows whose length is not a multiple of four, in the phased access mode: every
[E, T] array of the call at the same element phase (address / element size, mod 4), so
each row's four-step segments start at its own 16-byte boundary (rlk_engine.hpp load_seg,
kPhased).  Rows then start at every phase 0..3 within one call (row r at (phase0 + r*T)
mod 4); a row's first and last quads hold steps of its neighbours, which must be masked
and never stored.  Checked against the float64 oracle with the long-row tolerance, and
bfloat16 bit-identical to the float32 result rounded.  Through the C ABI, all arrays
(outputs too) are placed 1..3 elements into larger NaN-filled buffers (row 0 at phase
1..3): the steps a row's first and last quads read beyond the arrays are NaN, so a masking
slip shows, and the NaN around the output must survive the call.  A call whose outputs
sit at another phase than its inputs takes the element-aligned path instead; both against
the oracle.  A row's tiles are shifted to its four-element boundaries, which leaves up to
3 steps of the row outside them (backward scans: at the row's end, forward: at its start);
the first tile in scan order takes those as one more quad.  Lengths just below a multiple
of the tile (8190, 12287, 131071, 262143) put them beyond the last tile.
"""
import numpy as np
import pytest
import torch

from _common import OUTPUTS, assert_close, make_inputs, run_api, run_oracle, suite_atol

pytestmark = pytest.mark.gpu

CASES = [("gae", 5, 8190), ("gae_masked", 5, 4099), ("vtrace", 3, 12287),
         ("lambda_returns", 7, 4097), ("discounted_returns", 4, 65539),
         ("discounted_returns", 16, 131071), ("eligibility_traces", 6, 8193),
         ("prefix_sum", 8, 20001), ("prefix_sum", 3, 262143), ("backward_scan", 3, 16383),
         ("forward_scan", 9, 9001)]


def _inputs(op, E, T, seed):
    kw = {"p_done": 1e-3} if op in ("prefix_sum", "eligibility_traces") else {}
    boot = "full" if op in ("gae", "gae_masked", "vtrace", "lambda_returns",
                            "discounted_returns") else "row"
    return make_inputs(op, E, T, seed=seed, p_trunc=0.01, boot=boot, **kw)


@pytest.mark.parametrize("op,E,T", CASES, ids=lambda v: str(v))
def test_phased_rows_match_oracle(op, E, T, device):
    from rl_triton import _native
    print(f"[phased] {op} [{E},{T}]", flush=True)
    inp, params = _inputs(op, E, T, seed=E * 31 + T)
    got = run_api(op, inp, params, device)
    exp = run_oracle(op, inp, params)
    for name, g, e in zip(OUTPUTS[op], got, exp):
        assert_close(g.cpu().numpy(), e, 1e-5, suite_atol(op, inp, e, T), f"{op}[{E},{T}]:{name}")
    assert not _native.workspace_error(device)
    rounded = {k: (v if v is None else torch.as_tensor(v).to(torch.bfloat16).float().numpy())
               for k, v in inp.items()}
    got_b = run_api(op, rounded, params, device, dtype=torch.bfloat16)
    ref = run_api(op, rounded, params, device, dtype=torch.float32)
    for name, g, r in zip(OUTPUTS[op], got_b, ref):
        same = g.view(torch.int16) == r.to(torch.bfloat16).view(torch.int16)
        assert bool(same.all()), f"{op}[{E},{T}]:{name}: {int((~same).sum())} bfloat16 elements differ"


def _lib():
    from rl_triton import _native
    return _native.load()


def _placed(a, offset, device):
    """A float32 device copy of `a` (or NaN of its shape when a is a shape) starting `offset`
    elements into a larger buffer."""
    shape = a if isinstance(a, tuple) else a.shape
    n = int(np.prod(shape))
    buf = torch.full((n + offset + 3,), float("nan"), device=device)
    view = buf[offset:offset + n].view(shape)
    if not isinstance(a, tuple):
        view.copy_(torch.as_tensor(a))
    return buf, view


def _call(lib, op, inp, params, E, T, in_off, out_off, device):
    keep = []

    def put(k):
        if inp.get(k) is None:
            return None
        buf, view = _placed(inp[k], in_off, device)
        keep.append(buf)
        return view.data_ptr()

    obuf, out = _placed((E, T), out_off, device)
    wsb = lib.rlk_workspace_bytes(E, T)
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    if op == "gae":
        st = lib.rlk_gae(put("rewards"), put("values"), put("terminateds"), put("truncateds"),
                         put("bootstrap_values"), 2, out.data_ptr(), E, T, params["gamma"],
                         params["lambda_"], ws.data_ptr(), wsb, stream)
    elif op == "discounted_returns":
        st = lib.rlk_discounted_returns(put("rewards"), put("terminateds"), put("truncateds"),
                                        put("bootstrap_values"), 2, out.data_ptr(), E, T,
                                        params["gamma"], ws.data_ptr(), wsb, stream)
    else:
        seed = None
        if inp.get("seed_values") is not None:
            seed = torch.as_tensor(inp["seed_values"]).to(device)
            keep.append(seed)
        st = lib.rlk_prefix_sum(put("inputs"), put("dones"),
                                seed.data_ptr() if seed is not None else None, out.data_ptr(),
                                E, T, 1, ws.data_ptr(), wsb, stream)
    assert st == 0, f"{op}: status {st}"
    torch.cuda.synchronize()
    # nothing written outside the output's own elements
    assert bool(torch.isnan(obuf[:out_off]).all()) and bool(torch.isnan(obuf[out_off + E * T:]).all())
    return out.cpu().numpy()


@pytest.mark.parametrize("op,E,T", [("gae", 6, 12287), ("discounted_returns", 5, 40001),
                                    ("prefix_sum", 7, 70002)], ids=lambda v: str(v))
def test_phased_rows_at_every_base_phase(op, E, T, device):
    lib = _lib()
    inp, params = _inputs(op, E, T, seed=T)
    exp = run_oracle(op, inp, params)[0]
    tol = suite_atol(op, inp, exp, T)
    for in_off, out_off in [(1, 1), (2, 2), (3, 3), (0, 2), (3, 0)]:
        print(f"[phased-capi] {op} [{E},{T}] inputs +{in_off} outputs +{out_off}", flush=True)
        got = _call(lib, op, inp, params, E, T, in_off, out_off, device)
        assert_close(got, exp, 1e-5, tol, f"{op}[{E},{T}] +{in_off}/+{out_off}")
