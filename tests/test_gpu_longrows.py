"""The look-back path (rows longer than 2048 steps) in the layouts the BASELINE shapes do not
reach: more rows than counter slots (64), so that several rows share a slot; rows of many
tiles; one workspace serving calls of changing shapes in stream order; two streams at once;
the rare paths (a predecessor computed in its workgroup's place, a walk back past 64 tiles,
a wait that gives up) forced from the host; and every op at those shapes.  Against the float64 oracle with the long-row
tolerance of test_gpu_parity.py (atol = 1e-5 * sqrt(L_eff / 128) * max(1, max|expected|)),
and no look-back wait may give up (the workspace error flag stays clear).
"""
import math

import numpy as np
import pytest

from _common import OUTPUTS, assert_close, make_inputs, run_api, run_oracle

pytestmark = pytest.mark.gpu

OPS = ["gae", "gae_masked", "vtrace", "retrace", "lambda_returns", "discounted_returns",
       "eligibility_traces", "prefix_sum", "backward_scan", "forward_scan"]


def _longest_run(d):
    best = 0
    for row in np.asarray(d) > 0:
        idx = np.flatnonzero(np.concatenate(([True], row, [True])))
        best = max(best, int(np.max(np.diff(idx))))
    return best


def _atol(op, inp, exp):
    scale = max(1.0, float(np.max(np.abs(exp))))
    if op == "prefix_sum":
        l_eff = _longest_run(inp["dones"])
    elif op in ("discounted_returns", "backward_scan", "forward_scan"):
        l_eff = 1.0 / (1.0 - 0.99)
    else:
        l_eff = 1.0 / (1.0 - 0.99 * 0.95)
    return 1e-5 * math.sqrt(max(l_eff, 128) / 128.0) * scale


def _inputs(op, E, T, seed):
    kw = {"p_done": 1e-3} if op in ("prefix_sum", "eligibility_traces") else {}
    boot = "full" if op in ("gae", "gae_masked", "vtrace", "lambda_returns",
                            "discounted_returns") else "row"
    return make_inputs(op, E, T, seed=seed, p_trunc=0.01 if op != "retrace" else 0.0, boot=boot,
                       **kw)


def _check(op, E, T, seed, device):
    inp, params = _inputs(op, E, T, seed)
    got = run_api(op, inp, params, device)
    exp = run_oracle(op, inp, params)
    for name, g, e in zip(OUTPUTS[op], got, exp):
        assert_close(g.cpu().numpy(), e, 1e-5, _atol(op, inp, e), f"{op}[{E},{T}]:{name}")


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", [(65, 2049), (130, 4100), (200, 2052)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_more_rows_than_slots(op, shape, device):
    from rl_triton import _native
    _check(op, *shape, seed=21, device=device)
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("path", ["python", "fast"])
def test_one_workspace_across_changing_shapes(path, device, monkeypatch):
    """Calls of different shapes and ops back to back on one stream share the cached
    workspace (the Python path's, or the C++ fast path's), which grows as the shapes need;
    each call leaves it ready for the next."""
    from rl_triton import _native
    if path == "fast":
        monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
    seq = [("prefix_sum", 3, 70000), ("gae", 130, 2100), ("vtrace", 2, 131073),
           ("discounted_returns", 64, 4096), ("prefix_sum", 1, 300000), ("gae_masked", 5, 9000),
           ("retrace", 70, 2500), ("forward_scan", 9, 33333)]
    before = _native.fast.launched() if _native.fast is not None else 0
    for i, (op, E, T) in enumerate(seq * 2):
        _check(op, E, T, seed=100 + i, device=device)
    if path == "fast":
        assert _native.fast.launched() - before == 2 * len(seq), "a call left the fast path"
    assert not _native.workspace_error(device)


def test_concurrent_streams(device):
    """Long-row calls queued on two streams at once, with no synchronisation between them:
    each stream has its own workspace (counters, epoch and status words), and the two grids
    may share the GPU in any proportion, so a tile can wait on a predecessor whose
    workgroup is not resident yet (the look-back then computes that predecessor itself).
    Every result matches the oracle and no wait gives up."""
    import torch
    from rl_triton import _native
    jobs = [[("prefix_sum", 4, 150000), ("discounted_returns", 3, 200001), ("vtrace", 2, 131072)],
            [("eligibility_traces", 6, 90000), ("gae", 5, 70000), ("forward_scan", 8, 65537)]]
    streams = [torch.cuda.Stream(device), torch.cuda.Stream(device)]
    pending = []
    for rep in range(2):
        for k in range(3):
            for j, s in enumerate(streams):
                op, E, T = jobs[j][k]
                inp, params = _inputs(op, E, T, seed=300 + 10 * rep + 3 * j + k)
                with torch.cuda.stream(s):
                    pending.append((op, E, T, inp, params, run_api(op, inp, params, device)))
    torch.cuda.synchronize()
    for op, E, T, inp, params, got in pending:
        exp = run_oracle(op, inp, params)
        for name, g, e in zip(OUTPUTS[op], got, exp):
            assert_close(g.cpu().numpy(), e, 1e-5, _atol(op, inp, e), f"{op}[{E},{T}] concurrent:{name}")
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("path", ["python", "fast"])
def test_row_counts_change_on_a_new_workspace(path, device, monkeypatch):
    """A new stream (so a new, zeroed workspace) and long-row calls whose row counts change
    from call to call, growing and shrinking past the 64 slots: rows then fall in other
    slots and use other status words, so the words an earlier call published lie where a
    later call's rows now look.  One row first (the 19 tiles of row 0), then two rows of 10
    tiles (row 1's words are row 0's last nine): a word an earlier call left must never
    carry the current epoch of the slot that reads it.  Every result matches the oracle
    and no wait gives up."""
    import torch
    from rl_triton import _native
    if path == "fast":
        monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
    shapes = [("prefix_sum", 1, 600000), ("prefix_sum", 2, 300000), ("discounted_returns", 3, 200001),
              ("prefix_sum", 70, 9000), ("discounted_returns", 5, 100000), ("prefix_sum", 64, 12000),
              ("discounted_returns", 1, 400000), ("prefix_sum", 9, 65537)]
    stream = torch.cuda.Stream(device)
    pending = []
    with torch.cuda.stream(stream):
        for i, (op, E, T) in enumerate(shapes):
            inp, params = _inputs(op, E, T, seed=500 + i)
            pending.append((op, E, T, inp, params, run_api(op, inp, params, device)))
    torch.cuda.synchronize()
    for op, E, T, inp, params, got in pending:
        exp = run_oracle(op, inp, params)
        for name, g, e in zip(OUTPUTS[op], got, exp):
            assert_close(g.cpu().numpy(), e, 1e-5, _atol(op, inp, e), f"{op}[{E},{T}] in sequence:{name}")
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("path", ["python", "fast"])
def test_single_tile_rows_between_chained_calls(path, device, monkeypatch):
    """Calls of one tile per row skip the look-back protocol and leave the workspace as
    they found it.  On a new stream (a new, zeroed workspace), such calls queued between
    chained ones, of changing row counts: every chained call must still find its slots'
    epochs current and its counters at rest.  Every result matches the oracle and no wait
    gives up."""
    import torch
    from rl_triton import _native
    if path == "fast":
        monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
    shapes = [("prefix_sum", 300, 3000), ("prefix_sum", 2, 300000), ("discounted_returns", 1000, 2101),
              ("discounted_returns", 3, 200001), ("gae", 70, 4000), ("prefix_sum", 70, 9000),
              ("eligibility_traces", 512, 2500), ("prefix_sum", 1, 600000), ("vtrace", 100, 4096),
              ("vtrace", 2, 131073)]
    stream = torch.cuda.Stream(device)
    pending = []
    with torch.cuda.stream(stream):
        for i, (op, E, T) in enumerate(shapes * 2):
            inp, params = _inputs(op, E, T, seed=700 + i)
            pending.append((op, E, T, inp, params, run_api(op, inp, params, device)))
    torch.cuda.synchronize()
    for op, E, T, inp, params, got in pending:
        exp = run_oracle(op, inp, params)
        for name, g, e in zip(OUTPUTS[op], got, exp):
            assert_close(g.cpu().numpy(), e, 1e-5, _atol(op, inp, e), f"{op}[{E},{T}] in sequence:{name}")
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("op,shape", [("prefix_sum", (1, 1 << 23)), ("vtrace", (1, 1 << 21)),
                                      ("gae_masked", (1, 1 << 20)), ("backward_scan", (1, 3 << 20)),
                                      ("discounted_returns", (2, 1 << 21)),
                                      ("eligibility_traces", (1, (1 << 22) + 3))],
                         ids=lambda v: v if isinstance(v, str) else f"{v[0]}x{v[1]}")
def test_many_tiles_per_row(op, shape, device):
    """Rows of 128-512 tiles: the look-back walks back over several 64-tile windows of maps
    before it meets a tile's state."""
    from rl_triton import _native
    _check(op, *shape, seed=41, device=device)
    assert not _native.workspace_error(device)


def test_lookback_give_up_poisons_with_nan(device):
    """A look-back wait that gives up -- forced here from the host with a budget of zero
    polls (rlk_debug_lookback), so that every tile whose 64 nearest predecessors do not
    already lead to a published state at its first poll gives up at once -- sets the
    workspace error flag and writes NaN for its tile and every tile chained through it,
    never plausible wrong values.  The row has no dones, so no tile's map ignores its carry
    and every tile needs a state from up to 255 tiles before it: the far tiles cannot have
    one at their first poll, so some wait does give up.  NaN then covers whole tiles only,
    the row's first tile (which takes the row's own carry) is never NaN, every other
    element is right, and nothing waits: the kernel ends normally."""
    import torch
    from rl_triton import _native
    lib = _native.load()
    op, E, T = "prefix_sum", 1, 1 << 23
    inp, params = make_inputs(op, E, T, seed=13, p_done=0.0)
    exp = run_oracle(op, inp, params)[0]
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    tile = next(1024 * 4 * q for q in (8, 4, 2) if E * -(-T // (1024 * 4 * q)) >= cus or q == 2)
    stream = torch.cuda.Stream(device)
    assert lib.rlk_debug_lookback(0, -1) == 0
    try:
        with torch.cuda.stream(stream):
            got = run_api(op, inp, params, device)[0]
        torch.cuda.synchronize()
    finally:
        lib.rlk_debug_lookback(-1, -1)
    key = (torch.device(device).index, stream.cuda_stream)
    ws = _native._workspaces.pop(key)  # this stream's workspace: do not reuse its flag
    flagged = int(ws[24:32].cpu().view(torch.int64).item()) != 0
    g = got.cpu().numpy()
    nan = np.isnan(g)
    per_tile = nan.reshape(E, -1, tile)
    print(f"gave up: {flagged}, NaN tiles: {int(per_tile.all(axis=2).sum())} of {per_tile.shape[1]}")
    assert flagged and nan.any()
    assert np.array_equal(per_tile.any(axis=2), per_tile.all(axis=2)), "NaN covers part of a tile"
    assert not per_tile[:, 0].any(), "the row's first tile takes the row carry, never NaN"
    assert_close(g[~nan], exp[~nan], 1e-5, _atol(op, inp, exp), f"{op}[{E},{T}] outside the NaN tiles")


@pytest.mark.parametrize("path", ["python", "fast"])
def test_single_tile_rows_between_chained_calls(path, device, monkeypatch):
    """Calls of one tile per row skip the look-back protocol and leave the workspace as
    they found it.  On a new stream (a new, zeroed workspace), such calls queued between
    chained ones, of changing row counts: every chained call must still find its slots'
    epochs current and its counters at rest.  Every result matches the oracle and no wait
    gives up."""
    import torch
    from rl_triton import _native
    if path == "fast":
        monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
    shapes = [("prefix_sum", 300, 3000), ("prefix_sum", 2, 300000), ("discounted_returns", 1000, 2101),
              ("discounted_returns", 3, 200001), ("gae", 70, 4000), ("prefix_sum", 70, 9000),
              ("eligibility_traces", 512, 2500), ("prefix_sum", 1, 600000), ("vtrace", 100, 4096),
              ("vtrace", 2, 131073)]
    stream = torch.cuda.Stream(device)
    pending = []
    with torch.cuda.stream(stream):
        for i, (op, E, T) in enumerate(shapes * 2):
            inp, params = _inputs(op, E, T, seed=700 + i)
            pending.append((op, E, T, inp, params, run_api(op, inp, params, device)))
    torch.cuda.synchronize()
    for op, E, T, inp, params, got in pending:
        exp = run_oracle(op, inp, params)
        for name, g, e in zip(OUTPUTS[op], got, exp):
            assert_close(g.cpu().numpy(), e, 1e-5, _atol(op, inp, e), f"{op}[{E},{T}] in sequence:{name}")
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("op,shape", [("prefix_sum", (1, 1 << 23)), ("vtrace", (1, 1 << 21)),
                                      ("gae_masked", (2, 1 << 19)), ("retrace", (3, 70000)),
                                      ("discounted_returns", (16, 131072)),
                                      ("backward_scan", (1, 3 << 20))],
                         ids=lambda v: v if isinstance(v, str) else f"{v[0]}x{v[1]}")
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_lookback_fallback_paths_give_the_same_bits(op, shape, dtype, device):
    """With the fallback budget at zero polls (rlk_debug_lookback), a tile whose predecessor
    has published nothing at its first poll computes that predecessor itself, and a window
    of maps with no state sends the look-back further back at once -- the paths a call
    only takes when some workgroup of it is not running.  The results equal the ordinary
    run's bit for bit, and the oracle's."""
    import torch
    from rl_triton import _native
    lib = _native.load()
    inp, params = _inputs(op, *shape, seed=57)
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    plain = [t.clone() for t in run_api(op, inp, params, device, dt)]
    assert lib.rlk_debug_lookback(-1, 0) == 0
    try:
        forced = run_api(op, inp, params, device, dt)
        torch.cuda.synchronize()
    finally:
        lib.rlk_debug_lookback(-1, -1)
    for name, a, b in zip(OUTPUTS[op], plain, forced):
        assert torch.equal(a, b), f"{op}{shape} {dtype}:{name} differs under the fallback paths"
    assert not _native.workspace_error(device)
    if dtype == "bf16":
        return  # the bfloat16 results are pinned against float32 in test_gpu_bf16.py
    exp = run_oracle(op, inp, params)
    for name, g, e in zip(OUTPUTS[op], forced, exp):
        assert_close(g.cpu().numpy(), e, 1e-5, _atol(op, inp, e), f"{op}{shape}:{name}")
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("op", ["gae", "lambda_returns", "discounted_returns", "eligibility_traces",
                                "prefix_sum", "backward_scan", "forward_scan", "vtrace"])
@pytest.mark.parametrize("shape", [(64, 40000), (200, 10001), (257, 8192), (256, 16384),
                                   (171, 24576), (256, 8192)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_tiles_between_one_and_two_per_cu(op, shape, device):
    """Calls whose 8192-step tiles outnumber the compute units but not twice over: the
    ops whose tiles can double take 16384-step tiles, fewer than the CUs, in one round;
    V-trace, whose largest tile is 8192 steps, takes 512 x 2 so that two workgroups fit a
    CU.  Aligned and element-aligned rows, with truncations where the op has them, and
    bfloat16 bit-identical to the float32 result rounded.  On a 256-CU MI355X, 257 and 512
    tiles ([257,8192], [256,16384]) are the rules' edges and 513 and 256 ([171,24576],
    [256,8192]) fall just outside them."""
    import torch
    from rl_triton import _native
    _check(op, *shape, seed=61, device=device)
    assert not _native.workspace_error(device)
    inp, params = _inputs(op, *shape, 61)
    rounded = {k: (v if v is None or k == "actions" else
                   torch.as_tensor(v).to(torch.bfloat16).float().numpy()) for k, v in inp.items()}
    got_b = run_api(op, rounded, params, device, dtype=torch.bfloat16)
    ref = run_api(op, rounded, params, device, dtype=torch.float32)
    for g, r in zip(got_b, ref):
        assert torch.equal(g.view(torch.int16), r.to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", [(512, 2500), (1000, 2101), (256, 5000), (300, 10001),
                                   (64, 12000), (4096, 2561), (16, 40000), (24, 20001)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_rows_much_shorter_than_the_cu_tile(op, shape, device):
    """Many rows of a few thousand steps, where the tile that gives every CU one would be
    mostly padding: the launcher takes smaller tiles (4096 steps at 512 threads, or the
    op's 8192-step ones), one to three per row with a ragged last tile, aligned and
    element-aligned rows.  And few rows whose smallest CU-sized tiles leave CUs idle
    ([16,40000], [24,20001]): 4096-step tiles, five to ten per row.  Against the oracle,
    and bfloat16 bit-identical to the float32 result rounded."""
    import torch
    from rl_triton import _native
    print(f"[short-long rows] {op} {shape}", flush=True)
    _check(op, *shape, seed=67, device=device)
    assert not _native.workspace_error(device)
    inp, params = _inputs(op, *shape, 67)
    rounded = {k: (v if v is None or k == "actions" else
                   torch.as_tensor(v).to(torch.bfloat16).float().numpy()) for k, v in inp.items()}
    got_b = run_api(op, rounded, params, device, dtype=torch.bfloat16)
    ref = run_api(op, rounded, params, device, dtype=torch.float32)
    for g, r in zip(got_b, ref):
        assert torch.equal(g.view(torch.int16), r.to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("boot", ["none", "full"])
@pytest.mark.parametrize("shape", [(64, 65536), (300, 16385), (256, 16383), (1024, 1 << 16),
                                   (3, 500000), (8, 200001)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_discounted_returns_wide_tiles(shape, boot, device):
    """Discounted returns without truncations take 1024-thread tiles on two kinds of calls:
    four segments per thread where every compute unit gets a 16384-step tile (aligned rows,
    a ragged last tile, element-aligned rows, and 4096 tiles, far more than the GPU holds at
    once), two segments on a few long rows whose 8192-step tiles reach half the compute
    units ([3,500000], [8,200001]).  float32 against the oracle, and bfloat16 bit-identical
    to the float32 kernels' result rounded."""
    import torch
    from rl_triton import _native
    inp, params = make_inputs("discounted_returns", *shape, seed=88, boot=boot)
    got = run_api("discounted_returns", inp, params, device)
    exp = run_oracle("discounted_returns", inp, params)
    for name, g, e in zip(OUTPUTS["discounted_returns"], got, exp):
        assert_close(g.cpu().numpy(), e, 1e-5, _atol("discounted_returns", inp, e),
                     f"discounted{shape}:{name}")
    assert not _native.workspace_error(device)
    rounded = {k: (None if v is None else torch.as_tensor(v).to(torch.bfloat16).float().numpy())
               for k, v in inp.items()}
    got_b = run_api("discounted_returns", rounded, params, device, dtype=torch.bfloat16)
    ref = run_api("discounted_returns", rounded, params, device, dtype=torch.float32)
    for g, r in zip(got_b, ref):
        assert torch.equal(g.view(torch.int16), r.to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("op,shape", [("vtrace", (2048, 16384)), ("prefix_sum", (1024, 1 << 16)),
                                      ("gae_masked", (600, 12000))],
                         ids=lambda v: v if isinstance(v, str) else f"{v[0]}x{v[1]}")
def test_grids_larger_than_the_gpu(op, shape, device):
    """Thousands of multi-tile rows: far more workgroups than the GPU holds at once, so tiles
    wait on predecessors that may not have started; every result matches the oracle and no
    wait gives up."""
    from rl_triton import _native
    _check(op, *shape, seed=73, device=device)
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("path", ["python", "fast"])
def test_workspace_rezeroed_at_call_limit(path, device, monkeypatch):
    """Each binding zero-fills its cached workspace again after RLK_WORKSPACE_MAX_CALLS
    long-row calls (the status words' 30-bit call count would wrap after 2^30).  With the
    limit lowered to 3: once the stream's workspace has been re-zeroed (within the first
    few calls, however many calls it served before), nine more calls of changing shapes
    re-zero it exactly three more times; every call matches the oracle and no wait gives
    up.  The largest workspace comes first, so the cache never grows (which also resets
    the count) during the test."""
    import torch
    from rl_triton import _native
    seq = [("gae", 130, 2100), ("prefix_sum", 3, 70000), ("vtrace", 2, 131073),
           ("discounted_returns", 64, 4096), ("forward_scan", 9, 33333)]
    if path == "fast":
        monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")
        clears = _native.fast.workspace_clears
        prev = _native.fast.set_workspace_max_calls(3)
    else:
        clears = lambda: _native._ws_clears  # noqa: E731
        monkeypatch.setattr(_native, "WORKSPACE_MAX_CALLS", 3)
    try:
        stream = torch.cuda.Stream(device)
        with torch.cuda.stream(stream):
            _check(*seq[0], seed=499, device=device)  # the workspace exists, large enough
            start, i = clears(), 0
            while clears() == start:
                assert i < 4, "no re-zeroing within the call limit"
                _check(*seq[i % len(seq)], seed=500 + i, device=device)
                i += 1
            first = clears()
            for j in range(9):
                _check(*seq[(i + j) % len(seq)], seed=600 + j, device=device)
            torch.cuda.synchronize()
            assert clears() - first == 3
    finally:
        if path == "fast":
            _native.fast.set_workspace_max_calls(prev)
    assert not _native.workspace_error(device)


@pytest.mark.parametrize("op,shape", [("discounted_returns", (2, 65536)), ("prefix_sum", (2, 65536)),
                                      ("discounted_returns", (2, 2000)), ("prefix_sum", (2, 2000))],
                         ids=lambda v: v if isinstance(v, str) else f"{v[0]}x{v[1]}")
def test_non_finite_input_after_a_reset(op, shape, device):
    """An inf reward/input in a row with resets (dones every 300 steps).  The reference's
    sequential loop makes every later step in scan order non-finite, across resets too
    (0 * inf and 0 * nan are nan).  Rows of up to 2048 steps do exactly that.  A long row
    does it up to the end of the first tile, in scan order after the one holding the inf,
    whose map ignores its carry (a reset inside it): that tile publishes its outgoing value
    before it knows its carry, computed from a zero carry, so the tiles after it see a
    finite value.  There each step holds what the row gives with the inf replaced by 0 --
    a value the inf's episode cannot reach -- and never any other value.  So on every
    element: the oracle's finite values are matched; where the oracle is not finite the
    result is either not finite or the zeroed row's value; the non-finite elements form
    one run in scan order, starting at the inf."""
    import torch
    E, T = shape
    inp, params = make_inputs(op, E, T, seed=31, p_term=0.0, p_done=0.0)
    key = "rewards" if op == "discounted_returns" else "inputs"
    dkey = "terminateds" if op == "discounted_returns" else "dones"
    inp[dkey][:, 150::300] = 1.0
    at = (T * 3) // 4 if op == "discounted_returns" else T // 4  # backward / forward scans
    zeroed = {k: (v.copy() if v is not None else None) for k, v in inp.items()}
    inp[key][:, at] = np.inf
    zeroed[key][:, at] = 0.0
    exp = run_oracle(op, inp, params)[0]
    exp0 = run_oracle(op, zeroed, params)[0]
    got = run_api(op, inp, params, device)[0].cpu().numpy().astype(np.float64)
    torch.cuda.synchronize()
    fin_e, fin_g = np.isfinite(exp), np.isfinite(got)
    tol = 1e-4 * max(1.0, float(np.max(np.abs(exp0))))
    assert np.all(np.abs(got[fin_e] - exp[fin_e]) <= tol), "finite oracle values not matched"
    other = ~fin_e & fin_g
    assert np.all(np.abs(got[other] - exp0[other]) <= tol), "a finite value that is not the zeroed row's"
    for n in range(E):  # the non-finite run, in scan order, starts at the inf and is contiguous
        idx = np.flatnonzero(~fin_g[n])
        order = idx if op == "prefix_sum" else idx[::-1]
        assert order[0] == at, "the inf itself is not where the non-finite run starts"
        assert np.all(np.abs(np.diff(order)) == 1), "the non-finite elements are not one run"
    if T <= 2048:  # whole rows in one workgroup: the sequential loop's pattern exactly
        assert np.array_equal(fin_g, fin_e)
    else:
        assert np.any(other), "the long row was expected to stop the nan at a tile boundary"


def _shape_sweep(n=40, seed=4242):
    """Seeded (op, E, T) cases spread over the long-row tile-shape rules: from one 8192-step
    tile per call to about three per compute unit of a 256-CU GPU, one to forty tiles per
    row with a ragged last tile, aligned rows and element-aligned ones."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        op = OPS[i % len(OPS)]
        per_row = int(rng.choice([1, 2, 3, 5, 8, 16, 40]))
        tiles = int(rng.integers(1, 800))
        T = max(2052, per_row * 8192 - int(rng.integers(0, 8192)))
        if rng.random() < 0.6:
            T -= T % 4
        E = max(1, min(tiles // per_row, 4_000_000 // T))
        cases.append((op, E, T))
    return cases


@pytest.mark.parametrize("op,E,T", _shape_sweep(), ids=lambda v: str(v))
def test_long_row_shape_sweep(op, E, T, device):
    """Every tile shape the launcher picks for long rows (the op's own, the wide and few-row
    discounted-returns shapes, the half-width shapes at one to two tiles per CU) against the
    oracle, and bfloat16 bit-identical to the float32 result rounded."""
    import torch
    from rl_triton import _native
    print(f"[sweep] {op} [{E},{T}]", flush=True)
    _check(op, E, T, seed=E * 7 + T, device=device)
    assert not _native.workspace_error(device)
    inp, params = _inputs(op, E, T, E * 7 + T)
    rounded = {k: (v if v is None or k == "actions" else
                   torch.as_tensor(v).to(torch.bfloat16).float().numpy()) for k, v in inp.items()}
    got_b = run_api(op, rounded, params, device, dtype=torch.bfloat16)
    ref = run_api(op, rounded, params, device, dtype=torch.float32)
    for g, r in zip(got_b, ref):
        assert torch.equal(g.view(torch.int16), r.to(torch.bfloat16).view(torch.int16))
