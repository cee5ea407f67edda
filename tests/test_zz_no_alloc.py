"""rlk_gae_noalloc -- GAE with its look-back status words in the library's static device
buffer (no allocation, no caller workspace) -- against rlk_gae with a caller-allocated
workspace, through the C ABI (ctypes), on long rows: the two launch the same kernel with
the same arguments but the workspace pointer, so their results must be bit-identical.
Two calls in a row, the second on a smaller input, reuse the buffer the first left; a
graph-captured call clears the buffer itself on every replay; a call too large for the
buffer is refused before any launch.  Against the float64 oracle as well.  Runs alone in a
fresh process (the first call on the device clears the buffer) or after any other test.
"""
import ctypes

import numpy as np
import pytest
import torch

from _common import assert_close, make_inputs, run_oracle, suite_atol, to_device

pytestmark = pytest.mark.gpu


def _lib():
    from rl_triton import _native
    return _native.load()


def _args(d, out):
    boot = d.get("bootstrap_values")
    return (d["rewards"].data_ptr(), d["values"].data_ptr(), d["terminateds"].data_ptr(),
            d["truncateds"].data_ptr() if d.get("truncateds") is not None else None,
            boot.data_ptr() if boot is not None else None, 2 if boot is not None else 0,
            out.data_ptr())


def _both(lib, inp, E, T, stream):
    """(rlk_gae with a fresh zeroed workspace, rlk_gae_noalloc) on the same device inputs."""
    d = to_device(inp, "cuda")
    ref, got = torch.empty(E, T, device="cuda"), torch.empty(E, T, device="cuda")
    wsb = lib.rlk_workspace_bytes(E, T)
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device="cuda")
    assert lib.rlk_gae(*_args(d, ref), E, T, 0.99, 0.95, ws.data_ptr(), wsb, stream) == 0
    assert lib.rlk_gae_noalloc(*_args(d, got), E, T, 0.99, 0.95, stream) == 0
    torch.cuda.synchronize()
    if wsb:
        assert int(ws[24:32].view(torch.int64).item()) == 0
    return ref, got


def test_noalloc_matches_gae_with_workspace(device):
    lib = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    for i, (E, T) in enumerate([(16, 131072), (3, 5000), (1, 2000), (40, 4097)]):
        print(f"[case] rlk_gae_noalloc [{E},{T}]", flush=True)
        inp, params = make_inputs("gae", E, T, seed=70 + i, p_term=0.01, p_trunc=0.01, boot="full")
        ref, got = _both(lib, inp, E, T, stream)
        assert torch.equal(ref, got), f"[{E},{T}]: rlk_gae_noalloc differs from rlk_gae"
        exp = run_oracle("gae", inp, params)[0]
        assert_close(got.cpu().numpy(), exp, 1e-5, suite_atol("gae", inp, exp, T), f"[{E},{T}]")


def test_noalloc_refuses_calls_beyond_its_buffer(device):
    lib = _lib()
    E, T = 4096, 16384  # 16384 tiles of 4096 steps: 1.3 MB of status words > 1 MiB
    assert lib.rlk_workspace_bytes(E, T) > 1 << 20
    x = torch.zeros(1, device="cuda")
    p = x.data_ptr()
    assert lib.rlk_gae_noalloc(p, p, p, None, None, 0, p, E, T, 0.99, 0.95, None) == -4
    assert b"static buffer" in lib.rlk_status_string(-4)


def test_noalloc_under_graph_capture(device):
    """A captured call records the buffer's clear and the scan; each replay, with new inputs
    copied into the captured ones, equals rlk_gae on those inputs."""
    lib = _lib()
    E, T = 8, 40000
    inp, params = make_inputs("gae", E, T, seed=90, p_term=0.01, p_trunc=0.01, boot="full")
    static = to_device(inp, "cuda")
    out = torch.empty(E, T, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        assert lib.rlk_gae_noalloc(*_args(static, out), E, T, 0.99, 0.95, side.cuda_stream) == 0
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    for rep in range(3):
        new, _ = make_inputs("gae", E, T, seed=91 + rep, p_term=0.01, p_trunc=0.01, boot="full")
        for k, v in to_device(new, "cuda").items():
            if v is not None:
                static[k].copy_(v)
        graph.replay()
        torch.cuda.synchronize()
        ref, again = _both(lib, new, E, T, stream)  # eager calls between the replays
        assert torch.equal(out, ref), f"replay {rep} differs from rlk_gae"
        assert torch.equal(again, ref)
    del graph
