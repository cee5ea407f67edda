"""HIP-graph capture and replay of every op (the reference's ROADMAP.md:125-130 "graph
support for small-batch workloads"; torch.cuda.graph over the same public calls).

A captured call is replayed several times.  Between replays the static inputs are
overwritten with new data and other eager work (uncaptured calls of the same op, torch ops)
runs on the default stream; every replay's outputs must equal, bit for bit, an eager call on
the same inputs, and match the float64 oracle on those inputs at the suite's tolerances
(rtol = atol = 1e-5 up to 2048 steps, the horizon-scaled atol beyond; normalised advantages
with that tolerance divided by the batch std).  Rows longer than 2048 steps use the
look-back workspace: both the documented order (a warm-up call on the capture stream
creates it before capture) and a first call inside the capture are covered.  [3,5001]
takes the phased access of long rows whose length is not a multiple of four; [8193,300] the
tree that sums a normalised call's partials.
"""
import pytest
import torch

import numpy as np

from _common import OUTPUTS, assert_close, make_inputs, run_api, run_oracle, suite_atol, to_device

pytestmark = pytest.mark.gpu

OPS = ["gae", "gae_masked", "gae_normalized", "gae_normalized_masked", "vtrace", "retrace", "lambda_returns",
       "discounted_returns", "eligibility_traces", "prefix_sum", "backward_scan", "forward_scan"]


def _inputs(op, shape, seed):
    boot = ("full" if op in ("gae", "gae_masked", "gae_normalized", "gae_normalized_masked",
                             "vtrace", "lambda_returns", "discounted_returns") else "row")
    return make_inputs(op, *shape, seed=seed, p_trunc=0.02 if op != "retrace" else 0.0, boot=boot)


def _call(op, d, params):
    """run_api on already-placed device tensors (the static inputs of the graph)."""
    import rl_triton
    from rl_triton.ops._scan import _run_scan, _run_scan_forward
    g = d.get
    if op == "gae":
        return (rl_triton.compute_gae(g("rewards"), g("values"), g("terminateds"), g("truncateds"),
                                      bootstrap_values=g("bootstrap_values"),
                                      last_value=g("last_value"), **params),)
    if op == "gae_masked":
        return (rl_triton.compute_gae(g("rewards"), g("values"), g("terminateds"), g("truncateds"),
                                      bootstrap_values=g("bootstrap_values"),
                                      last_value=g("last_value"), mask=g("mask"), **params),)
    if op in ("gae_normalized", "gae_normalized_masked"):
        return rl_triton.compute_gae_normalized(g("rewards"), g("values"), g("terminateds"),
                                                g("truncateds"),
                                                bootstrap_values=g("bootstrap_values"),
                                                last_value=g("last_value"), mask=g("mask"),
                                                **params)
    if op == "vtrace":
        return rl_triton.compute_vtrace(g("log_pi_target"), g("log_pi_behavior"), g("values"),
                                        g("rewards"), g("terminateds"), g("truncateds"),
                                        bootstrap_values=g("bootstrap_values"),
                                        last_value=g("last_value"), **params)
    if op == "retrace":
        return rl_triton.compute_retrace(g("action_probs_target"), g("action_probs_behavior"),
                                         g("q_values"), g("next_q_values_all"), g("actions"),
                                         g("rewards"), g("terminateds"), g("truncateds"), **params)
    if op == "lambda_returns":
        return (rl_triton.compute_lambda_returns(g("rewards"), g("next_values"), g("terminateds"),
                                                 g("truncateds"),
                                                 bootstrap_values=g("bootstrap_values"), **params),)
    if op == "discounted_returns":
        return (rl_triton.compute_discounted_returns(g("rewards"), g("terminateds"),
                                                     g("truncateds"),
                                                     bootstrap_values=g("bootstrap_values"),
                                                     **params),)
    if op == "eligibility_traces":
        return (rl_triton.compute_eligibility_traces(g("gradients"), g("dones"), params["gamma"],
                                                     params["lambda_"],
                                                     seed_values=g("seed_values")),)
    if op == "prefix_sum":
        return (rl_triton.compute_episodic_prefix_sum(g("inputs"), g("dones"),
                                                      seed_values=g("seed_values"),
                                                      boundary=params.get("boundary", "ends_at")),)
    if op == "backward_scan":
        return (_run_scan(g("u"), g("v"), g("bootstrap")),)
    return (_run_scan_forward(g("u"), g("v"), g("seed")),)


def _same(a, b):
    return torch.equal(a.view(torch.int32), b.view(torch.int32))  # bitwise, nan included


def _against_oracle(op, inp, params, outs, T, what):
    exp = run_oracle(op, inp, params)
    if op.startswith("gae_normalized"):
        adv_exp, ret_exp = exp
        raw = ret_exp - np.asarray(inp["values"], np.float64)
        kept = raw if inp.get("mask") is None else raw[np.asarray(inp["mask"]) != 0]
        std = float(np.std(kept, ddof=1))
        base = suite_atol("gae", inp, raw, T)
        scale = max(1.0, float(np.max(np.abs(ret_exp))))
        assert_close(outs[1].cpu().numpy(), ret_exp, 1e-5, base + 1e-6 * scale, f"{what}:returns")
        assert_close(outs[0].cpu().numpy(), adv_exp, 1e-5, base / min(std, 1.0) + 1e-6,
                     f"{what}:advantages")
        return
    base_op = "gae" if op == "gae_masked" else op
    for name, o, e in zip(OUTPUTS[op], outs, exp):
        assert_close(o.cpu().numpy(), e, 1e-5, suite_atol(base_op, inp, e, T), f"{what}:{name}")


@pytest.mark.parametrize("warm", [True, False], ids=["warmed", "first-call-in-capture"])
@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("shape", [(64, 512), (16, 2048), (3, 5000), (3, 5001)],
                         ids=lambda s: f"{s[0]}x{s[1]}")
def test_graph_replays_match_eager(op, shape, warm, device, monkeypatch):
    monkeypatch.delenv("RL_TRITON_CORRECTNESS_WARNINGS")  # host-side scans cannot be captured
    inp, params = _inputs(op, shape, seed=41)
    static = to_device(inp, device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    if warm:
        with torch.cuda.stream(stream):
            _call(op, static, params)
        torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = _call(op, static, params)
    torch.cuda.synchronize()
    for rep in range(4):
        new, _ = _inputs(op, shape, seed=50 + rep)
        fresh = to_device(new, device)
        for k, v in fresh.items():
            if v is not None:
                static[k].copy_(v)
        graph.replay()
        # eager work between replays: an uncaptured call of the same op and a torch reduction
        _call(op, to_device(_inputs(op, shape, seed=90 + rep)[0], device), params)
        _ = (static[next(k for k, v in static.items() if v is not None and v.is_floating_point())]
             .sum())
        torch.cuda.synchronize()
        want = run_api(op, new, params, device)
        for o, w in zip(outs, want):
            assert _same(o, w), f"{op}{shape} replay {rep}: differs from the eager call"
        _against_oracle(op, new, params, outs, shape[1], f"{op}{shape} replay {rep}")
    del graph


@pytest.mark.parametrize("op", ["gae_normalized", "gae_normalized_masked"])
def test_graph_replays_with_a_partials_tree(op, device, monkeypatch):
    """[8193, 300]: 2049 workgroups in the statistics launch, so the captured call holds a
    level of the partials' tree (reduce_partials_kernel) between it and the normalisation."""
    test_graph_replays_match_eager(op, (8193, 300), True, device, monkeypatch)
