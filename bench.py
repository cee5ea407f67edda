"""Benchmark of the rl_triton return-estimation path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--configs all|none|names]

Workload (BASELINE.json configs[1] and configs[2], the configuration the metric is
quoted on): one STEP is one compute_gae call on a GAE [4096, 128] batch (terminations
Bernoulli(0.01), truncations Bernoulli(0.005), bootstrap values at truncations and at
t = T-1) plus one compute_vtrace call on a V-trace [4096, 128] batch (log-ratios
N(0, 0.5^2), last_value, terminations Bernoulli(0.01)), both fp32, through the public
Python API.  Steps rotate over enough input sets (> 3 x 256 MB) that the Infinity Cache
cannot hold them, so every call streams its inputs from HBM.

Printed JSON (one line, stdout):
  value          whole-job Gelem/s = 2 * 4096 * 128 elements / ms_per_step
  roofline       the dominant kernel (V-trace): algorithmic bytes per launch
                 (28 B/elem: 5 reads + 2 writes) / its average launch duration, timed with
                 HIP events on the launch stream around batches of launches that the GPU
                 runs back to back (queued behind a GPU spin), vs 8 TB/s; traffic = HBM
                 bytes per launch measured by rocprofv3 counters
                 (profiles/traffic_baseline_configs.json)
  host_issue     the host clock around each public call of the timed loop: host time per
                 step and per call (first steps apart); a step cannot end on the GPU before
                 the host has issued it
  graph_replay   the same steps replayed from a captured HIP graph (no host work per call)
  ops            per-op device time, Gelem/s, GB/s and %-of-peak for both kernels
  stream_ceiling the same byte pattern streamed with no scan (librlk_stream_ceiling.so:
                 5 reads + 1 write for GAE, 5 reads + 2 writes for V-trace, one 16-byte
                 non-temporal access per array per thread, 512-thread workgroups), timed
                 the same way; kernel_frac_of_ceiling = ceiling time / kernel time;
                 vtrace_pattern_sweep: the same 5r+2w kernel at 1x-64x the headline size,
                 fitted as time = fixed_us + bytes / asymptotic_gb_s; every configuration
                 below carries that fit at its bytes (stream_fit_us, frac_of_stream_fit)
  configs        the same figures for every BASELINE configuration (C1-C5,
                 tests/baseline_configs.py), each its own rotating input sets
  extensions     compute_gae_normalized (fused GAE + returns + advantage normalisation) at
                 [4096,128] against the torch composition it replaces
  element_aligned_rows
                 C2, C3 and the C5 prefix sum one step short of a multiple of four
                 ([4096,127], [8,2^20-1]): quads that are only element-aligned
  independent_ceilings
                 the same bytes moved by torch copy_ (hipMemcpyAsync device to device: a
                 copy of half the bytes reads and writes them all) on rotating buffers, and
                 the dispatch floor: back-to-back launches of a kernel that moves 32 KB
  cpu_baseline   the reference's sequential torch loops (restated in
                 oracle/torch_loops.py) on the host CPU, bounded sample: the headline step
                 (GAE C2 + V-trace C3) with the host's thread share and with 1 thread, and
                 C1's reference_gae at [64, 512] by the reference's _bench_cpu method; CPU
                 model and thread counts recorded.  This CPU leg also checks the headline
                 outputs against the float64 oracle (parity_max_abs_err) and against those
                 float32 loops (parity_vs_reference_loops_max_abs_err), and every
                 configuration's set-0 outputs against both (configs[*].max_abs_err,
                 max_abs_err_f32_loop: the reference's float32 loop's own error)
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "rl-triton_amd"), ROOT, os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "GAE & V-trace Gelem/s + achieved HBM GB/s (% of peak) at 4096×128 fp32"
PEAK_GBS = 8000.0
E, T = 4096, 128
GAE_BYTES_PER_ELEM = 24     # rewards, values, terminateds, truncateds, bootstrap_values in; advantages out
VTRACE_BYTES_PER_ELEM = 28  # log_pi_target, log_pi_behavior, values, rewards, terminateds in; 2 out
MALL_BYTES = 256 * 2 ** 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_sets(torch, dev, n_sets):
    """Input sets: set 0 from a seeded CPU generator (checked against the oracle),
    the rest drawn with the same distributions by a seeded device generator."""
    sets = []
    for i in range(n_sets):
        if i == 0:
            g, kw = torch.Generator().manual_seed(0), {}
        else:
            g, kw = torch.Generator(device=dev).manual_seed(1000 + i), {"device": dev}
        rn = lambda *s: torch.randn(*s, generator=g, **kw)  # noqa: E731
        ru = lambda *s: torch.rand(*s, generator=g, **kw)   # noqa: E731
        term = (ru(E, T) < 0.01).float()
        trunc = (ru(E, T) < 0.005).float() * (1.0 - term)
        boot = torch.where(trunc.bool(), rn(E, T), torch.zeros_like(term))
        boot[:, -1] = rn(E)
        gae = dict(rewards=rn(E, T), values=rn(E, T), terminateds=term, truncateds=trunc,
                   bootstrap_values=boot)
        vt = dict(log_pi_target=0.5 * rn(E, T), log_pi_behavior=torch.zeros_like(term),
                  values=rn(E, T), rewards=rn(E, T), terminateds=(ru(E, T) < 0.01).float(),
                  last_value=rn(E))
        to = lambda d: {k: v.to(dev).contiguous() for k, v in d.items()}  # noqa: E731
        g, v = to(gae), to(vt)
        # the timed loop's arguments as tuples, as a training loop holds its tensors
        args = ((g["rewards"], g["values"], g["terminateds"], g["truncateds"]), g["bootstrap_values"],
                (v["log_pi_target"], v["log_pi_behavior"], v["values"], v["rewards"], v["terminateds"]),
                v["last_value"])
        sets.append((g, v, (gae, vt) if i == 0 else None, args))
    return sets


def run_gae(rl, s):
    return rl.compute_gae(s["rewards"], s["values"], s["terminateds"], s["truncateds"],
                          gamma=0.99, lambda_=0.95, bootstrap_values=s["bootstrap_values"])


def run_vtrace(rl, s):
    return rl.compute_vtrace(s["log_pi_target"], s["log_pi_behavior"], s["values"], s["rewards"],
                             s["terminateds"], gamma=0.99, rho_bar=1.0, c_bar=1.0,
                             last_value=s["last_value"])


def measured_traffic(config):
    """HBM bytes per launch of `config`'s kernel (a name of tests/baseline_configs.py) from
    the committed rocprofv3 counter passes (FETCH_SIZE and WRITE_SIZE scaled by a known-size
    copy), or None if absent."""
    path = os.path.join(ROOT, "profiles", "traffic_baseline_configs.json")
    try:
        with open(path) as f:
            return json.load(f)["traffic_bytes_per_launch"][config]
    except (OSError, KeyError, ValueError):
        return None


def parity(np, cpu_sets, outs):
    from oracle import oracle as orc
    gae, vt = cpu_sets
    n = lambda t: t.numpy()  # noqa: E731
    e_adv = orc.gae(n(gae["rewards"]), n(gae["values"]), n(gae["terminateds"]), n(gae["truncateds"]),
                    0.99, 0.95, bootstrap=n(gae["bootstrap_values"]))
    e_tg, e_ad = orc.vtrace(n(vt["log_pi_target"]), n(vt["log_pi_behavior"]), n(vt["values"]),
                            n(vt["rewards"]), n(vt["terminateds"]), None, 0.99, 1.0, 1.0,
                            bootstrap=n(vt["last_value"]))
    errs = {"gae_advantages": float(np.max(np.abs(outs[0].cpu().numpy() - e_adv))),
            "vtrace_targets": float(np.max(np.abs(outs[1][0].cpu().numpy() - e_tg))),
            "vtrace_advantages": float(np.max(np.abs(outs[1][1].cpu().numpy() - e_ad)))}
    return errs


def parity_vs_loops(torch, cpu_sets, outs):
    """Max abs difference of set 0's outputs from the reference's own float32 sequential
    loops (restated in oracle/torch_loops.py), run on the host."""
    from oracle import torch_loops
    gae, vt = cpu_sets
    adv = torch_loops.gae_loop(gae["rewards"], gae["values"], gae["terminateds"], gae["truncateds"],
                               0.99, 0.95, bootstrap_values=gae["bootstrap_values"])
    tg, ad = torch_loops.vtrace_loop(vt["log_pi_target"], vt["log_pi_behavior"], vt["values"],
                                     vt["rewards"], vt["terminateds"], 0.99, 1.0, 1.0,
                                     last_value=vt["last_value"])
    d = lambda a, b: float((a.cpu() - b).abs().max())  # noqa: E731
    return {"gae_advantages": d(outs[0], adv), "vtrace_targets": d(outs[1][0], tg),
            "vtrace_advantages": d(outs[1][1], ad)}


def config_errors(np, kept):
    """Max abs error of each configuration's set-0 outputs against the float64 oracle, and
    the error of the reference's float32 sequential loop (oracle.loop32) on the same inputs:
    the north star's bar is the former no larger than (twice) the latter."""
    from _common import OUTPUTS, run_oracle
    from oracle import oracle as orc
    import baseline_configs as bc
    res = {}
    for name, (inp, params, outs) in kept.items():
        op = bc.CONFIGS[name][0]
        n = {k: v.numpy() for k, v in inp.items()}
        exp = run_oracle(op, n, params)
        loop = orc.loop32(op, n, params)
        err = max(float(np.max(np.abs(o.numpy().astype(np.float64) - e))) for o, e in zip(outs, exp))
        err_loop = max(float(np.max(np.abs(lp.astype(np.float64) - e))) for lp, e in zip(loop, exp))
        res[name] = {"max_abs_err": err, "max_abs_err_f32_loop": err_loop,
                     "outputs": list(OUTPUTS[op])}
        log(f"[bench] {name}: max abs err {err:.3e} vs float64 (the float32 loop: {err_loop:.3e})")
    return res


def time_ops(torch, rl, sets, iters, batch=100):
    """Average device duration of each op's kernel, from HIP events on the launch stream.
    Each batch of `batch` calls is queued behind a GPU spin, so the GPU runs the kernels
    back to back; an event before the first and after the last call brackets the batch."""
    stream = torch.cuda.current_stream()
    res = {}
    for name, fn, idx in (("gae", run_gae, 0), ("vtrace", run_vtrace, 1)):
        total_ms, n = 0.0, 0
        while n < iters:
            torch.cuda._sleep(20_000_000)  # ~10 ms of GPU spin: room to queue the batch
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for i in range(batch):
                fn(rl, sets[(n + i) % len(sets)][idx])
            b.record(stream)
            torch.cuda.synchronize()
            total_ms += a.elapsed_time(b)
            n += batch
        res[name] = total_ms / n
    return res


def time_configs(torch, names, min_launches=200, batch=50, dtype=None, keep=None):
    """Average kernel duration of every BASELINE configuration's public-API call (one
    kernel launch per call), from HIP events around batches of back-to-back launches queued
    behind a GPU spin, over rotating input sets of more than 3 x 256 MB.  dtype=bfloat16:
    the same calls with bfloat16 I/O (float32 arithmetic).  keep: a dict that receives each
    configuration's first input set and outputs, on the host."""
    import baseline_configs as bc
    dtype = dtype or torch.float32
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    res = {}
    for name in names:
        op, n_env, n_t, _ = bc.CONFIGS[name]
        bpe = bc.bytes_per_elem(name, dtype)
        set_bytes = bc.set_bytes(name) * bpe // bc.CONFIGS[name][3]
        n_sets = min(64, max(2, -(-3 * MALL_BYTES // set_bytes) + 1))
        sets = [bc.make(name, seed=100 + i, device=dev) for i in range(n_sets)]
        sets = [(bc.as_dtype(inp, dtype), params) for inp, params in sets]
        for i in range(min(n_sets, 8)):
            outs = bc.call(name, *sets[i])
            if i == 0 and keep is not None:  # set 0, its outputs, for the CPU leg's parity check
                keep[name] = ({k: v.cpu() for k, v in sets[0][0].items()}, sets[0][1],
                              [o.cpu() for o in outs])
        torch.cuda.synchronize()
        total_ms, n = 0.0, 0
        while n < min_launches:
            torch.cuda._sleep(20_000_000)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for i in range(batch):
                bc.call(name, *sets[(n + i) % n_sets])
            b.record(stream)
            torch.cuda.synchronize()
            total_ms += a.elapsed_time(b)
            n += batch
        del sets
        us = 1e3 * total_ms / n
        gbs = n_env * n_t * bpe / (us * 1e-6) / 1e9
        res[name] = {"op": op, "shape": [n_env, n_t], "device_us": round(us, 3),
                     "gelem_s": round(n_env * n_t / (us * 1e-6) / 1e9, 2), "gb_s": round(gbs, 1),
                     "pct_peak": round(100 * gbs / PEAK_GBS, 2), "bytes_per_elem": bpe,
                     "target_pct": (100 * bc.TARGETS[name]) if name in bc.TARGETS else None,
                     "traffic": measured_traffic(name if dtype is torch.float32 else name + "_bf16")}
        tag = "" if dtype is torch.float32 else " bf16"
        log(f"[bench] {name}{tag}: {us:.2f} us/launch, {gbs:.0f} GB/s ({100 * gbs / PEAK_GBS:.1f}% of 8 TB/s)")
    torch.cuda.empty_cache()
    return res


def _device_us(torch, fn, sets, min_launches=200, batch=50):
    """Average device time of fn(*set) from HIP events around batches of back-to-back calls
    queued behind a GPU spin, rotating over `sets`."""
    stream = torch.cuda.current_stream()
    for i in range(min(len(sets), 8)):
        fn(*sets[i])
    torch.cuda.synchronize()
    total_ms, n = 0.0, 0
    while n < min_launches:
        torch.cuda._sleep(20_000_000)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(batch):
            fn(*sets[(n + i) % len(sets)])
        b.record(stream)
        torch.cuda.synchronize()
        total_ms += a.elapsed_time(b)
        n += batch
    return 1e3 * total_ms / n


def time_element_aligned(torch, configs, min_launches=200):
    """Three BASELINE configurations one step short of a multiple of four (T % 4 != 0), so
    that their quads are only element-aligned, beside the aligned configuration's time."""
    import baseline_configs as bc
    dev = torch.device("cuda:0")
    res = {}
    for name, (E_, T_) in (("C2_gae_4096x128", (4096, 127)), ("C3_vtrace_4096x128", (4096, 127)),
                           ("C5_prefix_sum_8x1048576", (8, (1 << 20) - 1))):
        bpe = bc.bytes_per_elem(name)
        n_sets = min(64, max(2, -(-3 * MALL_BYTES // (E_ * T_ * bpe)) + 1))
        sets = [bc.make(name, seed=200 + i, device=dev, shape=(E_, T_)) for i in range(n_sets)]
        us = _device_us(torch, lambda inp, params: bc.call(name, inp, params), sets, min_launches)
        del sets
        gbs = E_ * T_ * bpe / (us * 1e-6) / 1e9
        res[f"{name.split('_')[0]}_{bc.CONFIGS[name][0]}_{E_}x{T_}"] = {
            "shape": [E_, T_], "device_us": round(us, 3), "gb_s": round(gbs, 1),
            "pct_peak": round(100 * gbs / PEAK_GBS, 2),
            "aligned_config_us": configs[name]["device_us"] if configs and name in configs else None}
        log(f"[bench] element-aligned {name} at [{E_},{T_}]: {us:.2f} us/launch ({100 * gbs / PEAK_GBS:.1f}% of 8 TB/s)")
    torch.cuda.empty_cache()
    return res


def time_stream_ceiling(torch, sets):
    """Device time of the streaming ceiling of each headline kernel's byte pattern
    (librlk_stream_ceiling.so: the same reads and writes, one 16-byte non-temporal access
    per array per thread in 512-thread workgroups, no scan) on the same rotating input
    sets, timed like the kernels themselves."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "rl-triton_amd", "rl_triton", "librlk_stream_ceiling.so"))
    fn = lib.rlk_stream_ceiling
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                   ctypes.c_int, ctypes.c_int64, ctypes.c_void_p]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = {}
    for name, key, n_out in (("gae", 0, 1), ("vtrace", 1, 2)):
        calls, keep = [], []
        for s in sets:
            ins = [t for t in s[key].values() if t.dim() == 2]
            outs = [torch.empty(E, T, device=ins[0].device) for _ in range(n_out)]
            keep.append((ins, outs))
            calls.append(((ctypes.c_void_p * len(ins))(*[t.data_ptr() for t in ins]), len(ins),
                          (ctypes.c_void_p * n_out)(*[t.data_ptr() for t in outs]), n_out))

        def run(pin, n_in, pout, n_o):
            if fn(pin, n_in, pout, n_o, E * T, stream) != 0:
                raise RuntimeError("rlk_stream_ceiling failed")

        run(*calls[0])
        ins, outs = keep[0]
        total = sum(ins[1:], ins[0].clone())
        for k, o in enumerate(outs):
            if not torch.allclose(o, total * (k + 1), rtol=1e-6, atol=1e-5):
                raise SystemExit(f"stream ceiling kernel wrote wrong values ({name})")
        us = _device_us(torch, run, calls)
        res[name] = {"device_us": round(us, 3), "reads": len(keep[0][0]), "writes": n_out,
                     "gb_s": round(E * T * 4 * (len(keep[0][0]) + n_out) / (us * 1e-6) / 1e9, 1)}
        log(f"[bench] stream ceiling {name} ({len(keep[0][0])} reads + {n_out} writes): {us:.2f} us/launch")
        del keep, calls

    # the V-trace pattern at 1x to 64x the headline size: t = fixed + bytes / bandwidth
    sweep = {"elements": [], "device_us": []}
    dev = torch.device("cuda:0")
    for scale in (1, 4, 16, 64):
        n = E * T * scale
        n_sets = max(2, -(-3 * MALL_BYTES // (7 * 4 * n)) + 1)
        keep = [([torch.randn(n, device=dev) for _ in range(5)], [torch.empty(n, device=dev) for _ in range(2)])
                for _ in range(n_sets)]
        calls = [((ctypes.c_void_p * 5)(*[t.data_ptr() for t in i]), 5,
                  (ctypes.c_void_p * 2)(*[t.data_ptr() for t in o]), 2) for i, o in keep]

        def run_n(pin, n_in, pout, n_o, n=n):
            if fn(pin, n_in, pout, n_o, n, stream) != 0:
                raise RuntimeError("rlk_stream_ceiling failed")

        sweep["elements"].append(n)
        sweep["device_us"].append(round(_device_us(torch, run_n, calls, min_launches=100), 3))
        del keep, calls
        torch.cuda.empty_cache()
    xs = [28.0 * n for n in sweep["elements"]]
    ys = sweep["device_us"]
    mx, my = sum(xs) / len(xs), sum(ys) / len(ys)
    slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
    sweep["fixed_us"] = round(my - slope * mx, 3)
    sweep["asymptotic_gb_s"] = round(1e-3 / slope, 1)
    log(f"[bench] stream ceiling sweep (V-trace pattern): {sweep}")
    res["vtrace_pattern_sweep"] = sweep
    return res


def time_independent_ceilings(torch, ops):
    """Ceilings measured without this project's kernels, timed like the kernels (batches of
    back-to-back calls queued behind a GPU spin, rotating over more than 3 x 256 MB):
      copy_  torch's device-to-device copy (hipMemcpyAsync) of half the headline kernel's
             bytes, so that its reads plus writes equal the kernel's algorithmic bytes;
      dispatch_floor  a launch of the streaming kernel over 8192 floats (2 workgroups,
             32 KB read and written): what any kernel launch costs back to back."""
    import ctypes
    dev = torch.device("cuda:0")
    res = {}
    for name in ("gae", "vtrace"):
        nbytes = ops[name]["bytes_per_launch"]
        n = nbytes // 2 // 4
        n_sets = max(2, -(-3 * MALL_BYTES // nbytes) + 1)
        bufs = [(torch.empty(n, device=dev), torch.empty(n, device=dev)) for _ in range(n_sets)]
        for src, _ in bufs:
            src.normal_()
        us = _device_us(torch, lambda src, dst: dst.copy_(src), bufs)
        gbs = nbytes / (us * 1e-6) / 1e9
        res[f"copy_{name}_bytes"] = {"device_us": round(us, 3), "bytes_moved": nbytes,
                                     "gb_s": round(gbs, 1), "pct_peak": round(100 * gbs / PEAK_GBS, 2),
                                     "kernel_frac_of_copy": round(us / ops[name]["device_us"], 3)}
        log(f"[bench] copy_ of {nbytes / 2 / 1e6:.2f} MB (moves {nbytes / 1e6:.2f} MB, like {name}): "
            f"{us:.2f} us/call, {gbs:.0f} GB/s")
        del bufs
    lib = ctypes.CDLL(os.path.join(ROOT, "rl-triton_amd", "rl_triton", "librlk_stream_ceiling.so"))
    fn = lib.rlk_stream_ceiling
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                   ctypes.c_int, ctypes.c_int64, ctypes.c_void_p]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    small = [(torch.empty(8192, device=dev), torch.empty(8192, device=dev)) for _ in range(4)]
    calls = [((ctypes.c_void_p * 1)(a.data_ptr()), (ctypes.c_void_p * 1)(b.data_ptr())) for a, b in small]

    def tiny(pin, pout):
        if fn(pin, 1, pout, 1, 8192, stream) != 0:
            raise RuntimeError("rlk_stream_ceiling failed")

    us = _device_us(torch, tiny, calls, min_launches=400, batch=100)
    res["dispatch_floor"] = {"device_us": round(us, 3), "workgroups": 2, "bytes_moved": 2 * 8192 * 4}
    log(f"[bench] dispatch floor (2-workgroup kernel back to back): {us:.2f} us/launch")
    torch.cuda.empty_cache()
    return res


def time_extensions(torch, min_launches=200, batch=50):
    """The paths beyond the reference's API (its ROADMAP.md items), on rotating HBM-resident
    sets of more than 3 x 256 MB:
      * compute_gae_normalized (GAE + returns + batch-normalised advantages) at the C2 shape,
        against the composition it replaces: compute_gae, then returns = A + values, then
        (A - A.mean()) / (A.std() + 1e-8) in torch;
      * compute_gae(..., mask=...) (skipped steps) and compute_gae_normalized(..., mask=...)
        at the C2 shape and distribution with a multi-turn mask (alternating kept/skipped
        spans, mean length 12), and the masked GAE at [16, 131072] (C5 shape,
        done ~ Bern(1e-4), last_value)."""
    import baseline_configs as bc
    import rl_triton
    dev = torch.device("cuda:0")
    out = {}
    name = "C2_gae_4096x128"
    _, n_env, n_t, _ = bc.CONFIGS[name]
    n_sets = min(64, -(-3 * MALL_BYTES // (n_env * n_t * 4 * 7)) + 1)
    sets = [bc.make(name, seed=200 + i, device=dev) for i in range(n_sets)]

    def fused(inp, params):
        return rl_triton.compute_gae_normalized(inp["rewards"], inp["values"], inp["terminateds"],
                                                inp["truncateds"],
                                                bootstrap_values=inp["bootstrap_values"], **params)

    def composed(inp, params):
        a = rl_triton.compute_gae(inp["rewards"], inp["values"], inp["terminateds"], inp["truncateds"],
                                  bootstrap_values=inp["bootstrap_values"], **params)
        ret = a + inp["values"]
        return (a - a.mean()) / (a.std() + 1e-8), ret

    us_f = _device_us(torch, fused, sets, min_launches, batch)
    us_c = _device_us(torch, composed, sets, min_launches, batch)
    elems = n_env * n_t
    out["gae_normalized_4096x128"] = {
        "shape": [n_env, n_t], "device_us": round(us_f, 3), "torch_composition_us": round(us_c, 3),
        "speedup": round(us_c / us_f, 2),
        "bytes_per_elem": 28,  # 5 inputs read, advantages and returns written, once each
        "gb_s": round(elems * 28 / (us_f * 1e-6) / 1e9, 1)}
    log(f"[bench] gae_normalized [{n_env},{n_t}]: {us_f:.2f} us/call fused vs "
        f"{us_c:.2f} us composed in torch")

    # masked GAE: the C2 sets with a multi-turn mask; then few long rows
    from baseline_configs import span_mask
    g = torch.Generator().manual_seed(300)
    masks = [span_mask(n_env, n_t, g).to(dev) for _ in range(4)]
    msets = [(dict(inp, mask=masks[i % len(masks)]), params) for i, (inp, params) in enumerate(sets)]

    def masked(inp, params):
        return rl_triton.compute_gae(inp["rewards"], inp["values"], inp["terminateds"],
                                     inp["truncateds"], bootstrap_values=inp["bootstrap_values"],
                                     mask=inp["mask"], **params)

    def masked_norm(inp, params):
        return rl_triton.compute_gae_normalized(inp["rewards"], inp["values"], inp["terminateds"],
                                                inp["truncateds"],
                                                bootstrap_values=inp["bootstrap_values"],
                                                mask=inp["mask"], **params)

    us_mn = _device_us(torch, masked_norm, msets, min_launches, batch)
    out["gae_normalized_masked_4096x128"] = {
        "shape": [n_env, n_t], "device_us": round(us_mn, 3),
        "bytes_per_elem": 32,  # 6 inputs read, advantages and returns written, once each
        "gb_s": round(elems * 32 / (us_mn * 1e-6) / 1e9, 1)}
    log(f"[bench] gae_normalized masked [{n_env},{n_t}]: {us_mn:.2f} us/call")
    us_m = _device_us(torch, masked, msets, min_launches, batch)
    us_p = _device_us(torch, lambda inp, params: bc.call(name, inp, params), sets, min_launches, batch)
    out["gae_masked_4096x128"] = {
        "shape": [n_env, n_t], "device_us": round(us_m, 3), "unmasked_device_us": round(us_p, 3),
        "bytes_per_elem": 28,  # the C2 inputs and the mask read, advantages written
        "gb_s": round(elems * 28 / (us_m * 1e-6) / 1e9, 1),
        "pct_peak": round(100 * elems * 28 / (us_m * 1e-6) / 1e9 / PEAK_GBS, 2),
        "traffic": measured_traffic("gae_masked_4096x128")}
    log(f"[bench] gae_masked [{n_env},{n_t}]: {us_m:.2f} us/call (unmasked {us_p:.2f} us), "
        f"{elems * 28 / (us_m * 1e-6) / 1e9:.0f} GB/s")
    del sets, msets, masks

    E, T = 16, 131072
    lsets = []
    for i in range(8):  # 8 x 42 MB (+ outputs) > 3 x 256 MB with the outputs
        gi = torch.Generator(device=dev).manual_seed(400 + i)
        lsets.append(({"rewards": torch.randn(E, T, generator=gi, device=dev),
                       "values": torch.randn(E, T, generator=gi, device=dev),
                       "terminateds": (torch.rand(E, T, generator=gi, device=dev) < 1e-4).float(),
                       "last_value": torch.randn(E, generator=gi, device=dev),
                       "mask": span_mask(E, T, g).to(dev)}, {"gamma": 0.99, "lambda_": 0.95}))

    def masked_long(inp, params):
        return rl_triton.compute_gae(inp["rewards"], inp["values"], inp["terminateds"],
                                     last_value=inp["last_value"], mask=inp["mask"], **params)

    us_l = _device_us(torch, masked_long, lsets, min_launches, batch)
    gbs = E * T * 20 / (us_l * 1e-6) / 1e9
    out["gae_masked_16x131072"] = {"shape": [E, T], "device_us": round(us_l, 3),
                                   "bytes_per_elem": 20, "gb_s": round(gbs, 1),
                                   "pct_peak": round(100 * gbs / PEAK_GBS, 2),
                                   "traffic": measured_traffic("gae_masked_16x131072")}
    log(f"[bench] gae_masked [{E},{T}]: {us_l:.2f} us/call, {gbs:.0f} GB/s")
    del lsets
    torch.cuda.empty_cache()
    return out


def time_graph_steps(torch, rl, sets, steps):
    """Steps replayed from a captured HIP graph (the same API calls, captured once per input
    set): the device-bound throughput without per-call host work."""
    n = min(len(sets), steps)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(n):  # warm the allocator on the capture stream
            run_gae(rl, sets[i][0])
            run_vtrace(rl, sets[i][1])
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(n):
            run_gae(rl, sets[i][0])
            run_vtrace(rl, sets[i][1])
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // n)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (reps * n)


def time_eager_ops(torch, rl, sets, calls=2000):
    """Each headline op alone, issued eagerly back to back through the public API (the
    reference's "full-call" figure, benchmarks.md:328): HIP events around `calls` calls on
    rotating input sets, per call, host time included."""
    res = {}
    for name, fn, idx in (("gae", run_gae, 0), ("vtrace", run_vtrace, 1)):
        for i in range(50):
            fn(rl, sets[i % len(sets)][idx])
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(calls):
            fn(rl, sets[i % len(sets)][idx])
        b.record()
        torch.cuda.synchronize()
        res[name] = round(1e3 * a.elapsed_time(b) / calls, 3)
    log(f"[bench] eager calls back to back (host-inclusive): GAE {res['gae']:.2f} us/call, "
        f"V-trace {res['vtrace']:.2f} us/call")
    return res


def time_launch_paths(torch, calls=2000):
    """The launch-bound path (the reference's ROADMAP.md:125-130 graph item): C1 [64, 512]
    GAE calls issued eagerly back to back (host-inclusive time per call) against the same
    calls replayed from a captured HIP graph (device time per call); and two C5 long-row
    configurations issued eagerly back to back (host-inclusive)."""
    import baseline_configs as bc
    dev = torch.device("cuda:0")
    name = "C1_gae_64x512"
    c1 = [bc.make(name, seed=500 + i, device=dev) for i in range(8)]

    def per_call_eager():
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(calls):
            bc.call(name, *c1[i % len(c1)])
        b.record()
        torch.cuda.synchronize()
        return 1e3 * a.elapsed_time(b) / calls

    per_call_eager()  # warm
    eager_us = per_call_eager()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for st in c1:
            bc.call(name, *st)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    per_graph = 64
    with torch.cuda.graph(g, stream=side):
        for i in range(per_graph):
            bc.call(name, *c1[i % len(c1)])
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, calls // per_graph)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    graph_us = 1e3 * a.elapsed_time(b) / (reps * per_graph)
    del g
    log(f"[bench] C1 [64,512] GAE: eager {eager_us:.2f} us/call (host-inclusive), "
        f"graph replay {graph_us:.2f} us/call")

    del c1
    res = {"c1_gae_64x512": {"eager_us_per_call": round(eager_us, 3),
                             "graph_us_per_call": round(graph_us, 3)}}

    # long rows (look-back workspace) issued eagerly: host-inclusive time per call, to set
    # beside the configurations' device time
    for name in ("C5_discounted_returns_16x131072", "C5_vtrace_16x131072"):
        n_sets = max(2, -(-3 * MALL_BYTES // bc.set_bytes(name)) + 1)
        sets = [bc.make(name, seed=600 + i, device=dev) for i in range(n_sets)]
        for st in sets:
            bc.call(name, *st)
        torch.cuda.synchronize()
        n = 400
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(n):
            bc.call(name, *sets[i % n_sets])
        b.record()
        torch.cuda.synchronize()
        us = 1e3 * a.elapsed_time(b) / n
        del sets
        log(f"[bench] {name}: eager {us:.2f} us/call (host-inclusive)")
        res[name] = {"eager_us_per_call": round(us, 3)}
    torch.cuda.empty_cache()
    return res


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _host_threads():
    """The host's thread share: os.cpu_count() (the thread count the CPU baseline is
    specified at), capped at this job's CPU share (OMP_NUM_THREADS, which the GPU box sets to
    16 for one GPU)."""
    n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    return min(n, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else n


def cpu_baseline(torch, cpu_sets, budget_s):
    """The reference's sequential torch loops on the host, as oracle/torch_loops.py restates
    them.  The headline step (GAE C2 + V-trace C3 at [4096, 128]) is timed for `budget_s`
    seconds with the host's thread share (the reported value) and again with one thread;
    C1's reference_gae at [64, 512] is timed by the reference's _bench_cpu method
    (tests/bench_utils.py:184-195: 3 warm-ups, then at least 0.5 s and 5 calls, mean).
    Per-step vectors of 64-4096 floats are below ATen's 32768-element grain for intra-op
    threads, so these loops run on one core whatever the thread count."""
    from oracle import torch_loops
    import baseline_configs as bc
    gae, vt = cpu_sets
    prev = torch.get_num_threads()

    def step():
        torch_loops.gae_loop(gae["rewards"], gae["values"], gae["terminateds"], gae["truncateds"],
                             0.99, 0.95, bootstrap_values=gae["bootstrap_values"])
        torch_loops.vtrace_loop(vt["log_pi_target"], vt["log_pi_behavior"], vt["values"],
                                vt["rewards"], vt["terminateds"], 0.99, 1.0, 1.0,
                                last_value=vt["last_value"])

    def timed_steps(seconds):
        n, t0 = 0, time.perf_counter()
        while True:
            step()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                return n, el

    threads = _host_threads()
    try:
        torch.set_num_threads(threads)
        used = torch.get_num_threads()
        n, el = timed_steps(budget_s)
        torch.set_num_threads(1)
        n1, el1 = timed_steps(budget_s / 2)
        # C1: reference_gae at [64, 512], terminateds 0, last_value (tests/test_gae.py:34-60)
        c1, c1p = bc.make("C1_gae_64x512", seed=0)
        torch.set_num_threads(threads)

        def c1_call():
            torch_loops.gae_loop(c1["rewards"], c1["values"], c1["terminateds"], None,
                                 c1p["gamma"], c1p["lambda_"], last_value=c1["last_value"])

        for _ in range(3):
            c1_call()
        k, t0 = 0, time.perf_counter()
        while k < 5 or time.perf_counter() - t0 < 0.5:
            c1_call()
            k += 1
        c1_ms = 1e3 * (time.perf_counter() - t0) / k
    finally:
        torch.set_num_threads(prev)
    model = _cpu_model()
    return {"value": 2 * E * T * n / el / 1e9, "unit": "Gelem/s", "cores": used, "kind": "port",
            "sample": f"{n} full steps (GAE C2 + V-trace C3 at [{E},{T}]) in {el:.1f} s, torch CPU "
                      f"loops of oracle/torch_loops.py, torch.set_num_threads({threads}) "
                      f"(os.cpu_count() = {os.cpu_count()}, capped at the job's CPU share), "
                      f"{model}; per-step vectors are below ATen's intra-op grain, so one core works",
            "ms_per_step": 1e3 * el / n, "cpu_model": model, "os_cpu_count": os.cpu_count(),
            "torch_threads": used,
            "one_thread": {"value": 2 * E * T * n1 / el1 / 1e9, "ms_per_step": 1e3 * el1 / n1,
                           "sample": f"{n1} steps in {el1:.1f} s, torch.set_num_threads(1)"},
            "c1_reference_gae_64x512": {
                "ms_per_call": round(c1_ms, 3), "gelem_s": round(64 * 512 / (c1_ms * 1e-3) / 1e9, 5),
                "calls": k, "method": "tests/bench_utils.py:184-195 (_bench_cpu): 3 warm-ups, "
                                      ">= 0.5 s and >= 5 calls, mean",
                "reference_published_ms": {"RTX 2000 Ada box host": 14.205, "H100 box host": 16.514}}}


def host_issue(stamps, steps, ms_step):
    """Host-side view of the timed loop: `stamps` holds the host clock before each public
    call (GAE, then V-trace, per step) and after the last one.  The GPU cannot finish a step
    before the host has issued it, so when the host needs longer per step than the kernels
    (issue_us_per_step against the GPU clock's us_per_step) the loop runs at the host's
    pace."""
    calls = [1e6 * (b - a) for a, b in zip(stamps, stamps[1:])]
    gae, vt = calls[0::2], calls[1::2]

    def dist(v):
        v = sorted(v)
        q = lambda f: round(v[min(len(v) - 1, int(f * (len(v) - 1) + 0.5))], 2)  # noqa: E731
        return {"median": q(0.5), "p10": q(0.1), "p90": q(0.9), "max": round(v[-1], 2)}

    later = calls[6:] or calls
    return {"issue_us_per_step": round(1e6 * (stamps[-1] - stamps[0]) / steps, 3),
            "gpu_us_per_step": round(1e3 * ms_step, 3),
            "gae_call_us": dist(gae), "vtrace_call_us": dist(vt),
            "first_steps_call_us": [round(c, 2) for c in calls[:6]],
            "later_steps_call_us_median": dist(later)["median"],
            "note": "host clock around each public call in the timed loop (two perf_counter "
                    "reads per step, ~0.1 us); a step cannot end on the GPU before the host "
                    "has issued it"}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--configs", default="all",
                    help="comma-separated BASELINE configuration names to time beside the headline "
                         "(tests/baseline_configs.py), 'all' or 'none'")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain elementwise copy (out = in * 1.0) of MIB MiB 20 times: "
                         "the known-size reference that scales rocprofv3 FETCH_SIZE/WRITE_SIZE")
    a = ap.parse_args(argv)
    if a.copy_calibration:
        import torch
        n = a.copy_calibration * 2 ** 20 // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 20 x (read {4 * n} B + write {4 * n} B)")
        return 0
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(rows are independent and would shard along num_envs with no exchange). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import rl_triton

    dev = torch.device("cuda:0")
    set_bytes = E * T * 4 * 10
    n_sets = max(8, int(3 * MALL_BYTES / set_bytes) + 1)
    log(f"[bench] {n_sets} input sets ({n_sets * set_bytes / 2**20:.0f} MiB) on {torch.cuda.get_device_name(0)}")
    sets = make_sets(torch, dev, n_sets)
    torch.cuda.synchronize()

    # outputs of the seeded CPU-drawn set 0, checked against the float64 oracle in the CPU leg
    outs = (run_gae(rl_triton, sets[0][0]), run_vtrace(rl_triton, sets[0][1]))
    cpu_sets = sets[0][2]

    for i in range(a.warmup):
        s = sets[i % n_sets]
        run_gae(rl_triton, s[0])
        run_vtrace(rl_triton, s[1])
    torch.cuda.synchronize()

    pc = time.perf_counter

    def timed_loop(first):
        """a.steps eager steps from input set `first` on: (GPU ms per step, host clock
        before each call and after the last, wall seconds)."""
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        stamps = [0.0] * (2 * a.steps + 1)
        torch.cuda.synchronize()
        start.record()
        t0 = pc()
        # The calls of run_gae and run_vtrace, their arguments unpacked from the set's tuples
        # rather than looked up in its dicts: that took ~1.3 us per step of the loop's own
        # host-cache misses off the driver's 20-step loop (mean of four runs each in fresh
        # processes, same box: 12.6 -> 11.3 us per step).
        for i in range(a.steps):
            gae, boot, vt, last = sets[(first + i) % n_sets][3]
            stamps[2 * i] = pc()
            rl_triton.compute_gae(*gae, gamma=0.99, lambda_=0.95, bootstrap_values=boot)
            stamps[2 * i + 1] = pc()
            rl_triton.compute_vtrace(*vt, gamma=0.99, rho_bar=1.0, c_bar=1.0, last_value=last)
        stamps[-1] = pc()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / a.steps, stamps, pc() - t0

    # from the set after the warm-up's last: the least recently used
    ms_step, stamps, wall = timed_loop(a.warmup)
    value = 2 * E * T / (ms_step * 1e-3) / 1e9
    host = host_issue(stamps, a.steps, ms_step)
    log(f"[bench] timed {a.steps} steps: {ms_step * 1e3:.2f} us/step on the GPU clock, "
        f"host issue {host['issue_us_per_step']:.2f} us/step, wall {wall * 1e6:.1f} us")
    log(f"[bench] host time per call (us): GAE median {host['gae_call_us']['median']}, "
        f"V-trace median {host['vtrace_call_us']['median']}; first three steps "
        f"{host['first_steps_call_us']}; later steps median {host['later_steps_call_us_median']}")
    # Diagnostic, not the value: the same loop on the next sets after a host-only pass that
    # reads every input tensor's metadata (no GPU work).  The timed loop's tensors were built
    # long before it and not touched since, so its calls start from cold host caches; this
    # loop shows what that costs.
    touched = 0
    for st in sets:
        for d in st[:2]:
            for t in d.values():
                if t is not None:
                    touched += t.data_ptr() != 0 and t.is_contiguous()
    ms_warm, stamps_warm, _ = timed_loop(a.warmup + a.steps)
    host["warm_metadata"] = {k: v for k, v in host_issue(stamps_warm, a.steps, ms_warm).items()
                             if k in ("issue_us_per_step", "gpu_us_per_step", "gae_call_us", "vtrace_call_us")}
    host["warm_metadata"]["note"] = (f"the same loop on the next {a.steps} sets after reading the host metadata "
                                     f"of all {touched} input tensors (no GPU work); not the value")
    log(f"[bench] same loop after a host-only pass over the inputs' metadata: {ms_warm * 1e3:.2f} us/step "
        f"on the GPU clock, host issue {host['warm_metadata']['issue_us_per_step']:.2f} us/step")

    op_ms = time_ops(torch, rl_triton, sets, max(200, min(a.steps, 2000)))
    ops = {}
    for name, bpe in (("gae", GAE_BYTES_PER_ELEM), ("vtrace", VTRACE_BYTES_PER_ELEM)):
        ms = op_ms[name]
        gbs = E * T * bpe / (ms * 1e-3) / 1e9
        ops[name] = {"device_us": round(ms * 1e3, 3), "gelem_s": round(E * T / (ms * 1e-3) / 1e9, 2),
                     "gb_s": round(gbs, 1), "pct_peak": round(100 * gbs / PEAK_GBS, 2),
                     "bytes_per_elem": bpe, "bytes_per_launch": E * T * bpe}
        log(f"[bench] {name}: {ms * 1e3:.2f} us/launch, {gbs:.0f} GB/s ({100 * gbs / PEAK_GBS:.1f}% of 8 TB/s)")
    dom = max(ops, key=lambda k: ops[k]["device_us"])
    roofline = {"bound": "hbm", "kernel": dom, "achieved": ops[dom]["gb_s"], "peak": PEAK_GBS,
                "unit": "GB/s", "frac": round(ops[dom]["gb_s"] / PEAK_GBS, 4),
                "traffic": measured_traffic({"gae": "C2_gae_4096x128", "vtrace": "C3_vtrace_4096x128"}[dom]),
                "bytes_per_launch": ops[dom]["bytes_per_launch"], "duration_us": ops[dom]["device_us"],
                "duration_source": "HIP events on the launch stream around batches of 100 launches "
                                   "queued back to back behind a GPU spin, no profiler attached"}

    ceiling = time_stream_ceiling(torch, sets)
    for name in ("gae", "vtrace"):
        ceiling[name]["kernel_frac_of_ceiling"] = round(ceiling[name]["device_us"] / ops[name]["device_us"], 3)
    independent = time_independent_ceilings(torch, ops)

    graph_ms = time_graph_steps(torch, rl_triton, sets, a.steps)
    log(f"[bench] graph-replayed step: {graph_ms * 1e3:.2f} us "
        f"({2 * E * T / (graph_ms * 1e-3) / 1e9:.1f} Gelem/s)")
    launch_paths = time_launch_paths(torch)
    eager_ops = time_eager_ops(torch, rl_triton, sets)
    launch_paths["C2_gae_4096x128"] = {"eager_us_per_call": eager_ops["gae"]}
    launch_paths["C3_vtrace_4096x128"] = {"eager_us_per_call": eager_ops["vtrace"]}
    del sets
    torch.cuda.empty_cache()

    cfg_names = []
    if a.configs == "all":
        import baseline_configs
        cfg_names = list(baseline_configs.CONFIGS)
    elif a.configs != "none":
        cfg_names = a.configs.split(",")
    kept = {} if not a.no_cpu_baseline else None
    configs = time_configs(torch, cfg_names, keep=kept) if cfg_names else None
    configs_bf16 = time_configs(torch, cfg_names, dtype=torch.bfloat16) if cfg_names else None
    extensions = time_extensions(torch) if a.configs != "none" else None
    element_aligned = time_element_aligned(torch, configs) if a.configs != "none" else None
    # every configuration against the streaming fit of this run (fixed cost + bytes / rate)
    fit = ceiling["vtrace_pattern_sweep"]
    for table in (configs, configs_bf16):
        for r in (table or {}).values():
            nbytes = r["shape"][0] * r["shape"][1] * r["bytes_per_elem"]
            fit_us = fit["fixed_us"] + nbytes / (fit["asymptotic_gb_s"] * 1e3)
            r["stream_fit_us"] = round(fit_us, 3)
            r["frac_of_stream_fit"] = round(fit_us / r["device_us"], 3)

    # CPU leg: the float64 oracle checks set 0's outputs, then the reference's sequential
    # loops are timed on the host
    cpu, errs, errs_loops = None, None, None
    if not a.no_cpu_baseline:
        errs = parity(np, cpu_sets, outs)
        log(f"[bench] parity vs float64 oracle (max abs err): {errs}")
        if max(errs.values()) > 1e-4:
            raise SystemExit(f"parity check failed: {errs}")
        errs_loops = parity_vs_loops(torch, cpu_sets, outs)
        log(f"[bench] parity vs the reference's float32 loops (max abs err): {errs_loops}")
        if max(errs_loops.values()) > 1e-4:
            raise SystemExit(f"parity check failed: {errs_loops}")
        if configs and kept:
            for name, r in config_errors(np, kept).items():
                configs[name].update(max_abs_err=r["max_abs_err"],
                                     max_abs_err_f32_loop=r["max_abs_err_f32_loop"])
            del kept
        log(f"[bench] CPU baseline ({a.cpu_seconds:.0f} s sample) ...")
        cpu = cpu_baseline(torch, cpu_sets, a.cpu_seconds)
        log(f"[bench] CPU baseline: {cpu['value']:.4f} Gelem/s ({cpu['ms_per_step']:.1f} ms/step)")

    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "Gelem/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded; BASELINE.json configs[1] GAE and configs[2] V-trace distributions)",
        "config": {"workload": "GAE [4096,128] term+trunc+bootstrap_values + V-trace [4096,128] "
                               "last_value, one public-API call each per step, inputs rotated over "
                               f"{n_sets} HBM-resident sets",
                   "num_envs": E, "seq_len": T, "gamma": 0.99, "lambda": 0.95,
                   "rho_bar": 1.0, "c_bar": 1.0,
                   "timing": "value: eager public-API calls, HIP events around the timed region; "
                             "the timed steps start at the input set after the warm-up's last "
                             "(the least recently used), so no timed call reads inputs the "
                             "warm-up left in the 256 MB MALL; each step's arguments are "
                             "unpacked from the set's tuples; host_issue holds the host clock's "
                             "view of the same loop"},
        "roofline": roofline, "ops": ops, "stream_ceiling": ceiling,
        "independent_ceilings": independent, "configs": configs, "configs_bf16_io": configs_bf16,
        "extensions": extensions, "element_aligned_rows": element_aligned,
        "graph_replay": {"ms_per_step": round(graph_ms, 6),
                         "gelem_s": round(2 * E * T / (graph_ms * 1e-3) / 1e9, 3)},
        "launch_paths": launch_paths, "host_issue": host,
        "parity_max_abs_err": errs, "parity_vs_reference_loops_max_abs_err": errs_loops,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
