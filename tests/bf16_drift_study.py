"""Precision drift of bfloat16 I/O (float32 arithmetic) against the float64 oracle, across
estimators and sequence lengths.  The reference lists this study as the prerequisite of
bfloat16 support (ROADMAP.md:82-99).

    python tests/bf16_drift_study.py            (needs a GPU; prints a markdown table)

Per (op, seq_len), on seeded float32 inputs of num_envs * seq_len = 2^20 elements (2^23 for
the million-step forward scans), every error is max |x - exact| / max |exact|, with exact
the float64 oracle on the float32 inputs:
  f32 I/O       the float32 kernels
  bf16 I/O      the bfloat16 kernels (inputs rounded to bfloat16, outputs bfloat16)
  quantisation  the float64 oracle on the bfloat16-rounded inputs, its result rounded to
                bfloat16: what any bfloat16-I/O implementation must lose
The bfloat16 kernels' error over the quantisation floor shows what float32 accumulation adds.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "rl-triton_amd"))
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from _common import OUTPUTS, make_inputs, run_api, run_oracle  # noqa: E402

OPS = ["gae", "vtrace", "retrace", "lambda_returns", "discounted_returns", "eligibility_traces",
       "prefix_sum"]
LENGTHS = [128, 2048, 131072]


def rounded(inp):
    return {k: (v if v is None or k == "actions" else
                torch.as_tensor(v).to(torch.bfloat16).float().numpy()) for k, v in inp.items()}


def rel(x, exact):
    scale = float(np.max(np.abs(exact))) or 1.0
    return float(np.max(np.abs(np.asarray(x, dtype=np.float64) - exact))) / scale


def main():
    dev = torch.device("cuda:0")
    rows = []
    for op in OPS:
        lengths = LENGTHS + ([1 << 20] if op in ("prefix_sum", "eligibility_traces") else [])
        for T in lengths:
            E = max(1, (1 << (23 if T == 1 << 20 else 20)) // T)
            kw = {"p_done": 1e-4} if op in ("prefix_sum", "eligibility_traces") else {}
            boot = "full" if op in ("gae", "vtrace", "lambda_returns", "discounted_returns") else "none"
            inp, params = make_inputs(op, E, T, seed=3, p_term=0.01,
                                      p_trunc=0.005 if op != "retrace" else 0.0, boot=boot, **kw)
            exact = run_oracle(op, inp, params)
            f32 = run_api(op, inp, params, dev)
            b16 = run_api(op, inp, params, dev, dtype=torch.bfloat16)
            quant = run_oracle(op, rounded(inp), params)
            for name, e, a, b, q in zip(OUTPUTS[op], exact, f32, b16, quant):
                qb = torch.as_tensor(np.asarray(q, dtype=np.float32)).to(torch.bfloat16).float()
                rows.append((op, name, E, T, rel(a.cpu().numpy(), e), rel(b.float().cpu().numpy(), e),
                             rel(qb.numpy(), e), float(np.max(np.abs(e)))))
            print(f"done {op} T={T}", file=sys.stderr, flush=True)
    print("| op | output | num_envs x seq_len | f32 I/O | bf16 I/O | quantisation floor | bf16 / floor | max abs exact |")
    print("|---|---|---|---|---|---|---|---|")
    for op, name, E, T, a, b, q, m in rows:
        print(f"| {op} | {name} | {E} x {T} | {a:.1e} | {b:.1e} | {q:.1e} | {b / q:.2f} | {m:.3g} |")


if __name__ == "__main__":
    main()
