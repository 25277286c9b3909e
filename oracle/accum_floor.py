"""Measures how far two FP32-accumulating implementations of a full-depth
step drift apart through BF16 rounding alone: c2 (Qwen2-0.5B shape, 24
layers, LoRA r=16 on q,k,v,o, B=4 x T=512) or c3 (Qwen2-1.5B shape, 28
layers, LoRA r=16 on all seven projections, B=1 x T=1024).

TEST INFRASTRUCTURE (a measurement of the oracle against itself): it runs
the CPU oracle twice on the same base, tokens and adapter state, once with
its FP64 accumulation (the exact side of every parity check) and once with
FP32 accumulators fed by 16-wide K blocks, as a tiled matrix-core GEMM
accumulates (or_set_accum_mode(1)); every BF16 rounding point of the
reference is the same in both.  The per-tensor relative L2 distance between
the two is the floor any FP32-accumulating implementation (cuBLAS included)
can be expected to sit at against the FP64 oracle, and it is what
tests/test_gpu_c2.py and tests/test_gpu_c3.py derive their bars from.  The
centroid sums (both oracles accumulate their own over the steps, as the
engine does) are measured the same way.

Same procedure as the tests: base seed and token stream seed per config
(assistant spans over almost every row), two steps, the second starting
from the FP64 side's adapter state after the first (so B != 0).

Usage: python oracle/accum_floor.py [c2|c3] [out.json]
(c2 about 20 min on 8 cores, c3 about 40 min).  Writes
tests/golden/<config>_accum_floor.json by default.
"""
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path[:0] = [HERE, os.path.join(ROOT, "tests")]

import numpy as np  # noqa: E402

import oracle as O  # noqa: E402
from step_util import base_tensors, pairs, rel, span_tokens  # noqa: E402

C2_MODEL = dict(vocab=151936, hidden=896, layers=24, n_q=14, n_kv=2, head_dim=64, inter=4864,
                rms_eps=1e-6, rope_theta=1e6, tie=1)
C2_ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b0001111, lr=1e-4, grad_clip=1.0, warmup=0,
                total_steps=20, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)
C3_MODEL = dict(vocab=151936, hidden=1536, layers=28, n_q=12, n_kv=2, head_dim=128, inter=8960,
                rms_eps=1e-6, rope_theta=1e6, tie=1)
C3_ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b1111111, lr=1e-4, grad_clip=1.0, warmup=0,
                total_steps=50, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)
# config -> (model, adapter, B, T, base seed, token seed); the tests use the same
CONFIGS = {"c2": (C2_MODEL, C2_ADAPT, 4, 512, 53, 59),
           "c3": (C3_MODEL, C3_ADAPT, 1, 1024, 79, 83)}
STATE = ("A", "B", "mA", "vA", "mB", "vB", "A16", "B16")


def measure(name="c2", steps=2):
    mc, ac, B, T, base_seed, tok_seed = CONFIGS[name]
    tens = base_tensors(mc, base_seed)
    exact, f32 = O.OracleModel(mc, ac), O.OracleModel(mc, ac)
    for n, a in tens.items():
        exact.set_weight(n, a)
        f32.set_weight(n, a)
    rng = np.random.default_rng(tok_seed)
    out = {"config": name, "B": B, "T": T, "steps": []}
    try:
        for step in range(steps):
            for l, t in pairs(mc, ac):
                for w in STATE:
                    f32.adapter(l, t, w)[:] = exact.adapter(l, t, w)
            toks = span_tokens(B, T, rng)
            inp, tgt = toks[:-1].copy(), toks[1:].copy()
            t0 = time.time()
            O.set_accum_mode(0)
            se = exact.step(inp, tgt, B, T)
            O.set_accum_mode(1)
            sf = f32.step(inp, tgt, B, T)
            O.set_accum_mode(0)
            rec = {"loss": [se["loss"], sf["loss"]], "gnorm_raw": [se["gnorm_raw"], sf["gnorm_raw"]],
                   "floor": {}}
            for l, t in pairs(mc, ac):
                for g in ("gA", "gB"):
                    if step == 0 and g == "gA":
                        continue  # B = 0 at the first step: every gA is exactly 0
                    rec["floor"][f"l{l}.{t}.{g}"] = rel(f32.adapter(l, t, g), exact.adapter(l, t, g))
            ce, we = exact.centroid()
            cf, wf = f32.centroid()
            rec["centroid"] = {"sums": rel(cf, ce), "weight": abs(wf - we) / we}
            out["steps"].append(rec)
            fl = list(rec["floor"].values())
            print(f"step {step}: {time.time() - t0:.0f}s, floor min {min(fl):.2e} "
                  f"median {np.median(fl):.2e} max {max(fl):.2e}, centroid "
                  f"{rec['centroid']['sums']:.2e}", flush=True)
    finally:
        O.set_accum_mode(0)
    return out


if __name__ == "__main__":
    name = sys.argv[1] if len(sys.argv) > 1 else "c2"
    dst = sys.argv[2] if len(sys.argv) > 2 else os.path.join(ROOT, "tests", "golden",
                                                             f"{name}_accum_floor.json")
    res = measure(name)
    with open(dst, "w") as f:
        json.dump(res, f, indent=1, sort_keys=True)
    print("wrote", dst)
