"""The Qwen2-0.5B configuration (24 layers, hidden 896, 14 Q / 2 KV heads,
head_dim 64, SwiGLU 4864, tied 151936-entry embedding; LoRA r=16 alpha=32
on q,k,v,o; B=4 x T=512) at full size against the CPU oracle, over two
steps: loss within 1e-3 relative, grad norm within 1e-2, every gB (step 1)
and every gA and gB (step 2, which starts from the oracle's state after
step 1, so B != 0) within the bars below, the updated adapters within the
same bars where the update is determined (check_band), the update
exactly AdamW of the engine's own gradients, and the centroid sums (all 24
layers, accumulated over both steps) within 2x their floor.

Bars from a measured floor, not 1e-2.  tests/golden/c2_accum_floor.json
(written by oracle/accum_floor.py, same seeds and procedure as this test)
holds, per tensor, the distance between two CPU oracles that differ only in
accumulation: the FP64 one and one with FP32 accumulators fed by 16-wide K
blocks, as a matrix-core GEMM accumulates; every BF16 rounding point of the
reference is the same in both.  That distance is 0.7e-2 to 3.1e-2 (median
2.3e-2; 1.9e-3 and 1.7e-3 for the centroid sums after steps 1 and 2): with
about 90% of the BF16 values one ulp apart after a few layers,
the differences of every layer's roundings add up over the 24 layers, so no
FP32-accumulating implementation (cuBLAS included) can meet 1e-2 here.
Each engine gradient must lie within 2x its tensor's floor, and the median
over tensors of (engine distance / floor) within 1.3: a GPU-side error
beyond accumulation order would shift that median (measured on MI355X:
medians 1.05 and 1.03, largest single ratio 1.42).

The token ids are uniform with an assistant span over almost every row, so
the trainer's masking keeps the targets."""
import json
import os

import numpy as np
import pytest

from step_util import make_pair, pairs, rel, span_tokens
from test_gpu_step import check_adamw_of_own_grads, check_band, snapshot, sync_state

pytestmark = pytest.mark.gpu

C2_MODEL = dict(vocab=151936, hidden=896, layers=24, n_q=14, n_kv=2, head_dim=64, inter=4864,
                rms_eps=1e-6, rope_theta=1e6, tie=1)
C2_ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b0001111, lr=1e-4, grad_clip=1.0, warmup=0,
                total_steps=20, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)
FLOOR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c2_accum_floor.json")


def test_c2_full_model_matches_oracle():
    mc, ac, B, T = C2_MODEL, C2_ADAPT, 4, 512
    floor = json.load(open(FLOOR))["steps"]
    orc, eng = make_pair(mc, ac, B, T, seed=53)
    rng = np.random.default_rng(59)
    for step in range(2):
        sync_state(orc, eng, mc, ac)
        state = snapshot(orc, mc, ac)
        toks = span_tokens(B, T, rng)
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        so = orc.step(inp, tgt, B, T)
        sg = eng.step(inp, tgt)
        print(f"step {step}: loss {sg['loss']:.6f} oracle {so['loss']:.6f} "
              f"gnorm {sg['gnorm_raw']:.5e} / {so['gnorm_raw']:.5e}", flush=True)
        assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (step, sg, so)
        assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (step, sg, so)
        fl = floor[step]["floor"]
        ratios, bad = [], []
        for l, t in pairs(mc, ac):
            for g in (("gB",) if step == 0 else ("gA", "gB")):
                key = f"l{l}.{t}.{g}"
                r = rel(eng.adapter(l, t, g), orc.adapter(l, t, g))
                ratios.append(r / fl[key])
                if r > 2.0 * fl[key]:
                    bad.append(f"{key}: {r:.3e} > 2 x floor {fl[key]:.3e}")
        med = float(np.median(ratios))
        print(f"step {step}: engine distance / FP32-order floor: median {med:.3f}, "
              f"max {max(ratios):.3f} over {len(ratios)} tensors", flush=True)
        assert not bad, "; ".join(bad)
        assert med <= 1.3, med
        check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])
        check_band(orc, eng, mc, ac, before={k: v for k, v in state.items() if k[2] in "AB"},
                   bar=lambda l, t, g: 2.0 * fl.get(f"l{l}.{t}.{g}", 5e-3))
        ca, cw = eng.centroid()
        oa, ow = orc.centroid()
        cf = floor[step]["centroid"]
        rc = rel(ca, oa)
        print(f"step {step}: centroid sums {rc:.3e} (floor {cf['sums']:.3e}), weight "
              f"{abs(cw - ow) / ow:.3e} (floor {cf['weight']:.3e})", flush=True)
        assert rc <= 2.0 * cf["sums"], (rc, cf)
        assert abs(cw - ow) <= 2.0 * max(cf["weight"], 1e-6) * ow, (cw, ow, cf)
    eng.close()
