"""One small LoRA training step of the gfx950 step engine on cuda:0, checked
against the CPU oracle (the oracle is only the checker).

Model: 1 layer, hidden 256, 4 Q / 2 KV heads of 64, SwiGLU 512, vocab 2048,
LoRA r=16 on all seven projections; batch 2 x 64 tokens.  Two steps: the
first has B = 0 (gB only), the second runs the full LoRA backward.  Checks:
loss within 1e-3 relative, raw gradient norm and every gradient within
1e-2 relative L2, and that the native library (not any fallback) ran.
"""
import numpy as np

import tadapt
from step_util import make_pair, pairs, rel

MODEL = dict(vocab=2048, hidden=256, layers=1, n_q=4, n_kv=2, head_dim=64, inter=512,
             rms_eps=1e-6, rope_theta=1e6, tie=1)
ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b1111111, lr=1e-3, grad_clip=10.0, warmup=0,
             total_steps=2, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)


def run() -> None:
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("smoke: no GPU visible")
    lib = tadapt.lib()
    print("smoke: library", lib._name, lib.ta_version().decode(), flush=True)
    B, T = 2, 64
    orc, eng = make_pair(MODEL, ADAPT, B, T, seed=3)
    rng = np.random.default_rng(1)
    for step in range(2):
        # same starting adapter state on both sides for every step
        for l, t in pairs(MODEL, ADAPT):
            for which in ("A", "B", "mA", "vA", "mB", "vB", "A16", "B16"):
                eng.write_adapter(l, t, which, orc.adapter(l, t, which))
        toks = rng.integers(0, MODEL["vocab"], B * T + 1).astype(np.int32)
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        so = orc.step(inp, tgt, B, T)
        sg = eng.step(inp, tgt)
        print(f"smoke: step {step + 1} loss gpu {sg['loss']:.6f} oracle {so['loss']:.6f} "
              f"gnorm gpu {sg['gnorm_raw']:.6e} oracle {so['gnorm_raw']:.6e}", flush=True)
        assert sg["step"] == so["step"] == step + 1
        assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (sg, so)
        assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (sg, so)
        worst = 0.0
        for l, t in pairs(MODEL, ADAPT):
            for which in (("gB",) if step == 0 else ("gA", "gB")):
                r = rel(eng.adapter(l, t, which), orc.adapter(l, t, which))
                worst = max(worst, r)
                assert r <= 1e-2, (step, l, t, which, r)
        print(f"smoke: step {step + 1} worst gradient rel-L2 {worst:.3e}", flush=True)
    del eng
    print("smoke: OK", flush=True)


if __name__ == "__main__":
    run()
