"""The Qwen2-0.5B configuration (24 layers, hidden 896, 14 Q / 2 KV heads,
head_dim 64, SwiGLU 4864, tied 151936-entry embedding; LoRA r=16 alpha=32
on q,k,v,o; B=4 x T=512) at full size against the CPU oracle, over two
steps: loss within 1e-3 relative, grad norm within 1e-2, every gB
(step 1) and every gA and gB (step 2, which starts from the oracle's state
after step 1, so B != 0) within 4e-2 relative L2, and the update exactly
AdamW of the engine's own gradients.

The per-tensor gradient bar is 4e-2 here, not 1e-2: every layer rounds its
residual stream, projections and norms to BF16, and where two
implementations sum a GEMM in different orders about half of those
roundings land one ulp apart.  Those differences add up over the 24
layers: measured 2.3e-2 to 2.8e-2 for every pair, against 4e-3 to 6e-3
for one 7B-shaped layer and under 1e-2 for the 1- and 2-layer configs,
which keep the 1e-2 bar.

The token ids are uniform with an assistant span over almost every row, so
the trainer's masking keeps the targets.  With uniform ids alone every
target is masked and the gradient is softmax(logits)/BT: loss and grad norm
then still agree (1.6e-7 and 8e-5 relative, measured) but the q/k gB of
any two BF16 pipelines sit 1.0e-2 to 1.4e-2 apart, since one-ulp BF16
differences in the logits move the probabilities by up to 0.4% and
nothing larger dominates the gradient."""
import numpy as np
import pytest

from step_util import make_pair, span_tokens
from test_gpu_step import check_adamw_of_own_grads, compare, snapshot, sync_state

pytestmark = pytest.mark.gpu

C2_MODEL = dict(vocab=151936, hidden=896, layers=24, n_q=14, n_kv=2, head_dim=64, inter=4864,
                rms_eps=1e-6, rope_theta=1e6, tie=1)
C2_ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b0001111, lr=1e-4, grad_clip=1.0, warmup=0,
                total_steps=20, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)


def test_c2_full_model_matches_oracle():
    mc, ac, B, T = C2_MODEL, C2_ADAPT, 4, 512
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
        compare(orc, eng, mc, ac, ("gB",) if step == 0 else ("gA", "gB"), bar=4e-2)
        check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])
    eng.close()
