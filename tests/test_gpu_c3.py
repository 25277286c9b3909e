"""The headline configuration: Qwen2-1.5B shape (28 layers, hidden 1536,
12 Q / 2 KV heads, head_dim 128, SwiGLU 8960, tied 151936-entry embedding),
LoRA r=16 alpha=32 on all seven projections, B=8 x T=1024.

- One c3-shaped layer against the CPU oracle over two steps (B=1 x T=1024,
  the full vocabulary, assistant-span tokens so the targets are kept), to
  the step bars: loss 1e-3 relative, every gB (step 1) and every gA and gB
  (step 2, which starts from the oracle's state after step 1, so B != 0)
  within 1e-2 relative L2, the updated adapters within 1e-2 where the
  update is determined (check_band), and the update exactly AdamW of the
  engine's own gradients.  This runs the kernels specific to the shape:
  the chained gate/up input-gradient GEMM over K = 2 x 8960, the SwiGLU-form
  gate/up GEMM at N = 8960 and the fused SwiGLU + gate/up LoRA backward over
  8960 columns, with head_dim 128 attention.
- The whole 28-layer model at B=1 x T=1024 against the CPU oracle over two
  steps, every gradient bounded by a measured accumulation floor (below).
- The whole 28-layer step at B=8 x T=1024, checked through properties that
  hold at any size: with B = 0 at the first step every gA is exactly zero
  and every gB finite and nonzero; the logits of unit-RMS rows against
  W ~ N(0, 0.02^2) are Gaussian with variance sigma^2 = 0.02^2 * H, so the
  initial loss is ln V + sigma^2 / 2 (V >> 1; uniform ids mask every
  target, so the loss is the logsumexp); AdamW's first update of B is
  -lr * g / (|g| + eps) element by element, g the clipped gradient the
  engine holds.  The second step's loss is finite and the step count 2.
"""
import json
import math
import os

import numpy as np
import pytest

import tadapt
from step_util import make_pair, pairs, rel, span_tokens
from test_gpu_step import check_adamw_of_own_grads, check_band, compare, snapshot, sync_state

pytestmark = pytest.mark.gpu

C3_MODEL = dict(vocab=151936, hidden=1536, layers=28, n_q=12, n_kv=2, head_dim=128, inter=8960,
                rms_eps=1e-6, rope_theta=1e6, tie=1)
C3_ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b1111111, lr=1e-4, grad_clip=1.0, warmup=0,
                total_steps=50, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)


def test_c3_layer_matches_oracle():
    mc = dict(C3_MODEL, layers=1)
    ac, B, T = C3_ADAPT, 1, 1024
    orc, eng = make_pair(mc, ac, B, T, seed=61)
    rng = np.random.default_rng(67)
    for step in range(2):
        sync_state(orc, eng, mc, ac)
        state = snapshot(orc, mc, ac)
        toks = span_tokens(B, T, rng)
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        so = orc.step(inp, tgt, B, T)
        sg = eng.step(inp, tgt)
        print(f"step {step}: loss {sg['loss']:.6f} oracle {so['loss']:.6f} "
              f"gnorm {sg['gnorm_raw']:.5e} / {so['gnorm_raw']:.5e}", flush=True)
        assert sg["valid_tokens"] == so["valid_tokens"] > 0
        assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (step, sg, so)
        assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (step, sg, so)
        compare(orc, eng, mc, ac, ("gB",) if step == 0 else ("gA", "gB"))
        if step == 0:
            assert not any(np.any(eng.adapter(l, t, "gA")) for l, t in pairs(mc, ac))
        check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])
        check_band(orc, eng, mc, ac, before={k: v for k, v in state.items() if k[2] in "AB"})
    eng.close()


FLOOR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c3_accum_floor.json")


@pytest.fixture(scope="module")
def c3_depth():
    """The engine / oracle pair of the full-depth comparison, shared by its
    two step tests (each step's oracle run takes about a minute and a half
    on the GPU host, so the steps are separate tests)."""
    mc, ac, B, T = C3_MODEL, C3_ADAPT, 1, 1024
    orc, eng = make_pair(mc, ac, B, T, seed=79)
    st = {"orc": orc, "eng": eng, "rng": np.random.default_rng(83), "done": 0,
          "floor": json.load(open(FLOOR))["steps"]}
    yield st
    eng.close()


def _c3_depth_step(st, step):
    """One step of the full-depth comparison (steps run in order; a later
    step first runs the ones before it)."""
    while st["done"] < step:
        _c3_depth_step(st, st["done"])
    mc, ac, B, T = C3_MODEL, C3_ADAPT, 1, 1024
    orc, eng, fl = st["orc"], st["eng"], st["floor"][step]["floor"]
    sync_state(orc, eng, mc, ac)
    state = snapshot(orc, mc, ac)
    toks = span_tokens(B, T, st["rng"])
    inp, tgt = toks[:-1].copy(), toks[1:].copy()
    sg = eng.step(inp, tgt)
    so = orc.step(inp, tgt, B, T)
    st["done"] = step + 1
    print(f"step {step}: loss {sg['loss']:.6f} oracle {so['loss']:.6f} "
          f"gnorm {sg['gnorm_raw']:.5e} / {so['gnorm_raw']:.5e}", flush=True)
    assert sg["valid_tokens"] == so["valid_tokens"] > 0
    assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (step, sg, so)
    assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (step, sg, so)
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
    if step == 0:
        assert not any(np.any(eng.adapter(l, t, "gA")) for l, t in pairs(mc, ac))
    check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])
    # at 28 layers the gradients differ from the FP64 oracle by their
    # FP32-accumulation floor (2-6% per tensor), so the band of
    # undetermined updates is wider than at one or two layers: at step 2 up
    # to 26% of an A tensor's elements fall inside it (measured, l11.o.A)
    check_band(orc, eng, mc, ac, before={k: v for k, v in state.items() if k[2] in "AB"},
               bar=lambda l, t, g: 2.0 * fl.get(f"l{l}.{t}.{g}", 5e-3), excl=0.35)
    ca, cw = eng.centroid()
    oa, ow = orc.centroid()
    cf = st["floor"][step]["centroid"]
    rc = rel(ca, oa)
    print(f"step {step}: centroid sums {rc:.3e} (floor {cf['sums']:.3e}), weight "
          f"{abs(cw - ow) / ow:.3e} (floor {cf['weight']:.3e})", flush=True)
    assert rc <= 2.0 * cf["sums"], (rc, cf)
    assert abs(cw - ow) <= 2.0 * max(cf["weight"], 1e-6) * ow, (cw, ow, cf)


def test_c3_full_depth_step1_matches_oracle(c3_depth):
    """All 28 layers of the headline shape at B=1 x T=1024 (the full 151936
    vocabulary, r=16 on all seven projections) against the CPU oracle
    (qwen2.cu:47-308, adapter_model.cu:96-220), first step: loss within 1e-3
    relative, grad norm within 1e-2, every gB within 2x its tensor's
    accumulation floor with the median over tensors of (engine distance /
    floor) at most 1.3 (every gA exactly 0: B = 0), the updated B likewise
    where the update is determined (check_band), the update exactly AdamW
    of the engine's own gradients, and the centroid sums of all 28 layers
    within 2x their floor.

    The floor: tests/golden/c3_accum_floor.json (oracle/accum_floor.py c3,
    the same seeds and procedure) holds, per tensor, the distance between
    the FP64 oracle and one with FP32 accumulators fed by 16-wide K blocks,
    as a matrix-core GEMM accumulates, every BF16 rounding point of the
    reference kept: 0.8e-2 to 7.1e-2 (median 4.3e-2) for the gradients,
    2.1e-3 for the centroid sums.  As at c2 (tests/test_gpu_c2.py), no
    FP32-accumulating implementation meets 1e-2 through 28 layers; an
    error beyond accumulation order would move the median ratio."""
    _c3_depth_step(c3_depth, 0)


def test_c3_full_depth_step2_matches_oracle(c3_depth):
    """The second step of the full-depth comparison, from the oracle's
    state after the first (B != 0): every gA and gB within 2x its floor
    (median ratio at most 1.3), the updated A and B where determined, the
    AdamW update and the cumulative centroid sums, as in step 1."""
    _c3_depth_step(c3_depth, 1)


def test_c3_full_step_properties():
    mc, ac, B, T = C3_MODEL, C3_ADAPT, 8, 1024
    eng = tadapt.Engine(mc, ac, B, T)
    eng.init_random(71)
    rng = np.random.default_rng(73)
    toks = rng.integers(0, mc["vocab"], B * T + 1).astype(np.int32)
    m = eng.step(toks[:-1].copy(), toks[1:].copy(), lr_override=ac["lr"])
    print(f"c3 step: loss {m['loss']:.5f} gnorm {m['gnorm_raw']:.4e} {m['step_ms']:.1f} ms",
          flush=True)
    expect = math.log(mc["vocab"]) + 0.5 * 0.02 ** 2 * mc["hidden"]
    assert abs(m["loss"] - expect) <= 2e-3 * expect, (m["loss"], expect)
    assert m["valid_tokens"] == B * T and m["step"] == 1
    for l, t in pairs(mc, ac):
        gA, gB = eng.adapter(l, t, "gA"), eng.adapter(l, t, "gB")
        assert not np.any(gA), (l, t)
        assert np.all(np.isfinite(gB)) and np.any(gB), (l, t)
        b = eng.adapter(l, t, "B").astype(np.float64)
        g = gB.astype(np.float64)
        want = -ac["lr"] * g / (np.abs(g) + ac["eps"])
        np.testing.assert_allclose(b, want, rtol=1e-4, atol=1e-6 * ac["lr"])
    toks = rng.integers(0, mc["vocab"], B * T + 1).astype(np.int32)
    m2 = eng.step(toks[:-1].copy(), toks[1:].copy(), lr_override=ac["lr"])
    assert m2["step"] == 2 and math.isfinite(m2["loss"]) and math.isfinite(m2["gnorm_raw"])
    assert abs(m2["loss"] - expect) <= 2e-3 * expect
    eng.close()
