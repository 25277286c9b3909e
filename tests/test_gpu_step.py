"""Full LoRA training step on the GPU engine vs the CPU oracle.

Same seeded BF16 base, same tokens, same adapter init on both sides; the
engine runs its gfx950 kernels through include/ta_engine.h.  Bars (from the
north star): loss within 1e-3 relative; per-tensor gradients and updated
adapters relative L2 <= 1e-2; token masking and step counters exact.
"""
import numpy as np
import pytest

import oracle as O
import tadapt
from step_util import chat_tokens, make_pair, pairs, rel

pytestmark = pytest.mark.gpu

C1_MODEL = dict(vocab=151936, hidden=896, layers=1, n_q=14, n_kv=2, head_dim=64, inter=4864,
                rms_eps=1e-6, rope_theta=1e6, tie=1)
C1_ADAPT = dict(rank=8, alpha=16.0, inject_mask=0b0000101, lr=1e-4, grad_clip=1.0, warmup=0,
                total_steps=1, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)
SMALL_MODEL = dict(vocab=2048, hidden=256, layers=2, n_q=4, n_kv=2, head_dim=64, inter=512,
                   rms_eps=1e-6, rope_theta=1e6, tie=1)
SMALL_ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b1111111, lr=1e-3, grad_clip=1.0, warmup=1,
                   total_steps=4, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)


def compare(orc, eng, mc, ac, what, bar=1e-2):
    bad = []
    for l, t in pairs(mc, ac):
        for which in what:
            r = rel(eng.adapter(l, t, which), orc.adapter(l, t, which))
            if r > bar:
                bad.append(f"l{l}.{t}.{which}: rel-L2 {r:.3e}")
    assert not bad, "; ".join(bad)


def check_band(orc, eng, mc, ac, before=None, bar=1e-2, excl=0.25):
    """Updated adapters vs the oracle where the update is determined.

    An AdamW update m_hat/(sqrt(v_hat)+eps) is a sign function of the
    gradient wherever the moments held nothing before (B at step 1, A at the
    first step with B != 0), so an element whose gradient lies inside the
    GPU-vs-oracle gradient error band can legitimately move the other way.
    Checked per tensor: over the elements where |g_oracle| exceeds 4x the
    RMS gradient difference, the update (updated - before; before = 0 for B
    at step 1) has relative L2 <= bar (1e-2, or a per-tensor bar given as
    bar(layer, target, "gA" | "gB")) against the oracle's; as a sanity
    bound on the gradient error, fewer
    than `excl` (25%) of elements are excluded (measured on MI355X: ~1% at
    c1, 3-10% on the 2-layer config whose gradients differ from the oracle
    by up to 1e-2: one-ulp BF16 rounding differences propagate through the
    layers)."""
    for l, t in pairs(mc, ac):
        for w in ("A", "B"):
            go, gg = orc.adapter(l, t, "g" + w), eng.adapter(l, t, "g" + w)
            if not np.any(go):
                continue
            b = bar(l, t, "g" + w) if callable(bar) else bar
            band = 4.0 * float(np.sqrt(np.mean((gg.astype(np.float64) - go) ** 2)))
            sure = np.abs(go) > band
            b0 = before[(l, t, w)] if before else np.zeros_like(go)
            uo = (orc.adapter(l, t, w).astype(np.float64) - b0)[sure]
            ug = (eng.adapter(l, t, w).astype(np.float64) - b0)[sure]
            assert rel(ug, uo) <= b, (l, t, w, rel(ug, uo), b)
            assert (~sure).mean() < excl, (l, t, w, float((~sure).mean()))


def check_adamw_of_own_grads(eng, mc, ac, state, lr, t, gnorm_raw):
    """The engine's update is exactly AdamW (bias correction, weight decay;
    ops.cu:1139-1158) of its own gradients from the given starting state.
    The gradients it holds after the step are the clipped ones, as
    clip_gradients leaves gA/gB (adapt_trainer.cu:55-70), so AdamW is
    applied to them as read; when the clip fired their global norm is
    clip * raw / (raw + 1e-6)."""
    if gnorm_raw > ac["grad_clip"]:
        ss = sum(O.sum_sq(eng.adapter(l, tg, "g" + w)) for l, tg in pairs(mc, ac) for w in "AB")
        want = ac["grad_clip"] * gnorm_raw / (gnorm_raw + 1e-6)
        assert abs(np.sqrt(ss) - want) <= 1e-5 * want, (np.sqrt(ss), want)
    for l, tg in pairs(mc, ac):
        for w in ("A", "B"):
            g = eng.adapter(l, tg, "g" + w)
            p = state[(l, tg, w)].copy()
            m = state[(l, tg, "m" + w)].copy()
            v = state[(l, tg, "v" + w)].copy()
            sh = np.empty(p.size, np.uint16)
            O.adamw_step(p, sh, m, v, np.ascontiguousarray(g, np.float32), lr, ac["b1"], ac["b2"],
                         ac["eps"], ac["wd"], t)
            got = eng.adapter(l, tg, w)
            tol = 1e-5 * np.abs(p) + 1e-6 * np.abs(p).max() + 1e-12
            assert np.all(np.abs(got - p) <= tol), (l, tg, w)
            mg = eng.adapter(l, tg, "m" + w)
            assert np.all(np.abs(mg - m) <= 1e-5 * np.abs(m) + 1e-6 * np.abs(m).max() + 1e-30)


def sync_state(orc, eng, mc, ac):
    """Give the engine the oracle's adapter state (masters, shadows, moments)."""
    for l, t in pairs(mc, ac):
        for which in ("A", "B", "mA", "vA", "mB", "vB", "A16", "B16"):
            eng.write_adapter(l, t, which, orc.adapter(l, t, which))


def snapshot(orc, mc, ac):
    return {(l, t, w): orc.adapter(l, t, w).copy() for l, t in pairs(mc, ac)
            for w in ("A", "B", "mA", "vA", "mB", "vB")}


def test_c1_single_step_matches_oracle():
    mc, ac, B, T = C1_MODEL, C1_ADAPT, 1, 128
    orc, eng = make_pair(mc, ac, B, T, seed=11)
    state = snapshot(orc, mc, ac)
    rng = np.random.default_rng(5)
    toks = chat_tokens(mc["vocab"], B, T + 1, rng)[:B * T + 1]
    inp, tgt = toks[:-1].copy(), toks[1:].copy()
    so = orc.step(inp, tgt, B, T, lr_override=1e-4)
    sg = eng.step(inp, tgt, lr_override=1e-4)
    assert sg["valid_tokens"] == so["valid_tokens"] > 0
    assert sg["step"] == so["step"] == 1
    assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"])
    # the random base gives near-uniform logits: loss ~ ln V (docs/lora_training.md:11)
    assert abs(so["loss"] - np.log(mc["vocab"])) < 0.5
    assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"]
    assert so["gnorm_raw"] < ac["grad_clip"]  # no clipping: raw grads are comparable
    compare(orc, eng, mc, ac, ("gB", "mB", "vB", "A", "A16"))
    # A grads are exactly zero at step 1 (B = 0)
    assert not np.any(eng.adapter(0, "q", "gA"))
    check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], 1, sg["gnorm_raw"])
    check_band(orc, eng, mc, ac)


def test_small_all_targets_multistep_matches_oracle():
    """Three steps over all seven targets, cosine schedule with warmup.  Before
    each step the engine receives the oracle's adapter state, so every step
    is compared from the same starting point (steps 2-3 have B != 0: the full
    LoRA backward runs)."""
    mc, ac, B, T = SMALL_MODEL, SMALL_ADAPT, 2, 64
    orc, eng = make_pair(mc, ac, B, T, seed=23)
    rng = np.random.default_rng(9)
    for step in range(3):
        sync_state(orc, eng, mc, ac)
        state = snapshot(orc, mc, ac)
        toks = rng.integers(0, mc["vocab"], B * T + 1).astype(np.int32)
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        so = orc.step(inp, tgt, B, T)
        sg = eng.step(inp, tgt)
        assert sg["step"] == so["step"] == step + 1
        assert abs(sg["lr"] - so["lr"]) <= 1e-7 * so["lr"]
        assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (step, sg, so)
        assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (step, sg, so)
        compare(orc, eng, mc, ac, ("gB",) if step == 0 else ("gA", "gB"))
        check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])
        check_band(orc, eng, mc, ac, before={k: v for k, v in state.items() if k[2] in "AB"})
    ca, cw = eng.centroid()
    oa, ow = orc.centroid()
    assert rel(ca, oa) < 1e-2 and abs(cw - ow) <= 1e-2 * ow


def test_small_clipped_steps_match_oracle():
    """grad_clip far below the gradient norm, so clip_gradients fires on both
    steps (adapt_trainer.cu:55-70).  The engine's gA/gB after a step are the
    clipped gradients, as the reference leaves them, and are compared with
    the oracle's clipped ones; the reported norm is min(norm, clip)
    (adapt_trainer.cu:250).  Step 2 starts from the oracle's state after
    step 1 (B != 0)."""
    mc, ac, B, T = SMALL_MODEL, dict(SMALL_ADAPT, grad_clip=1e-3), 2, 64
    orc, eng = make_pair(mc, ac, B, T, seed=27)
    rng = np.random.default_rng(19)
    for step in range(2):
        sync_state(orc, eng, mc, ac)
        state = snapshot(orc, mc, ac)
        toks = rng.integers(0, mc["vocab"], B * T + 1).astype(np.int32)
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        so = orc.step(inp, tgt, B, T)
        sg = eng.step(inp, tgt)
        assert so["gnorm_raw"] > 10 * ac["grad_clip"] and sg["gnorm_raw"] > 10 * ac["grad_clip"]
        assert sg["gnorm"] == so["gnorm"] == np.float32(ac["grad_clip"])
        assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (step, sg, so)
        assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (step, sg, so)
        compare(orc, eng, mc, ac, ("gB",) if step == 0 else ("gA", "gB"))
        check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])
        check_band(orc, eng, mc, ac, before={k: v for k, v in state.items() if k[2] in "AB"})


def test_small_long_batch_matches_oracle():
    """B*T = 1024 tokens: the fused SwiGLU backward + gate/up LoRA backward
    splits the tokens over two blocks (512 each) and the intermediate width
    over two column splits, so both of its partial reductions (dh over
    columns, gB over tokens) run with more than one term.  Step 2 starts
    from the oracle's state after step 1 (B != 0, so dh and gA are
    nonzero)."""
    mc, ac, B, T = SMALL_MODEL, SMALL_ADAPT, 2, 512
    orc, eng = make_pair(mc, ac, B, T, seed=31)
    rng = np.random.default_rng(13)
    for step in range(2):
        sync_state(orc, eng, mc, ac)
        state = snapshot(orc, mc, ac)
        toks = rng.integers(0, mc["vocab"], B * T + 1).astype(np.int32)
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        so = orc.step(inp, tgt, B, T)
        sg = eng.step(inp, tgt)
        assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (step, sg, so)
        assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (step, sg, so)
        compare(orc, eng, mc, ac, ("gB",) if step == 0 else ("gA", "gB"))
        check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])


@pytest.mark.parametrize("rank,mask", [(4, 0b1111111), (2, 0b0001111), (24, 0b1111111)])
def test_small_rank_not_multiple_of_16_matches_oracle(rank, mask):
    """Ranks the kernels do not take directly: the engine lays every adapter
    out at the rank rounded up to a multiple of 16, with the extra rows of A
    and columns of B zero (AdapterConfig::for_base picks rank 2 or 4 for
    bases under 800M parameters, adapter_config.cpp:53-127).  gA, gB, the
    moments and the updated masters match the oracle's rank-r adapter over
    two steps (step 2 from the oracle's state, B != 0), and the scale is
    alpha / r of the real rank.

    The updated adapters are compared at 2e-2 (check_band) instead of 1e-2:
    at rank 2 (alpha 4) the q/k gA sit at about AdamW's eps (1e-8), where
    the first update g / (|g| + eps) of A is no longer a sign function and
    carries the gradient's own relative error, weighted toward the smallest
    elements (the FP64 CPU oracle and an FP32-accumulating one differ by
    6.1e-3 in layer 0's k gA and by 6.1e-3 in its update).  The update is checked exactly against
    AdamW of the engine's own gradients in any case."""
    mc, B, T = SMALL_MODEL, 2, 64
    ac = dict(SMALL_ADAPT, rank=rank, alpha=2.0 * rank, inject_mask=mask)
    orc, eng = make_pair(mc, ac, B, T, seed=53 + rank)
    rng = np.random.default_rng(rank)
    for step in range(2):
        sync_state(orc, eng, mc, ac)
        state = snapshot(orc, mc, ac)
        toks = rng.integers(0, mc["vocab"], B * T + 1).astype(np.int32)
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        so = orc.step(inp, tgt, B, T)
        sg = eng.step(inp, tgt)
        assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (step, sg, so)
        assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (step, sg, so)
        compare(orc, eng, mc, ac, ("gB",) if step == 0 else ("gA", "gB"))
        check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])
        check_band(orc, eng, mc, ac, before={k: v for k, v in state.items() if k[2] in "AB"},
                   bar=2e-2)
    # the A init of a fresh engine is the reference's hash over the real rows
    fresh = tadapt.Engine(mc, ac, B, T)
    orc2 = O.OracleModel(mc, ac)
    for l, t in pairs(mc, ac):
        assert np.array_equal(fresh.adapter(l, t, "A16"), orc2.adapter(l, t, "A16")), (l, t)
        assert not np.any(fresh.adapter(l, t, "B"))
    fresh.close()


MID_MODEL = dict(vocab=2048, hidden=1024, layers=1, n_q=8, n_kv=2, head_dim=128, inter=3328,
                 rms_eps=1e-6, rope_theta=1e6, tie=1)


def test_mid_pipe_gemm_paths_match_oracle():
    """Sizes that take the large-GEMM kernel (M, N >= 1024) with its fused
    LoRA epilogues: the gate/up projections as one N-concatenated launch,
    the q/o/lm-head projections and the down-projection input gradient with
    rank-16 terms in the epilogue, split-K for the long-K products; and the
    fused SwiGLU backward with a partly filled last column block (3328 =
    6.5 x 512).  Step 2 starts from the oracle's state after step 1."""
    mc, ac, B, T = MID_MODEL, SMALL_ADAPT, 1, 1024
    orc, eng = make_pair(mc, ac, B, T, seed=41)
    rng = np.random.default_rng(17)
    for step in range(2):
        sync_state(orc, eng, mc, ac)
        state = snapshot(orc, mc, ac)
        toks = rng.integers(0, mc["vocab"], B * T + 1).astype(np.int32)
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        so = orc.step(inp, tgt, B, T)
        sg = eng.step(inp, tgt)
        assert abs(sg["loss"] - so["loss"]) <= 1e-3 * abs(so["loss"]), (step, sg, so)
        assert abs(sg["gnorm_raw"] - so["gnorm_raw"]) <= 1e-2 * so["gnorm_raw"], (step, sg, so)
        compare(orc, eng, mc, ac, ("gB",) if step == 0 else ("gA", "gB"))
        check_adamw_of_own_grads(eng, mc, ac, state, sg["lr"], step + 1, sg["gnorm_raw"])


def test_resident_step_rejects_out_of_range_ids():
    """Token ids resident in device memory are checked on the device (the
    host-buffer entry checks them on the host): an id outside [0, V) is
    never used as an index, the step returns an error and leaves the adapter
    state, step count and centroid sums as they were; the next valid batch
    then steps exactly as the host-buffer entry does."""
    import torch
    mc, ac, B, T = SMALL_MODEL, SMALL_ADAPT, 2, 64
    e_res, e_host = tadapt.Engine(mc, ac, B, T), tadapt.Engine(mc, ac, B, T)
    e_res.init_random(7)
    e_host.init_random(7)
    rng = np.random.default_rng(3)
    toks = rng.integers(0, mc["vocab"], B * T + 1).astype(np.int32)
    inp, tgt = toks[:-1].copy(), toks[1:].copy()
    bad = inp.copy()
    bad[5], bad[B * T - 2] = mc["vocab"] + 7, -3
    d_tgt = torch.from_numpy(tgt).cuda()
    before = {w: e_res.adapter(0, "q", w).copy() for w in ("A", "B", "mA", "A16")}
    c_before = e_res.centroid()[0].copy()
    with pytest.raises(tadapt.BackendError, match="outside"):
        e_res.step_resident(torch.from_numpy(bad).cuda(), d_tgt)
    for w, v in before.items():
        assert np.array_equal(e_res.adapter(0, "q", w), v), w
    assert np.array_equal(e_res.centroid()[0], c_before)
    m_res = e_res.step_resident(torch.from_numpy(inp).cuda(), d_tgt)
    m_host = e_host.step(inp, tgt)
    assert m_res["step"] == m_host["step"] == 1
    assert m_res["loss"] == m_host["loss"] and m_res["gnorm_raw"] == m_host["gnorm_raw"]
    for l, t in pairs(mc, ac):
        for w in ("A", "B", "gA", "gB"):
            assert np.array_equal(e_res.adapter(l, t, w), e_host.adapter(l, t, w)), (l, t, w)
    e_res.close()
    e_host.close()


def test_first_step_counts_nonfinite_logits():
    """The reference checks the logits of its first step for NaN and Inf and
    warns (adapt_trainer.cu:76-91,196-198).  Two embedding rows (the tied LM
    head's weights for two ids the batch never feeds in) carry a NaN each,
    so every row's logit for those ids is NaN: the first step reports
    exactly 2 * BT; a clean engine reports 0; later steps do not count (-1)."""
    mc, ac, B, T = SMALL_MODEL, SMALL_ADAPT, 2, 64
    rng = np.random.default_rng(29)
    toks = rng.integers(0, 1000, B * T + 1).astype(np.int32)
    inp, tgt = toks[:-1].copy(), toks[1:].copy()
    from step_util import base_tensors
    t = base_tensors(mc, 31)
    clean = tadapt.Engine(mc, ac, B, T)
    for n, a in t.items():
        clean.set_weight(n, a)
    assert clean.step(inp, tgt)["nonfinite_logits"] == 0
    assert clean.step(inp, tgt)["nonfinite_logits"] == -1
    clean.close()
    emb = t["model.embed_tokens.weight"].copy()
    emb[1500, 7] = 0x7fc0  # NaN
    emb[2000, 100] = 0xffc0  # NaN, sign set
    t["model.embed_tokens.weight"] = emb
    eng = tadapt.Engine(mc, ac, B, T)
    for n, a in t.items():
        eng.set_weight(n, a)
    m = eng.step(inp, tgt)
    assert m["nonfinite_logits"] == 2 * B * T, m
    assert eng.step(inp, tgt)["nonfinite_logits"] == -1
    eng.close()


def test_ce_in_dx_step_bit_identical():
    """TA_ENGINE_CE_IN_DX (the cross-entropy gradient formed inside the LM
    head's input-gradient GEMM from the logits and each row's normaliser,
    instead of a dlogits pass; ops.cu:958-1020, qwen2.cu:205) forms the same
    dlogits bits as the cross-entropy kernel and runs the same GEMM tiles in
    the same order, so at the headline shape (one c3 layer, B=8 x T=1024,
    the full 151936 vocabulary) two steps agree bit for bit with the default
    engine: loss, norm, the LM head's dX (dres), every gradient and every
    updated adapter."""
    mc = dict(vocab=151936, hidden=1536, layers=1, n_q=12, n_kv=2, head_dim=128, inter=8960,
              rms_eps=1e-6, rope_theta=1e6, tie=1)
    ac = dict(SMALL_ADAPT, total_steps=10)
    B, T = 8, 1024
    a, b = tadapt.Engine(mc, ac, B, T), tadapt.Engine(mc, ac, B, T, ce_in_dx=True)
    a.init_random(43)
    b.init_random(43)
    rng = np.random.default_rng(41)
    for step in range(2):
        toks = chat_tokens(mc["vocab"], B, T + 1, rng)[:B * T + 1]
        inp, tgt = toks[:-1].copy(), toks[1:].copy()
        ma, mb = a.step(inp, tgt), b.step(inp, tgt)
        assert ma["loss"] == mb["loss"] and ma["gnorm_raw"] == mb["gnorm_raw"], (ma, mb)
        assert np.array_equal(a.read_buffer("dres"), b.read_buffer("dres")), step
        for l, tg in pairs(mc, ac):
            for w in ("gA", "gB", "A", "B", "A16", "B16"):
                assert np.array_equal(a.adapter(l, tg, w), b.adapter(l, tg, w)), (step, l, tg, w)
    a.close()
    b.close()
