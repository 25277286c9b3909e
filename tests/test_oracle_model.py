"""Pins for the oracle's whole training step and centroid/k-means functions.

The step oracle (Qwen2 forward, CE, hand-written backward through every op,
LoRA gradients) is checked against torch float64 autograd of an
independently written Qwen2+LoRA forward (library routines: F.linear,
F.rms_norm, softmax, F.silu, logsumexp).  A dropped backward term, wrong
beta-accumulation or wrong cached tensor shows up as an O(1) gradient error;
BF16 rounding along the chain stays at the percent level.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O

TARGETS = O.TARGETS


def tiny_cfg(**kw):
    mc = dict(vocab=300, hidden=64, layers=2, n_q=4, n_kv=2, head_dim=16, inter=96,
              rms_eps=1e-6, rope_theta=10000.0, tie=1)
    ac = dict(rank=4, alpha=8.0, inject_mask=127, lr=1e-3, grad_clip=1e9, warmup=0,
              total_steps=10, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)
    mc.update(kw.get("mc", {}))
    ac.update(kw.get("ac", {}))
    return mc, ac


def make_weights(mc, rng, std=0.05):
    H, I, V = mc["hidden"], mc["inter"], mc["vocab"]
    qd, kvd = mc["n_q"] * mc["head_dim"], mc["n_kv"] * mc["head_dim"]
    W = {"model.embed_tokens.weight": (V, H), "model.norm.weight": None}
    for l in range(mc["layers"]):
        p = f"model.layers.{l}."
        W.update({p + "input_layernorm.weight": None, p + "post_attention_layernorm.weight": None,
                  p + "self_attn.q_proj.weight": (qd, H), p + "self_attn.q_proj.bias": (qd,),
                  p + "self_attn.k_proj.weight": (kvd, H), p + "self_attn.k_proj.bias": (kvd,),
                  p + "self_attn.v_proj.weight": (kvd, H), p + "self_attn.v_proj.bias": (kvd,),
                  p + "self_attn.o_proj.weight": (H, qd), p + "mlp.gate_proj.weight": (I, H),
                  p + "mlp.up_proj.weight": (I, H), p + "mlp.down_proj.weight": (H, I)})
    out = {}
    for k, shp in W.items():
        if shp is None:  # norm weights around 1
            out[k] = O.bf16_from_f32((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
        else:
            out[k] = O.bf16_from_f32((std * rng.standard_normal(shp)).astype(np.float32))
    return out


def torch_step_grads(mc, ac, W, AB, inp, tgt, B, T):
    """float64 autograd reference: per-token loss and d(loss_sum/N)/d{A,B}."""
    H, Hq, Hkv, hd, V = mc["hidden"], mc["n_q"], mc["n_kv"], mc["head_dim"], mc["vocab"]
    eps, theta = mc["rms_eps"], mc["rope_theta"]
    s = ac["alpha"] / ac["rank"]
    t = lambda k: torch.from_numpy(O.f32_from_bf16(W[k]).astype(np.float64))
    params = {}
    for (l, tg), (A, Bm) in AB.items():
        params[(l, tg)] = (torch.from_numpy(A.astype(np.float64)).requires_grad_(True),
                           torch.from_numpy(Bm.astype(np.float64)).requires_grad_(True))

    def lin(x, w, l, tg, b=None):
        y = F.linear(x, w, b)
        if (l, tg) in params:
            A, Bm = params[(l, tg)]
            y = y + s * ((x @ A.T) @ Bm.T)
        return y

    def rope(x, nh):  # x [B,T,nh*hd], interleaved pairs, complex rotation
        xc = x.view(B, T, nh, hd // 2, 2)
        z = torch.complex(xc[..., 0], xc[..., 1])
        i = np.arange(hd // 2)
        freq = np.float32(theta) ** (np.float32(-2.0) * i.astype(np.float32) / np.float32(hd))
        ang = (np.arange(T, dtype=np.float32)[:, None] * freq[None, :]).astype(np.float64)
        rot = torch.polar(torch.ones(T, hd // 2, dtype=torch.float64), torch.from_numpy(ang))
        z = z * rot[None, :, None, :]
        return torch.stack([z.real, z.imag], -1).view(B, T, nh * hd)

    emb = t("model.embed_tokens.weight")
    x = emb[torch.from_numpy(inp.astype(np.int64))].view(B, T, H)
    mask = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
    for l in range(mc["layers"]):
        p = f"model.layers.{l}."
        xn = F.rms_norm(x, (H,), t(p + "input_layernorm.weight"), eps)
        q = lin(xn, t(p + "self_attn.q_proj.weight"), l, "q", t(p + "self_attn.q_proj.bias"))
        k = lin(xn, t(p + "self_attn.k_proj.weight"), l, "k", t(p + "self_attn.k_proj.bias"))
        v = lin(xn, t(p + "self_attn.v_proj.weight"), l, "v", t(p + "self_attn.v_proj.bias"))
        q, k = rope(q, Hq), rope(k, Hkv)
        qh = q.view(B, T, Hq, hd).transpose(1, 2)
        kh = k.view(B, T, Hkv, hd).transpose(1, 2).repeat_interleave(Hq // Hkv, 1)
        vh = v.view(B, T, Hkv, hd).transpose(1, 2).repeat_interleave(Hq // Hkv, 1)
        sc = (qh @ kh.transpose(-1, -2)) / math.sqrt(hd)
        pr = torch.softmax(sc.masked_fill(mask, float("-inf")), -1)
        ao = (pr @ vh).transpose(1, 2).reshape(B, T, Hq * hd)
        x = x + lin(ao, t(p + "self_attn.o_proj.weight"), l, "o")
        xn2 = F.rms_norm(x, (H,), t(p + "post_attention_layernorm.weight"), eps)
        g = lin(xn2, t(p + "mlp.gate_proj.weight"), l, "gate")
        u = lin(xn2, t(p + "mlp.up_proj.weight"), l, "up")
        x = x + lin(F.silu(g) * u, t(p + "mlp.down_proj.weight"), l, "down")
    xf = F.rms_norm(x, (H,), t("model.norm.weight"), eps)
    logits = (xf @ emb.T).view(B * T, V)
    lse = torch.logsumexp(logits, -1)
    tg = torch.from_numpy(tgt.astype(np.int64))
    picked = torch.where(tg >= 0, logits.gather(1, tg.clamp(min=0)[:, None])[:, 0],
                         torch.zeros_like(lse))
    loss_tok = lse - picked
    grads = torch.autograd.grad(loss_tok.sum() / (B * T),
                                [w for pair in params.values() for w in pair])
    out = {}
    for i, key in enumerate(params):
        out[key] = (grads[2 * i].numpy(), grads[2 * i + 1].numpy())
    return loss_tok.detach().numpy(), out


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.parametrize("inject", [127, 1 | 4, 15])
def test_model_step_grads_vs_torch_autograd(inject):
    rng = np.random.default_rng(7)
    # real vocab size so the assistant-span tokens exist and some targets train
    mc, ac = tiny_cfg(mc={"vocab": 151936}, ac={"inject_mask": inject})
    W = make_weights(mc, rng)
    m = O.OracleModel(mc, ac)
    for k, v in W.items():
        m.set_weight(k, v)
    # give B (and A) non-trivial values so every gradient path is exercised
    AB = {}
    for l in range(mc["layers"]):
        for ti, tg in enumerate(TARGETS):
            if not inject & (1 << ti):
                assert m.adapter(l, tg, "A") is None
                continue
            A = m.adapter(l, tg, "A")
            Bm = m.adapter(l, tg, "B")
            Bm[:] = (0.2 * rng.standard_normal(Bm.size)).astype(np.float32)
            m.adapter(l, tg, "B16")[:] = O.bf16_from_f32(Bm)
            AB[(l, tg)] = (O.f32_from_bf16(m.adapter(l, tg, "A16")).reshape(ac["rank"], -1).copy(),
                           O.f32_from_bf16(m.adapter(l, tg, "B16")).reshape(-1, ac["rank"]).copy())
    B, T = 2, 12
    inp = rng.integers(0, mc["vocab"], B * T).astype(np.int32)
    tgt = rng.integers(0, mc["vocab"], B * T).astype(np.int32)
    # open an assistant span in row 0 so some targets are trained
    inp[2], inp[3], inp[8] = 151644, 77091, 151645
    masked = O.mask_targets(inp, tgt, B, T)
    assert 0 < np.count_nonzero(masked >= 0) < B * T
    m.keep_taps(True)
    out = m.step(inp, tgt, B, T)
    loss_ref, g_ref = torch_step_grads(mc, ac, W, AB, inp, masked, B, T)
    loss_or = m.tap("loss_tok")
    assert rel_l2(loss_or, loss_ref) < 1e-3
    valid = loss_ref[loss_ref > 1e-9]
    assert math.isclose(out["loss"], valid.mean(), rel_tol=1e-3)
    worst = 0.0
    for (l, tg), (gA, gB) in g_ref.items():
        eA = rel_l2(m.adapter(l, tg, "gA").reshape(gA.shape), gA)
        eB = rel_l2(m.adapter(l, tg, "gB").reshape(gB.shape), gB)
        worst = max(worst, eA, eB)
    assert worst < 5e-2, worst


def test_model_step_B0_gives_gA0_and_sign_update():
    rng = np.random.default_rng(3)
    mc, ac = tiny_cfg(ac={"inject_mask": 1 | 4, "lr": 1e-4, "wd": 0.01})
    W = make_weights(mc, rng, std=0.02)
    m = O.OracleModel(mc, ac)
    for k, v in W.items():
        m.set_weight(k, v)
    A0 = m.adapter(0, "q", "A").copy()
    B, T = 1, 16
    inp = rng.integers(0, mc["vocab"], B * T).astype(np.int32)
    out = m.step(inp, np.roll(inp, -1), B, T)
    # uniform random tokens: every target masked; loss is the mean log-sum-exp ~ ln V
    assert abs(out["loss"] - math.log(mc["vocab"])) < 0.05
    gA = m.adapter(0, "q", "gA")
    gB = m.adapter(0, "q", "gB")
    assert np.all(gA == 0) and np.any(gB != 0)
    # step 1 AdamW: A only decays; B = -lr * g/(|g|+eps)
    assert np.allclose(m.adapter(0, "q", "A"), A0 * (1 - 1e-4 * 0.01), rtol=1e-6)
    Bn = m.adapter(0, "q", "B")
    expect = -1e-4 * gB / (np.abs(gB) + 1e-8)
    assert np.allclose(Bn, expect, rtol=1e-5, atol=1e-12)
    assert m.adapter(0, "k", "A") is None


def test_grad_clip_and_report():
    rng = np.random.default_rng(5)
    mc, ac = tiny_cfg(ac={"grad_clip": 1e-6})
    W = make_weights(mc, rng)
    m = O.OracleModel(mc, ac)
    for k, v in W.items():
        m.set_weight(k, v)
    for l in range(mc["layers"]):
        for tg in TARGETS:
            Bm = m.adapter(l, tg, "B")
            Bm[:] = 0.1
            m.adapter(l, tg, "B16")[:] = O.bf16_from_f32(Bm)
    inp = rng.integers(0, mc["vocab"], 16).astype(np.int32)
    out = m.step(inp, inp, 1, 16)
    assert out["gnorm_raw"] > 1e-6 and out["gnorm"] == np.float32(1e-6)
    total = sum(O.sum_sq(m.adapter(l, tg, g)) for l in range(2) for tg in TARGETS for g in ("gA", "gB"))
    scale = 1e-6 / (out["gnorm_raw"] + 1e-6)
    assert math.isclose(math.sqrt(total), out["gnorm_raw"] * scale, rel_tol=1e-4)


def test_step_lr_schedule_and_counter():
    rng = np.random.default_rng(9)
    mc, ac = tiny_cfg(ac={"lr": 2e-4, "warmup": 3, "total_steps": 10})
    W = make_weights(mc, rng)
    m = O.OracleModel(mc, ac)
    for k, v in W.items():
        m.set_weight(k, v)
    inp = rng.integers(0, mc["vocab"], 8).astype(np.int32)
    lrs = [m.step(inp, inp, 1, 8)["lr"] for _ in range(4)]
    assert np.allclose(lrs, [2e-4 / 3, 4e-4 / 3, 2e-4, 2e-4], rtol=1e-6)


# ── centroid accumulate ──────────────────────────────────────
def test_centroid_equal_norms_is_mean():
    rng = np.random.default_rng(11)
    h = rng.standard_normal((1000, 64)).astype(np.float32)
    g = np.zeros((1000, 64), np.float32)
    g[:, 0] = 3.0
    acc, w = O.centroid_accumulate(h, g)
    assert math.isclose(w, 3000.0)
    assert np.allclose(acc / w, h.astype(np.float64).mean(0), rtol=1e-12, atol=1e-14)


def test_centroid_vs_numpy():
    rng = np.random.default_rng(12)
    h = rng.standard_normal((5000, 96)).astype(np.float32)
    g = rng.standard_normal((5000, 96)).astype(np.float32)
    acc, w, n = O.centroid_accumulate(h, g, want_norms=True)
    nn = np.linalg.norm(g.astype(np.float64), axis=1)
    assert np.allclose(n, nn, rtol=1e-13)
    assert np.allclose(acc, h.astype(np.float64).T @ nn, rtol=1e-11)
    assert math.isclose(w, nn.sum(), rel_tol=1e-12)
    acc2, w2 = O.centroid_accumulate_n(h, nn.astype(np.float32))
    assert np.allclose(acc2, h.astype(np.float64).T @ nn.astype(np.float32), rtol=1e-11)


# ── k-means, reference mode ──────────────────────────────────
def test_kmeans_ref_separated_clusters():
    rng = np.random.default_rng(13)
    means = np.array([[0, 0], [10, 0], [0, 10]], np.float32)
    lab = np.repeat(np.arange(3), 5)
    snaps = (means[lab] + 0.1 * rng.standard_normal((15, 2))).astype(np.float32)
    C, asg, it = O.kmeans_ref(snaps, 3)
    # init picks snapshots 0, 5, 10 = one per cluster => exact recovery in one pass
    assert np.array_equal(asg, lab)
    for c in range(3):
        assert np.allclose(C[c], snaps[lab == c].mean(0), rtol=1e-6)
    assert it == 1  # converged: second pass changed nothing


def test_kmeans_ref_empty_cluster_becomes_zero():
    a = np.array([1.0, 2.0], np.float32)
    b = np.array([3.0, 2.0], np.float32)
    c = np.array([3.5, 2.0], np.float32)
    snaps = np.stack([a, a, b, c])
    C, asg, it = O.kmeans_ref(snaps, 3)
    # init centers = s[(i*4)//3] = s[0], s[1], s[2] = a, a, b.
    # pass 1: a ties between centers 0 and 1 -> 0 (strict '<'); b, c -> 2 (changed).
    # update: center 0 = a, center 1 empty -> zero vector, center 2 = (b+c)/2.
    # pass 2: nothing changes -> stop after one update.
    assert np.array_equal(asg, [0, 0, 2, 2])
    assert np.allclose(C[0], a) and np.all(C[1] == 0) and np.allclose(C[2], [3.25, 2.0])
    assert it == 1
    # k larger than N clamps
    C2, _, _ = O.kmeans_ref(snaps, 9)
    assert C2.shape == (4, 2)


def test_kmeans_ref_first_pass_all_zero_stops_without_update():
    # assignments start at 0 (centroid_accumulator.cpp:125); if the first pass
    # assigns everything to center 0 nothing "changed" and the init is returned
    a = np.array([1.0, 2.0], np.float32)
    b = np.array([3.0, 2.0], np.float32)
    snaps = np.stack([a, a, a, b])
    C, asg, it = O.kmeans_ref(snaps, 3)
    assert np.array_equal(asg, [0, 0, 0, 0]) and it == 0
    assert np.all(C == a)


# ── k-means, c5 stress mode ──────────────────────────────────
def test_kmeans_pp_recovers_mixture_and_ranks_by_mass():
    rng = np.random.default_rng(17)
    K, D, N = 6, 32, 300
    means = rng.standard_normal((K, D)).astype(np.float32) * 4
    lab = rng.integers(0, K, N)
    snaps = (means[lab] + 0.1 * rng.standard_normal((N, D))).astype(np.float32)
    w = rng.lognormal(0, 1, N).astype(np.float32)
    C, asg, mass, seeds = O.kmeans_pp(snaps, w, K, 25, 1234)
    # each found cluster is pure and every component is found
    for c in range(K):
        assert len(set(lab[asg == c])) == 1
    assert len(set(lab[asg == c] [0] for c in range(K))) == K
    assert np.all(np.diff(mass) <= 0)
    assert math.isclose(mass.sum(), w.astype(np.float64).sum(), rel_tol=1e-12)
    for c in range(K):
        assert np.allclose(C[c], snaps[asg == c].mean(0), rtol=1e-5, atol=1e-6)
    assert len(set(seeds.tolist())) == K
