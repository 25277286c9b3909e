"""Golden vectors (tests/golden/, written by tests/golden/golden.py).

CPU: the oracle recomputes every committed output from the committed inputs
bit for bit (the fixtures pin the oracle against drift).
GPU: the gfx950 kernels, called through the C-ABI (and the step engine for
the init, masking and step cases), reproduce the committed outputs to the
bars written in each check.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import golden as G  # noqa: E402

CASES = sorted(G.CASES)
# host-only logic (Dataset::next_batch) has no device half: it is covered by
# the oracle check below and, bit-exact against the reference's compiled
# dataset.cpp, in tests/test_host_api.py
GPU_CASES = [c for c in CASES if c != "next_batch"]


@pytest.mark.parametrize("case", CASES)
def test_oracle_reproduces_golden(case):
    params, inputs, outputs = G.load(case)
    got = G.CASES[case][1](params, inputs)
    assert set(got) == set(outputs)
    for k, want in outputs.items():
        g = np.asarray(got[k]).reshape(want.shape).astype(want.dtype)
        assert np.array_equal(g, want), f"{case}.{k}"


# ── GPU ──────────────────────────────────────────────────────────────────
def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _gemm_ok(got, want, what):
    from gpu_util import f32
    r = _rel(f32(got), f32(want))
    exact = float((np.asarray(got) == np.asarray(want)).mean())
    assert r < 4e-3 and exact > 0.9, f"{what}: rel-L2 {r:.3e}, exact {exact:.4f}"


@pytest.mark.gpu
@pytest.mark.parametrize("case", GPU_CASES)
def test_gpu_matches_golden(case):
    print(f"case: golden {case}", flush=True)
    params, x, want = G.load(case)
    globals()["_gpu_" + case](params, x, want)


def _gpu_gemm_dx(p, x, want):
    from gpu_util import P, S, call, dev, host
    H, BT, KV = G.H, G.BT, G.HKV * G.HD
    dx = dev(np.zeros((BT, H), np.uint16))
    f = ctypes.c_float
    call("ta_gemm_bf16", 0, 0, H, BT, KV, f(1.0), P(dev(x["Wk"])), H, P(dev(x["dK"])), KV, f(0.0),
         P(dx), H, S())
    call("ta_gemm_bf16", 0, 0, H, BT, KV, f(1.0), P(dev(x["Wv"])), H, P(dev(x["dV"])), KV, f(1.0),
         P(dx), H, S())
    _gemm_ok(host(dx), want["dx"], "gemm_dx")


def _gpu_lora_bwd(p, x, want):
    from gpu_util import P, S, assert_bf16_close, call, dev, f32, host
    H, BT, R, OUT, s = G.H, G.BT, G.R, G.HQ * G.HD, p["s"]
    f = ctypes.c_float
    h = dev(np.zeros((BT, R), np.uint16))
    call("ta_gemm_bf16", 1, 0, R, BT, H, f(1.0), P(dev(x["A"])), H, P(dev(x["x"])), H, f(0.0),
         P(h), R, S())
    gB = dev(np.zeros((OUT, R), np.float32))
    call("ta_gemm_f32", 0, 1, R, OUT, BT, f(s), P(dev(f32(host(h)).copy())), R,
         P(dev(f32(x["go"]).copy())), OUT, f(1.0), P(gB), R, S())
    dh = dev(np.zeros((BT, R), np.uint16))
    call("ta_gemm_bf16", 0, 0, R, BT, OUT, f(1.0), P(dev(x["B"])), R, P(dev(x["go"])), OUT,
         f(0.0), P(dh), R, S())
    gA = dev(np.zeros((R, H), np.float32))
    call("ta_gemm_f32", 0, 1, H, R, BT, f(s), P(dev(f32(x["x"]).copy())), H,
         P(dev(f32(host(dh)).copy())), R, f(1.0), P(gA), H, S())
    gx = dev(x["grad_x"])
    call("ta_gemm_bf16", 0, 0, H, BT, R, f(s), P(dev(x["A"])), H, P(dh), R, f(1.0), P(gx), H, S())
    assert_bf16_close(host(h), want["h"], what="h")
    assert_bf16_close(host(dh), want["dh"], what="dh")
    # F32 weight gradients of BF16-valued operands: accumulation order only
    assert _rel(host(gB), want["gB"]) < 1e-5
    assert _rel(host(gA), want["gA"]) < 1e-5
    assert_bf16_close(host(gx), want["grad_x"], what="grad_x")


def _gpu_rms_norm(p, x, want):
    from gpu_util import P, S, assert_bf16_close, call, dev, empty_bf16, host
    import torch
    BT, H = G.BT, G.H
    out, dx = empty_bf16(BT, H), empty_bf16(BT, H)
    rms = dev(np.zeros(BT, np.float32))
    xd, wd = dev(x["x"]), dev(x["w"])
    f = ctypes.c_float(p["eps"])
    call("ta_rms_norm_fwd", P(xd), P(wd), P(out), P(rms), 1, BT, H, f, S())
    call("ta_rms_norm_bwd", P(dev(x["dy"])), P(xd), P(wd), P(rms), P(dx), None, 1, BT, H, f, S())
    torch.cuda.synchronize()
    assert_bf16_close(host(out), want["out"], what="rms out")
    assert _rel(host(rms), want["rms"]) < 1e-6
    assert_bf16_close(host(dx), want["dx"], what="rms dx")


def _gpu_rope(p, x, want):
    from gpu_util import P, S, assert_bf16_close, call, dev, host
    BT, f = G.BT, ctypes.c_float(p["theta"])
    q, dk = dev(x["q"]), dev(x["dk"])
    call("ta_rope_fwd", P(q), 1, BT, G.HQ, G.HD, f, S())
    call("ta_rope_bwd", P(dk), 1, BT, G.HKV, G.HD, f, S())
    assert_bf16_close(host(q), want["q_rot"], what="rope fwd")
    assert_bf16_close(host(dk), want["dk_rot"], what="rope bwd")


def _gpu_sdpa(p, x, want):
    from gpu_util import P, S, assert_bf16_close, call, dev, empty_bf16, f32, host
    BT, HQ, HKV, HD = G.BT, G.HQ, G.HKV, G.HD
    Q, K, V = dev(x["Q"]), dev(x["K"]), dev(x["V"])
    o = empty_bf16(BT, HQ * HD)
    Pm = dev(np.zeros((HQ, BT, BT), np.float32))
    call("ta_sdpa_fwd", P(Q), P(K), P(V), P(o), P(Pm), 1, BT, HQ, HKV, HD, S())
    assert _rel(host(Pm), want["P"]) < 1e-5
    assert_bf16_close(host(o), want["O"], frac_exact=0.95, what="attn out")
    dQ, dK, dV = empty_bf16(BT, HQ * HD), empty_bf16(BT, HKV * HD), empty_bf16(BT, HKV * HD)
    # backward from the oracle's P, so the comparison isolates the backward
    call("ta_sdpa_bwd", P(dev(x["dO"])), P(Q), P(K), P(V), P(dev(want["P"])), P(dQ), P(dK), P(dV),
         1, BT, HQ, HKV, HD, S())
    for name, t in (("dQ", dQ), ("dK", dK), ("dV", dV)):
        r = _rel(f32(host(t)), f32(want[name]))
        assert r < 1e-2, f"{name}: rel-L2 {r:.3e}"


def _gpu_silu_mul(p, x, want):
    from gpu_util import P, S, assert_bf16_close, call, dev, empty_bf16, host
    n = x["gate"].size
    g, u = dev(x["gate"]), dev(x["up"])
    out, dg, du = empty_bf16(n), empty_bf16(n), empty_bf16(n)
    call("ta_silu_mul_fwd", P(g), P(u), P(out), n, S())
    call("ta_silu_mul_bwd", P(dev(x["dout"])), P(g), P(u), P(dg), P(du), n, S())
    assert_bf16_close(host(out), want["out"].ravel(), what="silu out")
    assert_bf16_close(host(dg), want["dgate"].ravel(), what="dgate")
    assert_bf16_close(host(du), want["dup"].ravel(), what="dup")


def _gpu_cross_entropy(p, x, want):
    from gpu_util import P, S, assert_bf16_close, call, dev, empty_bf16, host
    N, V = x["logits"].shape
    loss = dev(np.zeros(N, np.float32))
    dl = empty_bf16(N, V)
    call("ta_cross_entropy_fwd", P(dev(x["logits"])), P(dev(x["targets"])), P(loss), P(dl), N, V,
         S())
    assert np.all(np.abs(host(loss) - want["loss"]) <= 1e-5 * np.abs(want["loss"]))
    assert_bf16_close(host(dl), want["dlogits"], what="dlogits")


def _gpu_adamw(p, x, want):
    from gpu_util import P, S, call, dev, host
    import oracle as O
    m32 = dev(x["master"].copy())
    sh = dev(O.bf16_from_f32(x["master"]))
    m = dev(np.zeros_like(x["master"]))
    v = dev(np.zeros_like(x["master"]))
    n = x["master"].size
    f = ctypes.c_float
    for t in range(x["grads"].shape[0]):
        call("ta_adamw_step", P(m32), P(sh), P(m), P(v), P(dev(np.ascontiguousarray(x["grads"][t]))),
             n, f(p["lr"]), f(p["b1"]), f(p["b2"]), f(p["eps"]), f(p["wd"]), t + 1, S())
    # F32 update math; contraction may differ from the oracle in the last bit
    for name, t in (("master", m32), ("m", m), ("v", v)):
        w = want[name]
        assert np.all(np.abs(host(t) - w) <= 1e-5 * np.abs(w) + 1e-6 * np.abs(w).max()), name
    d = np.abs(host(sh).astype(np.int32) - want["working"].astype(np.int32))
    assert d.max() <= 1
    acc = dev(np.zeros(1, np.float32))
    call("ta_sum_sq_into", P(dev(np.ascontiguousarray(x["grads"][0]))), P(acc), n, S())
    assert abs(float(host(acc)[0]) - want["sum_sq"][0]) <= 1e-5 * want["sum_sq"][0]


def _gpu_centroid(p, x, want):
    from gpu_util import P, S, call, dev, host
    acc = dev(np.zeros(G.H + 1, np.float64))
    call("ta_centroid_accumulate_bf16", P(dev(x["h"])), P(dev(x["g"])), G.BT, G.H, P(acc), S())
    got = host(acc)
    assert _rel(got[:-1], want["acc"][:-1]) < 1e-5
    assert abs(got[-1] - want["acc"][-1]) <= 1e-5 * want["acc"][-1]


def _gpu_kmeans(p, x, want):
    from gpu_util import P, S, call, dev, host
    N, D = x["snaps"].shape
    k = p["k"]
    c = dev(np.zeros((k, D), np.float32))
    a = dev(np.zeros(N, np.int32))
    it = dev(np.zeros(1, np.int32))
    call("ta_kmeans_ref", P(dev(x["snaps"])), N, D, k, 50, P(c), P(a), P(it), S())
    assert np.array_equal(host(c), want["centers"])
    assert np.array_equal(host(a), want["assign"])
    assert np.array_equal(host(it), want["iters"])
    mass = dev(np.zeros(k, np.float64))
    seeds = dev(np.zeros(k, np.int32))
    call("ta_kmeans_pp", P(dev(x["snaps"])), P(dev(x["weights"])), N, D, k, p["iters"],
         ctypes.c_uint64(p["seed"]), P(c), P(a), P(mass), P(seeds), S())
    assert np.array_equal(host(c), want["pp_centers"])
    assert np.array_equal(host(a), want["pp_assign"])
    assert np.array_equal(host(seeds), want["pp_seeds"])
    assert np.allclose(host(mass), want["pp_mass"], rtol=1e-6)


def _engine(mc, ac, B, T):
    import tadapt
    return tadapt.Engine(mc, ac, B, T)


def _gpu_kaiming_init(p, x, want):
    mc = dict(vocab=1024, hidden=p["in_dim"], layers=1, n_q=14, n_kv=2, head_dim=64, inter=512,
              rms_eps=1e-6, rope_theta=1e6, tie=1)
    ac = dict(rank=p["rank"], alpha=16.0, inject_mask=0b1001, lr=1e-4, grad_clip=1.0, warmup=0,
              total_steps=1, b1=0.9, b2=0.999, eps=1e-8, wd=0.0)
    e = _engine(mc, ac, 1, 64)
    for t in ("q", "o"):  # both have in_dim = 896: the same A (fixed seed)
        assert np.array_equal(e.adapter(0, t, "A16").reshape(want["A16"].shape), want["A16"])
        assert np.array_equal(e.adapter(0, t, "A").reshape(want["A32"].shape), want["A32"])


def _gpu_mask_targets(p, x, want):
    import torch
    mc = dict(vocab=151936, hidden=256, layers=1, n_q=4, n_kv=2, head_dim=64, inter=512,
              rms_eps=1e-6, rope_theta=1e6, tie=1)
    ac = dict(rank=8, alpha=16.0, inject_mask=0b1, lr=1e-4, grad_clip=1.0, warmup=0,
              total_steps=4, b1=0.9, b2=0.999, eps=1e-8, wd=0.0)
    e = _engine(mc, ac, p["B"], p["T"])
    e.init_random(seed=5, std=0.02)
    e.step(x["inputs"], x["targets"])  # host masking
    assert np.array_equal(e.read_buffer("targets").view(np.int32), want["masked"])
    e.step_resident(torch.from_numpy(x["inputs"]).cuda(), torch.from_numpy(x["targets"]).cuda())
    torch.cuda.synchronize()  # device masking
    assert np.array_equal(e.read_buffer("targets").view(np.int32), want["masked"])


def _gpu_step(p, x, want):
    from step_util import base_tensors, pairs
    e = _engine(p["model"], p["adapt"], p["B"], p["T"])
    for name, arr in base_tensors(p["model"], p["base_seed"]).items():
        e.set_weight(name, arr)
    m = e.step(x["inputs"], x["targets"])
    loss, gnorm, lr = want["metrics"]
    assert abs(m["loss"] - loss) <= 1e-3 * abs(loss)
    assert abs(m["gnorm_raw"] - gnorm) <= 1e-2 * gnorm
    assert abs(m["lr"] - lr) <= 1e-7 * lr
    for l, t in pairs(p["model"], p["adapt"]):
        go = want[f"gB_{t}"]
        gg = e.adapter(l, t, "gB").reshape(go.shape)
        assert _rel(gg, go) <= 1e-2, t
        # A: gA = 0 at step 1, so the update is the weight decay alone
        assert _rel(e.adapter(l, t, "A").reshape(want[f"A_{t}"].shape), want[f"A_{t}"]) < 1e-6
        # B at step 1 is a sign function of gB: compare where gB is determined
        band = 4.0 * float(np.sqrt(np.mean((gg.astype(np.float64) - go) ** 2)))
        sure = np.abs(go) > band
        assert (~sure).mean() < 0.25, t
        bg = e.adapter(l, t, "B").reshape(go.shape)
        assert _rel(bg[sure], want[f"B_{t}"][sure]) <= 1e-2, t


@pytest.mark.gpu
def test_gpu_mask_targets_multichunk():
    """Device masking over rows longer than one 1024-token scan chunk, with
    an assistant header split across each chunk seam and at the row end,
    bit-exact against the oracle's sequential state machine
    (adapt_trainer.cu:145-182)."""
    import torch
    import oracle as O
    B, T = 2, 2112  # chunks of 1024, 1024, 64
    print(f"case: mask_targets multichunk B={B} T={T}", flush=True)
    rng = np.random.default_rng(11)
    vocab = np.array([151644, 77091, 151645, 5, 6, 7, 8, 9], np.int32)
    prob = np.array([0.02, 0.03, 0.02, 0.23, 0.2, 0.2, 0.15, 0.15])
    inputs = rng.choice(vocab, size=(B, T), p=prob).astype(np.int32)
    # header opening at the last token of a chunk, role token in the next
    inputs[0, 1023], inputs[0, 1024] = 151644, 77091
    inputs[0, 1025:1500] = 5
    inputs[1, 2047], inputs[1, 2048] = 151644, 77091
    inputs[1, 2049:2111] = 6
    inputs[1, T - 1] = 151644  # opening at the row end: no next token
    inputs[0, 1024 - 3:1024 - 1] = (151645, 5)
    targets = rng.integers(0, 151936, size=(B, T), dtype=np.int32)
    want = O.mask_targets(inputs.ravel(), targets.ravel(), B, T).reshape(B, T)
    assert (want >= 0).sum() > 100 and (want < 0).sum() > 100
    mc = dict(vocab=151936, hidden=256, layers=1, n_q=4, n_kv=2, head_dim=64, inter=512,
              rms_eps=1e-6, rope_theta=1e6, tie=1)
    ac = dict(rank=8, alpha=16.0, inject_mask=0b1, lr=1e-4, grad_clip=1.0, warmup=0,
              total_steps=4, b1=0.9, b2=0.999, eps=1e-8, wd=0.0)
    e = _engine(mc, ac, B, T)
    e.init_random(seed=5, std=0.02)
    e.step_resident(torch.from_numpy(inputs).cuda(), torch.from_numpy(targets).cuda())
    torch.cuda.synchronize()
    got = e.read_buffer("targets").view(np.int32).reshape(B, T)
    assert np.array_equal(got, want)
