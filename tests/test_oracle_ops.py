"""Pins for the CPU oracle's per-op functions.

Each check comes from outside the oracle's own formula: torch float64
autograd (library routines), numpy float64 matmul, complex-number rotation,
closed forms and invariants.  Tolerances account for the reference's BF16
rounding points (BF16 has an 8-bit significand: relative step 2^-8).
"""
import math

import numpy as np
import pytest
import torch

import oracle as O

RNG = np.random.default_rng(1234)
BF = 2.0 ** -8  # one BF16 ulp, relative


def rand_bf16(*shape, scale=1.0, rng=RNG):
    return O.bf16_from_f32(rng.standard_normal(shape).astype(np.float32) * scale)


def f(x):
    return O.f32_from_bf16(x).astype(np.float64)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


# ── BF16 conversion vs torch's RNE cast ──────────────────────
def test_bf16_rne_matches_torch():
    x = np.concatenate([
        RNG.standard_normal(100000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, 65504.0, 3.3895314e38, 1e-40, -1e-40,
                  np.inf, -np.inf], np.float32),
        # exact ties: RNE must go to even
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    ours = O.bf16_from_f32(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    back = O.f32_from_bf16(ours)
    assert np.array_equal(back, torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_bf16_nan_kept():
    x = np.array([np.nan, -np.nan], np.float32)
    assert np.all(np.isnan(O.f32_from_bf16(O.bf16_from_f32(x))))


# ── GEMM: cuBLAS column-major semantics vs numpy float64 ─────
@pytest.mark.parametrize("tA,tB", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_bf16_column_major(tA, tB):
    M, N, K = 37, 29, 53
    lda = (K if tA else M) + 3
    ldb = (N if tB else K) + 2
    ldc = M + 5
    # column-major storage: element (r, c) of a matrix with leading dim ld is at r + c*ld
    A = rand_bf16((M if tA else K) * lda)
    B = rand_bf16((K if tB else N) * ldb)
    C = rand_bf16(N * ldc)
    C0 = C.copy()
    alpha, beta = 0.75, 1.0
    assert O.gemm_bf16(tA, tB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc) == 0
    Af, Bf, Cf = f(A), f(B), f(C0)
    if tA:  # stored as K x M col-major (ld = lda): opA = stored^T
        As = Af[:M * lda].reshape(M, lda)[:, :K]   # row i (of op) = column i of stored
    else:
        As = Af[:K * lda].reshape(K, lda)[:, :M].T
    if tB:
        Bs = Bf[:K * ldb].reshape(K, ldb)[:, :N]
    else:
        Bs = Bf[:N * ldb].reshape(N, ldb)[:, :K].T
    ref = alpha * (As @ Bs) + beta * Cf[:N * ldc].reshape(N, ldc)[:, :M].T
    got = f(C)[:N * ldc].reshape(N, ldc)[:, :M].T
    ref_bf = f(O.bf16_from_f32(ref.astype(np.float32)))
    # identical except where the f32 value straddles a BF16 rounding boundary
    mismatch = np.mean(got != ref_bf)
    assert mismatch < 0.01
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-3)) < 2 * BF
    # padding columns untouched
    pad = f(C)[:N * ldc].reshape(N, ldc)[:, M:]
    assert np.array_equal(pad, f(C0)[:N * ldc].reshape(N, ldc)[:, M:])


def test_gemm_validation():
    a = np.zeros(4, np.uint16)
    assert O.gemm_bf16(0, 0, 0, 1, 1, 1.0, a, 1, a, 1, 0.0, a, 1) == -1
    assert O.gemm_bf16(0, 0, 1, 1, 1, 1.0, a, 0, a, 1, 0.0, a, 1) == -1


def test_gemm_f32_vs_numpy():
    M, N, K = 16, 40, 300
    A = RNG.standard_normal((K, M)).astype(np.float32)  # col-major M x K with lda=M  <=> row-major K x M
    B = RNG.standard_normal((K, N)).astype(np.float32)  # opB(k,j) = B[j + k*ldb] with transB, ldb=N
    C = RNG.standard_normal((N, M)).astype(np.float32)
    C0 = C.copy()
    assert O.gemm_f32(0, 1, M, N, K, 2.0, A, M, B, N, 1.0, C, M) == 0
    ref = 2.0 * (A.astype(np.float64).T @ B.astype(np.float64)) + C0.T
    assert rel_l2(C.T, ref) < 1e-6


def test_fp32_accumulation_mode_matches_blocked_float32_sums():
    """The oracle's measurement mode (FP32 accumulators fed by 16-wide K
    blocks, oracle/accum_floor.py) against a numpy restatement: each block's
    products (exact in float32 for BF16-valued operands) summed in k order
    in float32 (cumsum is sequential), then added to the float32 running
    sum.  Bit for bit; the default FP64 mode is restored afterwards and
    differs from it by accumulation rounding only."""
    M, N, K = 5, 7, 70  # K not a multiple of 16: a short last block
    A = O.f32_from_bf16(O.bf16_from_f32(RNG.standard_normal((K, M)).astype(np.float32)))
    B = O.f32_from_bf16(O.bf16_from_f32(RNG.standard_normal((K, N)).astype(np.float32)))
    A, B = np.ascontiguousarray(A), np.ascontiguousarray(B)
    want = np.empty((N, M), np.float32)
    for i in range(M):
        for j in range(N):
            acc = np.float32(0)
            for k0 in range(0, K, 16):
                prod = (A[k0:k0 + 16, i] * B[k0:k0 + 16, j]).astype(np.float32)
                acc = np.float32(acc + np.cumsum(prod, dtype=np.float32)[-1])
            want[j, i] = acc
    C32 = np.zeros((N, M), np.float32)
    C64 = np.zeros((N, M), np.float32)
    try:
        O.set_accum_mode(1)
        assert O.gemm_f32(0, 1, M, N, K, 1.0, A, M, B, N, 0.0, C32, M) == 0
    finally:
        O.set_accum_mode(0)
    assert O.gemm_f32(0, 1, M, N, K, 1.0, A, M, B, N, 0.0, C64, M) == 0
    np.testing.assert_array_equal(C32.view(np.uint32), want.view(np.uint32))
    exact = (A.astype(np.float64).T @ B.astype(np.float64)).T
    assert np.max(np.abs(C64 - exact)) <= 1e-6 * np.abs(exact).max()
    assert 0 < np.max(np.abs(C32 - exact)) <= 1e-5 * np.abs(exact).max()


def test_c2_accumulation_floor_fixture():
    """tests/golden/c2_accum_floor.json (oracle/accum_floor.py): every gB of
    step 1 and every gA and gB of step 2 of c2's 24 x 4 pairs, each floor a
    positive distance well below the loss-level scale, the losses of the two
    accumulations within 1e-4 of each other (measured 1.9e-5 and 3.4e-6)."""
    import json
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "c2_accum_floor.json")
    f = json.load(open(path))
    assert [len(s["floor"]) for s in f["steps"]] == [96, 192]
    for s in f["steps"]:
        v = np.array(list(s["floor"].values()))
        assert np.all(v > 1e-3) and np.all(v < 0.1)
        a, b = s["loss"]
        assert abs(a - b) <= 1e-4 * abs(a)


# ── RMSNorm ──────────────────────────────────────────────────
def test_rms_norm_fwd_vs_torch():
    rows, D, eps = 64, 896, 1e-6
    x = rand_bf16(rows, D)
    w = rand_bf16(D, scale=0.5)
    out, inv = O.rms_norm_fwd(x, w, eps)
    xt = torch.from_numpy(f(x))
    ref_inv = torch.rsqrt(xt.pow(2).mean(-1) + eps)
    assert np.allclose(inv, ref_inv.numpy(), rtol=1e-6)
    ref = torch.nn.functional.rms_norm(xt, (D,), torch.from_numpy(f(w)), eps)
    assert rel_l2(f(out), ref.numpy()) < BF


def test_rms_norm_constant_row_closed_form():
    D, eps, c = 128, 1e-6, 0.375
    x = O.bf16_from_f32(np.full((3, D), c, np.float32))
    w = O.bf16_from_f32(np.linspace(-2, 2, D).astype(np.float32))
    out, inv = O.rms_norm_fwd(x, w, eps)
    expect = f(w) * c / math.sqrt(c * c + eps)
    assert np.allclose(f(out[1]), expect, rtol=BF, atol=1e-6)


def test_rms_norm_bwd_vs_torch_autograd():
    rows, D, eps = 48, 256, 1e-6
    x = rand_bf16(rows, D)
    w = rand_bf16(D, scale=0.5)
    dy = rand_bf16(rows, D)
    _, inv = O.rms_norm_fwd(x, w, eps)
    dx, dw = O.rms_norm_bwd(dy, x, w, inv, want_dw=True)
    xt = torch.from_numpy(f(x)).requires_grad_(True)
    wt = torch.from_numpy(f(w)).requires_grad_(True)
    y = torch.nn.functional.rms_norm(xt, (D,), wt, eps)
    gx, gw = torch.autograd.grad(y, (xt, wt), torch.from_numpy(f(dy)))
    assert rel_l2(f(dx), gx.numpy()) < 2 * BF
    assert rel_l2(dw, gw.numpy()) < 1e-5


def test_rms_norm_bwd_orthogonal_when_w_is_one():
    rows, D = 16, 512
    x = rand_bf16(rows, D)
    w = O.bf16_from_f32(np.ones(D, np.float32))
    dy = rand_bf16(rows, D)
    _, inv = O.rms_norm_fwd(x, w, 1e-6)
    dx = O.rms_norm_bwd(dy, x, w, inv)
    # d/dx of a scale-invariant function is orthogonal to x
    dots = np.sum(f(dx) * f(x), axis=1) / (np.linalg.norm(f(dx), axis=1) * np.linalg.norm(f(x), axis=1))
    assert np.max(np.abs(dots)) < 1e-2


# ── RoPE: interleaved pairs as complex rotation ──────────────
def rope_complex(x, B, T, H, hd, theta, inverse):
    xf = f(x).reshape(B, T, H, hd // 2, 2)
    z = xf[..., 0] + 1j * xf[..., 1]
    i = np.arange(hd // 2)
    freq = np.float32(theta) ** (np.float32(-2.0) * i.astype(np.float32) / np.float32(hd))
    ang = np.arange(T, dtype=np.float32)[:, None] * freq.astype(np.float32)[None, :]
    ang = ang.astype(np.float64) * (-1 if inverse else 1)
    z = z * np.exp(1j * ang)[None, :, None, :]
    return np.stack([z.real, z.imag], -1).reshape(B * T, H * hd)


@pytest.mark.parametrize("theta", [1e4, 1e6])
def test_rope_vs_complex_rotation(theta):
    B, T, H, hd = 2, 64, 3, 64
    x = rand_bf16(B * T, H * hd)
    y = O.rope(x, B, T, H, hd, theta, 0)
    ref = rope_complex(x, B, T, H, hd, theta, False)
    assert rel_l2(f(y), ref) < BF
    # t = 0 rows are unchanged
    assert np.array_equal(y.reshape(B, T, -1)[:, 0], x.reshape(B, T, -1)[:, 0])
    # pair norms preserved
    n0 = np.hypot(f(x)[:, 0::2], f(x)[:, 1::2])
    n1 = np.hypot(f(y)[:, 0::2], f(y)[:, 1::2])
    assert np.allclose(n0, n1, rtol=4 * BF, atol=1e-6)
    # inverse undoes forward up to bf16 rounding
    z = O.rope(y, B, T, H, hd, theta, 1)
    assert rel_l2(f(z), f(x)) < 2 * BF


def test_rope_hd2_closed_form():
    B, T, H, hd = 1, 5, 1, 2
    x = O.bf16_from_f32(np.tile(np.array([[1.0, 0.0]], np.float32), (T, 1)))
    y = f(O.rope(x, B, T, H, hd, 10000.0, 0))
    t = np.arange(T)
    assert np.allclose(y[:, 0], np.cos(t), atol=BF)
    assert np.allclose(y[:, 1], np.sin(t), atol=BF)


# ── attention (saved-P semantics) vs torch float64 ───────────
def torch_attn(Q, K, V, B, T, Hq, Hkv, hd):
    q = torch.from_numpy(f(Q)).view(B, T, Hq, hd).transpose(1, 2)
    k = torch.from_numpy(f(K)).view(B, T, Hkv, hd).transpose(1, 2)
    v = torch.from_numpy(f(V)).view(B, T, Hkv, hd).transpose(1, 2)
    return q, k, v


@pytest.mark.parametrize("Hq,Hkv", [(6, 2), (7, 1)])
def test_sdpa_fwd_vs_torch(Hq, Hkv):
    B, T, hd = 2, 40, 32
    Q, K, V = rand_bf16(B * T, Hq * hd), rand_bf16(B * T, Hkv * hd), rand_bf16(B * T, Hkv * hd)
    out, P = O.sdpa_fwd(Q, K, V, B, T, Hq, Hkv, hd)
    q, k, v = torch_attn(Q, K, V, B, T, Hq, Hkv, hd)
    rep = Hq // Hkv
    k = k.repeat_interleave(rep, 1)
    v = v.repeat_interleave(rep, 1)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(hd)
    mask = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
    p = torch.softmax(s.masked_fill(mask, float("-inf")), -1)
    o = (p @ v).transpose(1, 2).reshape(B * T, Hq * hd)
    assert np.allclose(P, p.numpy(), atol=1e-6)
    assert np.all(P[:, :, np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]] == 0)
    assert rel_l2(f(out), o.numpy()) < BF


def test_sdpa_equal_scores_uniform_rows():
    B, T, Hq, Hkv, hd = 1, 12, 2, 1, 16
    Q = O.bf16_from_f32(np.zeros((B * T, Hq * hd), np.float32))
    K = rand_bf16(B * T, Hkv * hd)
    V = rand_bf16(B * T, Hkv * hd)
    _, P = O.sdpa_fwd(Q, K, V, B, T, Hq, Hkv, hd)
    for tq in range(T):
        assert np.allclose(P[0, :, tq, :tq + 1], 1.0 / (tq + 1), rtol=1e-6)


@pytest.mark.parametrize("Hq,Hkv,T", [(6, 2, 24), (7, 1, 17)])
def test_sdpa_bwd_vs_torch_autograd(Hq, Hkv, T):
    B, hd = 2, 32
    Q, K, V = rand_bf16(B * T, Hq * hd), rand_bf16(B * T, Hkv * hd), rand_bf16(B * T, Hkv * hd)
    dO = rand_bf16(B * T, Hq * hd)
    _, P = O.sdpa_fwd(Q, K, V, B, T, Hq, Hkv, hd)
    dQ, dK, dV = O.sdpa_bwd(dO, Q, K, V, P, B, T, Hq, Hkv, hd)
    q, k, v = torch_attn(Q, K, V, B, T, Hq, Hkv, hd)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    rep = Hq // Hkv
    s = (q @ k.repeat_interleave(rep, 1).transpose(-1, -2)) / math.sqrt(hd)
    mask = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
    p = torch.softmax(s.masked_fill(mask, float("-inf")), -1)
    o = p @ v.repeat_interleave(rep, 1)
    g = torch.from_numpy(f(dO)).view(B, T, Hq, hd).transpose(1, 2)
    gq, gk, gv = torch.autograd.grad(o, (q, k, v), g)
    gq = gq.transpose(1, 2).reshape(B * T, -1).numpy()
    gk = gk.transpose(1, 2).reshape(B * T, -1).numpy()
    gv = gv.transpose(1, 2).reshape(B * T, -1).numpy()
    assert rel_l2(f(dQ), gq) < 2 * BF
    assert rel_l2(f(dK), gk) < 2 * BF
    assert rel_l2(f(dV), gv) < 2 * BF


def test_sdpa_bwd_T1_closed_form():
    B, T, Hq, Hkv, hd = 3, 1, 4, 2, 16
    Q, K, V = rand_bf16(B, Hq * hd), rand_bf16(B, Hkv * hd), rand_bf16(B, Hkv * hd)
    dO = rand_bf16(B, Hq * hd)
    _, P = O.sdpa_fwd(Q, K, V, B, T, Hq, Hkv, hd)
    assert np.all(P == 1.0)
    dQ, dK, dV = O.sdpa_bwd(dO, Q, K, V, P, B, T, Hq, Hkv, hd)
    assert np.all(f(dQ) == 0) and np.all(f(dK) == 0)
    grp = f(dO).reshape(B, Hkv, Hq // Hkv, hd).sum(2).reshape(B, -1)
    assert rel_l2(f(dV), grp) < BF


# ── SwiGLU ───────────────────────────────────────────────────
def test_silu_mul_vs_torch():
    n = 5000
    g, u, do = rand_bf16(n, scale=3), rand_bf16(n), rand_bf16(n)
    out = O.silu_mul_fwd(g, u)
    dg, du = O.silu_mul_bwd(do, g, u)
    gt = torch.from_numpy(f(g)).requires_grad_(True)
    ut = torch.from_numpy(f(u)).requires_grad_(True)
    y = torch.nn.functional.silu(gt) * ut
    rg, ru = torch.autograd.grad(y, (gt, ut), torch.from_numpy(f(do)))
    assert rel_l2(f(out), y.detach().numpy()) < BF
    assert rel_l2(f(dg), rg.numpy()) < BF
    assert rel_l2(f(du), ru.numpy()) < BF


def test_silu_bwd_at_zero_gate():
    n = 64
    g = np.zeros(n, np.uint16)
    u, do = rand_bf16(n), rand_bf16(n)
    dg, du = O.silu_mul_bwd(do, g, u)
    assert np.allclose(f(dg), f(do) * f(u) / 2, rtol=BF)
    assert np.all(f(du) == 0)


# ── cross entropy ────────────────────────────────────────────
def test_cross_entropy_vs_torch():
    N, V = 12, 3001
    L = rand_bf16(N, V, scale=2)
    tgt = RNG.integers(0, V, N).astype(np.int32)
    tgt[::3] = -1
    loss, dl = O.cross_entropy(L, tgt)
    Lt = torch.from_numpy(f(L)).requires_grad_(True)
    lse = torch.logsumexp(Lt, -1)
    picked = torch.where(torch.from_numpy(tgt) >= 0,
                         Lt.gather(1, torch.from_numpy(np.maximum(tgt, 0)).long()[:, None])[:, 0],
                         torch.zeros(N, dtype=torch.float64))
    lt = lse - picked
    (g,) = torch.autograd.grad(lt.sum() / N, Lt)
    assert np.allclose(loss, lt.detach().numpy(), rtol=1e-5)
    assert rel_l2(f(dl), g.numpy()) < BF


def test_cross_entropy_zero_logits_closed_form():
    N, V = 4, 151936
    L = np.zeros((N, V), np.uint16)
    tgt = np.array([-1, 5, 0, -1], np.int32)
    loss, dl = O.cross_entropy(L, tgt)
    assert np.allclose(loss, math.log(V), rtol=1e-5)
    assert abs(math.log(V) - 11.93121) < 1e-4
    pv = 1.0 / V / N
    assert np.allclose(f(dl[0]), pv, rtol=BF)
    assert np.isclose(f(dl[1, 5]), (1.0 / V - 1) / N, rtol=BF)


# ── small elementwise ops ────────────────────────────────────
def test_embed_bias_adds():
    V, D = 50, 24
    table = rand_bf16(V, D)
    tok = RNG.integers(0, V, 9).astype(np.int32)
    assert np.array_equal(O.embed_fwd(table, tok), table[tok])
    x, b, d = rand_bf16(9, D), rand_bf16(D), rand_bf16(9, D)
    assert np.array_equal(O.add_bias(x, b), O.bf16_from_f32((f(x) + f(b)).astype(np.float32)))
    assert np.array_equal(O.add_inplace(x, d), O.bf16_from_f32((f(x) + f(d)).astype(np.float32)))
    assert np.array_equal(O.lora_add(x, d, 2.0), O.bf16_from_f32((f(x) + 2 * f(d)).astype(np.float32)))


# ── AdamW vs torch.optim.AdamW (float64) ─────────────────────
def test_adamw_vs_torch_multistep():
    n = 1000
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.01
    p0 = RNG.standard_normal(n).astype(np.float32)
    master, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    work = np.zeros(n, np.uint16)
    pt = torch.from_numpy(p0.astype(np.float64)).requires_grad_(True)
    opt = torch.optim.AdamW([pt], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    for step in range(1, 6):
        g = RNG.standard_normal(n).astype(np.float32)
        O.adamw_step(master, work, m, v, g, lr, b1, b2, eps, wd, step)
        pt.grad = torch.from_numpy(g.astype(np.float64))
        opt.step()
        assert np.allclose(master, pt.detach().numpy(), rtol=1e-5, atol=1e-7)
    assert np.array_equal(work, O.bf16_from_f32(master))


def test_adamw_step1_closed_form():
    n = 64
    lr, wd, eps = 1e-4, 0.01, 1e-8
    p = RNG.standard_normal(n).astype(np.float32)
    g = RNG.standard_normal(n).astype(np.float32)
    g[::7] = 0
    master = p.copy()
    O.adamw_step(master, np.zeros(n, np.uint16), np.zeros(n, np.float32), np.zeros(n, np.float32),
                 g, lr, 0.9, 0.999, eps, wd, 1)
    expect = p.astype(np.float64) - lr * (g / (np.abs(g) + eps) + wd * p)
    assert np.allclose(master, expect, rtol=1e-5, atol=1e-9)


def test_sum_sq():
    g = RNG.standard_normal(10007).astype(np.float32)
    assert math.isclose(O.sum_sq(g), float(np.dot(g.astype(np.float64), g)), rel_tol=1e-12)


# ── LoRA A init hash (adapter_model.cu:15-39) ────────────────
def test_kaiming_init_hash_known_answers():
    """A-init hash of adapter_model.cu:15-39 (seed 0x1234, in_dim 96, rank 4),
    element by element, against values worked out by hand from its steps:

        r = seed ^ (i * 2654435761)   (32-bit)
        r ^= r >> 16;  r *= 0x45d9f3b (32-bit);  r ^= r >> 16
        u = (float)(r & 0xFFFFFF) / (float)0xFFFFFF * 2 - 1   (F32 ops)
        A = u * sqrtf(1 / (float)in_dim)

    i = 0:  r = 0x1234;  0x1234 ^ 0 = 0x1234;  0x1234 * 0x45d9f3b
            = 4660 * 73244475 = 341319253500 = 79 * 2^32 + 2016837116
            -> 0x78367dfc;  ^ 0x7836 -> 0x783605ca;  low 24 bits 0x3605ca
            = 3540426;  u = 3540426 / 16777215 * 2 - 1 = -0.57794833
            (F32 0xbf13f46c);  sqrtf(1/96) = 0.10206207 (0x3dd105ec);
            A = 0xbd719bf1.
    The other rows follow the same steps (i * 2654435761 mod 2^32 in the
    first column).  A wrong multiplier, shift or mask changes every one."""
    table = [  # i, i*2654435761 mod 2^32, r after xor-shift, after multiply, final r, A (F32 bits)
        (0, 0x00000000, 0x00001234, 0x78367dfc, 0x783605ca, 0xbd719bf1),
        (1, 0x9e3779b1, 0x9e37f5b2, 0x42292e06, 0x42296c2f, 0xbd8d615d),
        (2, 0x3c6ef362, 0x3c6edd38, 0x064ac3e8, 0x064ac5a2, 0xbd2dd786),
        (95, 0xb69628af, 0xb6968c0d, 0xaa6759ff, 0xaa67f398, 0xbc9d1577),
        (383, 0xb4ff0fcf, 0xb4ffa904, 0xf7596fec, 0xf75998b5, 0xbcfad9ba),
    ]
    a16, a32 = O.kaiming_init(96, 4)
    bits = a32.ravel().view(np.uint32)
    for i, prod, r1, r2, r3, want in table:
        # the table's own arithmetic, so a typo in it cannot pass silently
        assert prod == (i * 2654435761) & 0xFFFFFFFF
        assert r1 == (0x1234 ^ prod) ^ ((0x1234 ^ prod) >> 16)
        assert r2 == (r1 * 0x45D9F3B) & 0xFFFFFFFF and r3 == r2 ^ (r2 >> 16)
        assert int(bits[i]) == want, (i, hex(int(bits[i])), hex(want))
    assert np.array_equal(a16, O.bf16_from_f32(a32))
    assert a16.ravel()[0] == 0xbd72  # 0xbd719bf1 rounded to nearest even BF16
    big16, big32 = O.kaiming_init(896, 8)
    bound = math.sqrt(1 / 896)
    assert np.all(np.abs(big32) <= bound + 1e-7)
    # approximately uniform on [-bound, bound]
    u = big32.ravel() / bound
    assert abs(u.mean()) < 0.03 and abs(u.var() - 1 / 3) < 0.02
    # identical across calls (fixed seed, opts.seed unused)
    assert np.array_equal(O.kaiming_init(896, 8)[1], big32)


# ── masking state machine (adapt_trainer.cu:145-182) ─────────
def test_mask_targets_known_answers():
    S, A, E = 151644, 77091, 151645
    inp = np.array([[5, S, A, 7, 8, E, 9, S, 3, 4, 6, E]], np.int32)
    tgt = np.arange(100, 112, dtype=np.int32)[None, :]
    out = O.mask_targets(inp, tgt, 1, 12)
    # positions: 0 pre-turn (masked), 1 <|im_start|> (masked), 2 'assistant' (masked),
    # 3,4 in assistant span (trained), 5 <|im_end|> (trained), 6 after (masked),
    # 7 <|im_start|> not followed by assistant (masked), 8-10 user span (masked), 11 <|im_end|> (trained)
    expect = np.array([-1, -1, -1, 103, 104, 105, -1, -1, -1, -1, -1, 111], np.int32)
    assert np.array_equal(out.ravel(), expect)
    # start token at the end of a row cannot look ahead; rows are independent
    inp2 = np.array([[S, A, 1, 2], [3, 4, 5, S]], np.int32)
    out2 = O.mask_targets(inp2, np.ones((2, 4), np.int32), 2, 4)
    assert np.array_equal(out2, [[-1, -1, 1, 1], [-1, -1, -1, -1]])


def test_uniform_tokens_almost_all_masked():
    inp = RNG.integers(0, 151936, (4, 512)).astype(np.int32)
    out = O.mask_targets(inp, np.ones_like(inp), 4, 512)
    assert np.count_nonzero(out != -1) == np.count_nonzero(inp == 151645)


# ── cosine schedule closed forms ─────────────────────────────
def test_cosine_schedule():
    base = 2e-4
    assert math.isclose(O.cosine_lr(base, 10, 110, 0.1, 0), base / 10, rel_tol=1e-6)
    assert math.isclose(O.cosine_lr(base, 10, 110, 0.1, 9), base, rel_tol=1e-6)
    assert math.isclose(O.cosine_lr(base, 10, 110, 0.1, 10), base, rel_tol=1e-6)
    assert math.isclose(O.cosine_lr(base, 10, 110, 0.1, 60), 0.55 * base, rel_tol=1e-5)
    assert math.isclose(O.cosine_lr(base, 10, 110, 0.1, 500), 0.1 * base, rel_tol=1e-5)
    assert math.isclose(O.cosine_lr(1e-4, 0, 1, 0.1, 0), 1e-4, rel_tol=1e-6)


# ── Dataset::next_batch windows ──────────────────────────────
def test_next_batch_windows_wrap():
    tok = np.arange(10, dtype=np.uint32)
    inp, tgt, pos = O.next_batch(tok, 0, 2, 4)
    assert inp.tolist() == [0, 1, 2, 3, 4, 5, 6, 7]
    assert tgt.tolist() == [1, 2, 3, 4, 5, 6, 7, 8]
    assert pos == 8
    inp, tgt, pos = O.next_batch(tok, pos, 1, 4)
    assert inp.tolist() == [8, 9, 0, 1] and tgt.tolist() == [9, 0, 1, 2] and pos == 2
