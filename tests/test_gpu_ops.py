"""GPU parity of every backend entry point against the CPU oracle.

Each test runs the gfx950 kernel through the C-ABI (libtadapt.so) and the
oracle's restatement of the reference op on the same seeded inputs.
Tolerances (written per test): BF16 outputs of float math within 1 BF16 ulp
of the oracle for nearly every element; F32 reductions within the relative
bound stated; integer/index outputs bit-exact.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import (DEV, P, S, assert_bf16_close, call, dev, empty_bf16, f32, host,
                      rel_l2)

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20261201)


def rbf(*shape, scale=1.0):
    return O.bf16_from_f32(RNG.standard_normal(shape).astype(np.float32) * scale)


# ── elementwise ───────────────────────────────────────────────────────────
@pytest.mark.parametrize("n", [8 * 12345, 73 * 1000 + 5])
def test_silu_mul_fwd_bwd(n):
    g, u, d = rbf(n, scale=3), rbf(n), rbf(n)
    out = empty_bf16(n)
    call("ta_silu_mul_fwd", P(dev(g)), P(dev(u)), P(out), n, S())
    assert_bf16_close(host(out), O.silu_mul_fwd(g, u), what="silu fwd")
    dg, du = empty_bf16(n), empty_bf16(n)
    call("ta_silu_mul_bwd", P(dev(d)), P(dev(g)), P(dev(u)), P(dg), P(du), n, S())
    rg, ru = O.silu_mul_bwd(d, g, u)
    assert_bf16_close(host(dg), rg, what="dgate")
    assert_bf16_close(host(du), ru, what="dup")


def test_adds_and_bias():
    BT, D = 77, 896
    out, delta, bias = rbf(BT, D), rbf(BT, D), rbf(D)
    t = dev(out)
    call("ta_add_inplace", P(t), P(dev(delta)), BT * D, S())
    assert np.array_equal(host(t), O.add_inplace(out, delta))
    t = dev(out)
    call("ta_lora_add", P(t), P(dev(delta)), ctypes.c_float(2.0), BT * D, S())
    assert np.array_equal(host(t), O.lora_add(out, delta, 2.0))
    t = dev(out)
    call("ta_add_bias", P(t), P(dev(bias)), BT, D, S())
    assert np.array_equal(host(t), O.add_bias(out, bias))
    # odd width takes the scalar path
    o2, b2 = rbf(5, 13), rbf(13)
    t = dev(o2)
    call("ta_add_bias", P(t), P(dev(b2)), 5, 13, S())
    assert np.array_equal(host(t), O.add_bias(o2, b2))


def test_casts_and_embed():
    x = rbf(1000)
    f = torch.empty(1000, dtype=torch.float32, device=DEV)
    call("ta_cast_bf16_to_f32", P(dev(x)), P(f), 1000, S())
    assert np.array_equal(host(f), f32(x))
    y = RNG.standard_normal(1001).astype(np.float32)
    b = empty_bf16(1001)
    call("ta_cast_f32_to_bf16", P(dev(y)), P(b), 1001, S())
    assert np.array_equal(host(b), O.bf16_from_f32(y))
    V, D, BT = 500, 896, 64
    table = rbf(V, D)
    tok = RNG.integers(0, V, BT).astype(np.int32)
    out = empty_bf16(BT, D)
    call("ta_embed_fwd", P(dev(table)), P(dev(tok)), P(out), BT, D, S())
    assert np.array_equal(host(out), O.embed_fwd(table, tok))


# ── RMSNorm ───────────────────────────────────────────────────────────────
@pytest.mark.parametrize("rows,D", [(256, 896), (130, 1536), (64, 3584), (9, 100)])
def test_rms_norm_fwd(rows, D):
    x, w = rbf(rows, D), rbf(D, scale=0.5)
    out = empty_bf16(rows, D)
    rms = torch.empty(rows, dtype=torch.float32, device=DEV)
    call("ta_rms_norm_fwd", P(dev(x)), P(dev(w)), P(out), P(rms), 1, rows, D,
         ctypes.c_float(1e-6), S())
    ro, rr = O.rms_norm_fwd(x, w, 1e-6)
    assert np.allclose(host(rms), rr, rtol=2e-6)
    assert_bf16_close(host(out), ro, what="rms fwd")


@pytest.mark.parametrize("rows,D,want_dw", [(256, 896, False), (130, 1536, True),
                                            (64, 3584, False), (9, 100, True)])
def test_rms_norm_bwd(rows, D, want_dw):
    x, w, dy = rbf(rows, D), rbf(D, scale=0.5), rbf(rows, D)
    _, rms = O.rms_norm_fwd(x, w, 1e-6)
    dx = empty_bf16(rows, D)
    dw = torch.full((D,), 0.25, dtype=torch.float32, device=DEV) if want_dw else None
    call("ta_rms_norm_bwd", P(dev(dy)), P(dev(x)), P(dev(w)), P(dev(rms)), P(dx), P(dw), 1,
         rows, D, ctypes.c_float(1e-6), S())
    if want_dw:
        rdx, rdw = O.rms_norm_bwd(dy, x, w, rms, want_dw=True)
        assert np.allclose(host(dw), rdw + 0.25, rtol=1e-4, atol=1e-4)
    else:
        rdx = O.rms_norm_bwd(dy, x, w, rms)
    assert_bf16_close(host(dx), rdx, what="rms bwd")


# ── RoPE ──────────────────────────────────────────────────────────────────
@pytest.mark.parametrize("B,T,H,hd", [(1, 128, 14, 64), (2, 1024, 2, 128), (1, 17, 3, 6)])
@pytest.mark.parametrize("inverse", [0, 1])
def test_rope(B, T, H, hd, inverse):
    x = rbf(B * T, H * hd)
    t = dev(x)
    fn = "ta_rope_bwd" if inverse else "ta_rope_fwd"
    call(fn, P(t), B, T, H, hd, ctypes.c_float(1e6), S())
    assert_bf16_close(host(t), O.rope(x, B, T, H, hd, 1e6, inverse), frac_exact=0.98,
                      what="rope")


# ── cross entropy ─────────────────────────────────────────────────────────
# register-resident rows (V = 151936, 2048), the two-read kernel for rows
# too long for registers (200000) and ragged V (1001); in place as the
# engine calls it (dlogits over the logits)
@pytest.mark.parametrize("N,V,inplace", [(48, 151936, 0), (48, 151936, 1), (9, 2048, 1),
                                         (6, 200000, 1), (7, 1001, 0)])
def test_cross_entropy(N, V, inplace):
    logits = rbf(N, V, scale=2.0)
    tgt = RNG.integers(0, V, N).astype(np.int32)
    tgt[::3] = -1
    loss = torch.empty(N, dtype=torch.float32, device=DEV)
    lg = dev(logits)
    dl = lg if inplace else empty_bf16(N, V)
    call("ta_cross_entropy_fwd", P(lg), P(dev(tgt)), P(loss), P(dl), N, V, S())
    rl, rd = O.cross_entropy(logits, tgt)
    assert np.allclose(host(loss), rl, rtol=1e-5, atol=1e-5)
    assert_bf16_close(host(dl), rd, what="dlogits")


# ── AdamW / norms ─────────────────────────────────────────────────────────
def test_adamw_step_matches_oracle():
    n = 100003
    p = RNG.standard_normal(n).astype(np.float32) * 0.1
    m = RNG.standard_normal(n).astype(np.float32) * 1e-3
    v = np.abs(RNG.standard_normal(n).astype(np.float32)) * 1e-5
    g = RNG.standard_normal(n).astype(np.float32) * 1e-2
    tp, tm, tv, tw = dev(p), dev(m), dev(v), empty_bf16(n)
    call("ta_adamw_step", P(tp), P(tw), P(tm), P(tv), P(dev(g)), n, ctypes.c_float(1e-4),
         ctypes.c_float(0.9), ctypes.c_float(0.999), ctypes.c_float(1e-8), ctypes.c_float(0.01),
         3, S())
    rp, rm, rv, rw = p.copy(), m.copy(), v.copy(), np.empty(n, np.uint16)
    O.adamw_step(rp, rw, rm, rv, g, 1e-4, 0.9, 0.999, 1e-8, 0.01, 3)
    # F32 element math; the device may contract a*b+c into one FMA (so does
    # the reference's nvcc build): 1e-5 relative plus a floor at 1e-6 of scale
    for got, want in ((host(tm), rm), (host(tv), rv), (host(tp), rp)):
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())
    assert_bf16_close(host(tw), rw, what="shadow")


@pytest.mark.parametrize("scale,clip", [(1e-2, 1.0), (1.0, 1.0)])
def test_adamw_fused_norm_clip(scale, clip):
    n = 262147
    p = RNG.standard_normal(n).astype(np.float32) * 0.1
    g = RNG.standard_normal(n).astype(np.float32) * scale
    z = np.zeros(n, np.float32)
    tp, tm, tv, tw, tg = dev(p), dev(z), dev(z), empty_bf16(n), dev(g)
    norm = torch.zeros(1, dtype=torch.float32, device=DEV)
    call("ta_adamw_fused", P(tp), P(tw), P(tm), P(tv), P(tg), n, ctypes.c_float(1e-4),
         ctypes.c_float(0.9), ctypes.c_float(0.999), ctypes.c_float(1e-8), ctypes.c_float(0.01),
         1, ctypes.c_float(clip), P(norm), S())
    rn = float(np.sqrt(O.sum_sq(g)))
    gn = np.float32(host(norm)[0])
    assert abs(gn - rn) <= 1e-5 * rn
    gc = g * np.float32(clip / (rn + 1e-6)) if rn > clip else g
    # the gradient is left clipped in place, as clip_gradients leaves gA/gB
    # (adapt_trainer.cu:55-70): g * (clip / (norm + 1e-6)) in F32, bit for bit
    if rn > clip:
        sc = np.float32(clip) / (gn + np.float32(1e-6))
        assert np.array_equal(host(tg), (g * sc).astype(np.float32))
    else:
        assert np.array_equal(host(tg), g)
    rp, rm, rv, rw = p.copy(), z.copy(), z.copy(), np.empty(n, np.uint16)
    O.adamw_step(rp, rw, rm, rv, np.ascontiguousarray(gc, np.float32), 1e-4, 0.9, 0.999,
                 1e-8, 0.01, 1)
    assert rel_l2(host(tp), rp) < 1e-6
    assert rel_l2(host(tm), rm) < 1e-5


def test_sum_sq_into():
    g = RNG.standard_normal(1000001).astype(np.float32)
    acc = torch.full((1,), 2.0, dtype=torch.float32, device=DEV)
    call("ta_sum_sq_into", P(dev(g)), P(acc), g.size, S())
    assert abs(host(acc)[0] - (2.0 + O.sum_sq(g))) <= 1e-6 * O.sum_sq(g)


def test_scratch_release_on_a_stream_of_its_own():
    """An op on a new stream takes scratch of its own from the pool;
    ta_scratch_release frees it (after the stream is idle) and the next call
    on that stream allocates afresh and gives the same result."""
    g = RNG.standard_normal(300001).astype(np.float32)
    tg = dev(g)
    st = torch.cuda.Stream()
    out = []
    for _ in range(2):
        acc = dev(np.zeros(1, np.float32))
        torch.cuda.synchronize()
        call("ta_sum_sq_into", P(tg), P(acc), g.size, ctypes.c_void_p(st.cuda_stream))
        call("ta_scratch_release", ctypes.c_void_p(st.cuda_stream))
        out.append(host(acc)[0])
    assert out[0] == out[1] and abs(out[0] - O.sum_sq(g)) <= 1e-6 * O.sum_sq(g)


# ── GEMM ──────────────────────────────────────────────────────────────────
def check_gemm_close(got, want, what):
    r = rel_l2(f32(got), f32(want))
    exact = float((np.asarray(got) == np.asarray(want)).mean())
    assert r < 4e-3 and exact > 0.9, f"{what}: rel-L2 {r:.3e}, exact {exact:.4f}"


@pytest.mark.parametrize("tA,tB", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_bf16_column_major_all_transposes(tA, tB):
    M, N, K = 37, 29, 53
    lda = (K if tA else M) + 3
    ldb = (N if tB else K) + 2
    ldc = M + 5
    A = rbf((M if tA else K) * lda)
    B = rbf((K if tB else N) * ldb)
    C = rbf(N * ldc)
    tc = dev(C)
    call("ta_gemm_bf16", tA, tB, M, N, K, ctypes.c_float(0.75), P(dev(A)), lda, P(dev(B)), ldb,
         ctypes.c_float(1.0), P(tc), ldc, S())
    ref = C.copy()
    O.gemm_bf16(tA, tB, M, N, K, 0.75, A, lda, B, ldb, 1.0, ref, ldc)
    check_gemm_close(host(tc), ref, f"gemm tA={tA} tB={tB}")


def rm_ref(xk, yk, M, N, K, alpha, X, ldx, Y, ldy, beta, C, ldc):
    """oracle for the row-major form: C^T = op(Y) op(X) in column-major terms."""
    out = C.copy()
    O.gemm_bf16(yk, 0 if xk else 1, N, M, K, alpha, Y, ldy, X, ldx, beta, out, ldc)
    return out


@pytest.mark.parametrize("M,N,K", [(1024, 1536, 896), (4096, 4096, 256), (8192, 256, 1536),
                                   (200, 130, 72)])
def test_gemm_rm_kmajor_tiles(M, N, K):
    X, Y = rbf(M, K), rbf(N, K, scale=0.05)
    C = rbf(M, N)
    tc = dev(C)
    call("ta_gemm_rm", 1, 1, M, N, K, ctypes.c_float(1.0), P(dev(X)), K, P(dev(Y)), K,
         ctypes.c_float(1.0), P(tc), N, None, S())
    check_gemm_close(host(tc), rm_ref(1, 1, M, N, K, 1.0, X, K, Y, K, 1.0, C, N), "gemm_rm")


@pytest.mark.parametrize("M,N,K", [(2048, 1536, 1536), (1024, 3000, 320), (1280, 1100, 192),
                                   (1024, 1024, 64)])
def test_gemm_stage_forms_bit_identical(M, N, K):
    """The large-GEMM kernel forms that ta_gemm_rm_variant selects accumulate
    the same products in the same F32 order (64-k stages as two 32-k k
    steps each), so 17 and 18 (the default's two tile widths) equal 15 and
    16 (their 32-k-stage forms) bit for bit, with and without the bias
    and beta epilogues; the default (0) agrees with the oracle GEMM."""
    X, Y, b = rbf(M, K, scale=0.5), rbf(N, K, scale=0.02), rbf(N, scale=0.1)
    C0 = rbf(M, N)
    tX, tY, tb = dev(X), dev(Y), dev(b)

    def run(v, bias, beta):
        tc = dev(C0)
        call("ta_gemm_rm_variant", v, 1, 1, M, N, K, ctypes.c_float(1.0), P(tX), K, P(tY), K,
             ctypes.c_float(beta), P(tc), N, P(bias) if bias is not None else None, S())
        return host(tc)

    for a, c in ((15, 17), (16, 18)):
        for bias, beta in ((None, 0.0), (tb, 0.0), (None, 1.0)):
            ga, gc = run(a, bias, beta), run(c, bias, beta)
            assert np.array_equal(ga, gc), \
                f"variant {a} vs {c} (bias={bias is not None}, beta={beta}) differ"
    got = run(0, None, 1.0)
    # the variant held for that one call only: the plain entry runs the default
    tc = dev(C0)
    call("ta_gemm_rm", 1, 1, M, N, K, ctypes.c_float(1.0), P(tX), K, P(tY), K,
         ctypes.c_float(1.0), P(tc), N, None, S())
    assert np.array_equal(host(tc), got)
    check_gemm_close(got, rm_ref(1, 1, M, N, K, 1.0, X, K, Y, K, 1.0, C0, N), "gemm default")


@pytest.mark.parametrize("M,N,K", [(8192, 8960, 128), (2048, 8960, 192)])
def test_gemm_last_wave_split_bit_identical(M, N, K):
    """A last wave of at most half the CUs' 256 x 256 tiles (8192 x 8960:
    1120 tiles, 4.375 waves; 2048 x 8960: 280 tiles) runs its columns past
    the last whole wave (8192 ..) as 128-row tiles in a second launch.  Each
    output element keeps its k order, so the default equals the forced
    one-launch 256-wide form (variant 18) bit for bit, with the bias and
    beta epilogues too, and agrees with the oracle GEMM."""
    X, Y, b = rbf(M, K, scale=0.5), rbf(N, K, scale=0.02), rbf(N, scale=0.1)
    C0 = rbf(M, N)
    tX, tY, tb = dev(X), dev(Y), dev(b)

    def run(v, bias, beta):
        tc = dev(C0)
        call("ta_gemm_rm_variant", v, 1, 1, M, N, K, ctypes.c_float(1.0), P(tX), K, P(tY), K,
             ctypes.c_float(beta), P(tc), N, P(bias) if bias is not None else None, S())
        return host(tc)

    for bias, beta in ((None, 0.0), (tb, 0.0), (None, 1.0)):
        g0, g18 = run(0, bias, beta), run(18, bias, beta)
        assert np.array_equal(g0, g18), f"default vs 256-wide (bias={bias is not None}, beta={beta})"
    got = run(0, tb, 1.0)
    ref = O.add_bias(rm_ref(1, 1, M, N, K, 1.0, X, K, Y, K, 1.0, C0, N), b) if M <= 2048 else None
    if ref is not None:
        check_gemm_close(got, ref, "gemm last-wave split")


@pytest.mark.parametrize("M,N,K", [(2048, 896, 4864), (2048, 900, 16384), (1024, 1536, 16384),
                                   (1000, 900, 32768)])
def test_gemm_split_k_partials(M, N, K):
    """Long-K GEMMs on too few tiles to fill the chip (the Qwen2-0.5B shapes
    at B x T = 2048) run split-K, each split's F32 partials then the ordered
    reduce with alpha, beta and the bias.  Splits of about 10 stages (the
    first shape, 8 splits) take the direct-to-LDS kernel; splits of 32 or
    more the 64-k pipeline kernel, 256-wide (N = 900: the element stores;
    M = 1000: rows past M skipped) and 192-wide.  Checked against the
    oracle GEMM, with the bias and beta = 1."""
    X, Y, b = rbf(M, K, scale=0.5), rbf(N, K, scale=0.02), rbf(N, scale=0.1)
    C0 = rbf(M, N)
    tc = dev(C0)
    call("ta_gemm_rm", 1, 1, M, N, K, ctypes.c_float(1.0), P(dev(X)), K, P(dev(Y)), K,
         ctypes.c_float(1.0), P(tc), N, P(dev(b)), S())
    ref = O.add_bias(rm_ref(1, 1, M, N, K, 1.0, X, K, Y, K, 1.0, C0, N), b)
    check_gemm_close(host(tc), ref, "gemm split-K")


def test_gemm_rm_bias_epilogue():
    M, N, K = 256, 384, 128
    X, Y, b = rbf(M, K), rbf(N, K), rbf(N)
    tc = empty_bf16(M, N)
    call("ta_gemm_rm", 1, 1, M, N, K, ctypes.c_float(1.0), P(dev(X)), K, P(dev(Y)), K,
         ctypes.c_float(0.0), P(tc), N, P(dev(b)), S())
    ref = O.add_bias(rm_ref(1, 1, M, N, K, 1.0, X, K, Y, K, 0.0, np.zeros((M, N), np.uint16), N),
                     b)
    check_gemm_close(host(tc), ref, "gemm+bias")


@pytest.mark.parametrize("M,N,K", [(1536, 16, 8192), (16, 896, 4096), (8192, 16, 1536)])
def test_gemm_f32_weight_gradient_layouts(M, N, K):
    """LoRA weight-gradient shapes (reduction over tokens, K-strided operands),
    split-K path, F32 output with beta=1 (gemm_f32 as adapter_model.cu uses it)."""
    # column-major gemm_f32(transA=0, transB=1): C(MxN) = A(MxK) * B(NxK)^T
    A = f32(rbf(K, M)).copy()  # A[i + k*M]
    Bm = f32(rbf(K, N, scale=0.1)).copy()  # B[j + k*N]
    C = RNG.standard_normal(N * M).astype(np.float32)
    tc = dev(C)
    call("ta_gemm_f32", 0, 1, M, N, K, ctypes.c_float(0.5), P(dev(A)), M, P(dev(Bm)), N,
         ctypes.c_float(1.0), P(tc), M, S())
    ref = C.copy()
    O.gemm_f32(0, 1, M, N, K, 0.5, A, M, Bm, N, 1.0, ref, M)
    assert rel_l2(host(tc), ref) < 1e-5


def _cm_op(X, trans, rows, K, ld):
    """op(X) as a dense [rows, K] array from a column-major buffer."""
    if trans:  # op(X)(i,k) = X[k + i*ld]
        return X.reshape(rows, ld)[:, :K]
    return X.reshape(K, ld)[:, :rows].T  # op(X)(i,k) = X[i + k*ld]


@pytest.mark.parametrize("tA,tB,M,N,K", [(0, 0, 129, 67, 1000), (1, 0, 64, 300, 777),
                                         (0, 1, 1536, 16, 8192), (1, 1, 200, 130, 64),
                                         (0, 1, 8960, 40, 5000)])
def test_gemm_f32_general_operands(tA, tB, M, N, K):
    """gemm_f32 on F32 data that is not BF16-valued has cublasSgemm accuracy
    (tensor.cu:168-182): within 1e-5 relative L2 of the FP64-accumulated
    oracle, and each element within 1e-6 of alpha * sum_k |a||b| + |beta c|
    (BF16-rounded operands would miss both by about 3e-3).  Padded leading
    dimensions; the last shape takes three K chunks of the staging."""
    lda, ldb, ldc = (K if tA else M) + 3, (N if tB else K) + 2, M + 1
    A = RNG.standard_normal((M if tA else K) * lda).astype(np.float32)
    Bm = (RNG.standard_normal((K if tB else N) * ldb) * 1e-3).astype(np.float32)
    C = RNG.standard_normal(N * ldc).astype(np.float32)
    alpha, beta = 0.75, -0.5
    tc = dev(C)
    call("ta_gemm_f32", tA, tB, M, N, K, ctypes.c_float(alpha), P(dev(A)), lda, P(dev(Bm)), ldb,
         ctypes.c_float(beta), P(tc), ldc, S())
    ref = C.copy()
    assert O.gemm_f32(tA, tB, M, N, K, alpha, A, lda, Bm, ldb, beta, ref, ldc) == 0
    got = host(tc).reshape(N, ldc)[:, :M]
    want = ref.reshape(N, ldc)[:, :M]
    assert np.array_equal(host(tc).reshape(N, ldc)[:, M:], C.reshape(N, ldc)[:, M:])
    assert rel_l2(got, want) < 1e-5
    opa = _cm_op(A, tA, M, K, lda).astype(np.float64)            # [M, K]
    opb = _cm_op(Bm, not tB, N, K, ldb).astype(np.float64)       # [N, K]: op(B)(k,j) by j
    mag = abs(alpha) * (np.abs(opb) @ np.abs(opa).T) + abs(beta) * np.abs(C.reshape(N, ldc)[:, :M])
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-6 * mag)


# ── centroid accumulate / k-means ─────────────────────────────────────────
def test_centroid_accumulate_bf16():
    BT, D = 300, 896
    h, g = rbf(BT, D), rbf(BT, D, scale=1e-3)
    acc = torch.zeros(D + 1, dtype=torch.float64, device=DEV)
    for _ in range(2):
        call("ta_centroid_accumulate_bf16", P(dev(h)), P(dev(g)), BT, D, P(acc), S())
    ra, rw = O.centroid_accumulate(f32(h), f32(g))
    a = host(acc)
    assert rel_l2(a[:D], 2 * ra) < 1e-6
    assert abs(a[D] - 2 * rw) <= 1e-6 * 2 * rw


def test_centroid_accumulate_f32n():
    BT, D = 5000, 512
    h = RNG.standard_normal((BT, D)).astype(np.float32)
    n = RNG.lognormal(0, 1, BT).astype(np.float32)
    acc = torch.zeros(D + 1, dtype=torch.float64, device=DEV)
    call("ta_centroid_accumulate_f32n", P(dev(h)), P(dev(n)), BT, D, P(acc), S())
    ra, rw = O.centroid_accumulate_n(h, n)
    a = host(acc)
    assert np.max(np.abs(a[:D] - ra)) <= 1e-5 * np.max(np.abs(ra))
    assert abs(a[D] - rw) <= 1e-6 * rw


def mixture(N, D, comps, seed):
    r = np.random.default_rng(seed)
    means = r.standard_normal((comps, D)).astype(np.float32)
    lab = r.integers(0, comps, N)
    return (means[lab] + 0.3 * r.standard_normal((N, D))).astype(np.float32)


# (200, 128, 16): the center sums over four 64-snapshot ballots; (300, 256,
# 12): snapshots past the 128 KB LDS copy (read from global memory); D = 16:
# the per-output scan over every snapshot; D = 30: element-wise loads, no
# column permutation
@pytest.mark.parametrize("N,D,k", [(64, 512, 32), (50, 64, 8), (5, 16, 8), (200, 128, 16),
                                   (300, 256, 12), (20, 30, 4)])
def test_kmeans_ref_bit_exact(N, D, k):
    X = mixture(N, D, 16, N + D)
    kk = min(k, N)
    C = torch.empty(kk * D, dtype=torch.float32, device=DEV)
    A = torch.empty(N, dtype=torch.int32, device=DEV)
    it = torch.zeros(1, dtype=torch.int32, device=DEV)
    call("ta_kmeans_ref", P(dev(X)), N, D, k, 50, P(C), P(A), P(it), S())
    rc, ra, ri = O.kmeans_ref(X, k)
    assert np.array_equal(host(A), ra)
    assert np.array_equal(host(C).reshape(kk, D), rc)
    assert int(host(it)[0]) == ri


@pytest.mark.parametrize("N,D,k", [(64, 512, 32), (200, 128, 16), (300, 256, 12), (40, 48, 6)])
def test_kmeans_pp_bit_exact(N, D, k):
    X = mixture(N, D, 16, 7)
    W = np.random.default_rng(3).lognormal(0, 1, N).astype(np.float32)
    C = torch.empty(k * D, dtype=torch.float32, device=DEV)
    A = torch.empty(N, dtype=torch.int32, device=DEV)
    M = torch.empty(k, dtype=torch.float64, device=DEV)
    Sd = torch.empty(k, dtype=torch.int32, device=DEV)
    call("ta_kmeans_pp", P(dev(X)), P(dev(W)), N, D, k, 25, ctypes.c_uint64(12345), P(C), P(A),
         P(M), P(Sd), S())
    rc, ra, rm, rs = O.kmeans_pp(X, W, k, 25, 12345)
    assert np.array_equal(host(Sd), rs)
    assert np.array_equal(host(A), ra)
    assert np.array_equal(host(C).reshape(k, D), rc)
    assert np.allclose(host(M), rm, rtol=1e-12)


# ── attention ─────────────────────────────────────────────────────────────
ATTN_SHAPES = [(1, 128, 14, 2, 64), (2, 256, 12, 2, 128), (1, 100, 4, 2, 64), (1, 512, 14, 2, 64),
               (1, 1024, 12, 2, 128)]
ROWSTAT_SHAPES = [(1, 1024, 12, 2, 128), (2, 200, 14, 2, 64), (1, 100, 4, 2, 128),
                  (1, 512, 14, 2, 64), (1, 2048, 28, 4, 128)]


# Element-wise bar of the attention outputs (O, dQ, dK, dV) against the
# oracle: every element within 1 BF16 ulp, except where cancellation made
# the value tiny (within 2^-7 of the tensor's largest magnitude), at least
# 98% bit-identical, relative L2 at most 5e-4.  Measured on MI355X over all
# shapes of both tests: relative L2 at most 1.6e-4, at least 99.27% of the
# elements identical, and no element off by more than 0 ulp outside that
# cancellation band.
ATTN_BAR = dict(max_ulp=1, frac_exact=0.98, rl2=5e-4, floor=2.0 ** -7)


def _scores64(Q, K, B, T, Hq, Hkv, hd):
    """causal scores S * scale * log2(e) in float64, [B, Hq, T, T] (-inf above the diagonal)"""
    q = f32(Q).reshape(B, T, Hq, hd).astype(np.float64).transpose(0, 2, 1, 3)
    k = f32(K).reshape(B, T, Hkv, hd).astype(np.float64).transpose(0, 2, 3, 1)
    k = np.repeat(k, Hq // Hkv, axis=1)
    s = (q @ k) * (1.0 / np.sqrt(hd)) * np.log2(np.e)
    s[:, :, np.triu(np.ones((T, T), bool), 1)] = -np.inf
    return s


@pytest.mark.parametrize("B,T,Hq,Hkv,hd", ROWSTAT_SHAPES)
def test_attn_rowstats_fwd_bwd(B, T, Hq, Hkv, hd):
    """The step engine's attention (probabilities recomputed from each row's
    (max, 1/sum), never stored) against the oracle's sdpa_fwd/bwd
    (ops.cu:578-870): O as ta_sdpa_fwd's bar, O32 within 1e-4 relative L2
    of the float64 P.V, the row maximum (base-2 units) within 1e-5 of the
    float64 one and 1/sum within 1e-5 relative, dQ/dK/dV to the same
    element-wise bar as O.  Shapes: the headline layer (T=1024, 12/2 heads
    of 128), ragged T (100, 200), head_dim 64 and the 7B-shaped T=2048, 28/4."""
    print(f"case: attn rowstats B={B} T={T} Hq={Hq} Hkv={Hkv} hd={hd}", flush=True)
    Q, K, V = rbf(B * T, Hq * hd), rbf(B * T, Hkv * hd), rbf(B * T, Hkv * hd)
    dO = rbf(B * T, Hq * hd)
    tQ, tK, tV = dev(Q), dev(K), dev(V)
    out = empty_bf16(B * T, Hq * hd)
    o32 = torch.empty(B * T * Hq * hd, dtype=torch.float32, device=DEV)
    st = torch.empty(B * Hq * T * 2, dtype=torch.float32, device=DEV)
    call("ta_attn_fwd_rowstats", P(tQ), P(tK), P(tV), P(out), P(o32), P(st), B, T, Hq, Hkv, hd,
         S())
    rO, rP = O.sdpa_fwd(Q, K, V, B, T, Hq, Hkv, hd)
    assert_bf16_close(host(out), rO, what="attn O", **ATTN_BAR)
    s64 = _scores64(Q, K, B, T, Hq, Hkv, hd)
    m64 = s64.max(axis=-1)
    inv64 = 1.0 / np.exp2(s64 - m64[..., None]).sum(axis=-1)
    gst = host(st).reshape(B, Hq, T, 2)
    assert np.all(np.abs(gst[..., 0] - m64) <= 1e-5 * np.abs(m64) + 1e-5)
    np.testing.assert_allclose(gst[..., 1], inv64, rtol=1e-5)
    p64 = np.exp2(s64 - m64[..., None]) * inv64[..., None]
    v = f32(V).reshape(B, T, Hkv, hd).astype(np.float64).transpose(0, 2, 1, 3)
    o64 = (p64 @ np.repeat(v, Hq // Hkv, axis=1)).transpose(0, 2, 1, 3).reshape(B * T, Hq * hd)
    assert rel_l2(host(o32).reshape(B * T, Hq * hd), o64) < 1e-4
    dQ, dK, dV = empty_bf16(B * T, Hq * hd), empty_bf16(B * T, Hkv * hd), empty_bf16(B * T, Hkv * hd)
    call("ta_attn_bwd_rowstats", P(dev(dO)), P(tQ), P(tK), P(tV), P(st), P(o32), P(dQ), P(dK),
         P(dV), B, T, Hq, Hkv, hd, S())
    rdQ, rdK, rdV = O.sdpa_bwd(dO, Q, K, V, rP, B, T, Hq, Hkv, hd)
    for got, want, name in ((dQ, rdQ, "dQ"), (dK, rdK, "dK"), (dV, rdV, "dV")):
        assert_bf16_close(host(got), want, what=name, **ATTN_BAR)


@pytest.mark.parametrize("B,T,Hq,Hkv,hd", ATTN_SHAPES)
def test_sdpa_fwd_bwd(B, T, Hq, Hkv, hd):
    """P (F32) to 1e-5 relative; O, dQ, dK, dV to ATTN_BAR element-wise
    against the oracle's F32 products (P and dS feed the MFMA as BF16 hi/lo
    pairs, about 16 significant bits, where the reference used F32 GEMMs)."""
    Q, K, V = rbf(B * T, Hq * hd), rbf(B * T, Hkv * hd), rbf(B * T, Hkv * hd)
    dO = rbf(B * T, Hq * hd)
    out = empty_bf16(B * T, Hq * hd)
    Pd = torch.full((B * Hq * T * T,), 7.0, dtype=torch.float32, device=DEV)
    tQ, tK, tV = dev(Q), dev(K), dev(V)
    call("ta_sdpa_fwd", P(tQ), P(tK), P(tV), P(out), P(Pd), B, T, Hq, Hkv, hd, S())
    rO, rP = O.sdpa_fwd(Q, K, V, B, T, Hq, Hkv, hd)
    gP = host(Pd).reshape(B, Hq, T, T)
    assert np.allclose(gP, rP, rtol=1e-5, atol=1e-7)
    assert_bf16_close(host(out), rO, what="attn O", **ATTN_BAR)
    dQ, dK, dV = empty_bf16(B * T, Hq * hd), empty_bf16(B * T, Hkv * hd), empty_bf16(B * T, Hkv * hd)
    call("ta_sdpa_bwd", P(dev(dO)), P(tQ), P(tK), P(tV), P(Pd), P(dQ), P(dK), P(dV), B, T, Hq,
         Hkv, hd, S())
    rdQ, rdK, rdV = O.sdpa_bwd(dO, Q, K, V, rP, B, T, Hq, Hkv, hd)
    for got, want, name in ((dQ, rdQ, "dQ"), (dK, rdK, "dK"), (dV, rdV, "dV")):
        assert_bf16_close(host(got), want, what=name, **ATTN_BAR)
