"""ctypes binding for the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product.  Arrays are numpy; BF16
tensors travel as uint16 bit patterns.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_int = ctypes.c_int
c_vp = ctypes.c_void_p


class ModelCfg(ctypes.Structure):
    _fields_ = [("vocab", c_int), ("hidden", c_int), ("layers", c_int), ("n_q", c_int),
                ("n_kv", c_int), ("head_dim", c_int), ("inter", c_int),
                ("rms_eps", c_f32), ("rope_theta", c_f32), ("tie", c_int)]


class AdaptCfg(ctypes.Structure):
    _fields_ = [("rank", c_int), ("alpha", c_f32), ("inject_mask", c_int), ("lr", c_f32),
                ("grad_clip", c_f32), ("warmup", c_i64), ("total_steps", c_i64),
                ("b1", c_f32), ("b2", c_f32), ("eps", c_f32), ("wd", c_f32)]


class StepOut(ctypes.Structure):
    _fields_ = [("loss", c_f32), ("lr", c_f32), ("gnorm", c_f32), ("gnorm_raw", c_f32),
                ("valid_tokens", c_int), ("step", c_int)]


def build():
    subprocess.check_call([os.path.join(_HERE, "build.sh")])


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.or_sum_sq.restype = ctypes.c_double
        L.or_cosine_lr.restype = c_f32
        L.or_cosine_lr.argtypes = [c_f32, c_i64, c_i64, c_f32, c_i64]
        L.or_model_create.restype = c_vp
        L.or_model_adapter_ptr.restype = c_vp
        L.or_model_adapter_ptr.argtypes = [c_vp, c_int, c_int, c_int, ctypes.POINTER(c_i64)]
        L.or_model_tap.restype = c_i64
        L.or_model_tap.argtypes = [c_vp, ctypes.c_char_p, c_vp, ctypes.POINTER(c_int)]
        L.or_model_set_weight.argtypes = [c_vp, ctypes.c_char_p, c_vp, c_i64]
        L.or_model_step.argtypes = [c_vp, c_vp, c_vp, c_int, c_int, c_f32, ctypes.POINTER(StepOut)]
        L.or_model_destroy.argtypes = [c_vp]
        L.or_model_keep_taps.argtypes = [c_vp, c_int]
        L.or_model_centroid.argtypes = [c_vp, c_vp, c_vp]
        L.or_kmeans_pp.argtypes = [c_vp, c_vp, c_int, c_int, c_int, c_int, ctypes.c_uint64,
                                   c_vp, c_vp, c_vp, c_vp]
        _LIB = L
    return _LIB


def set_accum_mode(mode):
    """0: FP64 accumulation (default, the exact side of every check);
    1: FP32 accumulation in 16-wide K blocks, for measuring how far two
    FP32-accumulating implementations drift apart (process-wide)."""
    lib().or_set_accum_mode(c_int(mode))


def P(a):
    """data pointer of a contiguous numpy array (or None)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle needs contiguous arrays"
    return ctypes.c_void_p(a.ctypes.data)


# ── BF16 helpers (numpy) ─────────────────────────────────────
def bf16_from_f32(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_bf16_from_f32(P(x), P(y), c_i64(x.size))
    return y


def f32_from_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    return (x.astype(np.uint32) << 16).view(np.float32)


# ── op wrappers (in-place where the reference is in-place) ───
def gemm_bf16(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc):
    return lib().or_gemm_bf16(c_int(transA), c_int(transB), c_int(M), c_int(N), c_int(K),
                              c_f32(alpha), P(A), c_int(lda), P(B), c_int(ldb), c_f32(beta),
                              P(C), c_int(ldc))


def gemm_f32(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc):
    return lib().or_gemm_f32(c_int(transA), c_int(transB), c_int(M), c_int(N), c_int(K),
                             c_f32(alpha), P(A), c_int(lda), P(B), c_int(ldb), c_f32(beta),
                             P(C), c_int(ldc))


def rms_norm_fwd(x, w, eps):
    rows, D = x.shape
    out = np.empty_like(x)
    rms = np.empty(rows, np.float32)
    lib().or_rms_norm_fwd(P(x), P(w), P(out), P(rms), c_i64(rows), c_int(D), c_f32(eps))
    return out, rms


def rms_norm_bwd(dy, x, w, rms, want_dw=False):
    rows, D = x.shape
    dx = np.empty_like(x)
    dw = np.zeros(D, np.float32) if want_dw else None
    lib().or_rms_norm_bwd(P(dy), P(x), P(w), P(rms), P(dx), P(dw), c_i64(rows), c_int(D))
    return (dx, dw) if want_dw else dx


def rope(x, B, T, H, hd, theta, inverse):
    x = np.ascontiguousarray(x).copy()
    lib().or_rope(P(x), c_int(B), c_int(T), c_int(H), c_int(hd), c_f32(theta), c_int(inverse))
    return x


def sdpa_fwd(Q, K, V, B, T, Hq, Hkv, hd):
    out = np.empty((B * T, Hq * hd), np.uint16)
    attn = np.empty((B, Hq, T, T), np.float32)
    lib().or_sdpa_fwd(P(Q), P(K), P(V), P(out), P(attn), c_int(B), c_int(T), c_int(Hq),
                      c_int(Hkv), c_int(hd))
    return out, attn


def sdpa_bwd(dout, Q, K, V, attn, B, T, Hq, Hkv, hd):
    dQ = np.zeros((B * T, Hq * hd), np.uint16)
    dK = np.zeros((B * T, Hkv * hd), np.uint16)
    dV = np.zeros((B * T, Hkv * hd), np.uint16)
    lib().or_sdpa_bwd(P(dout), P(Q), P(K), P(V), P(attn), P(dQ), P(dK), P(dV), c_int(B),
                      c_int(T), c_int(Hq), c_int(Hkv), c_int(hd))
    return dQ, dK, dV


def silu_mul_fwd(gate, up):
    out = np.empty_like(gate)
    lib().or_silu_mul_fwd(P(gate), P(up), P(out), c_i64(gate.size))
    return out


def silu_mul_bwd(dout, gate, up):
    dg = np.empty_like(gate)
    du = np.empty_like(gate)
    lib().or_silu_mul_bwd(P(dout), P(gate), P(up), P(dg), P(du), c_i64(gate.size))
    return dg, du


def cross_entropy(logits, targets):
    N, V = logits.shape
    loss = np.empty(N, np.float32)
    dl = np.empty_like(logits)
    targets = np.ascontiguousarray(targets, np.int32)
    lib().or_cross_entropy(P(logits), P(targets), P(loss), P(dl), c_i64(N), c_i64(V))
    return loss, dl


def embed_fwd(table, tokens):
    V, D = table.shape
    tokens = np.ascontiguousarray(tokens, np.int32)
    out = np.empty((tokens.size, D), np.uint16)
    lib().or_embed_fwd(P(table), P(tokens), P(out), c_i64(tokens.size), c_int(D))
    return out


def add_bias(out, bias):
    out = out.copy()
    BT, D = out.shape
    lib().or_add_bias(P(out), P(bias), c_i64(BT), c_int(D))
    return out


def add_inplace(out, delta):
    out = out.copy()
    lib().or_add_inplace(P(out), P(delta), c_i64(out.size))
    return out


def lora_add(out, delta, scale):
    out = out.copy()
    lib().or_lora_add(P(out), P(delta), c_f32(scale), c_i64(out.size))
    return out


def adamw_step(master, working, m, v, grad, lr, b1, b2, eps, wd, step):
    """in place on master, working, m, v (like ops.cu:1139-1169)."""
    lib().or_adamw_step(P(master), P(working), P(m), P(v), P(grad), c_i64(master.size),
                        c_f32(lr), c_f32(b1), c_f32(b2), c_f32(eps), c_f32(wd), c_int(step))


def sum_sq(g):
    g = np.ascontiguousarray(g, np.float32)
    return lib().or_sum_sq(P(g), c_i64(g.size))


def kaiming_init(in_dim, rank, seed=0x1234):
    a16 = np.empty((rank, in_dim), np.uint16)
    a32 = np.empty((rank, in_dim), np.float32)
    lib().or_kaiming_init(P(a16), P(a32), c_int(in_dim), c_int(rank), ctypes.c_uint32(seed))
    return a16, a32


def mask_targets(inputs, targets, B, T):
    t = np.ascontiguousarray(targets, np.int32).copy()
    i = np.ascontiguousarray(inputs, np.int32)
    lib().or_mask_targets(P(i), P(t), c_int(B), c_int(T))
    return t


def cosine_lr(base, warmup, total, floor_frac, step):
    return lib().or_cosine_lr(base, warmup, total, floor_frac, step)


def next_batch(tokens, pos, B, T):
    tokens = np.ascontiguousarray(tokens, np.uint32)
    p = c_i64(pos)
    inp = np.empty(B * T, np.int32)
    tgt = np.empty(B * T, np.int32)
    lib().or_next_batch(P(tokens), c_i64(tokens.size), ctypes.byref(p), c_int(B), c_int(T),
                        P(inp), P(tgt))
    return inp, tgt, p.value


def centroid_accumulate(h, g, acc=None, acc_w=0.0, want_norms=False):
    BT, D = h.shape
    acc = np.zeros(D, np.float64) if acc is None else acc.copy()
    w = ctypes.c_double(acc_w)
    n = np.empty(BT, np.float64) if want_norms else None
    lib().or_centroid_accumulate(P(np.ascontiguousarray(h, np.float32)),
                                 P(np.ascontiguousarray(g, np.float32)), c_i64(BT), c_int(D),
                                 P(acc), ctypes.byref(w), P(n))
    return (acc, w.value, n) if want_norms else (acc, w.value)


def centroid_accumulate_n(h, n, acc=None, acc_w=0.0):
    BT, D = h.shape
    acc = np.zeros(D, np.float64) if acc is None else acc.copy()
    w = ctypes.c_double(acc_w)
    lib().or_centroid_accumulate_n(P(np.ascontiguousarray(h, np.float32)),
                                   P(np.ascontiguousarray(n, np.float32)), c_i64(BT), c_int(D),
                                   P(acc), ctypes.byref(w))
    return acc, w.value


def kmeans_ref(snaps, k):
    snaps = np.ascontiguousarray(snaps, np.float32)
    N, D = snaps.shape
    kk = min(k, N)
    centers = np.empty((kk, D), np.float32)
    assign = np.empty(N, np.int32)
    iters = c_int(0)
    lib().or_kmeans_ref(P(snaps), c_int(N), c_int(D), c_int(k), P(centers), P(assign),
                        ctypes.byref(iters))
    return centers, assign, iters.value


def kmeans_pp(snaps, weights, k, iters, seed):
    snaps = np.ascontiguousarray(snaps, np.float32)
    weights = np.ascontiguousarray(weights, np.float32)
    N, D = snaps.shape
    kk = min(k, N)
    centers = np.empty((kk, D), np.float32)
    assign = np.empty(N, np.int32)
    mass = np.empty(kk, np.float64)
    seeds = np.empty(kk, np.int32)
    lib().or_kmeans_pp(P(snaps), P(weights), N, D, k, iters, seed, P(centers), P(assign),
                       P(mass), P(seeds))
    return centers, assign, mass, seeds


# ── model-level oracle ───────────────────────────────────────
TARGETS = ("q", "k", "v", "o", "gate", "up", "down")
WHICH = {"A": 0, "B": 1, "mA": 2, "vA": 3, "mB": 4, "vB": 5, "gA": 6, "gB": 7,
         "A16": 8, "B16": 9}


class OracleModel:
    """One AdaptTrainer over a Qwen2 base, restated on the CPU."""

    def __init__(self, mcfg: dict, acfg: dict):
        self.mc = ModelCfg(**mcfg)
        self.ac = AdaptCfg(**acfg)
        self.h = lib().or_model_create(ctypes.byref(self.mc), ctypes.byref(self.ac))

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_destroy(self.h)
            self.h = None

    def set_weight(self, name, arr):
        arr = np.ascontiguousarray(arr, np.uint16)
        rc = lib().or_model_set_weight(self.h, name.encode(), P(arr), arr.size)
        if rc != 0:
            raise KeyError(name)

    def adapter(self, layer, target, which):
        n = c_i64(0)
        t = TARGETS.index(target) if isinstance(target, str) else target
        ptr = lib().or_model_adapter_ptr(self.h, layer, t, WHICH[which], ctypes.byref(n))
        if not ptr:
            return None
        ct = ctypes.c_uint16 if which in ("A16", "B16") else ctypes.c_float
        return np.ctypeslib.as_array((ct * n.value).from_address(ptr))

    def keep_taps(self, on=True):
        lib().or_model_keep_taps(self.h, 1 if on else 0)

    def tap(self, name):
        kind = c_int(0)
        n = lib().or_model_tap(self.h, name.encode(), None, ctypes.byref(kind))
        if n == 0:
            return None
        out = np.empty(n, np.uint16 if kind.value == 0 else np.float32)
        lib().or_model_tap(self.h, name.encode(), P(out), ctypes.byref(kind))
        return out

    def centroid(self):
        acc = np.empty(self.mc.hidden, np.float64)
        w = ctypes.c_double(0)
        lib().or_model_centroid(self.h, P(acc), ctypes.byref(w))
        return acc, w.value

    def step(self, inputs, targets, B, T, lr_override=0.0):
        so = StepOut()
        i = np.ascontiguousarray(inputs, np.int32)
        t = np.ascontiguousarray(targets, np.int32)
        lib().or_model_step(self.h, P(i), P(t), B, T, lr_override, ctypes.byref(so))
        return {k: getattr(so, k) for k, _ in StepOut._fields_}
