"""Golden vectors of the training-step path (test infrastructure).

c1-scale cases (one Qwen2-0.5B-shaped layer: H=896, 14 Q / 2 KV heads of 64,
SwiGLU 4864, vocab 151936, BT=128, LoRA r=8 alpha=16), plus reduced-N
centroid / k-means cases and one full step of a small model.  Inputs are
seeded; outputs are the CPU oracle's, which is pinned independently (closed
forms, PyTorch autograd, the reference's compiled host code: tests/
test_oracle_*.py, tests/test_host_api.py).

    python tests/golden/golden.py      # rewrites tests/golden/*.bin + manifest.json

Each array is a raw little-endian file <case>.input.<name>.bin or
<case>.output.<name>.bin; manifest.json
records dtype, shape, the per-output GPU bar and the case parameters.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)
import oracle as O  # noqa: E402

H, HQ, HKV, HD, I, V, BT, R, ALPHA = 896, 14, 2, 64, 4864, 151936, 128, 8, 16.0


def _bf(rng, *shape, scale=1.0):
    return O.bf16_from_f32((rng.standard_normal(shape) * scale).astype(np.float32))


# ── cases: inputs(rng) -> (params, inputs); compute(params, inputs) -> outputs
def gemm_dx_inputs(rng):
    # the k/v part of dx_normed = dQ Wq + dK Wk + dV Wv (a beta-1 chain,
    # qwen2.cu:283-285) as gemm_bf16 calls in column-major form:
    # C[in, BT] = W-view(in x out) * dY-view(out x BT)
    return {}, {"dK": _bf(rng, BT, HKV * HD), "Wk": _bf(rng, HKV * HD, H, scale=0.02),
                "dV": _bf(rng, BT, HKV * HD), "Wv": _bf(rng, HKV * HD, H, scale=0.02)}


def gemm_dx_compute(p, x):
    dx = np.zeros((BT, H), np.uint16)
    O.gemm_bf16(0, 0, H, BT, HKV * HD, 1.0, x["Wk"], H, x["dK"], HKV * HD, 0.0, dx, H)
    O.gemm_bf16(0, 0, H, BT, HKV * HD, 1.0, x["Wv"], H, x["dV"], HKV * HD, 1.0, dx, H)
    return {"dx": dx}


def lora_bwd_inputs(rng):
    # one q pair (adapter_model.cu:131-220), B != 0
    return {"s": ALPHA / R}, {"x": _bf(rng, BT, H), "go": _bf(rng, BT, HQ * HD, scale=0.1),
                               "A": _bf(rng, R, H, scale=0.05), "B": _bf(rng, HQ * HD, R, scale=0.05),
                               "grad_x": _bf(rng, BT, H, scale=0.1)}


def lora_bwd_compute(p, x):
    s, out = p["s"], HQ * HD
    # h = bf16(x A^T): C[r, BT] = A-view(r x in) * x-view(in x BT)
    h = np.zeros((BT, R), np.uint16)
    O.gemm_bf16(1, 0, R, BT, H, 1.0, x["A"], H, x["x"], H, 0.0, h, R)
    # gB[out, r] += s go^T h in F32: C[r, out] = h-view(r x BT) * go-view(BT x out)
    gB = np.zeros((out, R), np.float32)
    O.gemm_f32(0, 1, R, out, BT, s, O.f32_from_bf16(h).copy(), R,
               O.f32_from_bf16(x["go"]).copy(), out, 1.0, gB, R)
    # dh = bf16(go B): C[r, BT] = B-view(r x out) * go-view(out x BT)
    dh = np.zeros((BT, R), np.uint16)
    O.gemm_bf16(0, 0, R, BT, out, 1.0, x["B"], R, x["go"], out, 0.0, dh, R)
    # gA[r, in] += s dh^T x: C[in, r] = x-view(in x BT) * dh-view(BT x r)
    gA = np.zeros((R, H), np.float32)
    O.gemm_f32(0, 1, H, R, BT, s, O.f32_from_bf16(x["x"]).copy(), H,
               O.f32_from_bf16(dh).copy(), R, 1.0, gA, H)
    # grad_x = bf16(s dh A + grad_x): C[in, BT] = A-view(in x r) * dh-view(r x BT)
    gx = x["grad_x"].copy()
    O.gemm_bf16(0, 0, H, BT, R, s, x["A"], H, dh, R, 1.0, gx, H)
    return {"h": h, "gB": gB, "dh": dh, "gA": gA, "grad_x": gx}


def rms_inputs(rng):
    w = O.bf16_from_f32((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    return {"eps": 1e-6}, {"x": _bf(rng, BT, H), "w": w, "dy": _bf(rng, BT, H)}


def rms_compute(p, x):
    out, rms = O.rms_norm_fwd(x["x"], x["w"], p["eps"])
    dx = O.rms_norm_bwd(x["dy"], x["x"], x["w"], rms)
    return {"out": out, "rms": rms, "dx": dx}


def rope_inputs(rng):
    return {"theta": 1e6}, {"q": _bf(rng, BT, HQ * HD), "dk": _bf(rng, BT, HKV * HD)}


def rope_compute(p, x):
    return {"q_rot": O.rope(x["q"], 1, BT, HQ, HD, p["theta"], 0),
            "dk_rot": O.rope(x["dk"], 1, BT, HKV, HD, p["theta"], 1)}


def sdpa_inputs(rng):
    return {}, {"Q": _bf(rng, BT, HQ * HD), "K": _bf(rng, BT, HKV * HD),
                "V": _bf(rng, BT, HKV * HD), "dO": _bf(rng, BT, HQ * HD)}


def sdpa_compute(p, x):
    o, P_ = O.sdpa_fwd(x["Q"], x["K"], x["V"], 1, BT, HQ, HKV, HD)
    dQ, dK, dV = O.sdpa_bwd(x["dO"], x["Q"], x["K"], x["V"], P_, 1, BT, HQ, HKV, HD)
    return {"O": o, "P": P_.reshape(HQ, BT, BT), "dQ": dQ, "dK": dK, "dV": dV}


def silu_inputs(rng):
    n = (16, I)
    return {}, {"gate": _bf(rng, *n, scale=3.0), "up": _bf(rng, *n), "dout": _bf(rng, *n)}


def silu_compute(p, x):
    dg, du = O.silu_mul_bwd(x["dout"], x["gate"], x["up"])
    return {"out": O.silu_mul_fwd(x["gate"], x["up"]), "dgate": dg, "dup": du}


def ce_inputs(rng):
    return {}, {"logits": _bf(rng, 2, V, scale=2.0), "targets": np.array([17, -1], np.int32)}


def ce_compute(p, x):
    loss, dl = O.cross_entropy(x["logits"], x["targets"])
    return {"loss": loss, "dlogits": dl}


def adamw_inputs(rng):
    n = 4096
    master = (rng.standard_normal(n) * 0.05).astype(np.float32)
    grads = (rng.standard_normal((3, n)) * 1e-3).astype(np.float32)
    return ({"lr": 1e-3, "b1": 0.9, "b2": 0.999, "eps": 1e-8, "wd": 0.01},
            {"master": master, "grads": grads})


def adamw_compute(p, x):
    m32 = x["master"].copy()
    sh = O.bf16_from_f32(m32)
    m = np.zeros_like(m32)
    v = np.zeros_like(m32)
    for t in range(x["grads"].shape[0]):
        O.adamw_step(m32, sh, m, v, np.ascontiguousarray(x["grads"][t]), p["lr"], p["b1"],
                     p["b2"], p["eps"], p["wd"], t + 1)
    return {"master": m32, "working": sh, "m": m, "v": v,
            "sum_sq": np.array([O.sum_sq(x["grads"][0])], np.float64)}


def centroid_inputs(rng):
    return {}, {"h": _bf(rng, BT, H), "g": _bf(rng, BT, H, scale=0.3)}


def centroid_compute(p, x):
    acc, w = O.centroid_accumulate(O.f32_from_bf16(x["h"]).reshape(BT, H),
                                   O.f32_from_bf16(x["g"]).reshape(BT, H))
    return {"acc": np.concatenate([acc, [w]]).astype(np.float64)}


def kmeans_inputs(rng):
    # reduced c5: 64 snapshots of D=64 around 8 well-separated means, k=8
    means = rng.standard_normal((8, 64)).astype(np.float32) * 4
    lab = rng.integers(0, 8, 64)
    snaps = (means[lab] + 0.3 * rng.standard_normal((64, 64))).astype(np.float32)
    w = rng.lognormal(0.0, 1.0, 64).astype(np.float32)
    return {"k": 8, "iters": 25, "seed": 1234}, {"snaps": snaps, "weights": w}


def kmeans_compute(p, x):
    c, a, it = O.kmeans_ref(x["snaps"], p["k"])
    cp, ap, mass, seeds = O.kmeans_pp(x["snaps"], x["weights"], p["k"], p["iters"], p["seed"])
    return {"centers": c, "assign": a, "iters": np.array([it], np.int32), "pp_centers": cp,
            "pp_assign": ap, "pp_mass": mass, "pp_seeds": seeds}


def init_inputs(rng):
    return {"in_dim": H, "rank": R}, {}


def init_compute(p, x):
    a16, a32 = O.kaiming_init(p["in_dim"], p["rank"])
    return {"A16": a16, "A32": a32}


def mask_inputs(rng):
    B, T = 2, 64
    toks = rng.integers(0, 150000, B * T + 1).astype(np.int32)
    for b in range(B):  # one assistant span per row
        s = b * T + 5
        toks[s], toks[s + 1], toks[s + 20] = 151644, 77091, 151645
    toks[B * T - 3] = 151645
    return {"B": B, "T": T}, {"inputs": toks[:-1].copy(), "targets": toks[1:].copy()}


def mask_compute(p, x):
    return {"masked": O.mask_targets(x["inputs"], x["targets"], p["B"], p["T"])}


def batch_inputs(rng):
    return {"B": 2, "T": 100, "n": 3}, {"tokens": rng.integers(0, V, 500).astype(np.uint32)}


def batch_compute(p, x):
    pos, out = 0, []
    for _ in range(p["n"]):
        i, t, pos = O.next_batch(x["tokens"], pos, p["B"], p["T"])
        out += [i, t]
    return {"batches": np.concatenate(out)}


STEP_MODEL = dict(vocab=2048, hidden=256, layers=1, n_q=4, n_kv=2, head_dim=64, inter=512,
                  rms_eps=1e-6, rope_theta=1e6, tie=1)
STEP_ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b1111111, lr=1e-3, grad_clip=1.0, warmup=0,
                  total_steps=4, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)


def step_inputs(rng):
    toks = rng.integers(0, STEP_MODEL["vocab"], 2 * 64 + 1).astype(np.int32)
    return ({"model": STEP_MODEL, "adapt": STEP_ADAPT, "B": 2, "T": 64, "base_seed": 3},
            {"inputs": toks[:-1].copy(), "targets": toks[1:].copy()})


def step_compute(p, x):
    from step_util import base_tensors, pairs
    orc = O.OracleModel(p["model"], p["adapt"])
    for name, arr in base_tensors(p["model"], p["base_seed"]).items():
        orc.set_weight(name, arr)
    m = orc.step(x["inputs"], x["targets"], p["B"], p["T"])
    out = {"metrics": np.array([m["loss"], m["gnorm_raw"], m["lr"]], np.float64)}
    for l, t in pairs(p["model"], p["adapt"]):
        out[f"gB_{t}"] = orc.adapter(l, t, "gB").copy()
        out[f"B_{t}"] = orc.adapter(l, t, "B").copy()
        out[f"A_{t}"] = orc.adapter(l, t, "A").copy()
    return out


CASES = {
    "gemm_dx": (gemm_dx_inputs, gemm_dx_compute),
    "lora_bwd": (lora_bwd_inputs, lora_bwd_compute),
    "rms_norm": (rms_inputs, rms_compute),
    "rope": (rope_inputs, rope_compute),
    "sdpa": (sdpa_inputs, sdpa_compute),
    "silu_mul": (silu_inputs, silu_compute),
    "cross_entropy": (ce_inputs, ce_compute),
    "adamw": (adamw_inputs, adamw_compute),
    "centroid": (centroid_inputs, centroid_compute),
    "kmeans": (kmeans_inputs, kmeans_compute),
    "kaiming_init": (init_inputs, init_compute),
    "mask_targets": (mask_inputs, mask_compute),
    "next_batch": (batch_inputs, batch_compute),
    "step": (step_inputs, step_compute),
}


def _save(arrs, case, kind, man):
    for name, a in arrs.items():
        a = np.ascontiguousarray(a)
        fn = f"{case}.{kind[:-1]}.{name}.bin"
        a.tofile(os.path.join(HERE, fn))
        man[kind][name] = {"file": fn, "dtype": a.dtype.str, "shape": list(a.shape)}


def write_all():
    manifest = {}
    for i, (case, (mk, comp)) in enumerate(sorted(CASES.items())):
        rng = np.random.default_rng(1000 + i)
        params, inputs = mk(rng)
        outputs = comp(params, inputs)
        man = {"params": params, "inputs": {}, "outputs": {}}
        _save(inputs, case, "inputs", man)
        _save(outputs, case, "outputs", man)
        manifest[case] = man
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)


def load(case):
    with open(os.path.join(HERE, "manifest.json")) as f:
        man = json.load(f)[case]

    def rd(d):
        return {k: np.fromfile(os.path.join(HERE, v["file"]), np.dtype(v["dtype"])).reshape(
            v["shape"]) for k, v in d.items()}
    return man["params"], rd(man["inputs"]), rd(man["outputs"])


if __name__ == "__main__":
    O.build() if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")) else None
    write_all()
    tot = sum(os.path.getsize(os.path.join(HERE, f)) for f in os.listdir(HERE) if f.endswith(".bin"))
    print(f"wrote {len(CASES)} cases, {tot / 1e6:.2f} MB")
