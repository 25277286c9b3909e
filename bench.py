#!/usr/bin/env python3
"""Headline benchmark: LoRA training throughput of the MI355X step engine.

Workload ("c3"): Qwen2-1.5B shape — 28 layers,
hidden 1536, 12 Q / 2 KV heads, head_dim 128, SwiGLU 8960, vocab 151936,
tied embedding — BF16 frozen base ~N(0, 0.02) generated on the device from a
seed, LoRA r=16 alpha=32 on all seven projections, batch 8 x seq 1024 of
uniform random token ids (next-token targets as Dataset::next_batch makes
them), AdamW.  A step is one full training step (forward, cross entropy,
backward, centroid accumulation, grad norm/clip, AdamW) with the batch
already resident in HBM.

Prints one JSON line.  Besides tokens/s it carries:
  roofline     — the instrumented kernel with the largest share of step
                 time, every launch of it in every fifth timed step timed
                 with HIP events carried by its own dispatch on its launch
                 stream (timed launches cost a few microseconds of idle GPU
                 each, so not every step is timed): algorithmic flops (or bytes)
                 per launch / average launch time, against MI355X peak
                 (2.5 PFLOP/s dense BF16, 8 TB/s HBM); the bound is the
                 resource whose peak gives the longer time for that work.
  bwd_gemm_mfma_util, hbm_gbs, classes
               — the metric's other quantities: every kernel class of the
                 step (ta_engine_profile categories) event-timed for one
                 step each, with its algorithmic TFLOP/s and GB/s and their
                 fractions of the peaks; bwd_gemm_mfma_util is the
                 backward GEMMs' MFMA fraction (frozen-base input gradients
                 and the LM head's input gradient together), hbm_gbs the
                 norm, attention-backward and AdamW bandwidths.
  cpu_baseline — the CPU restatement of the reference step (oracle/, a
                 port: the reference has no CPU path) on this host's cores,
                 on a bounded sample, extrapolated to the c3 model.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tensor-adapt_amd"))

C3_MODEL = dict(vocab=151936, hidden=1536, layers=28, n_q=12, n_kv=2, head_dim=128, inter=8960,
                rms_eps=1e-6, rope_theta=1e6, tie=1)
C3_ADAPT = dict(rank=16, alpha=32.0, inject_mask=0b1111111, lr=1e-4, grad_clip=1.0, warmup=5,
                total_steps=50, b1=0.9, b2=0.999, eps=1e-8, wd=0.0)
C3_B, C3_T = 8, 1024
C3_WORK = ("c3: Qwen2-1.5B shape, LoRA r=16 alpha=32 on q,k,v,o,gate,up,down, batch 8 x seq 1024, "
           "AdamW, centroid accumulator on")
METRIC = "train tokens/s Qwen2-1.5B LoRA r=16 seq1024; bwd MFMA util %, HBM GB/s"
# the other BASELINE configs, for secondary measurements (--config); the
# headline line is c3
C2_MODEL = dict(vocab=151936, hidden=896, layers=24, n_q=14, n_kv=2, head_dim=64, inter=4864,
                rms_eps=1e-6, rope_theta=1e6, tie=1)
C2_ADAPT = dict(C3_ADAPT, inject_mask=0b0001111, total_steps=20)
C4_MODEL = dict(vocab=152064, hidden=3584, layers=28, n_q=28, n_kv=4, head_dim=128, inter=18944,
                rms_eps=1e-6, rope_theta=1e6, tie=0)
C4_ADAPT = dict(C3_ADAPT, rank=64, alpha=128.0, total_steps=20)
CONFIGS = {
    # name: (model, adapt, B, T, per-layer recompute, workload)
    "c3": (C3_MODEL, C3_ADAPT, C3_B, C3_T, False, C3_WORK),
    "c2": (C2_MODEL, C2_ADAPT, 4, 512, False,
           "c2: Qwen2-0.5B, tied embedding, LoRA r=16 alpha=32 on q,k,v,o, batch 4 x seq 512, "
           "AdamW, centroid accumulator on"),
    "c4": (C4_MODEL, C4_ADAPT, 4, 2048, True,
           "c4: Qwen2-7B shape, untied LM head, LoRA r=64 alpha=128 on q,k,v,o,gate,up,down, "
           "batch 4 x seq 2048, per-layer activation recompute, AdamW, centroid accumulator on"),
}

CAT_NAMES = ["gemm_fwd", "gemm_dx", "lm_head", "lora", "attn_fwd", "attn_bwd", "norm",
             "elementwise", "cross_entropy", "adamw_tail", "centroid", "lm_head_bwd"]
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def token_batches(n, B, T, V, seed):
    """n batches of Dataset::next_batch windows (src/data/dataset.cpp:56-71)
    over a uniform random uint32 token stream: input[b,t] = tok[pos+t],
    target = the next token, pos += T per row."""
    import numpy as np
    rng = np.random.default_rng(seed)
    stream = rng.integers(0, V, n * B * T + 1, dtype=np.int64).astype(np.int32)
    out = []
    pos = 0
    for _ in range(n):
        inp = np.empty(B * T, np.int32)
        tgt = np.empty(B * T, np.int32)
        for b in range(B):
            inp[b * T:(b + 1) * T] = stream[pos:pos + T]
            tgt[b * T:(b + 1) * T] = stream[pos + 1:pos + T + 1]
            pos += T
        out.append((inp, tgt))
    return out


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` measured with rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy's counters), as recorded
    in the traffic table under profiles/; None when no row names it."""
    path = os.path.join(ROOT, "profiles", "c3_traffic.md")
    if not kernel or not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip().strip("`") for c in line.split("|")]
        if len(cells) > 3 and cells[1] == kernel:
            try:
                return int(float(cells[-2]))
            except ValueError:
                return None
    return None


def cpu_baseline(model, adapt, cname="c3"):
    """Oracle (CPU restatement of the reference step) on this host, bounded
    sample: (A) one transformer layer of the config, forward+backward+AdamW,
    B=1 x T=1024, with a 2048-entry vocabulary so the LM head is negligible;
    (B) the LM head + cross entropy + final norm alone (0 layers, full
    vocabulary) on 256 tokens.  Per-token cost of the model =
    layers * A/1024 + B/256 (the head is linear in tokens, a layer is linear
    in B at fixed T=1024)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    rng = np.random.default_rng(7)

    def run(mc, B, T):
        m = O.OracleModel(mc, adapt)
        H, I, V = mc["hidden"], mc["inter"], mc["vocab"]
        qd, kvd = mc["n_q"] * mc["head_dim"], mc["n_kv"] * mc["head_dim"]
        w = lambda *s: O.bf16_from_f32((rng.standard_normal(s, np.float32) * 0.02))
        ones = O.bf16_from_f32(np.ones(H, np.float32))
        m.set_weight("model.embed_tokens.weight", w(V, H))
        m.set_weight("model.norm.weight", ones)
        if not mc["tie"]:
            m.set_weight("lm_head.weight", w(V, H))
        for l in range(mc["layers"]):
            p = f"model.layers.{l}."
            for n, a in (("input_layernorm.weight", ones), ("post_attention_layernorm.weight", ones),
                         ("self_attn.q_proj.weight", w(qd, H)), ("self_attn.k_proj.weight", w(kvd, H)),
                         ("self_attn.v_proj.weight", w(kvd, H)), ("self_attn.o_proj.weight", w(H, qd)),
                         ("self_attn.q_proj.bias", np.zeros(qd, np.uint16)),
                         ("self_attn.k_proj.bias", np.zeros(kvd, np.uint16)),
                         ("self_attn.v_proj.bias", np.zeros(kvd, np.uint16)),
                         ("mlp.gate_proj.weight", w(I, H)), ("mlp.up_proj.weight", w(I, H)),
                         ("mlp.down_proj.weight", w(H, I))):
                m.set_weight(p + n, a)
        toks = rng.integers(0, V, B * T + 1).astype(np.int32)
        t0 = time.perf_counter()
        m.step(toks[:-1], toks[1:], B, T)
        return time.perf_counter() - t0

    layer_mc = dict(model, layers=1, vocab=2048)
    head_mc = dict(model, layers=0)
    t_layer = run(layer_mc, 1, 1024)
    t_head = run(head_mc, 1, 256)
    per_tok = model["layers"] * t_layer / 1024.0 + t_head / 256.0
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(1.0 / per_tok, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": ("oracle step on one %s layer (B=1, T=1024, %.1f s) and the %s LM head + "
                       "CE on 256 tokens (%.1f s), extrapolated to %d layers"
                       % (cname, t_layer, cname, t_head, model["layers"]))}


C5 = dict(tokens=4 << 20, dim=512, chunk=65536, comps=16, k=32, iters=25)
C5_WORK = ("c5: centroid accumulator + merge stress, 4M F32 hidden states of dim 512 from a "
           "16-component Gaussian mixture, lognormal gradient norms, 64 cumulative snapshots, "
           "k-means++ k=32 with 25 Lloyd iterations")


def bench_c5(args):
    """c5: the Centroid Accumulator over 4M token states resident in HBM
    (one ta_centroid_accumulate_f32n call per 65536-token snapshot, each
    snapshot's sums copied to host memory), then the k-means merge on the 64
    snapshots.  A step is the whole job; tokens/s = 4M / step time.  The
    roofline is the accumulate call (partial-row and reduce launches),
    timed with events on the stream it is launched on; algorithmic bytes
    per call = chunk * (dim + 1) * 4 (h and n read once)."""
    import ctypes
    import numpy as np
    import torch
    import tadapt
    c = C5
    nchunk = c["tokens"] // c["chunk"]
    g = torch.Generator(device="cuda")
    g.manual_seed(2026)
    means = torch.randn(c["comps"], c["dim"], generator=g, device="cuda")
    h = torch.empty(c["tokens"], c["dim"], device="cuda")
    for i in range(nchunk):
        sl = slice(i * c["chunk"], (i + 1) * c["chunk"])
        lab = torch.randint(0, c["comps"], (c["chunk"],), generator=g, device="cuda")
        h[sl] = means[lab] + 0.3 * torch.randn(c["chunk"], c["dim"], generator=g, device="cuda")
    n = torch.exp(torch.randn(c["tokens"], generator=g, device="cuda"))  # lognormal(0, 1)
    acc = torch.zeros(c["dim"] + 1, dtype=torch.float64, device="cuda")
    snap_acc = torch.empty(nchunk, c["dim"] + 1, dtype=torch.float64, pin_memory=True)
    C = torch.empty(c["k"] * c["dim"], device="cuda")
    A = torch.empty(nchunk, dtype=torch.int32, device="cuda")
    M = torch.empty(c["k"], dtype=torch.float64, device="cuda")
    Sd = torch.empty(c["k"], dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(nchunk)]

    def job(timed):
        acc.zero_()
        for i in range(nchunk):
            off = i * c["chunk"]
            if timed:
                ev[i][0].record(stream)
            tadapt.call("ta_centroid_accumulate_f32n", h[off].data_ptr(), n[off:].data_ptr(),
                        c["chunk"], c["dim"], acc.data_ptr(), sp)
            if timed:
                ev[i][1].record(stream)
            snap_acc[i].copy_(acc, non_blocking=True)
        torch.cuda.synchronize()
        a = snap_acc.numpy()
        X = torch.from_numpy((a[:, :-1] / a[:, -1:]).astype(np.float32)).cuda()
        W = torch.from_numpy(a[:, -1].astype(np.float32)).cuda()
        tadapt.call("ta_kmeans_pp", X.data_ptr(), W.data_ptr(), nchunk, c["dim"], c["k"],
                    c["iters"], ctypes.c_uint64(5), C.data_ptr(), A.data_ptr(), M.data_ptr(),
                    Sd.data_ptr(), sp)

    for _ in range(args.warmup):
        job(False)
    launch_ms = 0.0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        job(True)
        torch.cuda.synchronize()
        launch_ms += sum(a.elapsed_time(b) for a, b in ev)
    dt = time.perf_counter() - t0
    calls = nchunk * args.steps
    per_call = launch_ms / calls
    bytes_call = c["chunk"] * (c["dim"] + 1) * 4
    achieved = bytes_call / (per_call * 1e-3) / 1e9
    out = {
        "metric": "c5 centroid accumulate + merge tokens/s",
        "value": round(c["tokens"] * args.steps / dt, 1),
        "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32/f64",
        "data": "synthetic (seeded Gaussian mixture generated on the device)",
        "config": {"workload": C5_WORK, "tokens": c["tokens"], "dim": c["dim"],
                   "snapshots": nchunk, "k": c["k"], "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "ta::k_centroid_part<false> + ta::k_centroid_reduce (one call)",
                     "launches": calls, "avg_launch_us": round(per_call * 1e3, 1),
                     "algorithmic_per_launch": {"bytes": bytes_call},
                     "share_of_step": round(launch_ms * 1e-3 / dt, 4)},
        "mass_top3": [round(float(x), 3) for x in M.cpu().numpy()[:3]],
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--config", choices=sorted(CONFIGS) + ["c5"], default="c3",
                    help="workload (default c3, the headline metric's config)")
    ap.add_argument("--categories", action="store_true",
                    help="print the per-kernel-class time split to stderr")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="run one plain device copy of MIB MiB first (counter calibration)")
    ap.add_argument("--ce-in-dx", action="store_true",
                    help="the measured alternative: cross-entropy gradient formed inside the LM "
                         "head's input-gradient GEMM (TA_ENGINE_CE_IN_DX)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU (one process, one MI355X); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    if args.config == "c5":
        return bench_c5(args)
    import torch
    import tadapt

    model, adapt, B, T, recompute, workload = CONFIGS[args.config]
    eng = tadapt.Engine(model, adapt, B, T, recompute=recompute, ce_in_dx=args.ce_in_dx)
    eng.init_random(seed=20261201, std=0.02)
    nb = args.warmup + args.steps + len(CAT_NAMES) + len(tadapt.KPROF_KERNELS)
    batches = token_batches(nb, B, T, model["vocab"], 1)
    dev = [(torch.from_numpy(i).cuda(), torch.from_numpy(t).cuda()) for i, t in batches]
    it = iter(dev)

    if args.copy_calibration:
        # a plain device copy of known size, for scaling the HBM byte
        # counters of a --pmc run (FETCH_SIZE / WRITE_SIZE of this kernel
        # against exactly copy_calibration MiB read and written)
        n = args.copy_calibration << 19
        src = torch.ones(n, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        eng.step_resident(*next(it))
    # one step per kernel class with that class's launches event-timed (not
    # part of the timed region): per-class time, algorithmic TFLOP/s and
    # GB/s against the MI355X peaks
    classes, raw = {}, {}
    for c in range(len(CAT_NAMES)):
        eng.profile(c)
        eng.step_resident(*next(it))
        v = eng.profile_read()
        sec = max(v["ms"], 1e-9) * 1e-3
        tf, gb = v["flops"] / sec / 1e12, v["bytes"] / sec / 1e9
        classes[CAT_NAMES[c]] = {"ms": round(v["ms"], 3), "launches": v["launches"],
                                 "tflops": round(tf, 1), "gbs": round(gb, 1),
                                 "mfma_frac": round(tf / PEAK_BF16_TFLOPS, 4),
                                 "hbm_frac": round(gb / PEAK_HBM_GBS, 4)}
        raw[CAT_NAMES[c]] = v
        if args.categories:
            print(f"  {CAT_NAMES[c]:14s} {v['ms']:8.2f} ms  {v['launches']:5d} launches  "
                  f"{tf:7.1f} TFLOP/s  {gb:7.1f} GB/s", file=sys.stderr)
    eng.profile(-1)
    bwd = [raw["gemm_dx"], raw["lm_head_bwd"]]
    bwd_util = round(sum(v["flops"] for v in bwd) / max(sum(v["ms"] for v in bwd), 1e-9) / 1e9
                     / PEAK_BF16_TFLOPS, 4)
    # survey: one step per instrumented kernel, to find the kernel with the
    # largest share of the step (not part of the timed region)
    split = {}
    for k in range(len(tadapt.KPROF_KERNELS)):
        tadapt.kprof_select(k)
        eng.step_resident(*next(it))
        split[k] = tadapt.kprof_read()
    tadapt.kprof_select(-1)
    dom = max(split, key=lambda k: split[k]["ms"])
    if args.categories:
        for k, v in split.items():
            if not v["launches"]:
                continue
            sec = v["ms"] * 1e-3
            print(f"  kernel {tadapt.KPROF_KERNELS[k]:14s} {v['ms']:7.2f} ms/step {v['launches']:4d} "
                  f"launches  {v['flops'] / sec / 1e12:7.1f} TFLOP/s  {v['bytes'] / sec / 1e9:7.1f} GB/s "
                  f"(algorithmic)  {tadapt.kprof_name(k)}", file=sys.stderr)

    # timed region; the dominant kernel is event-timed on its launch stream
    # in a sample of the steps (every fifth, or the last of fewer than five):
    # a timed launch costs a few microseconds of idle GPU on each side,
    # about 0.4 ms per c3 step for the chain GEMM's 56 launches
    sampled = [i for i in range(args.steps) if (i + 1) % 5 == 0] or [args.steps - 1]
    tadapt.kprof_select(dom)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    last = None
    for i in range(args.steps):
        tadapt.kprof_pause(i not in sampled)
        last = eng.step_resident(*next(it))
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    prof = tadapt.kprof_read()
    tadapt.kprof_select(-1)

    tokens = B * T * args.steps
    value = tokens / dt
    sec = prof["ms"] * 1e-3
    t_mfma = prof["flops"] / (PEAK_BF16_TFLOPS * 1e12)
    t_hbm = prof["bytes"] / (PEAK_HBM_GBS * 1e9)
    if t_mfma >= t_hbm:
        achieved = prof["flops"] / sec / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4)}
    else:
        achieved = prof["bytes"] / sec / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4)}
    name = tadapt.kprof_name(dom)
    # the recorded counter runs are of the c3 step
    roof["traffic"] = measured_traffic(name) if args.config == "c3" else None
    roof["kernel"] = name
    roof["launches"] = prof["launches"]
    roof["timed_steps"] = len(sampled)
    roof["avg_launch_us"] = round(prof["ms"] * 1e3 / max(prof["launches"], 1), 1)
    roof["algorithmic_per_launch"] = {
        "flops": round(prof["flops"] / max(prof["launches"], 1)),
        "bytes": round(prof["bytes"] / max(prof["launches"], 1))}
    # (the timed launches cover len(sampled) of the steps)
    roof["share_of_step"] = round(sec / len(sampled) / (dt / args.steps), 4)

    out = {
        "metric": METRIC if args.config == "c3" else f"train tokens/s ({args.config})",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform random token ids; random-init N(0,0.02) BF16 base)",
        "config": {"workload": workload + (" (cross-entropy gradient inside the LM head's "
                                           "input-gradient GEMM)" if args.ce_in_dx else ""),
                   "global_batch": B, "seq_len": T, "layers": model["layers"],
                   "hidden": model["hidden"], "parallelism": "single GPU"},
        "roofline": roof,
        # the metric's other two quantities, from the per-class timing:
        # MFMA utilisation of the backward GEMMs (the frozen-base input
        # gradients and the LM head's input gradient, flops over time) and
        # achieved HBM bandwidth of the norm, attention backward and AdamW
        # kernels, each against the MI355X peak
        "bwd_gemm_mfma_util": bwd_util,
        "hbm_gbs": {k: {"gbs": classes[c]["gbs"], "frac": classes[c]["hbm_frac"]}
                    for k, c in (("norm", "norm"), ("attention_bwd", "attn_bwd"),
                                 ("adamw", "adamw_tail"))},
        "classes": classes,
        "loss": round(last["loss"], 4),
    }
    del eng
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(model, adapt, args.config)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
