"""Shared helpers for full-step comparisons of the GPU engine with the CPU
oracle (test infrastructure): a seeded synthetic Qwen2 base under HF tensor
names, the engine/oracle pair built from it, and the comparison metric."""
import numpy as np

import oracle as O


def base_tensors(mc, seed):
    """HF-named synthetic Qwen2 base: N(0, 0.02) weights, unit norms, zero biases."""
    rng = np.random.default_rng(seed)
    H, I, V = mc["hidden"], mc["inter"], mc["vocab"]
    qd, kvd = mc["n_q"] * mc["head_dim"], mc["n_kv"] * mc["head_dim"]

    def w(*shape):
        return O.bf16_from_f32((rng.standard_normal(shape) * 0.02).astype(np.float32))

    one = lambda n: O.bf16_from_f32(np.ones(n, np.float32))
    zero = lambda n: np.zeros(n, np.uint16)
    t = {"model.embed_tokens.weight": w(V, H), "model.norm.weight": one(H)}
    if not mc.get("tie", 1):
        t["lm_head.weight"] = w(V, H)
    for l in range(mc["layers"]):
        p = f"model.layers.{l}."
        t[p + "input_layernorm.weight"] = one(H)
        t[p + "post_attention_layernorm.weight"] = one(H)
        t[p + "self_attn.q_proj.weight"] = w(qd, H)
        t[p + "self_attn.q_proj.bias"] = zero(qd)
        t[p + "self_attn.k_proj.weight"] = w(kvd, H)
        t[p + "self_attn.k_proj.bias"] = zero(kvd)
        t[p + "self_attn.v_proj.weight"] = w(kvd, H)
        t[p + "self_attn.v_proj.bias"] = zero(kvd)
        t[p + "self_attn.o_proj.weight"] = w(H, qd)
        t[p + "mlp.gate_proj.weight"] = w(I, H)
        t[p + "mlp.up_proj.weight"] = w(I, H)
        t[p + "mlp.down_proj.weight"] = w(H, I)
    return t


def make_pair(mc, ac, B, T, seed, recompute=False):
    tensors = base_tensors(mc, seed)
    orc = O.OracleModel(mc, ac)
    import tadapt
    eng = tadapt.Engine(mc, ac, B, T, recompute=recompute)
    for name, arr in tensors.items():
        orc.set_weight(name, arr)
        eng.set_weight(name, arr)
    return orc, eng


def chat_tokens(V, B, T, rng):
    """uniform ids with a few assistant spans (<|im_start|> assistant ... <|im_end|>)
    so that some targets survive the trainer's masking."""
    toks = rng.integers(0, min(V, 150000), B * T).astype(np.int32)
    if V > 151645:
        for b in range(B):
            s = b * T + 5
            toks[s], toks[s + 1] = 151644, 77091
            toks[s + 12] = 151645
    return toks


def span_tokens(B, T, rng):
    """Uniform ids with one assistant span (<|im_start|> assistant ...
    <|im_end|>) over almost every row, so the trainer's masking keeps
    nearly all targets."""
    toks = rng.integers(0, 150000, B * T + 1).astype(np.int32)
    for b in range(B):
        toks[b * T + 3], toks[b * T + 4] = 151644, 77091
        toks[b * T + T - 8] = 151645
    return toks


def rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / nb) if nb > 0 else float(np.linalg.norm(a))


def pairs(mc, ac):
    for l in range(mc["layers"]):
        for ti, t in enumerate(O.TARGETS):
            if (ac["inject_mask"] >> ti) & 1:
                yield l, t
