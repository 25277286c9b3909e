// per_op.cpp — the reference's per-op upper layers on this backend:
// Qwen2Base::forward / backward (src/base/arch/qwen2.cu:47-308),
// AdapterModel (src/adapter/adapter_model.cu:41-229) and AdamW
// (src/trainer/adamw.cu:9-38), composed from ops:: and the GEMM entry points
// on the Device's stream, with the reference's op order and BF16 rounding
// points.  Host code only.  Where the reference fills a buffer with zeros
// only for a call that overwrites it (a beta = 0 GEMM, sdpa_bwd) the fill is
// left out, and the frozen norms' weight gradients, which the reference
// computes and drops, are not computed (ops::rms_norm_bwd with dw = NULL).
#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "ta_backend.h"
#include <tensor/adapter/adapter_model.hpp>
#include <tensor/backend/cuda/ops.hpp>
#include <tensor/backend/cuda/tensor.hpp>
#include <tensor/base/arch/qwen2.hpp>
#include <tensor/trainer/adamw.hpp>

namespace {

using tensor::backend::cuda::bf16_t;
using tensor::backend::cuda::Device;
using tensor::backend::cuda::GemmParams;
using tensor::backend::cuda::Tensor;
using tensor::core::DType;
namespace ops = tensor::backend::cuda::ops;
using Sz = std::size_t;

// BLAS column-major C = alpha op(A) op(B) + beta C (row-major operands read
// as their transposes), BF16 or F32 in and out
void gemm16(const Device& dev, bool ta, bool tb, int M, int N, int K, float alpha, const bf16_t* A,
            int lda, const bf16_t* B, int ldb, float beta, bf16_t* C, int ldc) {
    GemmParams p;
    p.transA = ta;
    p.transB = tb;
    p.M = M;
    p.N = N;
    p.K = K;
    p.alpha = alpha;
    p.beta = beta;
    tensor::backend::cuda::gemm_bf16(dev, p, A, lda, B, ldb, C, ldc);
}
void gemm32(const Device& dev, bool ta, bool tb, int M, int N, int K, float alpha, const float* A,
            int lda, const float* B, int ldb, float beta, float* C, int ldc) {
    GemmParams p;
    p.transA = ta;
    p.transB = tb;
    p.M = M;
    p.N = N;
    p.K = K;
    p.alpha = alpha;
    p.beta = beta;
    tensor::backend::cuda::gemm_f32(dev, p, A, lda, B, ldb, C, ldc);
}

// y[BT, out] = bf16(x[BT, in] W^T), W [out, in]  (qwen2.cu:21-30)
void linear_fwd(const Device& dev, const Tensor& W, const Tensor& x, Tensor& y, int BT, int in,
                int out) {
    gemm16(dev, true, false, out, BT, in, 1.f, W.bf16(), in, x.bf16(), in, 0.f, y.bf16(), out);
}
// dx[BT, in] = bf16(dy[BT, out] W + beta dx)  (qwen2.cu:32-41)
void linear_dx(const Device& dev, const Tensor& W, const Tensor& dy, Tensor& dx, int BT, int out,
               int in, float beta) {
    gemm16(dev, false, false, in, BT, out, 1.f, W.bf16(), in, dy.bf16(), out, beta, dx.bf16(), in);
}

Tensor bf16_rows(Sz rows, Sz cols, const Device& dev) { return Tensor::empty_bf16({rows, cols}, dev); }

// a copy of src in a new tensor, on the device's stream
Tensor clone(const Tensor& src, const Device& dev) {
    Tensor t = Tensor::empty(src.shape(), src.dtype(), dev);
    const hipError_t e =
        hipMemcpyAsync(t.data(), src.data(), src.nbytes(), hipMemcpyDeviceToDevice, dev.stream());
    if (e != hipSuccess) throw std::runtime_error(std::string("clone: ") + hipGetErrorString(e));
    return t;
}

void need(bool ok, const std::string& what) {
    if (!ok) throw std::runtime_error(what);
}

}  // namespace

// ── Qwen2Base ───────────────────────────────────────────────────────────
namespace tensor::base::arch {

Qwen2ForwardResult Qwen2Base::forward(const FrozenBase& base, const Tensor& tokens, int B, int T,
                                      const Device& dev, adapter::AdapterModel* adapter) {
    const BaseConfig& c = base.config;
    const int BT = B * T, H = (int)c.hidden_size, I = (int)c.intermediate_size;
    const int Hq = (int)c.num_q_heads, Hkv = (int)c.num_kv_heads, hd = (int)c.head_dim;
    const int V = (int)c.vocab_size, qd = Hq * hd, kvd = Hkv * hd;
    const float eps = c.rms_norm_eps, theta = c.rope_theta;
    hipStream_t s = dev.stream();
    need(B > 0 && T > 0, "Qwen2Base::forward: B and T must be positive");
    need(base.layers.size() == c.num_layers, "Qwen2Base::forward: layer count mismatch");
    need(tokens.dtype() == DType::I32 && tokens.numel() >= (Sz)BT,
         "Qwen2Base::forward: tokens must be I32 with B*T elements");
    need(!adapter || adapter->layers.size() == c.num_layers,
         "Qwen2Base::forward: adapter layer count mismatch");

    Qwen2ForwardResult r;
    r.embed_in = bf16_rows(BT, H, dev);
    ops::embed_fwd(base.embed_w.bf16(), tokens.i32(), r.embed_in.bf16(), BT, H, s);
    Tensor res = clone(r.embed_in, dev);  // the residual stream
    r.layer_cache.resize(c.num_layers);

    for (Sz l = 0; l < c.num_layers; l++) {
        const LayerWeights& w = base.layers[l];
        Qwen2LayerCache& lc = r.layer_cache[l];
        // attention half: norm, q/k/v (+ bias, + LoRA), RoPE, attention, o (+ LoRA)
        lc.pre_attn_res = clone(res, dev);
        lc.in_norm_rms = Tensor::empty_f32({(Sz)BT}, dev);
        lc.x_normed = bf16_rows(BT, H, dev);
        ops::rms_norm_fwd(res.bf16(), w.input_norm_w.bf16(), lc.x_normed.bf16(),
                          lc.in_norm_rms.f32(), B, T, H, eps, s);
        lc.Q = bf16_rows(BT, qd, dev);
        lc.K = bf16_rows(BT, kvd, dev);
        lc.V = bf16_rows(BT, kvd, dev);
        linear_fwd(dev, w.q_proj_w, lc.x_normed, lc.Q, BT, H, qd);
        ops::add_bias(lc.Q.bf16(), w.q_proj_b.bf16(), BT, qd, s);
        linear_fwd(dev, w.k_proj_w, lc.x_normed, lc.K, BT, H, kvd);
        ops::add_bias(lc.K.bf16(), w.k_proj_b.bf16(), BT, kvd, s);
        linear_fwd(dev, w.v_proj_w, lc.x_normed, lc.V, BT, H, kvd);
        ops::add_bias(lc.V.bf16(), w.v_proj_b.bf16(), BT, kvd, s);
        if (adapter) {
            adapter::LayerAdapter& la = adapter->layers[l];
            adapter->apply_lora_fwd(l, la.lora_q, lc.x_normed, lc.Q, BT, dev);
            adapter->apply_lora_fwd(l, la.lora_k, lc.x_normed, lc.K, BT, dev);
            adapter->apply_lora_fwd(l, la.lora_v, lc.x_normed, lc.V, BT, dev);
        }
        ops::rope_fwd(lc.Q.bf16(), B, T, Hq, hd, theta, s);
        ops::rope_fwd(lc.K.bf16(), B, T, Hkv, hd, theta, s);
        lc.attn_out = bf16_rows(BT, qd, dev);
        lc.attn_w = Tensor::empty_f32({(Sz)B, (Sz)Hq, (Sz)T, (Sz)T}, dev);
        ops::sdpa_fwd(lc.Q.bf16(), lc.K.bf16(), lc.V.bf16(), lc.attn_out.bf16(), lc.attn_w.f32(),
                      B, T, Hq, Hkv, hd, dev);
        lc.h_mid = bf16_rows(BT, H, dev);
        linear_fwd(dev, w.o_proj_w, lc.attn_out, lc.h_mid, BT, qd, H);
        if (adapter)
            adapter->apply_lora_fwd(l, adapter->layers[l].lora_o, lc.attn_out, lc.h_mid, BT, dev);
        ops::add_inplace(res.bf16(), lc.h_mid.bf16(), BT * H, s);

        // MLP half: norm, gate and up, SiLU product, down
        lc.pre_ffn_res = clone(res, dev);
        lc.post_norm_rms = Tensor::empty_f32({(Sz)BT}, dev);
        lc.x_normed2 = bf16_rows(BT, H, dev);
        ops::rms_norm_fwd(res.bf16(), w.post_norm_w.bf16(), lc.x_normed2.bf16(),
                          lc.post_norm_rms.f32(), B, T, H, eps, s);
        lc.gate_out = bf16_rows(BT, I, dev);
        lc.up_out = bf16_rows(BT, I, dev);
        linear_fwd(dev, w.gate_proj_w, lc.x_normed2, lc.gate_out, BT, H, I);
        linear_fwd(dev, w.up_proj_w, lc.x_normed2, lc.up_out, BT, H, I);
        lc.act_out = bf16_rows(BT, I, dev);
        ops::silu_mul_fwd(lc.gate_out.bf16(), lc.up_out.bf16(), lc.act_out.bf16(), BT * I, s);
        lc.ffn_out = bf16_rows(BT, H, dev);
        linear_fwd(dev, w.down_proj_w, lc.act_out, lc.ffn_out, BT, I, H);
        ops::add_inplace(res.bf16(), lc.ffn_out.bf16(), BT * H, s);
    }

    // final norm and the LM head (the embedding when tied)
    r.x_final = clone(res, dev);
    r.final_rms = Tensor::empty_f32({(Sz)BT}, dev);
    Tensor xn = bf16_rows(BT, H, dev);
    ops::rms_norm_fwd(res.bf16(), base.final_norm_w.bf16(), xn.bf16(), r.final_rms.f32(), B, T,
                      H, eps, s);
    const Tensor& head = c.tie_embeddings ? base.embed_w : base.lm_head_w;
    r.logits = bf16_rows(BT, V, dev);
    r.dlogits = bf16_rows(BT, V, dev);
    linear_fwd(dev, head, xn, r.logits, BT, H, V);
    return r;
}

std::vector<Qwen2Base::LayerGrads> Qwen2Base::backward(const FrozenBase& base,
                                                       const Qwen2ForwardResult& fwd, int B, int T,
                                                       const Device& dev,
                                                       adapter::AdapterModel* adapter) {
    const BaseConfig& c = base.config;
    const int BT = B * T, H = (int)c.hidden_size, I = (int)c.intermediate_size;
    const int Hq = (int)c.num_q_heads, Hkv = (int)c.num_kv_heads, hd = (int)c.head_dim;
    const int V = (int)c.vocab_size, qd = Hq * hd, kvd = Hkv * hd;
    const float eps = c.rms_norm_eps, theta = c.rope_theta;
    hipStream_t s = dev.stream();
    need(fwd.layer_cache.size() == c.num_layers && base.layers.size() == c.num_layers,
         "Qwen2Base::backward: layer count mismatch");
    need(!adapter || adapter->layers.size() == c.num_layers,
         "Qwen2Base::backward: adapter layer count mismatch");

    std::vector<LayerGrads> out(c.num_layers);
    const Tensor& head = c.tie_embeddings ? base.embed_w : base.lm_head_w;
    Tensor dres = bf16_rows(BT, H, dev);
    linear_dx(dev, head, fwd.dlogits, dres, BT, V, H, 0.f);
    Tensor g = bf16_rows(BT, H, dev);  // gradient of the residual stream
    ops::rms_norm_bwd(dres.bf16(), fwd.x_final.bf16(), base.final_norm_w.bf16(),
                      fwd.final_rms.f32(), g.bf16(), nullptr, B, T, H, eps, s);

    for (int l = (int)c.num_layers - 1; l >= 0; l--) {
        const LayerWeights& w = base.layers[l];
        const Qwen2LayerCache& lc = fwd.layer_cache[l];
        LayerGrads& lg = out[l];

        // MLP half
        Tensor dact = bf16_rows(BT, I, dev);
        linear_dx(dev, w.down_proj_w, g, dact, BT, H, I, 0.f);
        Tensor dgate = bf16_rows(BT, I, dev), dup = bf16_rows(BT, I, dev);
        ops::silu_mul_bwd(dact.bf16(), lc.gate_out.bf16(), lc.up_out.bf16(), dgate.bf16(),
                          dup.bf16(), BT * I, s);
        Tensor dxn2 = bf16_rows(BT, H, dev);
        linear_dx(dev, w.gate_proj_w, dgate, dxn2, BT, I, H, 0.f);
        linear_dx(dev, w.up_proj_w, dup, dxn2, BT, I, H, 1.f);
        lg.dx_ffn_in = clone(dxn2, dev);
        Tensor dn2 = bf16_rows(BT, H, dev);
        ops::rms_norm_bwd(dxn2.bf16(), lc.pre_ffn_res.bf16(), w.post_norm_w.bf16(),
                          lc.post_norm_rms.f32(), dn2.bf16(), nullptr, B, T, H, eps, s);
        ops::add_inplace(g.bf16(), dn2.bf16(), BT * H, s);

        // attention half: o (+ LoRA), attention, RoPE, q/k/v (+ LoRA), norm
        lg.do_proj = clone(g, dev);
        Tensor dattn = bf16_rows(BT, qd, dev);
        linear_dx(dev, w.o_proj_w, g, dattn, BT, H, qd, 0.f);
        if (adapter) adapter->apply_lora_bwd(adapter->layers[l].lora_o, lc.attn_out, g, dattn, BT, dev);
        lg.dQ = bf16_rows(BT, qd, dev);
        lg.dK = bf16_rows(BT, kvd, dev);
        lg.dV = bf16_rows(BT, kvd, dev);
        ops::sdpa_bwd(dattn.bf16(), lc.Q.bf16(), lc.K.bf16(), lc.V.bf16(), lc.attn_w.f32(),
                      lg.dQ.bf16(), lg.dK.bf16(), lg.dV.bf16(), B, T, Hq, Hkv, hd, dev);
        ops::rope_bwd(lg.dQ.bf16(), B, T, Hq, hd, theta, s);
        ops::rope_bwd(lg.dK.bf16(), B, T, Hkv, hd, theta, s);
        Tensor dxn = bf16_rows(BT, H, dev);
        linear_dx(dev, w.q_proj_w, lg.dQ, dxn, BT, qd, H, 0.f);
        linear_dx(dev, w.k_proj_w, lg.dK, dxn, BT, kvd, H, 1.f);
        linear_dx(dev, w.v_proj_w, lg.dV, dxn, BT, kvd, H, 1.f);
        if (adapter) {
            adapter::LayerAdapter& la = adapter->layers[l];
            adapter->apply_lora_bwd(la.lora_q, lc.x_normed, lg.dQ, dxn, BT, dev);
            adapter->apply_lora_bwd(la.lora_k, lc.x_normed, lg.dK, dxn, BT, dev);
            adapter->apply_lora_bwd(la.lora_v, lc.x_normed, lg.dV, dxn, BT, dev);
        }
        lg.dx_attn_in = clone(dxn, dev);
        Tensor dn1 = bf16_rows(BT, H, dev);
        ops::rms_norm_bwd(dxn.bf16(), lc.pre_attn_res.bf16(), w.input_norm_w.bf16(),
                          lc.in_norm_rms.f32(), dn1.bf16(), nullptr, B, T, H, eps, s);
        ops::add_inplace(g.bf16(), dn1.bf16(), BT * H, s);
    }
    return out;
}

}  // namespace tensor::base::arch

// ── AdapterModel ────────────────────────────────────────────────────────
namespace tensor::adapter {

LoraPair AdapterModel::make_pair(int in_dim, int out_dim, int rank, const Device& dev) {
    LoraPair lp;
    lp.in_dim = in_dim;
    lp.out_dim = out_dim;
    lp.rank = rank;
    const Sz r = rank, in = in_dim, out = out_dim;
    lp.A_bf16 = Tensor::empty_bf16({r, in}, dev);
    lp.A_f32 = Tensor::empty_f32({r, in}, dev);
    tensor::backend::cuda::check_status(
        ta_lora_kaiming_init(lp.A_f32.f32(), lp.A_bf16.bf16(), (int64_t)r * in, in_dim,
                             dev.stream()),
        "AdapterModel: A init");
    lp.B_bf16 = Tensor::zeros({out, r}, DType::BF16, dev);
    lp.B_f32 = Tensor::zeros_f32({out, r}, dev);
    lp.mA = Tensor::zeros_f32({r, in}, dev);
    lp.vA = Tensor::zeros_f32({r, in}, dev);
    lp.gA = Tensor::zeros_f32({r, in}, dev);
    lp.mB = Tensor::zeros_f32({out, r}, dev);
    lp.vB = Tensor::zeros_f32({out, r}, dev);
    lp.gB = Tensor::zeros_f32({out, r}, dev);
    return lp;
}

AdapterModel AdapterModel::create(const base::FrozenBase& base, const AdapterConfig& cfg,
                                  const Device& dev) {
    need(cfg.rank > 0, "AdapterModel::create: rank must be positive");
    const base::BaseConfig& c = base.config;
    const int H = (int)c.hidden_size, qd = (int)(c.num_q_heads * c.head_dim),
              kvd = (int)(c.num_kv_heads * c.head_dim);
    AdapterModel m;
    m.cfg_ = cfg;
    m.layers.resize(c.num_layers);
    for (auto& la : m.layers) {
        la.lora_q = make_pair(H, qd, cfg.rank, dev);
        la.lora_k = make_pair(H, kvd, cfg.rank, dev);
        la.lora_v = make_pair(H, kvd, cfg.rank, dev);
        la.lora_o = make_pair(qd, H, cfg.rank, dev);
    }
    return m;
}

void AdapterModel::apply_lora_fwd(std::size_t, LoraPair& lp, const Tensor& x, Tensor& out, int BT,
                                  const Device& dev) {
    const int r = lp.rank, in = lp.in_dim, n = lp.out_dim;
    Tensor h = bf16_rows(BT, r, dev);  // x A^T
    gemm16(dev, true, false, r, BT, in, 1.f, lp.A_bf16.bf16(), in, x.bf16(), in, 0.f, h.bf16(), r);
    Tensor d = bf16_rows(BT, n, dev);  // h B^T
    gemm16(dev, true, false, n, BT, r, 1.f, lp.B_bf16.bf16(), r, h.bf16(), r, 0.f, d.bf16(), n);
    ops::lora_add(out.bf16(), d.bf16(), cfg_.alpha / (float)cfg_.rank, BT * n, dev.stream());
}

void AdapterModel::apply_lora_bwd(LoraPair& lp, const Tensor& x, const Tensor& grad_out,
                                  Tensor& grad_x, int BT, const Device& dev) {
    const int r = lp.rank, in = lp.in_dim, n = lp.out_dim;
    const float scale = cfg_.alpha / (float)cfg_.rank;
    hipStream_t s = dev.stream();
    Tensor h = bf16_rows(BT, r, dev);  // x A^T again
    gemm16(dev, true, false, r, BT, in, 1.f, lp.A_bf16.bf16(), in, x.bf16(), in, 0.f, h.bf16(), r);
    // the weight gradients run as F32 GEMMs of the BF16 values
    Tensor h32 = Tensor::empty_f32({(Sz)BT, (Sz)r}, dev);
    Tensor go32 = Tensor::empty_f32({(Sz)BT, (Sz)n}, dev);
    Tensor x32 = Tensor::empty_f32({(Sz)BT, (Sz)in}, dev);
    ops::cast_bf16_to_f32(h.bf16(), h32.f32(), BT * r, s);
    ops::cast_bf16_to_f32(grad_out.bf16(), go32.f32(), BT * n, s);
    ops::cast_bf16_to_f32(x.bf16(), x32.f32(), BT * in, s);
    // gB[n, r] += scale * grad_out^T h
    gemm32(dev, false, true, r, n, BT, scale, h32.f32(), r, go32.f32(), n, 1.f, lp.gB.f32(), r);
    // dh[BT, r] = bf16(grad_out B)
    Tensor dh = bf16_rows(BT, r, dev);
    gemm16(dev, false, false, r, BT, n, 1.f, lp.B_bf16.bf16(), r, grad_out.bf16(), n, 0.f,
           dh.bf16(), r);
    Tensor dh32 = Tensor::empty_f32({(Sz)BT, (Sz)r}, dev);
    ops::cast_bf16_to_f32(dh.bf16(), dh32.f32(), BT * r, s);
    // gA[r, in] += scale * dh^T x
    gemm32(dev, false, true, in, r, BT, scale, x32.f32(), in, dh32.f32(), r, 1.f, lp.gA.f32(), in);
    // grad_x = bf16(grad_x + scale * dh A)
    gemm16(dev, false, false, in, BT, r, scale, lp.A_bf16.bf16(), in, dh.bf16(), r, 1.f,
           grad_x.bf16(), in);
}

void AdapterModel::zero_grad(const Device& dev) {
    for (auto& la : layers)
        for (LoraPair* lp : {&la.lora_q, &la.lora_k, &la.lora_v, &la.lora_o}) {
            lp->gA.zero_(dev);
            lp->gB.zero_(dev);
        }
}

std::size_t AdapterModel::param_count() const {
    std::size_t n = 0;
    for (const auto& la : layers)
        for (const LoraPair* lp : {&la.lora_q, &la.lora_k, &la.lora_v, &la.lora_o})
            n += (std::size_t)lp->rank * (lp->in_dim + lp->out_dim);
    return n;
}

}  // namespace tensor::adapter

// ── AdamW ───────────────────────────────────────────────────────────────
namespace tensor::trainer {

void AdamW::step(adapter::LoraPair& lp, float lr, int step, const backend::cuda::Device& dev) const {
    const int nA = lp.rank * lp.in_dim, nB = lp.out_dim * lp.rank;
    ops::adamw_step(lp.A_f32.f32(), lp.A_bf16.bf16(), lp.mA.f32(), lp.vA.f32(), lp.gA.f32(), nA,
                    lr, beta1, beta2, eps, weight_decay, step, dev.stream());
    ops::adamw_step(lp.B_f32.f32(), lp.B_bf16.bf16(), lp.mB.f32(), lp.vB.f32(), lp.gB.f32(), nB,
                    lr, beta1, beta2, eps, weight_decay, step, dev.stream());
}

void AdamW::step_all(adapter::AdapterModel& model, float lr, int step,
                     const backend::cuda::Device& dev) const {
    for (auto& la : model.layers)
        for (adapter::LoraPair* lp : {&la.lora_q, &la.lora_k, &la.lora_v, &la.lora_o})
            this->step(*lp, lr, step, dev);
}

}  // namespace tensor::trainer
