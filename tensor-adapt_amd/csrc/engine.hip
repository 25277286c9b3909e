// engine.hip — the MI355X step engine behind include/ta_engine.h.
//
// One object owns everything a LoRA step touches, allocated once:
//   * the frozen base: every projection W [out,in] AND its transpose
//     W^T [in,out] (also E^T for the tied LM head), so both the forward
//     x*W^T and the input gradient dY*W are K-contiguous MFMA GEMMs;
//   * one flat adapter arena (F32 master, m, v, grad; BF16 shadow) so the
//     whole optimizer tail is two launches (optim.hip);
//   * the per-layer activation cache of Qwen2Base::forward
//     (src/base/arch/qwen2.hpp:17-35) and the backward scratch.
// A step replays qwen2.cu:47-308 / adapter_model.cu:96-220 /
// adapt_trainer.cu:130-277 op for op (same rounding points) on one stream
// with no allocation, no device-to-device copy of the residual stream and a
// single host synchronisation at the end (the reference synchronises for
// every attention call, every centroid layer and the grad norm).
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <initializer_list>
#include <map>
#include <string>
#include <vector>

#include "ta_backend.h"
#include "ta_engine.h"
#include "ta_internal.hpp"
#include <tensor/trainer/cosine_schedule.hpp>

namespace ta {

#define CK(x)                    \
    do {                         \
        int _rc = (x);           \
        if (_rc != 0) return _rc; \
    } while (0)

enum { PQ = 0, PK, PV, PO, PG, PU, PD, NPAIR };
static const char* kProj[NPAIR] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                   "self_attn.o_proj", "mlp.gate_proj",    "mlp.up_proj",
                                   "mlp.down_proj"};

struct Pair {
    bool on = false;
    int in = 0, out = 0;
    int64_t offA = 0, offB = 0;  // element offsets in the adapter arena
    bf16* h = nullptr;           // cached x*A^T [BT, r] from the forward
};

struct Layer {
    bf16 *in_norm = nullptr, *post_norm = nullptr, *bias[3] = {nullptr, nullptr, nullptr};
    bf16* W[NPAIR] = {};
    bf16* Wt[NPAIR] = {};
    bf16* Wgu = nullptr;  // gate/up weights interleaved in 128-row blocks (gemm_swiglu)
    Pair pr[NPAIR];
    // forward cache
    bf16 *res_in, *xn, *Q, *K, *V, *ao, *res_mid, *xn2, *gate, *up, *act;
    float *in_rms, *post_rms, *attn_st, *ao32;  // attn_st: rows' (max, 1/sum); ao32: output in F32
};

struct Engine {
    ta_model_config mc;
    ta_adapt_config ac;
    int B, T, BT, H, qd, kvd, I, V;
    // r: the rank every buffer and kernel of the engine is laid out for, the
    // requested rank r_real rounded up to a multiple of 16.  A holds r rows
    // [r, in] and B r columns [out, r]; rows and columns past r_real are zero
    // and stay zero (their h, dh, gradients and AdamW updates are exactly 0),
    // so the step computes the rank-r_real adapter.
    int r, r_real;
    float scale;  // alpha / r_real
    // per-layer activation recompute: only each layer's input (res_in) is
    // kept per layer; the other cached activations live in one shared set
    // that the backward refills by rerunning the layer's forward
    bool recompute = false;
    // the cross-entropy gradient formed inside the LM head's dX GEMM
    // (TA_ENGINE_CE_IN_DX): lse2 holds each row's base-2 normaliser
    bool ce_in_dx = false;
    float* lse2 = nullptr;
    hipStream_t s = nullptr;
    bool own_stream = false;
    std::vector<void*> allocs;
    std::map<std::string, std::pair<void*, std::pair<int64_t, int>>> named;

    bf16 *embed = nullptr, *embedT = nullptr, *lm = nullptr, *lmT = nullptr, *final_norm = nullptr;
    std::vector<Layer> L;

    int64_t nparam = 0;
    float *master = nullptr, *mom = nullptr, *vel = nullptr, *grad = nullptr;
    bf16* shadow = nullptr;
    bf16* shadowT = nullptr;       // A^T and B^T of every shadow (same offsets), per step
    // every adapter tensor for the tiled AdamW, which writes shadowT
    AdamTensor* atens = nullptr;
    int natens = 0;
    int64_t natiles = 0;
    // LoRA weight-gradient partials of one step (one arena slice per
    // product, in backward call order) and their batched reduction
    float* wg_arena = nullptr;
    WgradJob* wg_jobs = nullptr;   // device copy of wg_plan
    std::vector<WgradJob> wg_plan;
    int64_t wg_blocks = 0;
    double wg_elems = 0;
    size_t wg_cursor = 0;
    // SwiGLU backward fused with the gate/up LoRA backward (rank 16, both
    // pairs on, BT and I multiples of 64): its dh partials, split counts
    bool silu_fused = false;
    int sl_st = 0, sl_so = 0;
    float* dh_part = nullptr;
    // dh and gB of a group's pairs in one pass over their go (go_lora)
    float* go_part = nullptr;

    bf16 *x_final, *xfn, *logits, *g_res, *dres, *tmpH, *dact, *dgate, *dup, *dxn2, *dao, *dQ, *dK,
        *dV, *dxn, *delta, *dh, *dh_cat;
    float *final_rms, *loss_tok, *norm_dev, *Dbuf, *dkv_part;
    // (cos, sin) table of the inverse RoPE, taken by the attention backward
    // as it writes dQ and dK (the forward's rotation runs in the q/k/v GEMM)
    const float2* rope_bwd;
    double* cacc;          // the centroid sums the step adds into (own_cacc or the caller's)
    double* own_cacc = nullptr;
    int32_t *tok_dev, *tgt_dev;
    int32_t *tok_host, *tgt_host;  // pinned
    float *loss_host, *norm_host;  // pinned
    // set on the device when a token id of the batch lies outside [0, V):
    // the embedding then reads nothing for it, and the tail changes no state
    int32_t* bad_dev = nullptr;
    // NaN and Inf logits of the first step (the reference's step-0 check)
    int32_t* nonfinite_dev = nullptr;
    hipEvent_t ev[4];
    int64_t step_count = 0;
    float phase[3] = {0, 0, 0};
    const int32_t* tok_cur = nullptr;  // token ids the forward embeds

    // kernel-class timing (ta_engine_profile)
    int prof_cat = -1;
    std::vector<hipEvent_t> pev;  // per-launch event pairs of the timed category
    size_t pev_used = 0, pcall0 = 0;
    // per timed call: (flops, bytes) and its range of event pairs
    std::vector<std::pair<std::pair<double, double>, std::pair<size_t, size_t>>> pwork;
    double p_ms = 0, p_flops = 0, p_bytes = 0;
    int64_t p_n = 0;
};

// Time the launches of one call of category `cat` when that category is
// being timed: each kernel launch of the call carries a start/stop event
// pair in its own dispatch (tlaunch), so the sum is kernel time only.  Work
// figures are the algorithmic flops / HBM bytes of the call, computed from
// its shape.
static void prof_begin(Engine* e, int cat) {
    if (cat != e->prof_cat) return;
    KpArm& k = kprof_arm();
    k.pool = &e->pev;
    k.npairs = &e->pev_used;
    e->pcall0 = e->pev_used;
}
static void prof_end(Engine* e, int cat, double flops, double bytes) {
    if (cat != e->prof_cat) return;
    KpArm& k = kprof_arm();
    k.pool = nullptr;
    k.npairs = nullptr;
    e->pwork.push_back({{flops, bytes}, {e->pcall0, e->pev_used}});
}
static int prof_collect(Engine* e) {
    for (const auto& w : e->pwork) {
        for (size_t i = w.second.first; i < w.second.second; i++) {
            float ms = 0.f;
            TA_HIP(hipEventElapsedTime(&ms, e->pev[2 * i], e->pev[2 * i + 1]));
            e->p_ms += ms;
        }
        e->p_n++;
        e->p_flops += w.first.first;
        e->p_bytes += w.first.second;
    }
    e->pwork.clear();
    e->pev_used = 0;
    return 0;
}
#define TIMED(cat, flops, bytes, call)             \
    do {                                           \
        prof_begin(e, cat);                        \
        int _rc2 = (call);                         \
        prof_end(e, cat, (double)(flops), (double)(bytes)); \
        if (_rc2 != 0) return _rc2;                \
    } while (0)

static int dmalloc(Engine* e, void** p, size_t bytes, const char* what) {
    if (bytes == 0) bytes = 256;
    hipError_t err = hipMalloc(p, bytes);
    if (err != hipSuccess)
        return set_error(-2, "engine: hipMalloc(%zu) for %s failed: %s", bytes, what,
                         hipGetErrorString(err));
    e->allocs.push_back(*p);
    return 0;
}
template <typename T>
static int alloc(Engine* e, T** p, int64_t n, const char* name, int is_f32 = -1) {
    CK(dmalloc(e, (void**)p, (size_t)n * sizeof(T), name));
    if (is_f32 >= 0) e->named[name] = {(void*)*p, {n, is_f32}};
    return 0;
}

// Token splits of the gB partials when go_lora makes a group's dh and gB
// (rank 16, every on-pair's output a multiple of 64, BT a multiple of 32);
// 0 when the group runs the per-pair kernels.  Used by the plan and the step.
static int go_group_splits(Engine* e, const Layer& ly, std::initializer_list<int> group) {
    if (e->r != 16 || e->BT % 32 != 0) return 0;
    int ntot = 0;
    for (int p : group) {
        if (!ly.pr[p].on) continue;
        if (ly.pr[p].out % 64 != 0) return 0;
        ntot += ly.pr[p].out;
    }
    if (!ntot) return 0;
    int s_t = 0, s_o = 0;
    if (go_lora_splits(e->BT, ntot, &s_t, &s_o)) return 0;
    return s_t;
}

static int engine_alloc(Engine* e) {
    const int BT = e->BT, H = e->H, qd = e->qd, kvd = e->kvd, I = e->I, V = e->V, r = e->r;
    const ta_model_config& c = e->mc;
    CK(alloc(e, &e->embed, (int64_t)V * H, "embed"));
    CK(alloc(e, &e->final_norm, H, "final_norm"));
    if (c.tie) {
        CK(alloc(e, &e->embedT, (int64_t)H * V, "embedT"));
        e->lm = e->embed;
        e->lmT = e->embedT;
    } else {
        CK(alloc(e, &e->lm, (int64_t)V * H, "lm_head"));
        CK(alloc(e, &e->lmT, (int64_t)H * V, "lm_headT"));
    }
    int outs[NPAIR] = {qd, kvd, kvd, H, I, I, H};
    int ins[NPAIR] = {H, H, H, qd, H, H, I};
    e->L.resize(c.layers);
    // adapter arena layout: layer-major, targets in q,k,v,o,gate,up,down
    // order, A then B, each padded to 64 elements (256-byte aligned F32)
    int64_t off = 0;
    for (int l = 0; l < c.layers; l++)
        for (int p = 0; p < NPAIR; p++) {
            Pair& pr = e->L[l].pr[p];
            pr.on = (e->ac.inject_mask >> p) & 1;
            pr.in = ins[p];
            pr.out = outs[p];
            if (!pr.on) continue;
            pr.offA = off;
            off += ((int64_t)r * pr.in + 63) / 64 * 64;
            pr.offB = off;
            off += ((int64_t)pr.out * r + 63) / 64 * 64;
        }
    e->nparam = off;
    CK(alloc(e, &e->master, off, "adapter.master", 1));
    CK(alloc(e, &e->mom, off, "adapter.m", 1));
    CK(alloc(e, &e->vel, off, "adapter.v", 1));
    CK(alloc(e, &e->grad, off, "adapter.grad", 1));
    CK(alloc(e, &e->shadow, off, "adapter.shadow", 0));
    CK(alloc(e, &e->shadowT, off, "adapter.shadowT", 0));
    {
        // A [r, in] tiled by W columns, B [out, r] by W rows: W = 256 at
        // rank 16, else 64 (tiles of at most 4096 elements)
        std::vector<AdamTensor> td;
        int64_t blk = 0;
        const int lw = r <= 16 ? 8 : 6, W = 1 << lw;
        for (auto& ly : e->L)
            for (auto& pr : ly.pr)
                if (pr.on) {
                    td.push_back({pr.offA, blk, r, pr.in, 1, lw});
                    blk += (pr.in + W - 1) / W;
                    td.push_back({pr.offB, blk, pr.out, r, 0, lw});
                    blk += (pr.out + W - 1) / W;
                }
        e->natens = (int)td.size();
        e->natiles = blk;
        CK(dmalloc(e, (void**)&e->atens, td.size() * sizeof(AdamTensor) + 16, "adam_tensors"));
        if (!td.empty())
            TA_HIP(hipMemcpy(e->atens, td.data(), td.size() * sizeof(AdamTensor),
                             hipMemcpyHostToDevice));
    }
    for (int l = 0; l < c.layers; l++) {
        Layer& ly = e->L[l];
        std::string p = "l" + std::to_string(l) + ".";
        CK(alloc(e, &ly.in_norm, H, "w"));
        CK(alloc(e, &ly.post_norm, H, "w"));
        CK(alloc(e, &ly.bias[0], qd, "w"));
        CK(alloc(e, &ly.bias[1], kvd, "w"));
        CK(alloc(e, &ly.bias[2], kvd, "w"));
        for (int q = 0; q < NPAIR; q++) {
            CK(alloc(e, &ly.W[q], (int64_t)outs[q] * ins[q], "w"));
            CK(alloc(e, &ly.Wt[q], (int64_t)outs[q] * ins[q], "wt"));
            if (ly.pr[q].on) CK(alloc(e, &ly.pr[q].h, (int64_t)BT * r, "lora.h"));
        }
        if (I % 128 == 0) CK(alloc(e, &ly.Wgu, (int64_t)2 * I * H, "wgu"));
        CK(alloc(e, &ly.res_in, (int64_t)BT * H, (p + "res_in").c_str(), 0));
        if (e->recompute && l > 0) {
            // the shared activation set of layer 0 ("work." buffers)
            const Layer& l0 = e->L[0];
            ly.in_rms = l0.in_rms, ly.xn = l0.xn, ly.Q = l0.Q, ly.K = l0.K, ly.V = l0.V;
            ly.ao = l0.ao, ly.attn_st = l0.attn_st, ly.ao32 = l0.ao32, ly.res_mid = l0.res_mid;
            ly.post_rms = l0.post_rms, ly.xn2 = l0.xn2, ly.gate = l0.gate, ly.up = l0.up;
            ly.act = l0.act;
            continue;
        }
        if (e->recompute) p = "work.";
        CK(alloc(e, &ly.in_rms, BT, (p + "in_rms").c_str(), 1));
        CK(alloc(e, &ly.xn, (int64_t)BT * H, (p + "x_normed").c_str(), 0));
        CK(alloc(e, &ly.Q, (int64_t)BT * qd, (p + "Q").c_str(), 0));
        CK(alloc(e, &ly.K, (int64_t)BT * kvd, (p + "K").c_str(), 0));
        CK(alloc(e, &ly.V, (int64_t)BT * kvd, (p + "V").c_str(), 0));
        CK(alloc(e, &ly.ao, (int64_t)BT * qd, (p + "attn_out").c_str(), 0));
        // the attention probabilities are not kept: the backward recomputes
        // them from Q, K and each row's (max, 1/sum)
        CK(alloc(e, &ly.attn_st, (int64_t)2 * e->B * c.n_q * e->T, (p + "attn_stats").c_str(), 1));
        CK(alloc(e, &ly.ao32, (int64_t)BT * qd, (p + "attn_out32").c_str(), 1));
        CK(alloc(e, &ly.res_mid, (int64_t)BT * H, (p + "res_mid").c_str(), 0));
        CK(alloc(e, &ly.post_rms, BT, (p + "post_rms").c_str(), 1));
        CK(alloc(e, &ly.xn2, (int64_t)BT * H, (p + "x_normed2").c_str(), 0));
        CK(alloc(e, &ly.gate, (int64_t)BT * I, (p + "gate").c_str(), 0));
        CK(alloc(e, &ly.up, (int64_t)BT * I, (p + "up").c_str(), 0));
        CK(alloc(e, &ly.act, (int64_t)BT * I, (p + "act").c_str(), 0));
    }
    e->silu_fused = r == 16 && BT % 64 == 0 && I % 64 == 0;
    if (e->silu_fused) {
        CK(silu_lora_splits(BT, I, &e->sl_st, &e->sl_so));
        CK(alloc(e, &e->dh_part, (int64_t)e->sl_so * 2 * BT * 16, "lora.dh_partials"));
    }
    // weight-gradient jobs in the order lora_group_bwd issues them: layers
    // L-1..0; groups down, gate/up, o, q/k/v; per group gB of each on-pair,
    // then gA of the group.  (Reducing each layer's partials at the end of
    // its backward, with one arena every layer reuses, measured 0.35 ms per
    // c3 step slower: the partials were not cache-resident by then either.)
    {
        struct G {
            std::initializer_list<int> pairs;
            int in;
        };
        const G groups[4] = {{{PD}, I}, {{PG, PU}, H}, {{PO}, qd}, {{PQ, PK, PV}, H}};
        int64_t off = 0, blk = 0;
        auto add = [&](int NL, int NS, int trans, float* g0, float* g1, float* g2,
                       int splits) {
            int per = 0;
            WgradJob j{};
            j.splits = splits > 0 ? splits : lora_wgrad_splits(NL, BT, &per);
            j.NL = NL;
            j.NS = NS;
            j.r = r;
            j.trans = trans;
            j.scale = e->scale;
            j.g[0] = g0;
            j.g[1] = g1;
            j.g[2] = g2;
            j.n = (int64_t)NL * NS;
            j.blk0 = blk;
            j.part = (const float*)(intptr_t)off;  // arena offset until the arena exists
            blk += (j.n + 1023) / 1024;  // k_wgrad_reduce_jobs: 1024 elements per block
            off += ((int64_t)j.splits * j.n + 63) / 64 * 64;
            e->wg_elems += (double)j.n;
            e->wg_plan.push_back(j);
        };
        for (int l = c.layers - 1; l >= 0; l--)
            for (const G& g : groups) {
                float* ga[3] = {nullptr, nullptr, nullptr};
                int n = 0;
                // gB of the gate/up pairs come token-split from the fused kernel
                const bool fused = e->silu_fused && *g.pairs.begin() == PG &&
                                   e->L[l].pr[PG].on && e->L[l].pr[PU].on;
                const int go_st = fused ? 0 : go_group_splits(e, e->L[l], g.pairs);
                for (int p : g.pairs) {
                    Pair& pr = e->L[l].pr[p];
                    if (!pr.on) continue;
                    add(pr.out, r, 0, e->grad + pr.offB, nullptr, nullptr,
                        fused ? e->sl_st : go_st);
                    ga[n++] = e->grad + pr.offA;
                }
                // gA of the down pair comes token-split from the fused kernel too
                const bool fused_d = e->silu_fused && *g.pairs.begin() == PD &&
                                     e->L[l].pr[PG].on && e->L[l].pr[PU].on;
                if (n)
                    add(g.in, n * r, 1, ga[0], ga[1] ? ga[1] : ga[0], ga[2] ? ga[2] : ga[0],
                        fused_d ? e->sl_st : 0);
            }
        e->wg_blocks = blk;
        if (!e->wg_plan.empty()) {
            CK(alloc(e, &e->wg_arena, off, "lora.wgrad_partials"));
            for (WgradJob& j : e->wg_plan) j.part = e->wg_arena + (intptr_t)j.part;
            CK(dmalloc(e, (void**)&e->wg_jobs, e->wg_plan.size() * sizeof(WgradJob), "wg_jobs"));
            TA_HIP(hipMemcpy(e->wg_jobs, e->wg_plan.data(), e->wg_plan.size() * sizeof(WgradJob),
                             hipMemcpyHostToDevice));
        }
    }
    int maxout = std::max(std::max(qd, H), I);
    {
        // go_lora partials: [column blocks][3][BT][16] for the widest group
        const int wide = std::max(std::max(H, qd + 2 * kvd), 2 * I);
        CK(alloc(e, &e->go_part, (int64_t)((wide + 511) / 512) * 3 * BT * 16, "lora.go_partials"));
    }
    CK(alloc(e, &e->x_final, (int64_t)BT * H, "x_final", 0));
    CK(alloc(e, &e->final_rms, BT, "final_rms", 1));
    CK(alloc(e, &e->xfn, (int64_t)BT * H, "xfn", 0));
    CK(alloc(e, &e->logits, (int64_t)BT * V, "logits", 0));
    CK(alloc(e, &e->loss_tok, BT, "loss_tok", 1));
    if (e->ce_in_dx) CK(alloc(e, &e->lse2, BT, "lse2", 1));
    CK(alloc(e, &e->g_res, (int64_t)BT * H, "grad", 0));
    CK(alloc(e, &e->dres, (int64_t)BT * H, "dres", 0));
    CK(alloc(e, &e->tmpH, (int64_t)BT * H, "tmpH", 0));
    CK(alloc(e, &e->dact, (int64_t)BT * I, "dact", 0));
    CK(alloc(e, &e->dgate, (int64_t)BT * I, "dgate", 0));
    CK(alloc(e, &e->dup, (int64_t)BT * I, "dup", 0));
    CK(alloc(e, &e->dxn2, (int64_t)BT * H, "dx_normed2", 0));
    CK(alloc(e, &e->dao, (int64_t)BT * qd, "dattn_out", 0));
    CK(alloc(e, &e->dQ, (int64_t)BT * qd, "dQ", 0));
    CK(alloc(e, &e->dK, (int64_t)BT * kvd, "dK", 0));
    CK(alloc(e, &e->dV, (int64_t)BT * kvd, "dV", 0));
    CK(alloc(e, &e->dxn, (int64_t)BT * H, "dx_normed", 0));
    CK(alloc(e, &e->delta, (int64_t)BT * maxout, "delta", 0));
    CK(alloc(e, &e->dh, (int64_t)BT * r, "dh", 0));
    CK(alloc(e, &e->dh_cat, (int64_t)BT * r * 3, "dh_cat", 0));
    CK(alloc(e, &e->Dbuf, attn_bwd_rowbuf_floats(e->B, e->T, c.n_q), "Dbuf", 1));
    CK(alloc(e, &e->dkv_part, (int64_t)2 * e->B * c.n_q * e->T * c.head_dim, "dkv_part", 1));
    e->rope_bwd = rope_table(e->T, c.head_dim, c.rope_theta, -1.f, e->s);
    if (!e->rope_bwd) return set_error(-2, "engine: RoPE table allocation failed");
    CK(alloc(e, &e->norm_dev, 64, "norm", 1));
    e->bad_dev = (int32_t*)(e->norm_dev + 1);
    e->nonfinite_dev = (int32_t*)(e->norm_dev + 2);
    CK(alloc(e, &e->own_cacc, H + 1, "centroid"));
    e->cacc = e->own_cacc;
    CK(alloc(e, &e->tok_dev, BT, "tok"));
    CK(alloc(e, &e->tgt_dev, BT, "targets", 1));  // int32, 4-byte elements
    TA_HIP(hipHostMalloc((void**)&e->tok_host, BT * sizeof(int32_t)));
    TA_HIP(hipHostMalloc((void**)&e->tgt_host, BT * sizeof(int32_t)));
    TA_HIP(hipHostMalloc((void**)&e->loss_host, BT * sizeof(float)));
    TA_HIP(hipHostMalloc((void**)&e->norm_host, 64));
    for (int i = 0; i < 4; i++) TA_HIP(hipEventCreate(&e->ev[i]));
    return 0;
}

// A^T and B^T of every BF16 shadow, after shadows were written other than by
// the step's AdamW (creation, ta_engine_write_adapter)
static int refresh_shadowT(Engine* e) {
    return adamw_tiles_impl(e->master, e->shadow, e->shadowT, e->mom, e->vel, e->grad, e->nparam,
                            e->atens, e->natens, e->natiles, false, 0.f, 0.f, 0.f, 0.f, 0.f, 1,
                            0.f, nullptr, nullptr, e->s);
}

// Adapter state at creation (AdapterModel::create, adapter_model.cu:41-90):
// A from the fixed-seed hash, B = 0, moments 0.
static int adapter_init(Engine* e) {
    TA_HIP(hipMemsetAsync(e->master, 0, e->nparam * 4, e->s));
    TA_HIP(hipMemsetAsync(e->mom, 0, e->nparam * 4, e->s));
    TA_HIP(hipMemsetAsync(e->vel, 0, e->nparam * 4, e->s));
    TA_HIP(hipMemsetAsync(e->grad, 0, e->nparam * 4, e->s));
    TA_HIP(hipMemsetAsync(e->shadow, 0, e->nparam * 2, e->s));
    for (auto& ly : e->L)
        for (auto& p : ly.pr)
            if (p.on)
                CK(kaiming_init(e->master + p.offA, e->shadow + p.offA, (int64_t)e->r_real * p.in,
                                p.in, e->s));
    TA_HIP(hipMemsetAsync(e->cacc, 0, (e->H + 1) * sizeof(double), e->s));
    TA_HIP(hipMemsetAsync(e->shadowT, 0, e->nparam * 2, e->s));
    return refresh_shadowT(e);
}

// ── one LoRA pair (adapter_model.cu:96-129 forward, 131-220 backward) ────
// algorithmic work of an M x N x K GEMM: flops, and bytes of one read of
// each operand plus the output (read too when accumulating)
static inline double gflops(double M, double N, double K) { return 2.0 * M * N * K; }
static inline double gbytes(double M, double N, double K, double in_b, double out_b, bool acc) {
    return (M * K + K * N) * in_b + M * N * out_b * (acc ? 2.0 : 1.0);
}

// LoRA forward, first half, for the on-pairs of one input-sharing group (q,k,v
// on x_normed; gate,up on x_normed2; o; down): h_p = bf16(x A_p^T) in one
// pass over x (adapter_model.cu:104-114).  The second half,
// y_p = bf16(y_p + s * bf16(h_p B_p^T)) (adapter_model.cu:116-127), runs in
// the epilogue of y_p's projection GEMM (fwd_epi).
static int lora_group_h(Engine* e, Layer& ly, std::initializer_list<int> group, const bf16* x,
                        int in) {
    const bf16* Ay[3];
    bf16* hs[3];
    int n = 0;
    for (int p : group)
        if (ly.pr[p].on) {
            Ay[n] = e->shadow + ly.pr[p].offA;
            hs[n++] = ly.pr[p].h;
        }
    if (!n) return 0;
    const double BT = e->BT, r = e->r;
    TIMED(TA_CAT_LORA, gflops(BT, n * r, in), BT * in * 2 + BT * n * r * 2,
          lora_skinny_nt(x, in, e->BT, in, e->r, Ay, hs, e->r, n, e->s));
    return 0;
}

static LoraEpi fwd_epi(Engine* e, const Pair& pr) {
    LoraEpi ep{};
    if (!pr.on) return ep;
    ep.n = 1;
    ep.r = e->r;
    ep.delta = true;
    ep.s = e->scale;
    ep.u[0] = pr.h;
    ep.ldu[0] = e->r;
    ep.v_nk[0] = ep.v_alt[0] = e->shadow + pr.offB;
    return ep;
}

// Arena slice of the next weight-gradient product of the step; the call
// sequence must be the one the plan was built from.
static int next_wgrad(Engine* e, int NL, int NS, float** part) {
    if (e->wg_cursor >= e->wg_plan.size())
        return set_error(-1, "engine: more weight-gradient products than planned");
    const WgradJob& j = e->wg_plan[e->wg_cursor++];
    if (j.NL != NL || j.NS != NS)
        return set_error(-1, "engine: weight-gradient product %zu is %dx%d, planned %dx%d",
                         e->wg_cursor - 1, NL, NS, j.NL, j.NS);
    *part = (float*)j.part;
    return 0;
}

// LoRA backward for one group, adapter_model.cu:131-220, pairs in order:
//   dh_p = bf16(go_p B_p)            (B^T shadow, one pass over go_p)
//   gB_p += s * go_p^T h_p           (h_p cached by the forward)
//   gA_p += s * dh_p^T x             (all pairs of the group in one pass over x)
// and returns the terms gx = bf16(s * dh_p A_p + gx) (pairs in order) for
// the epilogue of the last input-gradient GEMM of the group.  dh_ready: dh_p
// and the gB products were made already (the fused SwiGLU backward);
// gA_part: the gA product is left to the caller, which receives its
// partials slice (the fused SwiGLU backward makes it for the down pair).
// The group's gA product, when the caller launches it after the input-
// gradient GEMM (defer): the GEMM reads dh_cat, the product reads dh_cat
// and x, and neither writes them, so the order between the two is free.
struct GaDeferred {
    const bf16* x = nullptr;
    int in = 0;
    int64_t ldh = 0;
    float* part = nullptr;
};
static int lora_group_bwd(Engine* e, Layer& ly, std::initializer_list<int> group, const bf16* x,
                          int in, const bf16* const* gos, LoraEpi* ep, bool dh_ready = false,
                          float** gA_part = nullptr, GaDeferred* defer = nullptr) {
    *ep = LoraEpi{};
    int on[3], n = 0, i = 0;
    const bf16* go_on[3];
    for (int p : group) {
        if (ly.pr[p].on) {
            on[n] = p;
            go_on[n++] = gos[i];
        }
        i++;
    }
    if (!n) return 0;
    const int BT = e->BT, r = e->r;
    const double dBT = BT;
    const int64_t ldh = (int64_t)n * r;
    if (!dh_ready && go_group_splits(e, ly, group) > 0) {
        // dh and gB of every pair in one pass over their go
        const bf16* bt[3];
        const bf16* hs[3];
        float* parts[3];
        int64_t ld[3];
        int outs[3];
        double bytes = 0.0, fl = 0.0;
        for (int q = 0; q < n; q++) {
            Pair& pr = ly.pr[on[q]];
            CK(next_wgrad(e, pr.out, r, &parts[q]));
            bt[q] = e->shadowT + pr.offB;
            hs[q] = pr.h;
            ld[q] = pr.out;
            outs[q] = pr.out;
            bytes += dBT * pr.out * 2 + dBT * r * 4;
            fl += 2.0 * gflops(dBT, r, pr.out);
        }
        TIMED(TA_CAT_LORA, fl, bytes,
              go_lora(go_on, ld, bt, hs, parts, outs, n, BT, e->go_part, e->dh_cat, ldh, e->s));
    }
    for (int q = 0; q < n && !dh_ready && go_group_splits(e, ly, group) == 0; q++) {
        Pair& pr = ly.pr[on[q]];
        const bf16* Yt[1] = {e->shadowT + pr.offB};
        bf16* C[1] = {e->dh_cat + q * r};
        TIMED(TA_CAT_LORA, gflops(dBT, r, pr.out), dBT * pr.out * 2 + dBT * r * 2,
              lora_skinny_nt(go_on[q], pr.out, BT, pr.out, r, Yt, C, ldh, 1, e->s));
        float* part = nullptr;
        CK(next_wgrad(e, pr.out, r, &part));
        TIMED(TA_CAT_LORA, gflops(pr.out, r, dBT), dBT * (pr.out + r) * 2,
              lora_wgrad_part(go_on[q], pr.out, pr.out, pr.h, r, r, BT, part, e->s));
    }
    ep->n = n;
    ep->r = r;
    ep->delta = false;
    ep->s = e->scale;
    for (int q = 0; q < n; q++) {
        Pair& pr = ly.pr[on[q]];
        ep->u[q] = e->dh_cat + q * r;
        ep->ldu[q] = ldh;
        ep->v_nk[q] = e->shadowT + pr.offA;
        ep->v_alt[q] = e->shadow + pr.offA;
    }
    float* part = nullptr;
    CK(next_wgrad(e, in, (int)ldh, &part));
    if (gA_part) {
        *gA_part = part;
        return 0;
    }
    if (defer) {
        *defer = GaDeferred{x, in, ldh, part};
        return 0;
    }
    TIMED(TA_CAT_LORA, gflops(ldh, in, dBT), dBT * (in + ldh) * 2,
          lora_wgrad_part(x, in, in, e->dh_cat, ldh, (int)ldh, BT, part, e->s));
    return 0;
}
static int ga_launch(Engine* e, const GaDeferred& d) {
    if (!d.part) return 0;
    const double dBT = e->BT;
    TIMED(TA_CAT_LORA, gflops(d.ldh, d.in, dBT), dBT * (d.in + d.ldh) * 2,
          lora_wgrad_part(d.x, d.in, d.in, e->dh_cat, d.ldh, (int)d.ldh, e->BT, d.part, e->s));
    return 0;
}

// proj_fwd (qwen2.cu:21-30) with the bias add fused: y = bf16(bf16(x W^T) + b)
// (with the pair's LoRA delta, when given, in the same epilogue)
static int proj_fwd(Engine* e, const bf16* W, const bf16* x, bf16* y, int in, int out,
                    const bf16* bias, const LoraEpi* lora = nullptr) {
    TIMED(TA_CAT_GEMM_FWD, gflops(e->BT, out, in), gbytes(e->BT, out, in, 2, 2, false),
          gemm_dispatch(true, true, e->BT, out, in, 1.f, x, in, W, in, 0.f, y, out, bias, false,
                        e->s, 0, lora && lora->n ? lora : nullptr));
    return 0;
}
// proj_bwd_x (qwen2.cu:32-41): dx = bf16(dy W + beta dx), W^T resident
// (with the group's LoRA dx terms, when given, in the same epilogue)
static int proj_bwd_x(Engine* e, const bf16* Wt, const bf16* dy, bf16* dx, int out, int in,
                      float beta, const LoraEpi* lora = nullptr) {
    TIMED(TA_CAT_GEMM_DX, gflops(e->BT, in, out), gbytes(e->BT, in, out, 2, 2, beta != 0.f),
          gemm_dispatch(true, true, e->BT, in, out, 1.f, dy, out, Wt, out, beta, dx, in, nullptr,
                        false, e->s, 0, lora && lora->n ? lora : nullptr));
    return 0;
}

static void mask_targets(const int32_t* in, int32_t* tgt, int B, int T) {
    // adapt_trainer.cu:145-182 (151644 <|im_start|>, 77091 "assistant", 151645 <|im_end|>)
    for (int b = 0; b < B; ++b) {
        bool in_asst = false;
        int off = b * T;
        for (int t = 0; t < T; ++t) {
            int idx = off + t, tok = in[idx];
            if (tok == 151644) in_asst = (t + 1 < T && in[off + t + 1] == 77091);
            bool mask = !in_asst;
            if (tok == 151644 || tok == 77091) mask = true;
            if (tok == 151645) {
                in_asst = false;
                mask = false;
            }
            if (mask) tgt[idx] = -1;
        }
    }
}

// CosineSchedule::lr_at (include/tensor/trainer/cosine_schedule.hpp:18-29)
static float cosine_lr(float base, int64_t warmup, int64_t total, float floor_frac, int64_t step) {
    tensor::trainer::CosineSchedule cs{base, (size_t)warmup, (size_t)total, floor_frac};
    return cs.lr_at((size_t)step);
}

// One layer's forward (qwen2.cu:80-157) from its normed input ly.xn up to
// act and the down pair's h: everything the layer's backward reads.  The
// down projection and the residual add follow in forward().
static int layer_fwd_body(Engine* e, Layer& ly) {
    const ta_model_config& c = e->mc;
    const int BT = e->BT, H = e->H, qd = e->qd, kvd = e->kvd, I = e->I;
    const double dBT = BT, tri = (double)e->B * c.n_q * e->T * (e->T + 1) / 2.0;
    hipStream_t s = e->s;
    const double nrm_b = dBT * H * 4 + H * 2 + dBT * 4;
    CK(lora_group_h(e, ly, {PQ, PK, PV}, ly.xn, H));
    {
        // q, k and v projections (qwen2.cu:21-30, each with its bias and
        // LoRA delta) in one launch over the three weight matrices, with
        // the RoPE of Q and K (qwen2.cu:109-110) on the rounded outputs
        LoraEpi eq = fwd_epi(e, ly.pr[PQ]), ek = fwd_epi(e, ly.pr[PK]), ev = fwd_epi(e, ly.pr[PV]);
        const GemmGroup gr[3] = {{qd, ly.W[PQ], ly.Q, qd, ly.bias[0], &eq, true},
                                 {kvd, ly.W[PK], ly.K, kvd, ly.bias[1], &ek, true},
                                 {kvd, ly.W[PV], ly.V, kvd, ly.bias[2], &ev, false}};
        const RopeSpec rope{e->B, e->T, c.head_dim, c.rope_theta};
        TIMED(TA_CAT_GEMM_FWD, gflops(BT, qd + 2.0 * kvd, H),
              gbytes(BT, qd + 2.0 * kvd, H, 2, 2, false),
              gemm_groups(BT, H, ly.xn, H, H, gr, 3, s, &rope));
    }
    // sdpa_fwd (ops.cu:578-681) without the probabilities buffer: the
    // rows' (max, 1/sum) are kept instead
    TIMED(TA_CAT_ATTN_FWD, 4.0 * tri * c.head_dim,
          dBT * (2.0 * qd + 2.0 * kvd) * 2 + dBT * qd * 4 + 8.0 * e->B * c.n_q * e->T,
          attn_fwd(ly.Q, ly.K, ly.V, ly.ao, ly.ao32, nullptr, ly.attn_st, e->B, e->T, c.n_q,
                   c.n_kv, c.head_dim, false, s));
    CK(lora_group_h(e, ly, {PO}, ly.ao, qd));
    {
        LoraEpi eo = fwd_epi(e, ly.pr[PO]);
        CK(proj_fwd(e, ly.W[PO], ly.ao, e->tmpH, qd, H, nullptr, &eo));
    }
    // res_mid = bf16(res_in + o_proj) and its post-attention norm, one pass
    TIMED(TA_CAT_NORM, 0, nrm_b + dBT * H * 4,
          rms_fwd_res(ly.res_in, e->tmpH, ly.res_mid, ly.post_norm, ly.xn2, ly.post_rms, BT, H,
                      c.rms_eps, s));
    CK(lora_group_h(e, ly, {PG, PU}, ly.xn2, H));
    {
        // gate and up projections (qwen2.cu:21-30, each with its LoRA
        // delta) and act = silu_mul_fwd(gate, up) (ops.cu:913-923) in one
        // launch over the interleaved gate/up weights
        LoraEpi eg = fwd_epi(e, ly.pr[PG]), eu = fwd_epi(e, ly.pr[PU]);
        TIMED(TA_CAT_GEMM_FWD, 2.0 * gflops(BT, I, H),
              2.0 * gbytes(BT, I, H, 2, 2, false) + dBT * I * 2,
              gemm_swiglu(BT, H, ly.xn2, H, ly.Wgu, ly.W[PG], ly.W[PU], ly.gate, ly.up, ly.act,
                          I, &eg, &eu, s));
    }
    CK(lora_group_h(e, ly, {PD}, ly.act, I));
    return 0;
}

static int forward(Engine* e) {
    const ta_model_config& c = e->mc;
    const int BT = e->BT, H = e->H, I = e->I;
    const double dBT = BT;
    hipStream_t s = e->s;
    TIMED(TA_CAT_ELEMWISE, 0, dBT * H * 4,
          embed_fwd_checked(e->embed, e->tok_cur, e->L[0].res_in, BT, H, e->V, e->bad_dev, s));
    const double nrm_b = dBT * H * 4 + H * 2 + dBT * 4;
    for (int l = 0; l < c.layers; l++) {
        Layer& ly = e->L[l];
        bf16* res_out = (l + 1 < c.layers) ? e->L[l + 1].res_in : e->x_final;
        // (the input norm of layers after the first runs fused with the
        // previous layer's residual add, below)
        if (l == 0)
            TIMED(TA_CAT_NORM, 0, nrm_b,
                  ta_rms_norm_fwd(ly.res_in, ly.in_norm, ly.xn, ly.in_rms, 1, BT, H, c.rms_eps, s));
        CK(layer_fwd_body(e, ly));
        {
            LoraEpi ed = fwd_epi(e, ly.pr[PD]);
            CK(proj_fwd(e, ly.W[PD], ly.act, e->tmpH, I, H, nullptr, &ed));
        }
        // res_out = bf16(res_mid + down_proj) and the next norm (the next
        // layer's input norm, or the final norm), one pass
        const bool last = l + 1 == c.layers;
        TIMED(TA_CAT_NORM, 0, nrm_b + dBT * H * 4,
              rms_fwd_res(ly.res_mid, e->tmpH, res_out, last ? e->final_norm : e->L[l + 1].in_norm,
                          last ? e->xfn : e->L[l + 1].xn, last ? e->final_rms : e->L[l + 1].in_rms,
                          BT, H, c.rms_eps, s));
    }
    // LM head (qwen2.cu:163-175), tied to the embedding when c.tie
    TIMED(TA_CAT_LMHEAD, gflops(BT, e->V, H), gbytes(BT, e->V, H, 2, 2, false),
          gemm_dispatch(true, true, BT, e->V, H, 1.f, e->xfn, H, e->lm, H, 0.f, e->logits, e->V,
                        nullptr, false, s, 0, nullptr));
    // loss (adapt_trainer.cu:201-205): dlogits overwrite the logits in place
    // (one read and one write of BT x V BF16); the first step also counts
    // the NaN and Inf logits (adapt_trainer.cu:196-198)
    if (e->ce_in_dx)  // loss and row normalisers only: one read of the logits
        TIMED(TA_CAT_CE, 0, dBT * e->V * 2,
              cross_entropy(e->logits, e->tgt_dev, e->loss_tok, nullptr, BT, e->V,
                            e->step_count == 0 ? e->nonfinite_dev : nullptr, s, e->lse2));
    else
        TIMED(TA_CAT_CE, 0, dBT * e->V * 4,
              cross_entropy(e->logits, e->tgt_dev, e->loss_tok, e->logits, BT, e->V,
                            e->step_count == 0 ? e->nonfinite_dev : nullptr, s));
    return 0;
}

static int backward(Engine* e) {
    const ta_model_config& c = e->mc;
    const int BT = e->BT, H = e->H, qd = e->qd, kvd = e->kvd, I = e->I;
    const double dBT = BT, tri = (double)e->B * c.n_q * e->T * (e->T + 1) / 2.0;
    hipStream_t s = e->s;
    const double nrm_b = dBT * H * 6 + H * 2 + dBT * 4;
    e->wg_cursor = 0;
    // dres = dlogits * W_lm (qwen2.cu:205); grad = rms_norm_bwd(final)
    if (e->ce_in_dx)
        TIMED(TA_CAT_LMHEAD_BWD, gflops(BT, H, e->V), gbytes(BT, H, e->V, 2, 2, false),
              gemm_ce_dx(BT, H, e->V, e->logits, e->lmT, e->dres, e->lse2, e->tgt_dev,
                         1.f / (float)BT, s));
    else
        TIMED(TA_CAT_LMHEAD_BWD, gflops(BT, H, e->V), gbytes(BT, H, e->V, 2, 2, false),
              gemm_dispatch(true, true, BT, H, e->V, 1.f, e->logits, e->V, e->lmT, e->V, 0.f,
                            e->dres, H, nullptr, false, s, 0, nullptr));
    TIMED(TA_CAT_NORM, 0, nrm_b,
          ta_rms_norm_bwd(e->dres, e->x_final, e->final_norm, e->final_rms, e->g_res, nullptr, 1,
                          BT, H, c.rms_eps, s));
    for (int l = c.layers - 1; l >= 0; l--) {
        Layer& ly = e->L[l];
        if (e->recompute && l + 1 < c.layers) {
            // refill the shared activation set with this layer's forward
            // (the last layer's is still there from the forward).  The
            // input norm gives the same bits as the fused residual-add form
            // that made it in the forward: both normalise the stored BF16 row.
            TIMED(TA_CAT_NORM, 0, dBT * H * 4 + H * 2 + dBT * 4,
                  ta_rms_norm_fwd(ly.res_in, ly.in_norm, ly.xn, ly.in_rms, 1, BT, H, c.rms_eps, s));
            CK(layer_fwd_body(e, ly));
        }
        // FFN (qwen2.cu:222-246)
        const bool fused = e->silu_fused && ly.pr[PG].on && ly.pr[PU].on;
        float* ga_down = nullptr;  // the down pair's gA partials, made by the fused kernel
        {
            const bf16* gos[1] = {e->g_res};
            LoraEpi ep;
            CK(lora_group_bwd(e, ly, {PD}, ly.act, I, gos, &ep, false, fused ? &ga_down : nullptr));
            CK(proj_bwd_x(e, ly.Wt[PD], e->g_res, e->dact, H, I, 0.f, &ep));
        }
        if (fused) {
            // dgate, dup, dh of both pairs and their gB partials in one pass
            // (and the down pair's gA = act^T dh_down, act recomputed)
            float *pg = nullptr, *pu = nullptr;
            CK(next_wgrad(e, I, e->r, &pg));
            CK(next_wgrad(e, I, e->r, &pu));
            const Pair &PRg = ly.pr[PG], &PRu = ly.pr[PU];
            TIMED(TA_CAT_ELEMWISE, (ga_down ? 5.0 : 4.0) * gflops(BT, e->r, I),
                  dBT * I * 10 + dBT * 96,
                  silu_bwd_lora(e->dact, ly.gate, ly.up, e->dgate, e->dup, e->shadowT + PRg.offB,
                                e->shadowT + PRu.offB, PRg.h, PRu.h, e->dh_part, pg, pu,
                                ga_down ? e->dh_cat : nullptr, ga_down, BT, I, s));
            TIMED(TA_CAT_LORA, 0, dBT * 128.0 * e->sl_so + dBT * 64,
                  dh_reduce2(e->dh_part, e->sl_so, BT, e->dh_cat, 2 * e->r, s));
        } else {
            TIMED(TA_CAT_ELEMWISE, 0, dBT * I * 10,
                  ta_silu_mul_bwd(e->dact, ly.gate, ly.up, e->dgate, e->dup, (int64_t)BT * I, s));
        }
        {
            const bf16* gos[2] = {e->dgate, e->dup};
            LoraEpi ep;
            GaDeferred ga;
            CK(lora_group_bwd(e, ly, {PG, PU}, ly.xn2, H, gos, &ep, fused, nullptr, &ga));
            // proj_bwd_x of gate (beta 0) then up (beta 1), qwen2.cu:233-234
            const GemmSeg sg[2] = {{I, e->dgate, I, ly.Wt[PG], I}, {I, e->dup, I, ly.Wt[PU], I}};
            TIMED(TA_CAT_GEMM_DX, 2.0 * gflops(BT, H, I), 2.0 * gbytes(BT, H, I, 2, 2, false),
                  gemm_chain(BT, H, sg, 2, e->dxn2, H, ep.n ? &ep : nullptr, s));
            CK(ga_launch(e, ga));
        }
        // grad += bf16(rms_norm_bwd(dx_normed2)), one pass
        TIMED(TA_CAT_NORM, 0, nrm_b + dBT * H * 2,
              rms_bwd_acc(e->dxn2, ly.res_mid, ly.post_norm, ly.post_rms, e->g_res, e->tmpH, BT, H,
                          s));
        // attention (qwen2.cu:250-304)
        {
            const bf16* gos[1] = {e->g_res};
            LoraEpi ep;
            GaDeferred ga;
            CK(lora_group_bwd(e, ly, {PO}, ly.ao, qd, gos, &ep, false, nullptr, &ga));
            CK(proj_bwd_x(e, ly.Wt[PO], e->g_res, e->dao, H, qd, 0.f, &ep));
            CK(ga_launch(e, ga));
        }
        TIMED(TA_CAT_ATTN_BWD, 12.0 * tri * c.head_dim,
              16.0 * e->B * c.n_q * e->T + dBT * (2.0 * qd + 2.0 * kvd) * 2 +
                  dBT * (qd + 2.0 * kvd) * 2 + dBT * qd * 4,
              attn_bwd(e->dao, ly.Q, ly.K, ly.V, nullptr, ly.attn_st, ly.ao32, e->dQ, e->dK, e->dV,
                       e->B, e->T, c.n_q, c.n_kv, c.head_dim, e->Dbuf, e->dkv_part, s,
                       e->rope_bwd));
        {
            const bf16* gos[3] = {e->dQ, e->dK, e->dV};
            LoraEpi ep;
            GaDeferred ga;
            CK(lora_group_bwd(e, ly, {PQ, PK, PV}, ly.xn, H, gos, &ep, false, nullptr, &ga));
            // proj_bwd_x of q (beta 0), k and v (beta 1), qwen2.cu:283-285
            const GemmSeg sg[3] = {{qd, e->dQ, qd, ly.Wt[PQ], qd},
                                   {kvd, e->dK, kvd, ly.Wt[PK], kvd},
                                   {kvd, e->dV, kvd, ly.Wt[PV], kvd}};
            TIMED(TA_CAT_GEMM_DX, gflops(BT, H, qd + 2.0 * kvd),
                  gbytes(BT, H, qd + 2.0 * kvd, 2, 2, false),
                  gemm_chain(BT, H, sg, 3, e->dxn, H, ep.n ? &ep : nullptr, s));
            CK(ga_launch(e, ga));
        }
        // centroid side channel (adapt_trainer.cu:210-232): h = x_normed,
        // g = dx_attn_in of this layer
        TIMED(TA_CAT_CENTROID, 0, dBT * H * 4,
              centroid_acc_bf16(ly.xn, e->dxn, BT, H, e->cacc, e->bad_dev, s));
        // grad += bf16(rms_norm_bwd(dx_normed)), one pass
        TIMED(TA_CAT_NORM, 0, nrm_b + dBT * H * 2,
              rms_bwd_acc(e->dxn, ly.res_in, ly.in_norm, ly.in_rms, e->g_res, e->tmpH, BT, H, s));
    }
    // every gA / gB += scale * (its ordered partial sum), one launch
    if (e->wg_cursor != e->wg_plan.size())
        return set_error(-1, "engine: %zu weight-gradient products run, %zu planned", e->wg_cursor,
                         e->wg_plan.size());
    TIMED(TA_CAT_LORA, 0, e->wg_elems * 8.0,
          lora_wgrad_reduce_jobs(e->wg_jobs, (int)e->wg_plan.size(), e->wg_blocks, e->wg_elems, s));
    return 0;
}

// The step body; the batch is already in e->tok_cur / e->tgt_dev (masked).
static int engine_step_body(Engine* e, float lr_override, ta_step_metrics* m,
                            std::chrono::steady_clock::time_point t0) {
    const int BT = e->BT;
    // zero_grad (adapter_model.cu:222-229)
    TA_HIP(hipMemsetAsync(e->grad, 0, e->nparam * sizeof(float), e->s));
    TA_HIP(hipMemsetAsync(e->bad_dev, 0, 2 * sizeof(int32_t), e->s));  // and nonfinite_dev
    TA_HIP(hipEventRecord(e->ev[0], e->s));
    CK(forward(e));
    TA_HIP(hipEventRecord(e->ev[1], e->s));
    CK(backward(e));
    TA_HIP(hipEventRecord(e->ev[2], e->s));
    // tail: loss read-back, grad norm + clip + AdamW on the device
    TA_HIP(hipMemcpyAsync(e->loss_host, e->loss_tok, BT * 4, hipMemcpyDeviceToHost, e->s));
    float lr = (lr_override > 0.f)
                   ? lr_override
                   : cosine_lr(e->ac.lr, e->ac.warmup, e->ac.total_steps, 0.1f, e->step_count);
    int t = (int)e->step_count + 1;
    TIMED(TA_CAT_TAIL, 0, (double)e->nparam * 34,
          adamw_tiles_impl(e->master, e->shadow, e->shadowT, e->mom, e->vel, e->grad, e->nparam,
                           e->atens, e->natens, e->natiles, true, lr, e->ac.b1, e->ac.b2,
                           e->ac.eps, e->ac.wd, t, e->ac.grad_clip, e->norm_dev, e->bad_dev,
                           e->s));
    // the norm and the bad-id flag behind it
    TA_HIP(hipMemcpyAsync(e->norm_host, e->norm_dev, 12, hipMemcpyDeviceToHost, e->s));
    TA_HIP(hipEventRecord(e->ev[3], e->s));
    TA_HIP(hipStreamSynchronize(e->s));
    for (int i = 0; i < 3; i++) TA_HIP(hipEventElapsedTime(&e->phase[i], e->ev[i], e->ev[i + 1]));
    CK(prof_collect(e));
    // adapt_trainer.cu:237-246: mean over tokens whose loss > 1e-9
    float mean = 0.f;
    int valid = 0;
    for (int i = 0; i < BT; i++)
        if (e->loss_host[i] > 1e-9f) {
            mean += e->loss_host[i];
            valid++;
        }
    if (valid > 0) mean /= (float)valid;
    float norm = e->norm_host[0];
    int32_t bad, nonfinite;
    memcpy(&bad, e->norm_host + 1, sizeof bad);
    memcpy(&nonfinite, e->norm_host + 2, sizeof nonfinite);
    const bool first = e->step_count == 0;
    if (bad)
        return set_error(-1,
                         "engine_step: a token id of the batch lies outside [0, %d); the step was "
                         "not applied (adapter state, step count and centroid unchanged)",
                         e->V);
    e->step_count++;
    if (m) {
        m->loss = mean;
        m->lr = lr;
        m->gnorm_raw = norm;
        m->gnorm = std::min(norm, e->ac.grad_clip);
        m->valid_tokens = valid;
        m->step = (int)e->step_count;
        m->nonfinite_logits = first ? nonfinite : -1;
        m->step_ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    }
    return 0;
}

static int engine_step(Engine* e, const int32_t* inputs, const int32_t* targets, float lr_override,
                       ta_step_metrics* m) {
    auto t0 = std::chrono::steady_clock::now();
    const int BT = e->BT;
    memcpy(e->tok_host, inputs, BT * sizeof(int32_t));
    memcpy(e->tgt_host, targets, BT * sizeof(int32_t));
    mask_targets(e->tok_host, e->tgt_host, e->B, e->T);
    TA_HIP(hipMemcpyAsync(e->tok_dev, e->tok_host, BT * 4, hipMemcpyHostToDevice, e->s));
    TA_HIP(hipMemcpyAsync(e->tgt_dev, e->tgt_host, BT * 4, hipMemcpyHostToDevice, e->s));
    e->tok_cur = e->tok_dev;
    return engine_step_body(e, lr_override, m, t0);
}

static bf16** weight_slot(Engine* e, const std::string& name, int64_t* n, int* layer, int* proj) {
    const int H = e->H;
    *layer = -1;
    *proj = -1;
    if (name == "model.embed_tokens.weight") {
        *n = (int64_t)e->V * H;
        return &e->embed;
    }
    if (name == "model.norm.weight") {
        *n = H;
        return &e->final_norm;
    }
    if (name == "lm_head.weight") {
        *n = (int64_t)e->V * H;
        return e->mc.tie ? nullptr : &e->lm;
    }
    const std::string pre = "model.layers.";
    if (name.compare(0, pre.size(), pre) != 0) return nullptr;
    size_t dot = name.find('.', pre.size());
    if (dot == std::string::npos) return nullptr;
    int l = atoi(name.substr(pre.size(), dot - pre.size()).c_str());
    if (l < 0 || l >= (int)e->L.size()) return nullptr;
    std::string k = name.substr(dot + 1);
    Layer& ly = e->L[l];
    *layer = l;
    if (k == "input_layernorm.weight") {
        *n = H;
        return &ly.in_norm;
    }
    if (k == "post_attention_layernorm.weight") {
        *n = H;
        return &ly.post_norm;
    }
    for (int b = 0; b < 3; b++)
        if (k == std::string(kProj[b]) + ".bias") {
            *n = b == 0 ? e->qd : e->kvd;
            return &ly.bias[b];
        }
    for (int p = 0; p < NPAIR; p++)
        if (k == std::string(kProj[p]) + ".weight") {
            *n = (int64_t)ly.pr[p].in * ly.pr[p].out;
            *proj = p;
            return &ly.W[p];
        }
    return nullptr;
}

// after a projection (or the LM head / embedding) changes: refresh W^T
static int refresh_transpose(Engine* e, const std::string& name, int layer, int proj) {
    if (proj >= 0) {
        Layer& ly = e->L[layer];
        Pair& p = ly.pr[proj];
        if ((proj == PG || proj == PU) && ly.Wgu) {
            // 128-row blocks of gate and up alternate in Wgu
            const size_t blk = (size_t)128 * p.in * sizeof(bf16);
            TA_HIP(hipMemcpy2DAsync(ly.Wgu + (proj == PU ? (size_t)128 * p.in : 0), 2 * blk,
                                    ly.W[proj], blk, blk, p.out / 128, hipMemcpyDeviceToDevice,
                                    e->s));
        }
        return transpose_bf16(ly.W[proj], ly.Wt[proj], p.out, p.in, e->s);
    }
    if (name == "model.embed_tokens.weight" && e->mc.tie)
        return transpose_bf16(e->embed, e->embedT, e->V, e->H, e->s);
    if (name == "lm_head.weight") return transpose_bf16(e->lm, e->lmT, e->V, e->H, e->s);
    return 0;
}

}  // namespace ta

using namespace ta;

extern "C" {

void* ta_engine_create(const ta_model_config* mc, const ta_adapt_config* ac, int B, int T,
                       void* stream) {
    return ta_engine_create_ex(mc, ac, B, T, stream, 0);
}

void* ta_engine_create_ex(const ta_model_config* mc, const ta_adapt_config* ac, int B, int T,
                          void* stream, int flags) {
    if (!mc || !ac || B <= 0 || T <= 0 ||
        (flags & ~(TA_ENGINE_RECOMPUTE | TA_ENGINE_CE_IN_DX)) != 0) {
        set_error(-1, "engine_create: bad arguments");
        return nullptr;
    }
    if (mc->n_kv <= 0 || mc->n_q % mc->n_kv != 0 || mc->hidden <= 0 || mc->layers <= 0 ||
        (mc->head_dim != 64 && mc->head_dim != 128) || ac->rank <= 0 || ac->rank > 64 ||
        mc->vocab <= 0) {
        // (rank 64 is the top of the reference's rank ladder, adapter_config.cpp:53-127)
        set_error(-1, "engine_create: unsupported shape (head_dim 64/128, n_q %% n_kv == 0, "
                      "LoRA rank 1..64)");
        return nullptr;
    }
    Engine* e = new Engine();
    e->mc = *mc;
    e->ac = *ac;
    e->B = B;
    e->T = T;
    e->BT = B * T;
    e->H = mc->hidden;
    e->qd = mc->n_q * mc->head_dim;
    e->kvd = mc->n_kv * mc->head_dim;
    e->I = mc->inter;
    e->V = mc->vocab;
    e->r_real = ac->rank;
    e->r = (ac->rank + 15) / 16 * 16;
    e->scale = ac->alpha / (float)ac->rank;  // adapter_model.cu:139
    e->recompute = (flags & TA_ENGINE_RECOMPUTE) != 0;
    // (the CE kernel's row-in-registers form and the GEMM's tile shapes)
    e->ce_in_dx = (flags & TA_ENGINE_CE_IN_DX) != 0 && e->V % 64 == 0 && e->V <= 163840 &&
                  e->H >= 192 && e->H % 8 == 0 && e->BT >= 256;
    if (stream) {
        e->s = (hipStream_t)stream;
    } else {
        if (hipStreamCreate(&e->s) != hipSuccess) {
            set_error(-2, "engine_create: hipStreamCreate failed");
            delete e;
            return nullptr;
        }
        e->own_stream = true;
    }
    if (engine_alloc(e) != 0 || adapter_init(e) != 0) {
        std::string msg = ta_last_error();
        ta_engine_destroy(e);
        set_error(-2, "%s", msg.c_str());
        return nullptr;
    }
    return e;
}

int ta_engine_destroy(void* ep) {
    Engine* e = (Engine*)ep;
    if (!e) return 0;
    if (e->s) (void)hipStreamSynchronize(e->s);
    for (void* p : e->allocs) (void)hipFree(p);
    for (void* p : {(void*)e->tok_host, (void*)e->tgt_host, (void*)e->loss_host,
                    (void*)e->norm_host})
        if (p) (void)hipHostFree(p);
    for (auto& ev : e->ev)
        if (ev) (void)hipEventDestroy(ev);
    for (auto& ev : e->pev) (void)hipEventDestroy(ev);
    if (e->own_stream) (void)hipStreamDestroy(e->s);
    delete e;
    return 0;
}

int ta_engine_set_weight(void* ep, const char* name, const uint16_t* host, int64_t n) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && name && host, "engine_set_weight: null argument");
    int64_t want = 0;
    int layer, proj;
    bf16** slot = weight_slot(e, name, &want, &layer, &proj);
    TA_REQUIRE(slot, "engine_set_weight: unknown tensor '%s'", name);
    TA_REQUIRE(n == want, "engine_set_weight: '%s' has %lld elements, expected %lld", name,
               (long long)n, (long long)want);
    TA_HIP(hipMemcpyAsync(*slot, host, n * 2, hipMemcpyHostToDevice, e->s));
    CK(refresh_transpose(e, name, layer, proj));
    TA_HIP(hipStreamSynchronize(e->s));
    return 0;
}

int ta_engine_set_weight_device(void* ep, const char* name, const uint16_t* src, int64_t n) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && name && src, "engine_set_weight_device: null argument");
    int64_t want = 0;
    int layer, proj;
    bf16** slot = weight_slot(e, name, &want, &layer, &proj);
    TA_REQUIRE(slot, "engine_set_weight_device: unknown tensor '%s'", name);
    TA_REQUIRE(n == want, "engine_set_weight_device: '%s' has %lld elements, expected %lld", name,
               (long long)n, (long long)want);
    TA_HIP(hipMemcpyAsync(*slot, src, n * 2, hipMemcpyDeviceToDevice, e->s));
    CK(refresh_transpose(e, name, layer, proj));
    return 0;
}

int ta_engine_set_centroid(void* ep, double* acc) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e, "engine_set_centroid: null engine");
    e->cacc = acc ? acc : e->own_cacc;
    return 0;
}

int ta_engine_set_step(void* ep, int64_t step) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && step >= 0, "engine_set_step: bad arguments");
    e->step_count = step;
    return 0;
}

int ta_engine_init_random(void* ep, uint64_t seed, float std) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e, "engine_init_random: null engine");
    uint64_t sid = 0;
    CK(fill_normal_bf16(e->embed, (int64_t)e->V * e->H, seed, sid++, std, e->s));
    CK(refresh_transpose(e, "model.embed_tokens.weight", -1, -1));
    if (!e->mc.tie) {
        CK(fill_normal_bf16(e->lm, (int64_t)e->V * e->H, seed, sid++, std, e->s));
        CK(refresh_transpose(e, "lm_head.weight", -1, -1));
    }
    CK(fill_bf16(e->final_norm, e->H, 1.f, e->s));
    for (int l = 0; l < (int)e->L.size(); l++) {
        Layer& ly = e->L[l];
        CK(fill_bf16(ly.in_norm, e->H, 1.f, e->s));
        CK(fill_bf16(ly.post_norm, e->H, 1.f, e->s));
        CK(fill_bf16(ly.bias[0], e->qd, 0.f, e->s));
        CK(fill_bf16(ly.bias[1], e->kvd, 0.f, e->s));
        CK(fill_bf16(ly.bias[2], e->kvd, 0.f, e->s));
        for (int p = 0; p < NPAIR; p++) {
            CK(fill_normal_bf16(ly.W[p], (int64_t)ly.pr[p].in * ly.pr[p].out, seed,
                                1000 + l * 16 + p, std, e->s));
            CK(refresh_transpose(e, "", l, p));
        }
    }
    TA_HIP(hipStreamSynchronize(e->s));
    return 0;
}

int ta_engine_step(void* ep, const int32_t* inputs, const int32_t* targets, float lr_override,
                   ta_step_metrics* m) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && inputs && targets, "engine_step: null argument");
    for (int i = 0; i < e->BT; i++)
        TA_REQUIRE(inputs[i] >= 0 && inputs[i] < e->V, "engine_step: token id %d out of range",
                   inputs[i]);
    return engine_step(e, inputs, targets, lr_override, m);
}

// Locate one adapter tensor: device pointer, element count and element size,
// and its layout in the arena: `rows` rows of `width` elements `pitch` apart
// (B [out, r_real] sits in the columns of B [out, r]; A [r_real, in] is the
// first r_real rows of A [r, in], contiguous).
struct Slot {
    void* ptr;
    int64_t cnt, rows, width, pitch;
    size_t es;
};
static int adapter_slot(Engine* e, int layer, int target, int which, Slot* sl) {
    TA_REQUIRE(layer >= 0 && layer < (int)e->L.size() && target >= 0 && target < NPAIR,
               "engine adapter: bad layer/target");
    Pair& p = e->L[layer].pr[target];
    TA_REQUIRE(p.on, "engine adapter: target %d not injected", target);
    bool isA = (which == 0 || which == 2 || which == 3 || which == 6 || which == 8);
    sl->cnt = isA ? (int64_t)e->r_real * p.in : (int64_t)p.out * e->r_real;
    sl->rows = isA ? 1 : p.out;
    sl->width = isA ? sl->cnt : e->r_real;
    sl->pitch = isA ? sl->cnt : e->r;
    int64_t off = isA ? p.offA : p.offB;
    sl->es = 4;
    switch (which) {
        case 0: case 1: sl->ptr = e->master + off; break;
        case 2: case 4: sl->ptr = e->mom + off; break;
        case 3: case 5: sl->ptr = e->vel + off; break;
        case 6: case 7: sl->ptr = e->grad + off; break;
        case 8: case 9: sl->ptr = e->shadow + off; sl->es = 2; break;
        default: return set_error(-1, "engine adapter: bad which=%d", which);
    }
    return 0;
}

// host <-> adapter tensor copy on the engine's stream, then wait for it
static int adapter_copy(Engine* e, const Slot& sl, void* host, bool to_host) {
    const size_t hp = (size_t)sl.width * sl.es, dp = (size_t)sl.pitch * sl.es;
    if (to_host)
        TA_HIP(hipMemcpy2DAsync(host, hp, sl.ptr, dp, hp, sl.rows, hipMemcpyDeviceToHost, e->s));
    else
        TA_HIP(hipMemcpy2DAsync(sl.ptr, dp, host, hp, hp, sl.rows, hipMemcpyHostToDevice, e->s));
    TA_HIP(hipStreamSynchronize(e->s));
    return 0;
}

int ta_engine_write_adapter(void* ep, int layer, int target, int which, const void* host,
                            int64_t n) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && host, "engine_write_adapter: null argument");
    Slot sl;
    CK(adapter_slot(e, layer, target, which, &sl));
    TA_REQUIRE(n == sl.cnt, "engine_write_adapter: n=%lld, tensor has %lld", (long long)n,
               (long long)sl.cnt);
    CK(adapter_copy(e, sl, const_cast<void*>(host), false));
    if (which == 8 || which == 9) {  // the transposed copy the LoRA backward reads
        CK(refresh_shadowT(e));
        TA_HIP(hipStreamSynchronize(e->s));
    }
    return 0;
}

int ta_engine_step_resident(void* ep, const int32_t* d_inputs, const int32_t* d_targets,
                            float lr_override, ta_step_metrics* m) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && d_inputs && d_targets, "engine_step_resident: null argument");
    auto t0 = std::chrono::steady_clock::now();
    CK(mask_targets_dev(d_inputs, d_targets, e->tgt_dev, e->B, e->T, e->s));
    e->tok_cur = d_inputs;
    return engine_step_body(e, lr_override, m, t0);
}

int ta_engine_profile(void* ep, int category) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e, "engine_profile: null engine");
    TA_REQUIRE(category >= -1 && category < TA_NCAT, "engine_profile: bad category %d", category);
    e->prof_cat = category;
    e->p_ms = e->p_flops = e->p_bytes = 0;
    e->p_n = 0;
    return 0;
}

int ta_engine_profile_read(void* ep, double* ms, int64_t* n, double* flops, double* bytes) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e, "engine_profile_read: null engine");
    if (ms) *ms = e->p_ms;
    if (n) *n = e->p_n;
    if (flops) *flops = e->p_flops;
    if (bytes) *bytes = e->p_bytes;
    e->p_ms = e->p_flops = e->p_bytes = 0;
    e->p_n = 0;
    return 0;
}

int ta_engine_read_adapter(void* ep, int layer, int target, int which, void* host, int64_t n) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && host, "engine_read_adapter: null argument");
    Slot sl;
    CK(adapter_slot(e, layer, target, which, &sl));
    TA_REQUIRE(n == sl.cnt, "engine_read_adapter: n=%lld, tensor has %lld", (long long)n,
               (long long)sl.cnt);
    return adapter_copy(e, sl, host, true);
}

int ta_engine_centroid(void* ep, double* host) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && host, "engine_centroid: null argument");
    TA_HIP(hipMemcpyAsync(host, e->cacc, (e->H + 1) * sizeof(double), hipMemcpyDeviceToHost, e->s));
    TA_HIP(hipStreamSynchronize(e->s));
    return 0;
}

void* ta_engine_buffer(void* ep, const char* name, int64_t* n, int* is_f32) {
    Engine* e = (Engine*)ep;
    if (!e || !name) return nullptr;
    auto it = e->named.find(name);
    if (it == e->named.end()) {
        set_error(-1, "engine_buffer: no buffer '%s'", name);
        return nullptr;
    }
    if (n) *n = it->second.second.first;
    if (is_f32) *is_f32 = it->second.second.second;
    return it->second.first;
}

int ta_engine_read_buffer(void* ep, const char* name, void* host, int64_t n) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e && name && host, "engine_read_buffer: null argument");
    auto it = e->named.find(name);
    TA_REQUIRE(it != e->named.end(), "engine_read_buffer: no buffer '%s'", name);
    TA_REQUIRE(n >= 0 && n <= it->second.second.first, "engine_read_buffer: n=%lld too large",
               (long long)n);
    size_t es = it->second.second.second ? 4 : 2;
    TA_HIP(hipStreamSynchronize(e->s));
    TA_HIP(hipMemcpy(host, it->second.first, n * es, hipMemcpyDeviceToHost));
    return 0;
}

int ta_engine_phase_ms(void* ep, float* f, float* b, float* t) {
    Engine* e = (Engine*)ep;
    TA_REQUIRE(e, "engine_phase_ms: null engine");
    if (f) *f = e->phase[0];
    if (b) *b = e->phase[1];
    if (t) *t = e->phase[2];
    return 0;
}

}  // extern "C"

extern "C" float ta_cosine_lr(float base_lr, int64_t warmup, int64_t total, float floor_frac,
                              int64_t step) {
    return cosine_lr(base_lr, warmup, total, floor_frac, step);
}
