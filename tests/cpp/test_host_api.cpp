// Tests of the C++ host API (include/tensor/**) as a caller of the
// reference's interface would use it: Device, Tensor, GEMM, ops::, the
// Centroid Accumulator (snapshot / merge file formats) and Dataset.
//
//   test_host_api cpu <dir>   no device use; writes <dir>/batches.bin and
//                             <dir>/lr.bin for the Python side to compare
//                             with the reference's compiled host code
//   test_host_api gpu <dir>   device paths on hip:0
//   test_host_api perop <dir> the per-op classes against the step engine
// Exit status 0 when every check passed; each failure prints one line.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <functional>
#include <string>
#include <vector>

#include "ta_backend.h"
#include "ta_engine.h"
#include <tensor/backend/cuda/device.hpp>
#include <tensor/backend/cuda/ops.hpp>
#include <tensor/backend/cuda/tensor.hpp>
#include <tensor/centroid/centroid_accumulator.hpp>
#include <tensor/centroid/centroid_merge.hpp>
#include <tensor/core/tensor_view.hpp>
#include <tensor/data/dataset.hpp>
#include <tensor/adapter/adapter_config.hpp>
#include <tensor/base/frozen_base.hpp>
#include <tensor/checkpoint/adapter_writer.hpp>
#include <tensor/adapter/adapter_model.hpp>
#include <tensor/base/arch/qwen2.hpp>
#include <tensor/trainer/adamw.hpp>
#include <tensor/trainer/adapt_trainer.hpp>
#include <tensor/trainer/cosine_schedule.hpp>

namespace fs = std::filesystem;
using namespace tensor;
using backend::cuda::CudaError;
using backend::cuda::Device;
using backend::cuda::GemmParams;
using backend::cuda::Tensor;
using core::DType;
using core::Shape;
using core::TensorView;
namespace ops = backend::cuda::ops;

static int g_fail = 0;
#define CHECK(cond)                                                            \
    do {                                                                       \
        if (!(cond)) {                                                         \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);        \
            g_fail++;                                                          \
        }                                                                      \
    } while (0)

template <typename E>
static bool throws(const std::function<void()>& f, const char* prefix = nullptr) {
    try {
        f();
    } catch (const E& e) {
        return !prefix || std::strncmp(e.what(), prefix, std::strlen(prefix)) == 0;
    } catch (...) {
        return false;
    }
    return false;
}

static uint16_t f2bf(float f) {  // round to nearest even
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static float bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
static uint32_t lcg(uint32_t& s) { return s = s * 1664525u + 1013904223u; }
static float urand(uint32_t& s) { return (float)(lcg(s) >> 8) / 16777216.f * 2.f - 1.f; }

template <typename T>
static void write_file(const fs::path& p, const std::vector<T>& v) {
    std::ofstream f(p, std::ios::binary);
    f.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * sizeof(T)));
}
static std::vector<char> read_file(const fs::path& p) {
    std::ifstream f(p, std::ios::binary);
    return std::vector<char>(std::istreambuf_iterator<char>(f), {});
}

static void writer_tests(const fs::path& dir);

static void cpu_tests(const fs::path& dir) {
    // core types
    CHECK(core::dtype_size(DType::BF16) == 2 && core::dtype_size(DType::F64) == 8);
    CHECK(core::to_string(DType::F8_E4M3) == "F8_E4M3");
    CHECK((Shape{}.numel() == 1 && Shape{3, 4, 5}.numel() == 60 && Shape{3, 0}.numel() == 0));
    std::vector<float> host(6, 1.f);
    TensorView tv{host.data(), DType::F32, Shape{2, 3}};
    CHECK(tv.nbytes() == 24 && tv.as<float>().size() == 6);
    CHECK(throws<std::invalid_argument>([&] { (void)tv.as<uint16_t>(); }));

    // device spec errors (reference message prefix)
    CHECK(throws<CudaError>([] { (void)Device::open("gpu:0"); },
                            "CudaError: invalid device spec"));
    CHECK(throws<CudaError>([] { (void)Device::open("cuda:x"); },
                            "CudaError: invalid device index"));
    CHECK(throws<std::runtime_error>([] { (void)Device::open("hip:-1"); }));

    // Dataset: two files concatenated in name order, wrap-around windows
    fs::create_directories(dir / "data");
    std::vector<uint32_t> a(37), b(29);
    uint32_t s = 7;
    for (auto& t : a) t = lcg(s) % 151936u;
    for (auto& t : b) t = lcg(s) % 151936u;
    write_file(dir / "data" / "b.bin", b);
    write_file(dir / "data" / "a.bin", a);
    write_file(dir / "data" / "skip.txt", a);
    auto ds = data::Dataset::load((dir / "data").string());
    CHECK(ds.total_tokens() == 66);
    std::vector<int32_t> out;
    const int B = 3, T = 10, NB = 5;  // 150 tokens: wraps twice
    for (int i = 0; i < NB; i++) {
        auto [in, tg] = ds.next_batch(B, T);
        CHECK(in.size() == (size_t)B * T && tg.size() == (size_t)B * T);
        out.insert(out.end(), in.begin(), in.end());
        out.insert(out.end(), tg.begin(), tg.end());
    }
    CHECK(ds.tokens_consumed() == (size_t)NB * B * T);
    write_file(dir / "batches.bin", out);
    CHECK(throws<data::DataError>([&] { (void)data::Dataset::load((dir / "missing").string()); },
                                  "DataError: path not found"));
    fs::create_directories(dir / "empty");
    CHECK(throws<data::DataError>([&] { (void)data::Dataset::load((dir / "empty").string()); },
                                  "DataError: no .bin files"));
    CHECK(throws<std::runtime_error>(
        [&] { backend::cuda::Tensor t; (void)t.to_host_f32(); }) == false);  // empty F32: fine

    // learning-rate schedule over a grid, for comparison with the reference
    std::vector<float> lr;
    for (int warm : {0, 1, 5, 100})
        for (int total : {1, 50, 1000})
            for (int step = 0; step < 60; step++) {
                if (total <= warm) continue;
                trainer::CosineSchedule cs{3e-4f, (size_t)warm, (size_t)total};
                lr.push_back(cs.lr_at((size_t)step));
            }
    write_file(dir / "lr.bin", lr);

    // merging an empty directory is an error, as in the reference
    fs::create_directories(dir / "no_snapshots");
    CHECK(throws<std::runtime_error>(
        [&] { centroid::CentroidMerge::run((dir / "no_snapshots").string(), "x", 4); },
        "No .centroid files"));

    writer_tests(dir / "writer");
}

// AdapterWriter: a checkpoint and a final adapter from known tensors (the
// Python side checks the files against independent readers), and the
// checkpoint read back exactly.
static void writer_tests(const fs::path& dir) {
    using checkpoint::AdapterTensor;
    std::vector<AdapterTensor> ts;
    uint32_t s = 11;
    for (int l = 0; l < 2; l++)
        for (int p : {0, 2, 6})
            for (int ab = 0; ab < 2; ab++) {
                AdapterTensor t;
                t.name = checkpoint::lora_prefix(l, p) + (ab ? ".lora_B" : ".lora_A");
                const size_t n = 8 + 3 * l + p + ab;
                for (size_t i = 0; i < n; i++) {
                    t.value.push_back(urand(s) * 0.05f);
                    t.exp_avg.push_back(urand(s) * 1e-3f);
                    t.exp_avg_sq.push_back(std::fabs(urand(s)) * 1e-6f);
                }
                // BF16 ties: 1 + 2^-8 rounds down to even, 1 + 3*2^-8 up to even
                t.value[0] = 1.00390625f;
                t.value[1] = -1.01171875f;
                ts.push_back(std::move(t));
            }
    std::vector<double> sums(17);
    for (auto& v : sums) v = urand(s) * 1e3;
    adapter::AdapterConfig cfg;
    cfg.rank = 4;
    cfg.alpha = 0.1f;
    cfg.inject_k = false;
    cfg.inject_down = true;
    base::FrozenBase fb;
    fb.config.arch_name = "qwen2";
    fb.config.base_sha = "abc123";
    fb.config.num_layers = 2;
    fb.config.hidden_size = 16;
    checkpoint::AdapterWriter w(dir.string());
    w.save_checkpoint(ts, sums, cfg, fb, "golang/gin \"x\"", 7, 3584, (dir / "ckpt").string());
    w.save_final(ts, cfg, fb, "golang/gin", 9, 4608, (dir / "final").string());
    checkpoint::TrainState st = checkpoint::load_checkpoint((dir / "ckpt").string());
    CHECK(st.step == 7 && st.tokens_consumed == 3584 && st.centroid_sums == sums);
    CHECK(st.tensors.size() == ts.size());
    for (const auto& t : ts) {
        bool found = false;
        for (const auto& r : st.tensors)
            if (r.name == t.name) {
                found = true;
                CHECK(r.value == t.value && r.exp_avg == t.exp_avg && r.exp_avg_sq == t.exp_avg_sq);
            }
        CHECK(found);
    }
    CHECK(!fs::exists(dir / "final" / "train_state.json"));
    CHECK(throws<std::runtime_error>(
        [&] { (void)checkpoint::load_checkpoint((dir / "absent").string()); }));
    // the tensors' names and F32 values, in order, for the Python side
    std::ofstream names(dir / "names.txt");
    std::vector<float> vals;
    for (const auto& t : ts) {
        names << t.name << " " << t.value.size() << "\n";
        vals.insert(vals.end(), t.value.begin(), t.value.end());
    }
    write_file(dir / "values.bin", vals);
    write_file(dir / "sums.bin", sums);
}

static void trainer_tests(const Device& dev, const fs::path& dir);

static void gpu_tests(const fs::path& dir) {
    Device dev = Device::open("hip:0");
    CHECK(dev.supports_bf16_gemm() && dev.sm_major() >= 9);
    CHECK(dev.arch().rfind("gfx950", 0) == 0);
    { Device d2 = Device::open("cuda:0"); CHECK(d2.id() == 0); }

    // Tensor round trips and dtype checks
    std::vector<uint16_t> hb(1000);
    uint32_t s = 3;
    for (auto& v : hb) v = f2bf(urand(s));
    Tensor tb = Tensor::from_host(TensorView{hb.data(), DType::BF16, Shape{10, 100}}, dev);
    CHECK(tb.to_host_bf16() == hb);
    CHECK(throws<std::runtime_error>([&] { (void)tb.to_host_f32(); }));
    Tensor tz = Tensor::zeros_f32(Shape{257}, dev);
    auto z = tz.to_host_f32();
    CHECK(z.size() == 257 && std::all_of(z.begin(), z.end(), [](float x) { return x == 0.f; }));
    std::vector<int32_t> hi = {5, -1, 151645, 0};
    Tensor ti = Tensor::from_host(TensorView{hi.data(), DType::I32, Shape{4}}, dev);
    auto u = ti.to_host_u32();
    CHECK(u.size() == 4 && u[0] == 5 && u[1] == 0xffffffffu && u[2] == 151645u);
    Tensor moved = std::move(tb);
    CHECK(tb.empty() && !moved.empty() && moved.numel() == 1000);

    // GEMM: column-major semantics vs a double brute force (one BF16 rounding)
    {
        const int M = 37, N = 45, K = 96;
        std::vector<uint16_t> A(M * K), Bm(K * N), C(M * N);
        for (auto& v : A) v = f2bf(urand(s));
        for (auto& v : Bm) v = f2bf(urand(s));
        for (auto& v : C) v = f2bf(urand(s));
        for (int ta = 0; ta < 2; ta++)
            for (int tb2 = 0; tb2 < 2; tb2++) {
                int lda = ta ? K : M, ldb = tb2 ? N : K;
                Tensor dA = Tensor::from_host(TensorView{A.data(), DType::BF16, Shape{A.size()}}, dev);
                Tensor dB = Tensor::from_host(TensorView{Bm.data(), DType::BF16, Shape{Bm.size()}}, dev);
                Tensor dC = Tensor::from_host(TensorView{C.data(), DType::BF16, Shape{C.size()}}, dev);
                GemmParams p{(bool)ta, (bool)tb2, M, N, K, 0.5f, 1.0f};
                backend::cuda::gemm_bf16(dev, p, dA.bf16(), lda, dB.bf16(), ldb, dC.bf16(), M);
                auto got = dC.to_host_bf16();
                int bad = 0;
                for (int i = 0; i < M; i++)
                    for (int j = 0; j < N; j++) {
                        double acc = 0;
                        for (int k = 0; k < K; k++) {
                            float a = bf2f(ta ? A[k + i * lda] : A[i + k * lda]);
                            float b = bf2f(tb2 ? Bm[j + k * ldb] : Bm[k + j * ldb]);
                            acc += (double)a * b;
                        }
                        double want = 0.5 * acc + bf2f(C[i + j * M]);
                        double g = bf2f(got[i + j * M]);
                        if (std::fabs(g - want) > std::fabs(want) * (1.0 / 128) + 1e-6) bad++;
                    }
                CHECK(bad == 0);
            }
        Tensor dA = Tensor::empty_bf16(Shape{4}, dev);
        CHECK(throws<CudaError>([&] {
            backend::cuda::gemm_bf16(dev, GemmParams{false, false, 0, 1, 1}, dA.bf16(), 1,
                                     dA.bf16(), 1, dA.bf16(), 1);
        }, "CudaError: gemm_bf16: M/N/K must be > 0"));
        CHECK(throws<CudaError>([&] {
            backend::cuda::gemm_bf16(dev, GemmParams{false, false, 1, 1, 1}, dA.bf16(), 0,
                                     dA.bf16(), 1, dA.bf16(), 1);
        }, "CudaError: gemm_bf16: leading dims must be > 0"));
    }

    // ops: RMSNorm of a constant row is w*c/sqrt(c^2+eps); rms_out = inverse RMS
    {
        const int D = 1536, rows = 4;
        std::vector<uint16_t> x(rows * D), w(D, f2bf(1.f));
        for (int r = 0; r < rows; r++)
            for (int d = 0; d < D; d++) x[r * D + d] = f2bf(0.25f * (r + 1));
        Tensor dx = Tensor::from_host(TensorView{x.data(), DType::BF16, Shape{(size_t)rows, (size_t)D}}, dev);
        Tensor dw = Tensor::from_host(TensorView{w.data(), DType::BF16, Shape{(size_t)D}}, dev);
        Tensor out = Tensor::empty_bf16(Shape{(size_t)rows, (size_t)D}, dev);
        Tensor rms = Tensor::empty_f32(Shape{(size_t)rows}, dev);
        ops::rms_norm_fwd(dx.bf16(), dw.bf16(), out.bf16(), rms.f32(), 1, rows, D, 1e-6f,
                          dev.stream());
        auto o = out.to_host_bf16();
        auto r = rms.to_host_f32();
        for (int i = 0; i < rows; i++) {
            double c = 0.25 * (i + 1);
            CHECK(std::fabs(r[i] - 1.0 / std::sqrt(c * c + 1e-6)) < 1e-5 / c);
            CHECK(std::fabs(bf2f(o[i * D + 7]) - c / std::sqrt(c * c + 1e-6)) < 4e-3);
        }
        CHECK(throws<CudaError>([&] {
            ops::rms_norm_fwd(dx.bf16(), dw.bf16(), out.bf16(), rms.f32(), 1, rows, -1, 1e-6f,
                              dev.stream());
        }));
    }

    // ops: cross entropy of zero logits is ln V with gradient (1/V - onehot)/N
    {
        const int N = 3, V = 151936;
        Tensor lg = Tensor::zeros(Shape{(size_t)N, (size_t)V}, DType::BF16, dev);
        std::vector<int32_t> tg = {5, -1, V - 1};
        Tensor dt = Tensor::from_host(TensorView{tg.data(), DType::I32, Shape{3}}, dev);
        Tensor loss = Tensor::empty_f32(Shape{(size_t)N}, dev);
        ops::cross_entropy_fwd(lg.bf16(), dt.i32(), loss.f32(), lg.bf16(), N, V, dev.stream());
        auto l = loss.to_host_f32();
        for (int i = 0; i < N; i++) CHECK(std::fabs(l[i] - std::log((double)V)) < 1e-4);
        auto g = lg.to_host_bf16();
        CHECK(std::fabs(bf2f(g[5]) - (1.0 / V - 1.0) / N) < 2e-3);
        CHECK(bf2f(g[(size_t)V + 9]) == bf2f(f2bf((float)(1.0 / V / N))));
    }

    // Centroid Accumulator: equal gradient norms -> centroid = mean of h;
    // snapshot and merged files in the reference's byte layout
    {
        const int D = 64, BT = 200;
        fs::path sdir = dir / "snapshots";
        fs::remove_all(sdir);
        centroid::CentroidAccumulator acc(D, sdir.string());
        std::vector<uint16_t> h(BT * D), g(BT * D, 0);
        std::vector<double> mean(D, 0.0);
        for (int t = 0; t < BT; t++) {
            for (int d = 0; d < D; d++) {
                h[t * D + d] = f2bf(urand(s));
                mean[d] += bf2f(h[t * D + d]) / BT;
            }
            g[t * D + (t % D)] = f2bf((t & 1) ? -2.f : 2.f);  // ||g_t|| = 2
        }
        Tensor th = Tensor::from_host(TensorView{h.data(), DType::BF16, Shape{(size_t)BT, (size_t)D}}, dev);
        Tensor tg = Tensor::from_host(TensorView{g.data(), DType::BF16, Shape{(size_t)BT, (size_t)D}}, dev);
        acc.write_snapshot(0);  // W == 0: no file
        CHECK(!fs::exists(sdir / "step-0.centroid"));
        acc.accumulate(th, tg, dev);
        Tensor wrong = Tensor::empty_bf16(Shape{(size_t)BT, 32}, dev);
        acc.accumulate(wrong, wrong, dev);  // other D: ignored
        acc.write_snapshot(10);
        auto bytes = read_file(sdir / "step-10.centroid");
        CHECK(bytes.size() == 4 + 4 * D + 4);
        int32_t d0;
        std::memcpy(&d0, bytes.data(), 4);
        CHECK(d0 == D);
        std::vector<float> c(D);
        std::memcpy(c.data(), bytes.data() + 4, 4 * D);
        float w;
        std::memcpy(&w, bytes.data() + 4 + 4 * D, 4);
        CHECK(w == 400.f);
        double err = 0;
        for (int d = 0; d < D; d++) err = std::max(err, std::fabs(c[d] - mean[d]));
        CHECK(err < 1e-6);
        // F32 inputs take the same path as the BF16 ones
        std::vector<float> hf(BT * D), gf(BT * D);
        for (int i = 0; i < BT * D; i++) {
            hf[i] = bf2f(h[i]);
            gf[i] = bf2f(g[i]);
        }
        Tensor thf = Tensor::from_host(TensorView{hf.data(), DType::F32, Shape{(size_t)BT, (size_t)D}}, dev);
        Tensor tgf = Tensor::from_host(TensorView{gf.data(), DType::F32, Shape{(size_t)BT, (size_t)D}}, dev);
        acc.accumulate(thf, tgf, dev);
        auto sums = acc.sums();
        CHECK(sums[D] == 800.0);
        for (int d = 0; d < D; d++) CHECK(std::fabs(sums[d] / 800.0 - mean[d]) < 1e-6);
        acc.write_snapshot(20);
        // merge: k = 1 keeps the first snapshot (the first assignment pass
        // changes nothing, so the loop stops before any update)
        acc.merge_and_write(1, (dir / "merged1.centroid").string());
        auto m = read_file(dir / "merged1.centroid");
        CHECK(m.size() == 8 + 4 * D);
        int32_t hk[2];
        std::memcpy(hk, m.data(), 8);
        CHECK(hk[0] == 1 && hk[1] == D);
        CHECK(std::memcmp(m.data() + 8, bytes.data() + 4, 4 * D) == 0);
        // standalone merge over the directory, k clamped to the snapshot count
        for (int i = 0; i < 4; i++) {
            std::vector<float> v(D, (i < 2 ? 1.f : 100.f) + 0.01f * i);
            std::ofstream f(sdir / ("step-" + std::to_string(100 + i) + ".centroid"),
                            std::ios::binary);
            int32_t dd = D;
            float ww = 1.f;
            f.write((const char*)&dd, 4);
            f.write((const char*)v.data(), 4 * D);
            f.write((const char*)&ww, 4);
        }
        centroid::CentroidMerge::run(sdir.string(), (dir / "merged.centroid").string(), 9);
        auto mm = read_file(dir / "merged.centroid");
        std::memcpy(hk, mm.data(), 8);
        CHECK(hk[0] == 6 && hk[1] == D && mm.size() == 8 + 4 * 6 * D);
    }

    // memory: every block is back in the cache once the tensors are gone
    {
        int64_t in_use = -1, cached = -1;
        {
            Tensor t1 = Tensor::empty_f32(Shape{1 << 20}, dev);
            ta_mem_stats(0, &in_use, &cached);
            CHECK(in_use >= (4 << 20));
        }
        int64_t in2 = -1, cached2 = -1;
        ta_mem_stats(0, &in2, &cached2);
        CHECK(in2 < in_use && cached2 >= (4 << 20));
        void* p = nullptr;
        CHECK(ta_mem_free(&p, 0) != 0);  // not ours: rejected
    }
    dev.sync();
    trainer_tests(dev, dir / "trainer");
}

// A small Qwen2 base (V=1024 unless given, H=256, 2 layers, 4 Q / 2 KV
// heads of 64, I=512) in device tensors, N(0, 0.02) weights, unit norms,
// zero biases.
static base::FrozenBase small_base(const Device& dev, size_t V = 1024) {
    base::FrozenBase b;
    base::BaseConfig& c = b.config;
    c.arch_name = "qwen2";
    c.arch = base::ArchType::Qwen2;
    c.vocab_size = V;
    c.hidden_size = 256;
    c.num_layers = 2;
    c.num_q_heads = 4;
    c.num_kv_heads = 2;
    c.head_dim = 64;
    c.intermediate_size = 512;
    c.rms_norm_eps = 1e-6f;
    c.rope_theta = 1e6f;
    c.tie_embeddings = true;
    uint32_t s = 17;
    auto mk = [&](std::initializer_list<size_t> shape, float scale, float fill) {
        Shape sh(shape);
        std::vector<uint16_t> h(sh.numel());
        for (auto& v : h) v = f2bf(scale > 0 ? urand(s) * scale * 1.7320508f : fill);
        return Tensor::from_host(TensorView{h.data(), DType::BF16, sh}, dev);
    };
    const size_t H = 256, q = 256, kv = 128, I = 512;
    b.embed_w = mk({V, H}, 0.02f, 0.f);
    b.final_norm_w = mk({H}, 0.f, 1.f);
    for (int l = 0; l < 2; l++) {
        base::LayerWeights w;
        w.input_norm_w = mk({H}, 0.f, 1.f);
        w.post_norm_w = mk({H}, 0.f, 1.f);
        w.q_proj_w = mk({q, H}, 0.02f, 0.f);
        w.q_proj_b = mk({q}, 0.f, 0.f);
        w.k_proj_w = mk({kv, H}, 0.02f, 0.f);
        w.k_proj_b = mk({kv}, 0.f, 0.f);
        w.v_proj_w = mk({kv, H}, 0.02f, 0.f);
        w.v_proj_b = mk({kv}, 0.f, 0.f);
        w.o_proj_w = mk({H, q}, 0.02f, 0.f);
        w.gate_proj_w = mk({I, H}, 0.02f, 0.f);
        w.up_proj_w = mk({I, H}, 0.02f, 0.f);
        w.down_proj_w = mk({H, I}, 0.02f, 0.f);
        b.layers.push_back(std::move(w));
    }
    return b;
}

// every adapter tensor of a trainer's engine (masters, moments, shadows)
static std::vector<std::vector<char>> adapter_state(void* eng, int mask, const base::BaseConfig& c,
                                                    int r) {
    std::vector<std::vector<char>> out;
    const int64_t H = c.hidden_size, q = c.num_q_heads * c.head_dim,
                  kv = c.num_kv_heads * c.head_dim, I = c.intermediate_size;
    const int64_t in[7] = {H, H, H, q, H, H, I}, o[7] = {q, kv, kv, H, I, I, H};
    for (int l = 0; l < (int)c.num_layers; l++)
        for (int p = 0; p < 7; p++) {
            if (!((mask >> p) & 1)) continue;
            for (int which = 0; which < 10; which++) {
                const bool isA = which == 0 || which == 2 || which == 3 || which == 6 || which == 8;
                const int64_t n = isA ? r * in[p] : o[p] * r;
                std::vector<char> buf(n * (which >= 8 ? 2 : 4));
                CHECK(ta_engine_read_adapter(eng, l, p, which, buf.data(), n) == 0);
                out.push_back(std::move(buf));
            }
        }
    return out;
}

// AdaptTrainer driven as tools/tensor-adapt.cpp drives it (Device, an
// in-memory FrozenBase, AdapterConfig, Dataset, AdaptOptions, run()), then
// checkpoint + resume: a trainer resumed from the step-2 checkpoint takes
// step 3 to exactly the state, loss and centroid sums of the original run.
static void trainer_tests(const Device& dev, const fs::path& dir) {
    fs::create_directories(dir / "data");
    std::vector<uint32_t> toks(5000);
    uint32_t s = 23;
    for (auto& t : toks) t = lcg(s) % 1024u;
    write_file(dir / "data" / "tokens.bin", toks);
    base::FrozenBase fb = small_base(dev);
    adapter::AdapterConfig cfg;
    cfg.rank = 8;
    cfg.alpha = 16.f;
    cfg.inject_k = cfg.inject_o = false;
    cfg.inject_gate = cfg.inject_down = true;
    cfg.lr = 1e-3f;
    cfg.warmup_steps = 1;
    cfg.weight_decay = 0.01f;
    cfg.batch_size = 2;
    cfg.seq_len = 64;
    const size_t bt = 128;

    {  // run() to the token budget: 5 steps, checkpoints at 2 and 4
        auto ds = data::Dataset::load((dir / "data").string());
        trainer::AdaptOptions opts;
        opts.domain = "test/domain";
        opts.output_dir = (dir / "run").string();
        opts.checkpoint_every = 2;
        opts.tokens = 5 * bt;
        opts.log_to_stdout = false;
        auto tr = trainer::AdaptTrainer::create(fb, cfg, ds, opts, dev);
        CHECK(!tr.done());
        tr.run();
        CHECK(tr.done() && ds.tokens_consumed() == 5 * bt);
        for (const char* f : {"adapter.safetensors", "adapter.json", "adapter.centroid",
                              "centroids/step-2.centroid", "centroids/step-4.centroid",
                              "centroids/step-5.centroid", "step-2/optimizer.safetensors",
                              "step-4/train_state.json"})
            CHECK(fs::exists(dir / "run" / f));
        auto js = read_file(dir / "run" / "adapter.json");
        std::string j(js.begin(), js.end());
        CHECK(j.find("\"step\": 5") != std::string::npos &&
              j.find("\"tokens_trained\": 640") != std::string::npos);
    }
    // step by step, checkpoint at 2; then a trainer resumed from it
    auto dsA = data::Dataset::load((dir / "data").string());
    trainer::AdaptOptions oa;
    oa.output_dir = (dir / "a").string();
    oa.checkpoint_every = 2;
    oa.tokens = 10 * bt;
    oa.log_to_stdout = false;
    auto A = trainer::AdaptTrainer::create(fb, cfg, dsA, oa, dev);
    trainer::StepMetrics ma{};
    for (int i = 0; i < 3; i++) {
        ma = A.step();
        CHECK(ma.step == (size_t)i + 1 && ma.tokens_consumed == (i + 1) * bt);
        CHECK(std::isfinite(ma.loss) && ma.loss > 0.f && ma.grad_norm > 0.f);
        CHECK(ma.grad_norm <= cfg.grad_clip && ma.learning_rate > 0.f);
    }
    CHECK(fs::exists(dir / "a" / "step-2" / "optimizer.safetensors"));
    auto stA = adapter_state(A.engine(), cfg.inject_mask(), fb.config, cfg.rank);
    std::vector<double> cA(257);
    CHECK(ta_engine_centroid(A.engine(), cA.data()) == 0);

    auto dsB = data::Dataset::load((dir / "data").string());
    trainer::AdaptOptions ob = oa;
    ob.output_dir = (dir / "b").string();
    ob.resume_from = (dir / "a" / "step-2").string();
    auto Bt = trainer::AdaptTrainer::create(fb, cfg, dsB, ob, dev);
    trainer::StepMetrics mb = Bt.step();
    CHECK(mb.step == 3 && mb.tokens_consumed == 3 * bt && dsB.tokens_consumed() == 3 * bt);
    CHECK(mb.loss == ma.loss && mb.grad_norm == ma.grad_norm &&
          mb.learning_rate == ma.learning_rate);
    auto stB = adapter_state(Bt.engine(), cfg.inject_mask(), fb.config, cfg.rank);
    CHECK(stA.size() == stB.size());
    size_t diff = 0;
    for (size_t i = 0; i < stA.size() && i < stB.size(); i++) diff += stA[i] != stB[i];
    CHECK(diff == 0);
    std::vector<double> cB(257);
    CHECK(ta_engine_centroid(Bt.engine(), cB.data()) == 0);
    CHECK(cA == cB && cA[256] > 0);
    // a checkpoint of another configuration is refused
    adapter::AdapterConfig other = cfg;
    other.inject_k = true;
    auto dsC = data::Dataset::load((dir / "data").string());
    CHECK(throws<std::runtime_error>(
        [&] { (void)trainer::AdaptTrainer::create(fb, other, dsC, ob, dev); }, "resume:"));
}

// BASELINE configs[1] (c2) run through AdaptTrainer on its own schedule:
// Qwen2-0.5B shape (24 layers, hidden 896, 14/2 heads of 64, SwiGLU 4864,
// tied 151936-entry embedding), r=16 alpha=32 on q,k,v,o, batch 4 x 512,
// lr 1e-4 with the cosine schedule over 20 steps, weight decay 0.01 and a
// centroid snapshot every 10 steps (centroid_accumulator.cpp:72-91).  Checks
// the two snapshot files' byte layout ([i32 D][D f32][f32 W]) and that each
// is the cumulative C / W of the accumulator at its step (the sums are not
// reset by a snapshot), the schedule's lr at every step, finite losses and
// norms, and the merged file ([i32 k][i32 D][k x D f32]): with k >= the 2
// snapshots every snapshot is its own center.
static void c2_schedule_tests(const fs::path& dir) {
    Device dev = Device::open("hip:0");
    const size_t V = 151936, H = 896, L = 24, q = 896, kv = 128, I = 4864, B = 4, T = 512;
    base::FrozenBase fb;
    base::BaseConfig& c = fb.config;
    c.arch_name = "qwen2";
    c.arch = base::ArchType::Qwen2;
    c.vocab_size = V;
    c.hidden_size = H;
    c.num_layers = L;
    c.num_q_heads = 14;
    c.num_kv_heads = 2;
    c.head_dim = 64;
    c.intermediate_size = I;
    c.rms_norm_eps = 1e-6f;
    c.rope_theta = 1e6f;
    c.tie_embeddings = true;
    uint32_t s = 91;
    auto mk = [&](std::initializer_list<size_t> shape, float scale, float fill) {
        Shape sh(shape);
        std::vector<uint16_t> h(sh.numel());
        for (auto& v : h) v = f2bf(scale > 0 ? urand(s) * scale * 1.7320508f : fill);
        return Tensor::from_host(TensorView{h.data(), DType::BF16, sh}, dev);
    };
    fb.embed_w = mk({V, H}, 0.02f, 0.f);
    fb.final_norm_w = mk({H}, 0.f, 1.f);
    for (size_t l = 0; l < L; l++) {
        base::LayerWeights w;
        w.input_norm_w = mk({H}, 0.f, 1.f);
        w.post_norm_w = mk({H}, 0.f, 1.f);
        w.q_proj_w = mk({q, H}, 0.02f, 0.f);
        w.q_proj_b = mk({q}, 0.f, 0.f);
        w.k_proj_w = mk({kv, H}, 0.02f, 0.f);
        w.k_proj_b = mk({kv}, 0.f, 0.f);
        w.v_proj_w = mk({kv, H}, 0.02f, 0.f);
        w.v_proj_b = mk({kv}, 0.f, 0.f);
        w.o_proj_w = mk({H, q}, 0.02f, 0.f);
        w.gate_proj_w = mk({I, H}, 0.02f, 0.f);
        w.up_proj_w = mk({I, H}, 0.02f, 0.f);
        w.down_proj_w = mk({H, I}, 0.02f, 0.f);
        fb.layers.push_back(std::move(w));
    }
    // uniform ids with an assistant span over almost every 512-token row, so
    // the trainer's masking keeps the targets
    fs::create_directories(dir / "data");
    std::vector<uint32_t> toks(20 * B * T + 1);
    for (auto& t : toks) t = lcg(s) % 150000u;
    for (size_t r = 0; r + T <= toks.size(); r += T) {
        toks[r + 3] = 151644;
        toks[r + 4] = 77091;
        toks[r + T - 8] = 151645;
    }
    write_file(dir / "data" / "tokens.bin", toks);
    adapter::AdapterConfig cfg;
    cfg.rank = 16;
    cfg.alpha = 32.f;
    cfg.lr = 1e-4f;
    cfg.warmup_steps = 0;
    cfg.weight_decay = 0.01f;
    cfg.batch_size = B;
    cfg.seq_len = T;
    auto ds = data::Dataset::load((dir / "data").string());
    trainer::AdaptOptions opts;
    opts.domain = "c2/schedule";
    opts.output_dir = (dir / "run").string();
    opts.checkpoint_every = 10;
    opts.tokens = 20 * B * T;
    opts.log_to_stdout = false;
    auto tr = trainer::AdaptTrainer::create(fb, cfg, ds, opts, dev);
    std::vector<double> acc[2];
    for (int i = 1; i <= 20; i++) {
        trainer::StepMetrics m = tr.step();
        CHECK(m.step == (size_t)i && std::isfinite(m.loss) && m.loss > 10.f && m.loss < 14.f);
        CHECK(std::isfinite(m.grad_norm) && m.grad_norm > 0.f && m.grad_norm <= cfg.grad_clip);
        CHECK(m.learning_rate == ta_cosine_lr(cfg.lr, 0, 20, 0.1f, i - 1));
        if (i % 10 == 0) {
            acc[i / 10 - 1].resize(H + 1);
            CHECK(ta_engine_centroid(tr.engine(), acc[i / 10 - 1].data()) == 0);
        }
    }
    CHECK(tr.done());
    CHECK(acc[0][H] > 0 && acc[1][H] > acc[0][H]);  // cumulative weight
    for (int k = 0; k < 2; k++) {
        auto f = read_file(dir / "run" / "centroids" / ("step-" + std::to_string(10 * (k + 1)) + ".centroid"));
        CHECK(f.size() == 4 + 4 * H + 4);
        if (f.size() != 4 + 4 * H + 4) continue;
        int32_t D;
        std::memcpy(&D, f.data(), 4);
        CHECK(D == (int32_t)H);
        size_t same = 0;
        for (size_t d = 0; d < H; d++) {
            float v;
            std::memcpy(&v, f.data() + 4 + 4 * d, 4);
            same += v == (float)(acc[k][d] / acc[k][H]);
        }
        CHECK(same == H);
        float w;
        std::memcpy(&w, f.data() + 4 + 4 * H, 4);
        CHECK(w == (float)acc[k][H]);
    }
    tr.save_adapter((dir / "out").string());
    auto m = read_file(dir / "out" / "adapter.centroid");
    CHECK(m.size() == 8 + 2 * 4 * H);
    if (m.size() == 8 + 2 * 4 * H) {
        int32_t k, D;
        std::memcpy(&k, m.data(), 4);
        std::memcpy(&D, m.data() + 4, 4);
        CHECK(k == 2 && D == (int32_t)H);
        for (int j = 0; j < 2; j++) {
            size_t same = 0;
            for (size_t d = 0; d < H; d++) {
                float v;
                std::memcpy(&v, m.data() + 8 + 4 * (j * H + d), 4);
                same += v == (float)(acc[j][d] / acc[j][H]);
            }
            CHECK(same == H);
        }
    }
}

// relative L2 distance of two F32 vectors
static double rel_l2(const std::vector<float>& a, const std::vector<float>& b) {
    double d = 0, n = 0;
    for (size_t i = 0; i < a.size() && i < b.size(); i++) {
        d += ((double)a[i] - b[i]) * ((double)a[i] - b[i]);
        n += (double)b[i] * b[i];
    }
    return n > 0 ? std::sqrt(d / n) : std::sqrt(d);
}

// The per-op classes (Qwen2Base, AdapterModel, AdamW) composed into the
// reference trainer's step (adapt_trainer.cu:189-253: zero_grad, forward,
// cross entropy over B*T rows, backward, mean of the positive per-token
// losses, AdamW::step_all; no clip at grad_clip = 1e30), two steps, against
// the step engine on the same base and batches.  Both start from the same
// adapter (the reference's hashed A, B = 0); before step 2 the engine takes
// the per-op model's state (masters, moments, BF16 weights), so each step's
// gradients are compared from one state.  The two paths take the reference's
// BF16 rounding points and differ in accumulation order and in the attention
// backward's form (stored P here, recomputed P in the engine): loss within
// 1e-3 relative, every gB (step 1; every gA is exactly 0 on both, B being 0)
// and every gA and gB (step 2) within 1e-2 relative L2.  AdamW::step_all is
// checked against the update written out from the model's own gradients
// (first step: m = (1 - b1) g, v = (1 - b2) g^2, bias corrections 1 - b^1;
// decoupled decay), and every BF16 weight against its master's rounding.
static void perop_tests() {
    Device dev = Device::open("hip:0");
    const size_t V = 151936;  // the chat-template ids fit: targets survive the masking
    base::FrozenBase fb = small_base(dev, V);
    const base::BaseConfig& c = fb.config;
    const int B = 2, T = 128, BT = B * T, L = (int)c.num_layers, R = 8;
    adapter::AdapterConfig cfg;
    cfg.rank = R;
    cfg.alpha = 16.f;
    cfg.weight_decay = 0.01f;
    cfg.grad_clip = 1e30f;
    const float lr = 1e-3f;

    ta_model_config mc{(int)V, 256, L, 4, 2, 64, 512, c.rms_norm_eps, c.rope_theta, 1};
    ta_adapt_config ac{R, cfg.alpha, 0b1111, lr, cfg.grad_clip, 0, 100, cfg.adam_beta1,
                       cfg.adam_beta2, 1e-8f, cfg.weight_decay};
    void* eng = ta_engine_create(&mc, &ac, B, T, dev.stream());
    CHECK(eng != nullptr);
    if (!eng) return;
    auto set = [&](const std::string& name, const Tensor& t) {
        CHECK(ta_engine_set_weight_device(eng, name.c_str(), t.bf16(), (int64_t)t.numel()) == 0);
    };
    set("model.embed_tokens.weight", fb.embed_w);
    set("model.norm.weight", fb.final_norm_w);
    for (int l = 0; l < L; l++) {
        const base::LayerWeights& w = fb.layers[l];
        const std::string p = "model.layers." + std::to_string(l) + ".";
        set(p + "input_layernorm.weight", w.input_norm_w);
        set(p + "post_attention_layernorm.weight", w.post_norm_w);
        set(p + "self_attn.q_proj.weight", w.q_proj_w);
        set(p + "self_attn.q_proj.bias", w.q_proj_b);
        set(p + "self_attn.k_proj.weight", w.k_proj_w);
        set(p + "self_attn.k_proj.bias", w.k_proj_b);
        set(p + "self_attn.v_proj.weight", w.v_proj_w);
        set(p + "self_attn.v_proj.bias", w.v_proj_b);
        set(p + "self_attn.o_proj.weight", w.o_proj_w);
        set(p + "mlp.gate_proj.weight", w.gate_proj_w);
        set(p + "mlp.up_proj.weight", w.up_proj_w);
        set(p + "mlp.down_proj.weight", w.down_proj_w);
    }

    adapter::AdapterModel m = adapter::AdapterModel::create(fb, cfg, dev);
    const int64_t in[4] = {256, 256, 256, 256}, out[4] = {256, 128, 128, 256};
    CHECK(m.layers.size() == (size_t)L &&
          m.param_count() == (size_t)L * R * ((256 + 256) + 2 * (256 + 128) + (256 + 256)));
    const trainer::AdamW opt(cfg);
    CHECK(opt.beta1 == cfg.adam_beta1 && opt.weight_decay == cfg.weight_decay && opt.eps == 1e-8f);
    auto pairs = [&](int l) {
        return std::vector<adapter::LoraPair*>{&m.layers[l].lora_q, &m.layers[l].lora_k,
                                               &m.layers[l].lora_v, &m.layers[l].lora_o};
    };
    // the engine starts from the same A (the hashed init) and B = 0
    for (int l = 0; l < L; l++)
        for (int p = 0; p < 4; p++) {
            std::vector<float> e(R * in[p]);
            CHECK(ta_engine_read_adapter(eng, l, p, 0, e.data(), R * in[p]) == 0);
            CHECK(e == pairs(l)[p]->A_f32.to_host_f32());
        }
    uint32_t rs = 91;
    for (int k = 1; k <= 2; k++) {
        // one assistant span per row, so the masking keeps most targets
        std::vector<int32_t> toks(BT + 1);
        for (auto& t : toks) t = (int32_t)(lcg(rs) % 150000u);
        for (int b = 0; b < B; b++) {
            toks[b * T + 3] = 151644;
            toks[b * T + 4] = 77091;
            toks[b * T + T - 8] = 151645;
        }
        std::vector<int32_t> inp(toks.begin(), toks.begin() + BT), tgt(toks.begin() + 1, toks.end());
        ta_step_metrics met{};
        CHECK(ta_engine_step(eng, inp.data(), tgt.data(), lr, &met) == 0);
        std::vector<int32_t> masked(BT);
        CHECK(ta_engine_read_buffer(eng, "targets", masked.data(), BT) == 0);

        Tensor tok_d = Tensor::from_host(TensorView{inp.data(), DType::I32, Shape({(size_t)BT})}, dev);
        Tensor tgt_d = Tensor::from_host(TensorView{masked.data(), DType::I32, Shape({(size_t)BT})}, dev);
        m.zero_grad(dev);
        auto fwd = base::arch::Qwen2Base::forward(fb, tok_d, B, T, dev, &m);
        CHECK(fwd.layer_cache.size() == (size_t)L && fwd.logits.numel() == (size_t)BT * V);
        Tensor loss_tok = Tensor::empty_f32(Shape({(size_t)BT}), dev);
        ops::cross_entropy_fwd(fwd.logits.bf16(), tgt_d.i32(), loss_tok.f32(), fwd.dlogits.bf16(),
                               BT, (int)V, dev.stream());
        auto grads = base::arch::Qwen2Base::backward(fb, fwd, B, T, dev, &m);
        CHECK(grads.size() == (size_t)L && grads[0].dx_attn_in.numel() == (size_t)BT * 256);
        double sum = 0;
        int nv = 0;
        for (float l : loss_tok.to_host_f32())
            if (l > 1e-9f) {
                sum += l;
                nv++;
            }
        const double loss = nv ? sum / nv : 0.0;
        std::printf("perop step %d: loss %.6f engine %.6f\n", k, loss, (double)met.loss);
        CHECK(std::fabs(loss - met.loss) <= 1e-3 * std::fabs(met.loss));
        double worst = 0;
        for (int l = 0; l < L; l++)
            for (int p = 0; p < 4; p++)
                for (int which : {6, 7}) {
                    const bool isA = which == 6;
                    const int64_t n = isA ? R * in[p] : out[p] * R;
                    std::vector<float> e(n);
                    CHECK(ta_engine_read_adapter(eng, l, p, which, e.data(), n) == 0);
                    const std::vector<float> g = (isA ? pairs(l)[p]->gA : pairs(l)[p]->gB).to_host_f32();
                    if (k == 1 && isA) {
                        bool zero = true;
                        for (size_t i = 0; i < g.size(); i++) zero = zero && g[i] == 0.f && e[i] == 0.f;
                        CHECK(zero);
                        continue;
                    }
                    const double d = rel_l2(g, e);
                    worst = std::max(worst, d);
                    if (d > 1e-2)
                        std::printf("FAIL layer %d pair %d %s: rel L2 %.3e\n", l, p, isA ? "gA" : "gB", d);
                    CHECK(d <= 1e-2);
                }
        std::printf("perop step %d: worst gradient rel L2 %.3e\n", k, worst);

        // AdamW::step_all against the update written out from the model's
        // own gradients and state
        std::vector<std::vector<float>> w0, m0, v0, gg;
        for (int l = 0; l < L; l++)
            for (adapter::LoraPair* lp : pairs(l)) {
                w0.push_back(lp->A_f32.to_host_f32());
                w0.push_back(lp->B_f32.to_host_f32());
                m0.push_back(lp->mA.to_host_f32());
                m0.push_back(lp->mB.to_host_f32());
                v0.push_back(lp->vA.to_host_f32());
                v0.push_back(lp->vB.to_host_f32());
                gg.push_back(lp->gA.to_host_f32());
                gg.push_back(lp->gB.to_host_f32());
            }
        opt.step_all(m, lr, k, dev);
        const double b1 = cfg.adam_beta1, b2 = cfg.adam_beta2, wd = cfg.weight_decay;
        const double c1 = 1.0 - std::pow(b1, k), c2 = 1.0 - std::pow(b2, k);
        double wu = 0;
        size_t bad_bf = 0, ti = 0;
        for (int l = 0; l < L; l++)
            for (adapter::LoraPair* lp : pairs(l))
                for (int ab = 0; ab < 2; ab++, ti++) {
                    const std::vector<float> w1 = (ab ? lp->B_f32 : lp->A_f32).to_host_f32();
                    const std::vector<uint16_t> h1 = (ab ? lp->B_bf16 : lp->A_bf16).to_host_bf16();
                    std::vector<float> want(w1.size());
                    for (size_t i = 0; i < w1.size(); i++) {
                        const double g = gg[ti][i];
                        const double mm = b1 * m0[ti][i] + (1 - b1) * g;
                        const double vv = b2 * v0[ti][i] + (1 - b2) * g * g;
                        const double w = w0[ti][i];
                        want[i] = (float)(w - lr * (mm / c1 / (std::sqrt(vv / c2) + 1e-8) + wd * w));
                        bad_bf += h1[i] != f2bf(w1[i]);
                    }
                    wu = std::max(wu, rel_l2(w1, want));
                }
        std::printf("perop step %d: AdamW worst rel L2 %.3e, BF16 mismatches %zu\n", k, wu, bad_bf);
        CHECK(wu <= 1e-5 && bad_bf == 0);

        // the engine takes the model's state for the next step
        if (k == 1)
            for (int l = 0; l < L; l++)
                for (int p = 0; p < 4; p++) {
                    adapter::LoraPair* lp = pairs(l)[p];
                    const Tensor* t32[6] = {&lp->A_f32, &lp->B_f32, &lp->mA, &lp->vA, &lp->mB, &lp->vB};
                    for (int which = 0; which < 6; which++) {
                        auto v = t32[which]->to_host_f32();
                        CHECK(ta_engine_write_adapter(eng, l, p, which, v.data(), (int64_t)v.size()) == 0);
                    }
                    for (int which : {8, 9}) {
                        auto v = (which == 8 ? lp->A_bf16 : lp->B_bf16).to_host_bf16();
                        CHECK(ta_engine_write_adapter(eng, l, p, which, v.data(), (int64_t)v.size()) == 0);
                    }
                }
    }
    CHECK(ta_engine_destroy(eng) == 0);
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::printf("usage: %s cpu|gpu <dir>\n", argv[0]);
        return 2;
    }
    fs::path dir = argv[2];
    fs::create_directories(dir);
    std::string mode = argv[1];
    try {
        if (mode == "cpu")
            cpu_tests(dir);
        else if (mode == "gpu")
            gpu_tests(dir);
        else if (mode == "c2sched")
            c2_schedule_tests(dir);
        else if (mode == "perop")
            perop_tests();
        else
            return 2;
    } catch (const std::exception& e) {
        std::printf("FAIL uncaught exception: %s\n", e.what());
        g_fail++;
    }
    std::printf("%s: %s (%d failures)\n", argv[0], g_fail ? "FAILED" : "OK", g_fail);
    return g_fail ? 1 : 0;
}
