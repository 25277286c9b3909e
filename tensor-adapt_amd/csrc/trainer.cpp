// trainer.cpp — the trainer layer of the C++ host API: AdapterConfig's
// factory, the adapter/checkpoint writer and AdaptTrainer over the step
// engine (include/tensor/adapter/adapter_config.hpp,
// include/tensor/checkpoint/adapter_writer.hpp,
// include/tensor/trainer/adapt_trainer.hpp).  Host code only; every device
// operation goes through a ta_* entry point.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "ta_backend.h"
#include "ta_engine.h"
#include <tensor/adapter/adapter_config.hpp>
#include <tensor/backend/cuda/device.hpp>
#include <tensor/base/frozen_base.hpp>
#include <tensor/centroid/centroid_accumulator.hpp>
#include <tensor/checkpoint/adapter_writer.hpp>
#include <tensor/data/dataset.hpp>
#include <tensor/trainer/adapt_trainer.hpp>

namespace fs = std::filesystem;

namespace {

// ── JSON text in the form the reference's files have (nlohmann::json's
//    dump(): object keys in sorted order, no spaces when compact, two-space
//    indentation and ": " otherwise, doubles as the shortest text that reads
//    back to the same value) ───────────────────────────────────────────────

std::string json_string(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\b': o += "\\b"; break;
            case '\f': o += "\\f"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            default:
                if (c < 0x20) {
                    char b[8];
                    std::snprintf(b, sizeof b, "\\u%04x", c);
                    o += b;
                } else {
                    o += (char)c;
                }
        }
    }
    return o + "\"";
}

// Shortest decimal digits d (no leading zeros) and exponent e with
// x = 0.d * 10^e ... written as digits and the decimal point position n
// (x = d[0..n) . d[n..)), then laid out as the reference's serializer does:
// plain for -4 < n <= 15 (a ".0" is appended to integral values), otherwise
// d.ddd e±XX with at least two exponent digits.
std::string json_double(double x) {
    if (x == 0) return std::signbit(x) ? "-0.0" : "0.0";
    std::string sign = x < 0 ? "-" : "";
    double a = std::fabs(x);
    char buf[64];
    std::string digits;
    int exp10 = 0;
    for (int p = 1; p <= 17; p++) {
        std::snprintf(buf, sizeof buf, "%.*e", p - 1, a);
        if (std::strtod(buf, nullptr) == a || p == 17) {
            const char* e = std::strchr(buf, 'e');
            exp10 = std::atoi(e + 1);
            for (const char* c = buf; c < e; c++)
                if (*c >= '0' && *c <= '9') digits += *c;
            break;
        }
    }
    while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
    const int k = (int)digits.size(), n = exp10 + 1;
    std::string o;
    if (k <= n && n <= 15) {
        o = digits + std::string(n - k, '0') + ".0";
    } else if (0 < n && n <= 15) {
        o = digits.substr(0, n) + "." + digits.substr(n);
    } else if (-4 < n && n <= 0) {
        o = "0." + std::string(-n, '0') + digits;
    } else {
        o = digits.substr(0, 1);
        if (k > 1) o += "." + digits.substr(1);
        int e = n - 1;
        o += e < 0 ? "e-" : "e+";
        e = std::abs(e);
        char eb[8];
        std::snprintf(eb, sizeof eb, e < 10 ? "0%d" : "%d", e);
        o += eb;
    }
    return sign + o;
}

// ── a small JSON reader for the files this library writes ─────────────────
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0;
    std::string text;  // Str, or Num's literal
    std::vector<JVal> arr;
    std::map<std::string, JVal> obj;
};

struct JParser {
    const std::string& s;
    size_t i = 0;
    explicit JParser(const std::string& t) : s(t) {}
    [[noreturn]] void fail(const char* what) {
        throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(i));
    }
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) i++;
    }
    bool lit(const char* w) {
        size_t n = std::strlen(w);
        if (s.compare(i, n, w) == 0) {
            i += n;
            return true;
        }
        return false;
    }
    std::string str() {
        if (s[i] != '"') fail("string expected");
        i++;
        std::string o;
        while (i < s.size() && s[i] != '"') {
            char c = s[i++];
            if (c == '\\') {
                if (i >= s.size()) fail("bad escape");
                char e = s[i++];
                switch (e) {
                    case 'b': o += '\b'; break;
                    case 'f': o += '\f'; break;
                    case 'n': o += '\n'; break;
                    case 'r': o += '\r'; break;
                    case 't': o += '\t'; break;
                    case 'u': {
                        if (i + 4 > s.size()) fail("bad escape");
                        unsigned v = (unsigned)std::strtoul(s.substr(i, 4).c_str(), nullptr, 16);
                        i += 4;
                        if (v >= 0x80) fail("non-ASCII escape");
                        o += (char)v;
                        break;
                    }
                    default: o += e;
                }
            } else {
                o += c;
            }
        }
        if (i >= s.size()) fail("unterminated string");
        i++;
        return o;
    }
    JVal value() {
        ws();
        if (i >= s.size()) fail("value expected");
        JVal v;
        char c = s[i];
        if (c == '{') {
            v.kind = JVal::Obj;
            i++;
            ws();
            if (s[i] == '}') {
                i++;
                return v;
            }
            for (;;) {
                ws();
                std::string k = str();
                ws();
                if (s[i++] != ':') fail("':' expected");
                v.obj[k] = value();
                ws();
                if (s[i] == ',') {
                    i++;
                    continue;
                }
                if (s[i] == '}') {
                    i++;
                    return v;
                }
                fail("',' or '}' expected");
            }
        }
        if (c == '[') {
            v.kind = JVal::Arr;
            i++;
            ws();
            if (s[i] == ']') {
                i++;
                return v;
            }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (s[i] == ',') {
                    i++;
                    continue;
                }
                if (s[i] == ']') {
                    i++;
                    return v;
                }
                fail("',' or ']' expected");
            }
        }
        if (c == '"') {
            v.kind = JVal::Str;
            v.text = str();
            return v;
        }
        if (lit("true")) {
            v.kind = JVal::Bool;
            v.b = true;
            return v;
        }
        if (lit("false")) {
            v.kind = JVal::Bool;
            return v;
        }
        if (lit("null")) return v;
        size_t j = i;
        while (j < s.size() && std::strchr("+-0123456789.eE", s[j])) j++;
        if (j == i) fail("unexpected character");
        v.kind = JVal::Num;
        v.text = s.substr(i, j - i);
        v.num = std::strtod(v.text.c_str(), nullptr);
        i = j;
        return v;
    }
};

JVal parse_json(const std::string& text) {
    JParser p(text);
    JVal v = p.value();
    p.ws();
    if (p.i != text.size()) p.fail("trailing characters");
    return v;
}

std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot read " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

uint16_t bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// One safetensors entry: name, dtype, element count and raw bytes.
struct StEntry {
    std::string name, dtype;
    size_t n;
    std::vector<char> bytes;
};

// [u64 header length][header JSON, spaces to a multiple of 8][data in entry order]
void write_safetensors(const std::string& path, const std::vector<StEntry>& entries) {
    std::map<std::string, std::string> fields;  // sorted, as the reference's header
    size_t off = 0;
    for (const auto& e : entries) {
        if (fields.count(e.name)) throw std::runtime_error("safetensors: duplicate " + e.name);
        fields[e.name] = "{\"data_offsets\":[" + std::to_string(off) + "," +
                         std::to_string(off + e.bytes.size()) + "],\"dtype\":" +
                         json_string(e.dtype) + ",\"shape\":[" + std::to_string(e.n) + "]}";
        off += e.bytes.size();
    }
    std::string h = "{";
    bool first = true;
    for (const auto& kv : fields) {
        if (!first) h += ",";
        first = false;
        h += json_string(kv.first) + ":" + kv.second;
    }
    h += "}";
    while (h.size() % 8 != 0) h += ' ';
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot write " + path);
    uint64_t hl = h.size();
    f.write(reinterpret_cast<const char*>(&hl), 8);
    f.write(h.data(), (std::streamsize)h.size());
    for (const auto& e : entries) f.write(e.bytes.data(), (std::streamsize)e.bytes.size());
    if (!f) throw std::runtime_error("write failed: " + path);
}

template <typename T>
StEntry entry(const std::string& name, const char* dtype, const std::vector<T>& v) {
    StEntry e{name, dtype, v.size(), std::vector<char>(v.size() * sizeof(T))};
    if (!v.empty()) std::memcpy(e.bytes.data(), v.data(), e.bytes.size());
    return e;
}

// name -> (dtype, data bytes) of a safetensors file
std::map<std::string, std::pair<std::string, std::vector<char>>> read_safetensors(
    const std::string& path) {
    std::string all = read_file(path);
    if (all.size() < 8) throw std::runtime_error("safetensors: short file " + path);
    uint64_t hl;
    std::memcpy(&hl, all.data(), 8);
    if (8 + hl > all.size()) throw std::runtime_error("safetensors: bad header length in " + path);
    JVal h = parse_json(all.substr(8, hl));
    if (h.kind != JVal::Obj) throw std::runtime_error("safetensors: header is not an object");
    const size_t base = 8 + hl;
    std::map<std::string, std::pair<std::string, std::vector<char>>> out;
    for (const auto& kv : h.obj) {
        if (kv.first == "__metadata__") continue;
        const JVal& t = kv.second;
        auto it = t.obj.find("data_offsets");
        auto dt = t.obj.find("dtype");
        if (it == t.obj.end() || dt == t.obj.end() || it->second.arr.size() != 2)
            throw std::runtime_error("safetensors: malformed entry " + kv.first);
        size_t a = (size_t)it->second.arr[0].num, b = (size_t)it->second.arr[1].num;
        if (a > b || base + b > all.size())
            throw std::runtime_error("safetensors: offsets out of range for " + kv.first);
        out[kv.first] = {dt->second.text, std::vector<char>(all.begin() + base + a,
                                                              all.begin() + base + b)};
    }
    return out;
}

template <typename T>
std::vector<T> as_vec(const std::pair<std::string, std::vector<char>>& e, const char* dtype,
                      const std::string& name) {
    if (e.first != dtype || e.second.size() % sizeof(T) != 0)
        throw std::runtime_error("checkpoint: " + name + " is not " + dtype);
    std::vector<T> v(e.second.size() / sizeof(T));
    if (!v.empty()) std::memcpy(v.data(), e.second.data(), e.second.size());
    return v;
}

const char* kProjName[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                            "self_attn.o_proj", "mlp.gate_proj",    "mlp.up_proj",
                            "mlp.down_proj"};

}  // namespace

// ── AdapterConfig ──────────────────────────────────────────────────────────
namespace tensor::adapter {

AdapterConfig AdapterConfig::for_base(const base::FrozenBase& b, const backend::cuda::Device& dev) {
    const base::BaseConfig& bc = b.config;
    // parameter count as the reference estimates it (adapter_config.cpp:58-64)
    const std::size_t params =
        bc.vocab_size * bc.hidden_size +
        bc.num_layers * (4 * bc.hidden_size * bc.hidden_size +
                         2 * bc.hidden_size * bc.num_kv_heads * bc.head_dim +
                         3 * bc.hidden_size * bc.intermediate_size);
    AdapterConfig cfg;
    cfg.architecture = bc.arch_name;
    cfg.base_parameters = params;
    // rank ladder (rank = alpha), up/down from 800M parameters on
    struct Rung {
        std::size_t below;
        int rank;
        bool mlp;
    };
    static const Rung ladder[] = {{200'000'000ULL, 2, false},     {800'000'000ULL, 4, false},
                                  {2'000'000'000ULL, 8, true},    {8'000'000'000ULL, 16, true},
                                  {20'000'000'000ULL, 32, true}};
    cfg.rank = 64;
    cfg.inject_up = cfg.inject_down = true;
    for (const Rung& r : ladder)
        if (params < r.below) {
            cfg.rank = r.rank;
            cfg.inject_up = cfg.inject_down = r.mlp;
            break;
        }
    cfg.alpha = (float)cfg.rank;
    // batch / sequence from the memory left after the base (256 MB headroom)
    if (hipSetDevice(dev.id()) != hipSuccess)
        throw backend::cuda::CudaError("AdapterConfig::for_base: hipSetDevice failed");
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess)
        throw backend::cuda::CudaError("AdapterConfig::for_base: hipMemGetInfo failed");
    const size_t headroom = 256ull << 20;
    const size_t budget = free_b > headroom ? free_b - headroom : 0;
    struct Tier {
        size_t min_free, batch, seq;
    };
    static const Tier tiers[] = {{16ull << 30, 8, 2048}, {8ull << 30, 4, 1024},
                                 {4ull << 30, 2, 1024},  {2ull << 30, 1, 512},
                                 {1ull << 30, 1, 256},   {0, 1, 128}};
    for (const Tier& t : tiers)
        if (budget >= t.min_free) {
            cfg.batch_size = t.batch;
            cfg.seq_len = t.seq;
            break;
        }
    cfg.warmup_steps = params < 1'000'000'000ULL ? 100 : params < 8'000'000'000ULL ? 200 : 500;
    std::cerr << "[adapter] VRAM free=" << (free_b >> 20) << " MB total=" << (total_b >> 20)
              << " MB -> batch=" << cfg.batch_size << " seq=" << cfg.seq_len << "\n";
    return cfg;
}

}  // namespace tensor::adapter

// ── AdapterWriter ──────────────────────────────────────────────────────────
namespace tensor::checkpoint {

std::string lora_prefix(std::size_t layer, int proj) {
    if (proj < 0 || proj > 6) throw std::runtime_error("lora_prefix: projection out of range");
    return "layers." + std::to_string(layer) + "." + kProjName[proj];
}

void write_adapter_safetensors(const std::string& path, const std::vector<AdapterTensor>& ts) {
    std::vector<StEntry> es;
    es.reserve(ts.size());
    for (const auto& t : ts) {
        std::vector<uint16_t> b(t.value.size());
        for (size_t i = 0; i < b.size(); i++) b[i] = bf16_rne(t.value[i]);
        es.push_back(entry(t.name, "BF16", b));
    }
    write_safetensors(path, es);
}

void write_optimizer_safetensors(const std::string& path, const std::vector<AdapterTensor>& ts,
                                 const std::vector<double>& centroid_sums) {
    std::vector<StEntry> es;
    for (const auto& t : ts) {
        if (t.exp_avg.size() != t.value.size() || t.exp_avg_sq.size() != t.value.size())
            throw std::runtime_error("optimizer state of " + t.name + " is incomplete");
        es.push_back(entry(t.name, "F32", t.value));
        es.push_back(entry(t.name + ".exp_avg", "F32", t.exp_avg));
        es.push_back(entry(t.name + ".exp_avg_sq", "F32", t.exp_avg_sq));
    }
    if (!centroid_sums.empty()) es.push_back(entry("centroid.sums", "F64", centroid_sums));
    write_safetensors(path, es);
}

std::string adapter_json(const adapter::AdapterConfig& cfg, const base::BaseConfig& bc,
                         const std::string& domain, std::size_t step, std::size_t tokens) {
    // the reference's fields (adapter_writer.cpp:101-121); inject_gate only
    // when set (no reference counterpart)
    std::map<std::string, std::string> f;
    auto b = [](bool v) { return std::string(v ? "true" : "false"); };
    f["domain"] = json_string(domain);
    f["architecture"] = json_string(bc.arch_name);
    f["base_model"] = json_string("unknown");
    f["base_sha"] = json_string(bc.base_sha);
    f["rank"] = std::to_string(cfg.rank);
    f["alpha"] = json_double((double)cfg.alpha);
    f["target_begin"] = "0";
    f["target_end"] = std::to_string((int)bc.num_layers - 1);
    f["inject_q"] = b(cfg.inject_q);
    f["inject_k"] = b(cfg.inject_k);
    f["inject_v"] = b(cfg.inject_v);
    f["inject_o"] = b(cfg.inject_o);
    f["inject_up"] = b(cfg.inject_up);
    f["inject_down"] = b(cfg.inject_down);
    if (cfg.inject_gate) f["inject_gate"] = "true";
    f["tokens_trained"] = std::to_string(tokens);
    f["centroid_dim"] = std::to_string(bc.hidden_size);
    f["centroid_count"] = "16";
    f["step"] = std::to_string(step);
    f["tensor_adapt_version"] = json_string("0.1.0");
    std::string o = "{\n";
    bool first = true;
    for (const auto& kv : f) {
        if (!first) o += ",\n";
        first = false;
        o += "  " + json_string(kv.first) + ": " + kv.second;
    }
    return o + "\n}";
}

AdapterWriter::AdapterWriter(const std::string& dir) : base_dir_(dir) {
    fs::create_directories(dir);
}

void AdapterWriter::save_checkpoint(const std::vector<AdapterTensor>& ts,
                                    const std::vector<double>& centroid_sums,
                                    const adapter::AdapterConfig& cfg,
                                    const base::FrozenBase& base, const std::string& domain,
                                    std::size_t step, std::size_t tokens,
                                    const std::string& dir) {
    fs::create_directories(dir);
    write_adapter_safetensors(dir + "/adapter.safetensors", ts);
    std::ofstream(dir + "/adapter.json") << adapter_json(cfg, base.config, domain, step, tokens);
    std::ofstream(dir + "/train_state.json")
        << "{\n  \"step\": " << step << ",\n  \"tokens_consumed\": " << tokens << "\n}";
    write_optimizer_safetensors(dir + "/optimizer.safetensors", ts, centroid_sums);
    std::cerr << "[writer] checkpoint saved -> " << dir << "\n";
}

void AdapterWriter::save_final(const std::vector<AdapterTensor>& ts,
                               const adapter::AdapterConfig& cfg, const base::FrozenBase& base,
                               const std::string& domain, std::size_t step, std::size_t tokens,
                               const std::string& dir) {
    fs::create_directories(dir);
    write_adapter_safetensors(dir + "/adapter.safetensors", ts);
    std::ofstream(dir + "/adapter.json") << adapter_json(cfg, base.config, domain, step, tokens);
    std::cerr << "[writer] final adapter saved -> " << dir << "\n";
}

TrainState load_checkpoint(const std::string& dir) {
    TrainState st;
    JVal s = parse_json(read_file(dir + "/train_state.json"));
    auto num = [&](const char* k) -> std::size_t {
        auto it = s.obj.find(k);
        if (s.kind != JVal::Obj || it == s.obj.end() || it->second.kind != JVal::Num)
            throw std::runtime_error("checkpoint: train_state.json lacks " + std::string(k));
        return (std::size_t)std::strtoull(it->second.text.c_str(), nullptr, 10);
    };
    st.step = num("step");
    st.tokens_consumed = num("tokens_consumed");
    auto ent = read_safetensors(dir + "/optimizer.safetensors");
    auto cs = ent.find("centroid.sums");
    if (cs != ent.end()) st.centroid_sums = as_vec<double>(cs->second, "F64", "centroid.sums");
    for (const auto& kv : ent) {
        const std::string& n = kv.first;
        if (n == "centroid.sums" || n.size() < 7) continue;
        if (n.compare(n.size() - 7, 7, ".lora_A") != 0 && n.compare(n.size() - 7, 7, ".lora_B") != 0)
            continue;
        AdapterTensor t;
        t.name = n;
        t.value = as_vec<float>(kv.second, "F32", n);
        auto m = ent.find(n + ".exp_avg"), v = ent.find(n + ".exp_avg_sq");
        if (m == ent.end() || v == ent.end())
            throw std::runtime_error("checkpoint: moments of " + n + " missing");
        t.exp_avg = as_vec<float>(m->second, "F32", n + ".exp_avg");
        t.exp_avg_sq = as_vec<float>(v->second, "F32", n + ".exp_avg_sq");
        if (t.exp_avg.size() != t.value.size() || t.exp_avg_sq.size() != t.value.size())
            throw std::runtime_error("checkpoint: moments of " + n + " have the wrong size");
        st.tensors.push_back(std::move(t));
    }
    return st;
}

}  // namespace tensor::checkpoint

// ── AdaptTrainer ───────────────────────────────────────────────────────────
namespace tensor::trainer {

using backend::cuda::check_status;
using backend::cuda::CudaError;
using Clock = std::chrono::steady_clock;

struct AdaptTrainer::Impl {
    const base::FrozenBase* base;
    adapter::AdapterConfig cfg;
    data::Dataset* dataset;
    AdaptOptions opts;
    const backend::cuda::Device* dev;
    void* eng = nullptr;
    centroid::CentroidAccumulator centroid_acc;
    checkpoint::AdapterWriter writer;
    std::size_t step_count = 0, tokens_seen = 0, total_steps = 0;
    double ema_ms = 0.0;
    static constexpr double kEmaAlpha = 0.1;
    int B, T;

    Impl(const base::FrozenBase* b, const adapter::AdapterConfig& c, data::Dataset* ds,
         const AdaptOptions& o, const backend::cuda::Device* d)
        : base(b), cfg(c), dataset(ds), opts(o), dev(d),
          centroid_acc((int)b->config.hidden_size, o.output_dir + "/centroids"),
          writer(o.output_dir) {
        const base::BaseConfig& bc = b->config;
        B = (int)cfg.batch_size;
        T = (int)cfg.seq_len;
        if (B <= 0 || T <= 0 || cfg.rank <= 0)
            throw std::runtime_error("AdaptTrainer: batch_size, seq_len and rank must be > 0");
        if (opts.checkpoint_every == 0)
            throw std::runtime_error("AdaptTrainer: checkpoint_every must be > 0");
        total_steps = opts.tokens / ((std::size_t)B * T);
        ta_model_config mc{(int)bc.vocab_size, (int)bc.hidden_size, (int)bc.num_layers,
                           (int)bc.num_q_heads, (int)bc.num_kv_heads, (int)bc.head_dim,
                           (int)bc.intermediate_size, bc.rms_norm_eps, bc.rope_theta,
                           bc.tie_embeddings ? 1 : 0};
        ta_adapt_config ac{cfg.rank, cfg.alpha, cfg.inject_mask(), cfg.lr, cfg.grad_clip,
                           (int64_t)cfg.warmup_steps, (int64_t)total_steps, cfg.adam_beta1,
                           cfg.adam_beta2, cfg.adam_eps, cfg.weight_decay};
        if (hipSetDevice(dev->id()) != hipSuccess)
            throw CudaError("AdaptTrainer: hipSetDevice failed");
        // the reference trains q, k, v and o whatever the flags say
        // (adapter_model.cu:83-86); here every flag is honoured
        if (cfg.inject_gate || cfg.inject_up || cfg.inject_down || !cfg.inject_q ||
            !cfg.inject_k || !cfg.inject_v || !cfg.inject_o)
            std::cerr << "[trainer] note: training LoRA on the projections the inject flags name ("
                      << (cfg.inject_q ? "q " : "") << (cfg.inject_k ? "k " : "")
                      << (cfg.inject_v ? "v " : "") << (cfg.inject_o ? "o " : "")
                      << (cfg.inject_gate ? "gate " : "") << (cfg.inject_up ? "up " : "")
                      << (cfg.inject_down ? "down " : "")
                      << "); the reference trains q, k, v and o only, so adapter.safetensors "
                         "holds a different tensor set\n";
        eng = ta_engine_create(&mc, &ac, B, T, dev->stream());
        if (!eng) throw CudaError(std::string("AdaptTrainer: ") + ta_last_error());
        try {
            upload_base();
            check_status(ta_engine_set_centroid(eng, centroid_acc.device_sums(*dev)),
                         "AdaptTrainer: centroid");
            if (!opts.resume_from.empty()) resume(opts.resume_from);
            dev->sync();
        } catch (...) {
            ta_engine_destroy(eng);
            eng = nullptr;
            throw;
        }
    }
    ~Impl() {
        if (eng) ta_engine_destroy(eng);
    }

    void set(const std::string& name, const backend::cuda::Tensor& t) {
        if (t.empty() || t.dtype() != core::DType::BF16)
            throw base::BaseError("tensor " + name + " is missing or not BF16");
        check_status(ta_engine_set_weight_device(eng, name.c_str(), t.bf16(), (int64_t)t.numel()),
                     "AdaptTrainer: base weight");
    }

    void upload_base() {
        const base::FrozenBase& b = *base;
        if (b.layers.size() != b.config.num_layers)
            throw base::BaseError("FrozenBase has " + std::to_string(b.layers.size()) +
                                  " layers, config says " + std::to_string(b.config.num_layers));
        set("model.embed_tokens.weight", b.embed_w);
        set("model.norm.weight", b.final_norm_w);
        if (!b.config.tie_embeddings) set("lm_head.weight", b.lm_head_w);
        for (std::size_t l = 0; l < b.layers.size(); l++) {
            const base::LayerWeights& w = b.layers[l];
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
    }

    // element counts of projection p's A [r, in] and B [out, r]
    void dims(int p, int64_t* nA, int64_t* nB) const {
        const base::BaseConfig& bc = base->config;
        const int64_t H = bc.hidden_size, q = bc.num_q_heads * bc.head_dim,
                      kv = bc.num_kv_heads * bc.head_dim, I = bc.intermediate_size;
        const int64_t in[7] = {H, H, H, q, H, H, I}, out[7] = {q, kv, kv, H, I, I, H};
        *nA = cfg.rank * in[p];
        *nB = out[p] * cfg.rank;
    }

    // every injected A and B in the reference's order, with the moments when asked
    std::vector<checkpoint::AdapterTensor> gather(bool moments) {
        std::vector<checkpoint::AdapterTensor> ts;
        const int mask = cfg.inject_mask();
        for (std::size_t l = 0; l < base->config.num_layers; l++)
            for (int p = 0; p < 7; p++) {
                if (!((mask >> p) & 1)) continue;
                int64_t n[2];
                dims(p, &n[0], &n[1]);
                for (int ab = 0; ab < 2; ab++) {
                    checkpoint::AdapterTensor t;
                    t.name = checkpoint::lora_prefix(l, p) + (ab ? ".lora_B" : ".lora_A");
                    t.value.resize(n[ab]);
                    check_status(ta_engine_read_adapter(eng, (int)l, p, ab, t.value.data(), n[ab]),
                                 "AdaptTrainer: read adapter");
                    if (moments) {
                        t.exp_avg.resize(n[ab]);
                        t.exp_avg_sq.resize(n[ab]);
                        check_status(ta_engine_read_adapter(eng, (int)l, p, ab ? 4 : 2,
                                                            t.exp_avg.data(), n[ab]),
                                     "AdaptTrainer: read adapter");
                        check_status(ta_engine_read_adapter(eng, (int)l, p, ab ? 5 : 3,
                                                            t.exp_avg_sq.data(), n[ab]),
                                     "AdaptTrainer: read adapter");
                    }
                    ts.push_back(std::move(t));
                }
            }
        return ts;
    }

    void resume(const std::string& dir) {
        checkpoint::TrainState st = checkpoint::load_checkpoint(dir);
        std::map<std::string, const checkpoint::AdapterTensor*> by;
        for (const auto& t : st.tensors) by[t.name] = &t;
        const int mask = cfg.inject_mask();
        std::size_t used = 0;
        for (std::size_t l = 0; l < base->config.num_layers; l++)
            for (int p = 0; p < 7; p++) {
                if (!((mask >> p) & 1)) continue;
                int64_t n[2];
                dims(p, &n[0], &n[1]);
                for (int ab = 0; ab < 2; ab++) {
                    const std::string name =
                        checkpoint::lora_prefix(l, p) + (ab ? ".lora_B" : ".lora_A");
                    auto it = by.find(name);
                    if (it == by.end())
                        throw std::runtime_error("resume: " + name + " not in " + dir);
                    const checkpoint::AdapterTensor& t = *it->second;
                    if ((int64_t)t.value.size() != n[ab])
                        throw std::runtime_error("resume: " + name + " has the wrong size");
                    std::vector<uint16_t> shadow(t.value.size());
                    for (size_t i = 0; i < shadow.size(); i++) shadow[i] = bf16_rne(t.value[i]);
                    const int w_master = ab, w_m = ab ? 4 : 2, w_v = ab ? 5 : 3, w_sh = 8 + ab;
                    check_status(ta_engine_write_adapter(eng, (int)l, p, w_master, t.value.data(), n[ab]),
                                 "resume");
                    check_status(ta_engine_write_adapter(eng, (int)l, p, w_m, t.exp_avg.data(), n[ab]),
                                 "resume");
                    check_status(ta_engine_write_adapter(eng, (int)l, p, w_v, t.exp_avg_sq.data(), n[ab]),
                                 "resume");
                    check_status(ta_engine_write_adapter(eng, (int)l, p, w_sh, shadow.data(), n[ab]),
                                 "resume");
                    used++;
                }
            }
        if (used != st.tensors.size())
            throw std::runtime_error("resume: " + dir + " holds adapter tensors this configuration "
                                     "does not inject");
        check_status(ta_engine_set_step(eng, (int64_t)st.step), "resume");
        if (!st.centroid_sums.empty()) {
            if (st.centroid_sums.size() != base->config.hidden_size + 1)
                throw std::runtime_error("resume: centroid sums have the wrong size");
            if (hipMemcpy(centroid_acc.device_sums(*dev), st.centroid_sums.data(),
                          st.centroid_sums.size() * sizeof(double),
                          hipMemcpyHostToDevice) != hipSuccess)
                throw CudaError("resume: centroid sums upload failed");
        }
        // the data position the run had reached: one batch per step
        for (std::size_t s = 0; s < st.step; s++) (void)dataset->next_batch(B, T);
        step_count = st.step;
        tokens_seen = st.tokens_consumed;
        std::cerr << "[trainer] resumed from " << dir << " at step " << step_count << "\n";
    }

    void checkpoint_to(const std::string& dir) {
        dev->sync();
        centroid_acc.write_snapshot(step_count);
        std::vector<double> sums = centroid_acc.sums();
        writer.save_checkpoint(gather(true), sums, cfg, *base, opts.domain, step_count,
                               tokens_seen, dir);
    }

    StepMetrics do_step() {
        const auto t0 = Clock::now();
        auto batch = dataset->next_batch(B, T);
        ta_step_metrics m{};
        check_status(ta_engine_step(eng, batch.first.data(), batch.second.data(), 0.f, &m),
                     "AdaptTrainer::step");
        // the logits check of the first step (adapt_trainer.cu:76-91,196-198)
        if (step_count == 0 && m.nonfinite_logits > 0)
            std::cerr << "[trainer] WARNING: " << m.nonfinite_logits << " NaNs in logits at step 0\n";
        step_count++;
        tokens_seen += (std::size_t)B * T;
        const double ms = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
        ema_ms = step_count == 1 ? ms : kEmaAlpha * ms + (1.0 - kEmaAlpha) * ema_ms;
        const double tps = ema_ms > 0.0 ? (double)B * T * 1000.0 / ema_ms : 0.0;
        if (step_count % opts.checkpoint_every == 0)
            checkpoint_to(opts.output_dir + "/step-" + std::to_string(step_count));
        return StepMetrics{step_count, tokens_seen, m.loss, m.lr, m.gnorm, ms, ema_ms, tps};
    }
};

AdaptTrainer AdaptTrainer::create(const base::FrozenBase& base, const adapter::AdapterConfig& cfg,
                                  data::Dataset& dataset, const AdaptOptions& opts,
                                  const backend::cuda::Device& dev) {
    fs::create_directories(opts.output_dir);
    return AdaptTrainer(std::make_unique<Impl>(&base, cfg, &dataset, opts, &dev));
}

AdaptTrainer::AdaptTrainer(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
AdaptTrainer::~AdaptTrainer() = default;
AdaptTrainer::AdaptTrainer(AdaptTrainer&&) noexcept = default;
AdaptTrainer& AdaptTrainer::operator=(AdaptTrainer&&) noexcept = default;

bool AdaptTrainer::done() const { return impl_->tokens_seen >= impl_->opts.tokens; }
StepMetrics AdaptTrainer::step() { return impl_->do_step(); }
void* AdaptTrainer::engine() const { return impl_->eng; }

void AdaptTrainer::run() {
    while (!done()) {
        StepMetrics m = step();
        if (impl_->opts.log_to_stdout && impl_->step_count % 10 == 0)
            std::cerr << "[step " << m.step << "/" << impl_->total_steps << "] loss=" << m.loss
                      << " lr=" << m.learning_rate << " grad=" << m.grad_norm
                      << " tok=" << m.tokens_consumed << " ms=" << (int)m.step_ms
                      << " ema=" << (int)m.ema_ms << " tok/s=" << (int)m.tokens_per_sec << "\n";
    }
    save_adapter(impl_->opts.output_dir);
}

void AdaptTrainer::save_checkpoint(const std::string& dir) { impl_->checkpoint_to(dir); }

void AdaptTrainer::save_adapter(const std::string& dir) {
    impl_->dev->sync();
    impl_->centroid_acc.write_snapshot(impl_->step_count);
    // (the reference merges before its writer creates dir, so into a new
    // directory its unchecked stream writes no adapter.centroid)
    fs::create_directories(dir);
    impl_->centroid_acc.merge_and_write(16, dir + "/adapter.centroid");
    impl_->writer.save_final(impl_->gather(false), impl_->cfg, *impl_->base, impl_->opts.domain,
                             impl_->step_count, impl_->tokens_seen, dir);
    std::cerr << "[trainer] adapter saved -> " << dir << "\n";
}

}  // namespace tensor::trainer
