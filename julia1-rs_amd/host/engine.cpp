// Host side of the HIP backend: checkpoint config, safetensors, weight
// resolution and the micro-batching engine (include/julia1_engine.h).
// Restates the reference runtime's src/config.rs, src/weights.rs,
// src/model.rs and src/engine.rs below the text front end.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <deque>
#include <fstream>
#include <memory>
#include <mutex>
#include <numeric>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/julia1_engine.h"
#include "../../include/julia1_hip.h"
#include "../csrc/abi_util.hpp"
#include "json.hpp"

namespace {

using jh::Json;

[[noreturn]] void invalid(const std::string& msg) { throw jh_error(JH_ERR_INVALID, msg); }

std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) invalid("reading " + path + ": cannot open");
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

Json read_json(const std::string& path) {
    std::string text = read_file(path);
    try {
        return jh::parse_json(text);
    } catch (const std::exception& e) {
        invalid("parsing " + path + ": " + e.what());
    }
}

bool file_exists(const std::string& p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0;
}

// ------------------------------------------------------------ ModelConfig (src/config.rs:6-96)
struct ModelConfig {
    uint32_t hidden = 0, heads = 0, head_dim = 0, intermediate = 0, layers = 0;
    std::vector<uint8_t> global;
    uint32_t half_window = 0;
    std::vector<float> rope_theta;
    float norm_eps = 1e-5f;
    uint32_t vocab = 0, max_positions = 0, head_layers = 0, head_heads = 0, head_ff = 0;
    // weight_dtype "bfloat16": tensors may be stored as BF16 (an extension; the
    // reference reads "float32" checkpoints only).
    bool bf16_checkpoint = false;

    jh_config view() const {
        return jh_config{hidden, heads, head_dim, intermediate, layers, global.data(), half_window,
                         rope_theta.data(), norm_eps, vocab, max_positions, head_layers, head_heads, head_ff};
    }
};

uint32_t usize_of(const Json& v, const char* key) {
    const Json* x = v.get(key);
    if (!x || !x->is_uint() || x->num > 4294967295.0) invalid(std::string("config is missing ") + key);
    return (uint32_t)x->num;
}

bool json_eq_str(const Json* v, const char* s) { return v && v->kind == Json::String && v->str == s; }

// `ModelConfig::from_values` (src/config.rs:43-96): same checks, same derived fields.
ModelConfig config_from_values(const Json& julia, const Json& enc) {
    const Json* fv = julia.get("format_version");
    if (!fv || !fv->is_uint() || fv->num != 1.0) invalid("Unsupported Julia checkpoint format");
    const Json* wd = julia.get("weight_dtype");  // absent or not a string reads as "float32"
    const bool bf16 = wd && wd->kind == Json::String && wd->str == "bfloat16";
    if (wd && wd->kind == Json::String && wd->str != "float32" && !bf16)
        invalid("Only float32 Julia checkpoints are supported");
    if (!json_eq_str(enc.get("model_type"), "modernbert")) invalid("Encoder must be ModernBERT");
    for (const char* key : {"attention_bias", "mlp_bias", "norm_bias"}) {
        const Json* v = enc.get(key);
        if (!v || v->kind != Json::Bool || v->b) invalid(std::string("Unsupported encoder setting ") + key);
    }
    if (!json_eq_str(enc.get("hidden_activation"), "gelu")) invalid("Unsupported encoder activation");
    ModelConfig c;
    c.bf16_checkpoint = bf16;
    c.hidden = usize_of(enc, "hidden_size");
    c.heads = usize_of(enc, "num_attention_heads");
    c.layers = usize_of(enc, "num_hidden_layers");
    const uint32_t every = usize_of(enc, "global_attn_every_n_layers");
    const uint32_t local = usize_of(enc, "local_attention");
    if (c.heads == 0 || c.hidden % c.heads != 0 || c.hidden / c.heads != 64) invalid("Runtime kernels require head_dim 64");
    if (every == 0) invalid("config is missing global_attn_every_n_layers");
    std::vector<std::string> types;
    const Json* lt = enc.get("layer_types");
    if (lt && lt->kind == Json::Array) {
        for (const Json& t : lt->arr) types.push_back(t.kind == Json::String ? t.str : std::string());
    } else {
        for (uint32_t i = 0; i < c.layers; ++i) types.push_back(i % every == 0 ? "full_attention" : "sliding_attention");
    }
    if (types.size() != c.layers) invalid("layer_types must list every layer");
    auto theta = [&](const std::string& kind) -> float {
        const Json* rp = enc.get("rope_parameters");
        const Json* p = rp ? rp->get(kind) : nullptr;
        if (p) {
            if (!json_eq_str(p->get("rope_type"), "default")) invalid("Only default RoPE is supported");
            const Json* t = p->get("rope_theta");
            if (!t || t->kind != Json::Number) invalid("rope_theta");
            return (float)t->num;
        }
        const char* key = kind == "full_attention" ? "global_rope_theta" : "local_rope_theta";
        const Json* t = enc.get(key);
        if (!t || t->kind != Json::Number) invalid(std::string("missing ") + key);
        return (float)t->num;
    };
    for (const auto& t : types) c.rope_theta.push_back(theta(t));
    c.head_layers = usize_of(julia, "head_layers");
    c.head_dim = c.hidden / c.heads;
    c.intermediate = usize_of(enc, "intermediate_size");
    // ModernBertAttention: sliding iff layer_id % global_attn_every_n_layers != 0.
    for (uint32_t i = 0; i < c.layers; ++i) c.global.push_back(i % every == 0 ? 1 : 0);
    c.half_window = local / 2;
    const Json* eps = enc.get("norm_eps");
    c.norm_eps = eps && eps->kind == Json::Number ? (float)eps->num : 1e-5f;
    c.vocab = usize_of(enc, "vocab_size");
    c.max_positions = usize_of(enc, "max_position_embeddings");
    c.head_heads = std::max<uint32_t>(c.hidden / 64, 1);
    c.head_ff = 4 * c.hidden;
    return c;
}

ModelConfig load_config(const std::string& root) {
    return config_from_values(read_json(root + "/julia_config.json"), read_json(root + "/encoder/config.json"));
}

// ------------------------------------------------------------ SafeTensors (src/weights.rs:32-94)
class SafeTensors {
public:
    // allow_bf16: BF16 tensors are accepted next to F32 ones and widened to
    // FP32 on access (exact: a BF16 value is the top half of its FP32 bits).
    SafeTensors(const std::string& path, bool allow_bf16) : allow_bf16_(allow_bf16) {
        int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) invalid("opening " + path + ": cannot open");
        struct stat st;
        if (fstat(fd, &st) != 0) {
            ::close(fd);
            invalid("opening " + path + ": cannot stat");
        }
        size_ = (size_t)st.st_size;
        if (size_) {
            void* p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
            if (p == MAP_FAILED) {
                ::close(fd);
                invalid("mapping " + path + " failed");
            }
            base_ = (const uint8_t*)p;
        }
        ::close(fd);
        try {
            parse();
        } catch (...) {
            if (base_) munmap((void*)base_, size_);
            base_ = nullptr;
            throw;
        }
    }
    ~SafeTensors() {
        if (base_) munmap((void*)base_, size_);
    }
    SafeTensors(const SafeTensors&) = delete;
    SafeTensors& operator=(const SafeTensors&) = delete;

    // F32: borrowed when 4-byte aligned (the usual case), copied otherwise.
    // BF16: widened into an owned FP32 copy.
    const float* f32(const std::string& name, std::initializer_list<size_t> shape) {
        auto it = std::find_if(tensors_.begin(), tensors_.end(), [&](const Entry& e) { return e.name == name; });
        if (it == tensors_.end()) invalid("missing tensor " + name);
        if (!std::equal(shape.begin(), shape.end(), it->shape.begin(), it->shape.end()))
            invalid(name + ": expected shape " + fmt(std::vector<size_t>(shape)) + ", found " + fmt(it->shape));
        size_t elems = 1;
        for (size_t d : shape) elems *= d;
        const size_t esize = it->bf16 ? 2 : 4;
        if (it->end - it->begin != elems * esize) invalid(name + ": data length does not match its shape");
        const uint8_t* p = base_ + it->begin;
        if (!it->bf16 && ((uintptr_t)p & 3) == 0) return (const float*)p;
        copies_.emplace_back(elems);
        float* dst = copies_.back().data();
        if (!it->bf16) {
            std::memcpy(dst, p, elems * 4);
        } else {
            for (size_t j = 0; j < elems; ++j) {
                uint16_t b;
                std::memcpy(&b, p + 2 * j, 2);
                const uint32_t u = (uint32_t)b << 16;
                std::memcpy(dst + j, &u, 4);
            }
        }
        return dst;
    }
    size_t count() const { return tensors_.size(); }
    size_t bf16_count() const {
        return (size_t)std::count_if(tensors_.begin(), tensors_.end(), [](const Entry& e) { return e.bf16; });
    }
    size_t bytes() const { return size_; }

private:
    struct Entry {
        std::string name;
        std::vector<size_t> shape;
        size_t begin, end;
        bool bf16;
    };
    bool allow_bf16_;
    const uint8_t* base_ = nullptr;
    size_t size_ = 0;
    std::vector<Entry> tensors_;
    std::vector<std::vector<float>> copies_;

    static std::string fmt(const std::vector<size_t>& s) {
        std::string o = "[";
        for (size_t i = 0; i < s.size(); ++i) o += (i ? ", " : "") + std::to_string(s[i]);
        return o + "]";
    }

    void parse() {
        static const char lfs[] = "version https://git-lfs.github.com/spec/v1";
        if (size_ >= sizeof(lfs) - 1 && std::memcmp(base_, lfs, sizeof(lfs) - 1) == 0)
            invalid("Checkpoint contains Git LFS pointers; fetch the real model weights first");
        if (size_ < 8) invalid("Truncated safetensors file");
        uint64_t n = 0;
        std::memcpy(&n, base_, 8);
        if (n > size_ - 8) invalid("Truncated safetensors header");
        Json header;
        try {
            header = jh::JsonParser((const char*)base_ + 8, (size_t)n).parse();
        } catch (const std::exception& e) {
            invalid(std::string("safetensors header: ") + e.what());
        }
        if (header.kind != Json::Object) invalid("safetensors header");
        for (const auto& kv : header.obj) {
            if (kv.first == "__metadata__") continue;
            const Json& info = kv.second;
            const bool bf16 = allow_bf16_ && json_eq_str(info.get("dtype"), "BF16");
            if (!bf16 && !json_eq_str(info.get("dtype"), "F32"))
                invalid(kv.first + (allow_bf16_ ? ": only F32 and BF16 tensors are supported"
                                                : ": only F32 tensors are supported"));
            const Json* shape = info.get("shape");
            const Json* offs = info.get("data_offsets");
            if (!shape || shape->kind != Json::Array) invalid("shape");
            if (!offs || offs->kind != Json::Array || offs->arr.size() != 2) invalid("data_offsets");
            Entry e;
            e.name = kv.first;
            e.bf16 = bf16;
            for (const Json& d : shape->arr) {
                uint64_t dim = 0;
                if (!d.as_u64(dim)) invalid("shape");
                e.shape.push_back((size_t)dim);
            }
            // Offsets are read from their literal text and checked without
            // wrap-around: n <= size_ - 8 was checked above (weights.rs slices
            // the mapping with bounds checks, src/weights.rs:79-89).
            uint64_t a = 0, b = 0;
            if (!offs->arr[0].as_u64(a) || !offs->arr[1].as_u64(b)) invalid("data_offsets");
            if (a > b || b > (uint64_t)(size_ - 8) - n) invalid(kv.first + ": data out of bounds");
            e.begin = 8 + n + a;
            e.end = 8 + n + b;
            tensors_.push_back(std::move(e));
        }
    }
};

// ------------------------------------------------------------ HostWeights (src/model.rs:55-110)
struct HostWeights {
    std::vector<jh_encoder_layer> layers;
    std::vector<jh_head_layer> head;
    jh_weights w{};
};

HostWeights load_weights(SafeTensors& t, const ModelConfig& c) {
    const size_t h = c.hidden, i = c.intermediate, ff = c.head_ff;
    HostWeights hw;
    hw.w.embedding = t.f32("encoder.embeddings.tok_embeddings.weight", {c.vocab, h});
    for (uint32_t l = 0; l < c.layers; ++l) {
        const std::string p = "encoder.layers." + std::to_string(l) + ".";
        jh_encoder_layer L{};
        L.attn_norm = l == 0 ? nullptr : t.f32(p + "attn_norm.weight", {h});
        L.wqkv = t.f32(p + "attn.Wqkv.weight", {3 * h, h});
        L.wo = t.f32(p + "attn.Wo.weight", {h, h});
        L.mlp_norm = t.f32(p + "mlp_norm.weight", {h});
        L.wi = t.f32(p + "mlp.Wi.weight", {2 * i, h});
        L.wo2 = t.f32(p + "mlp.Wo.weight", {h, i});
        hw.layers.push_back(L);
    }
    for (uint32_t l = 0; l < c.head_layers; ++l) {
        const std::string p = "head.layers." + std::to_string(l) + ".";
        jh_head_layer L{};
        L.norm1_w = t.f32(p + "norm1.weight", {h});
        L.norm1_b = t.f32(p + "norm1.bias", {h});
        L.in_w = t.f32(p + "self_attn.in_proj_weight", {3 * h, h});
        L.in_b = t.f32(p + "self_attn.in_proj_bias", {3 * h});
        L.out_w = t.f32(p + "self_attn.out_proj.weight", {h, h});
        L.out_b = t.f32(p + "self_attn.out_proj.bias", {h});
        L.norm2_w = t.f32(p + "norm2.weight", {h});
        L.norm2_b = t.f32(p + "norm2.bias", {h});
        L.lin1_w = t.f32(p + "linear1.weight", {ff, h});
        L.lin1_b = t.f32(p + "linear1.bias", {ff});
        L.lin2_w = t.f32(p + "linear2.weight", {h, ff});
        L.lin2_b = t.f32(p + "linear2.bias", {h});
        hw.head.push_back(L);
    }
    hw.w.scorer_norm_w = t.f32("scorer.0.weight", {h});
    hw.w.scorer_norm_b = t.f32("scorer.0.bias", {h});
    hw.w.scorer_w1 = t.f32("scorer.1.weight", {h, h});
    hw.w.scorer_b1 = t.f32("scorer.1.bias", {h});
    hw.w.scorer_w2 = t.f32("scorer.3.weight", {1, h});
    hw.w.scorer_b2 = t.f32("scorer.3.bias", {1})[0];
    hw.w.emb_norm = t.f32("encoder.embeddings.norm.weight", {h});
    hw.w.final_norm = t.f32("encoder.final_norm.weight", {h});
    hw.w.type_emb = t.f32("type_emb.weight", {3, h});
    hw.w.layers = hw.layers.data();
    hw.w.head = hw.head.data();
    return hw;
}

}  // namespace

struct je_engine {
    ModelConfig config;
    je_options options{};
    jh_model* model = nullptr;
    std::string name;
    std::mutex lock;  // Engine::lock: one logits call at a time (src/engine.rs:78,226)
    uint64_t forwards = 0;

    ~je_engine() {
        if (model) jh_destroy(model);
    }
};

extern "C" {

void je_default_options(je_options* out) {
    if (out) *out = je_options{0, 0, 16, 65536};
}

int je_parse_device(const char* s, int* ordinal) {
    return jh_guarded([&] {
        if (!s || !ordinal) invalid("null argument");
        std::string d(s);
        if (d == "hip") {
            *ordinal = 0;
            return;
        }
        if (d.rfind("hip:", 0) == 0 && d.size() > 4 &&
            std::all_of(d.begin() + 4, d.end(), [](char c) { return c >= '0' && c <= '9'; }) && d.size() < 14) {
            *ordinal = std::stoi(d.substr(4));
            return;
        }
        invalid("device must be hip or hip:N");
    });
}

int je_inspect(const char* dir, char* summary, size_t capacity) {
    return jh_guarded([&] {
        if (!dir) invalid("null checkpoint path");
        const std::string root(dir);
        ModelConfig c = load_config(root);
        SafeTensors t(root + "/model.safetensors", c.bf16_checkpoint);
        HostWeights hw = load_weights(t, c);
        (void)hw;
        std::string s = "{\"hidden\":" + std::to_string(c.hidden) + ",\"layers\":" + std::to_string(c.layers) +
                        ",\"head_layers\":" + std::to_string(c.head_layers) + ",\"tensors\":" +
                        std::to_string(t.count()) + ",\"bf16_tensors\":" + std::to_string(t.bf16_count()) +
                        ",\"bytes\":" + std::to_string(t.bytes()) + "}";
        if (summary && capacity) {
            size_t n = std::min(capacity - 1, s.size());
            std::memcpy(summary, s.data(), n);
            summary[n] = 0;
        }
    });
}

int je_load(const char* dir, const je_options* options, je_engine** out) {
    return jh_guarded([&] {
        if (!dir || !out) invalid("null argument");
        *out = nullptr;
        je_options opts;
        je_default_options(&opts);
        if (options) opts = *options;
        const std::string root(dir);
        auto e = std::make_unique<je_engine>();
        e->config = load_config(root);
        const uint32_t max_length = opts.max_length ? opts.max_length : e->config.max_positions;
        if (max_length < 1 || max_length > e->config.max_positions)
            invalid("max_length must be an integer between 1 and " + std::to_string(e->config.max_positions));
        if (file_exists(root + "/INCOMPLETE") || file_exists(root + "/quantization.json"))
            invalid("INT8 checkpoints are not supported by this runtime");
        SafeTensors t(root + "/model.safetensors", e->config.bf16_checkpoint);
        // assemble (src/engine.rs:147-172)
        if (opts.batch_size < 1 || opts.max_batch_tokens < max_length) invalid("Invalid batch size / token budget");
        HostWeights hw = load_weights(t, e->config);
        jh_config cfg = e->config.view();
        int rc = jh_create(&cfg, &hw.w, opts.device_ordinal, &e->model);
        if (rc != JH_OK) throw jh_error(rc, jh_last_error());
        opts.max_length = max_length;
        e->options = opts;
        e->name = jh_name(e->model);
        *out = e.release();
    });
}

int je_logits_encoded(je_engine* e, size_t n, const uint32_t* ids, const size_t* id_off, const uint32_t* markers,
                      const size_t* mk_off, const uint8_t* qtypes, float* logits) {
    return jh_guarded([&] {
        if (!e) invalid("null engine");
        if (n == 0) return;
        if (!ids || !id_off || !mk_off || !qtypes || (mk_off[n] && (!markers || !logits))) invalid("null argument");
        std::lock_guard<std::mutex> guard(e->lock);
        for (size_t i = 0; i < n; ++i) {
            if (id_off[i + 1] < id_off[i] || mk_off[i + 1] < mk_off[i]) invalid("offsets must be non-decreasing");
            const size_t len = id_off[i + 1] - id_off[i];
            if (len > e->options.max_length) invalid("encoded row longer than max_length");
            for (size_t j = mk_off[i]; j < mk_off[i + 1]; ++j)
                if (markers[j] >= len) invalid("marker outside its row");
        }
        // Length-sorted micro-batches (src/engine.rs:191-210): stable by length,
        // cut at batch_size rows or max_batch_tokens tokens.
        std::vector<size_t> order(n);
        std::iota(order.begin(), order.end(), 0);
        std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
            return id_off[a + 1] - id_off[a] < id_off[b + 1] - id_off[b];
        });
        std::vector<std::vector<size_t>> batches;
        std::vector<size_t> group;
        size_t tokens = 0;
        for (size_t i : order) {
            const size_t len = id_off[i + 1] - id_off[i];
            if (!group.empty() && (group.size() == e->options.batch_size || tokens + len > e->options.max_batch_tokens)) {
                batches.push_back(std::move(group));
                group.clear();
                tokens = 0;
            }
            group.push_back(i);
            tokens += len;
        }
        if (!group.empty()) batches.push_back(std::move(group));
        // Engine::forward per micro-batch: Batch::new packing (src/model.rs:127-147),
        // the backend, then the nonfinite check (src/engine.rs:212-223).  The
        // reference waits for each forward before packing the next; here up to
        // JH_MAX_INFLIGHT micro-batches are submitted ahead, so the host packs
        // and enqueues batch i+1 while the GPU runs batch i.
        struct InFlight {
            uint64_t ticket;
            size_t batch, markers;
        };
        std::deque<InFlight> inflight;
        std::vector<float> scores;
        // A failure leaves no ticket behind: outstanding ones are collected and dropped.
        struct Drain {
            je_engine* e;
            std::deque<InFlight>& q;
            ~Drain() {
                std::vector<float> sink;
                for (const InFlight& f : q) {
                    sink.resize(f.markers);
                    (void)jh_collect(e->model, f.ticket, sink.data(), f.markers);
                }
            }
        } drain{e, inflight};
        auto finish = [&] {
            const InFlight f = inflight.front();
            scores.assign(f.markers, 0.0f);
            const int rc = jh_collect(e->model, f.ticket, scores.data(), f.markers);
            inflight.pop_front();
            if (rc != JH_OK) throw jh_error(rc, jh_last_error());
            ++e->forwards;
            for (float v : scores)
                if (!std::isfinite(v)) throw jh_error(JH_ERR_NONFINITE, "Inference returned nonfinite logits");
            size_t k = 0;
            for (size_t i : batches[f.batch])
                for (size_t j = mk_off[i]; j < mk_off[i + 1]; ++j) logits[j] = scores[k++];
        };
        std::vector<uint32_t> bids, starts, lens, rows;
        std::vector<uint8_t> bq;
        for (size_t bi = 0; bi < batches.size(); ++bi) {
            bids.clear(); starts.clear(); lens.clear(); rows.clear(); bq.clear();
            for (size_t i : batches[bi]) {
                const uint32_t start = (uint32_t)bids.size();
                starts.push_back(start);
                lens.push_back((uint32_t)(id_off[i + 1] - id_off[i]));
                bq.push_back(qtypes[i]);
                bids.insert(bids.end(), ids + id_off[i], ids + id_off[i + 1]);
                for (size_t j = mk_off[i]; j < mk_off[i + 1]; ++j) rows.push_back(start + markers[j]);
            }
            if (inflight.size() == JH_MAX_INFLIGHT) finish();
            uint64_t ticket = 0;
            const int rc = jh_submit(e->model, bids.data(), bids.size(), starts.data(), lens.data(), bq.data(),
                                     batches[bi].size(), rows.data(), rows.size(), &ticket);
            if (rc != JH_OK) throw jh_error(rc, jh_last_error());
            inflight.push_back({ticket, bi, rows.size()});
        }
        while (!inflight.empty()) finish();
    });
}

int je_config(je_engine* e, jh_config* out) {
    return jh_guarded([&] {
        if (!e || !out) invalid("null argument");
        *out = e->config.view();
    });
}

int je_get_options(je_engine* e, je_options* out) {
    return jh_guarded([&] {
        if (!e || !out) invalid("null argument");
        *out = e->options;
    });
}

const char* je_device_name(je_engine* e) { return e ? e->name.c_str() : ""; }

uint64_t je_forward_count(je_engine* e) { return e ? e->forwards : 0; }

void je_destroy(je_engine* e) { delete e; }

}  // extern "C"
