// The HIP backend model: device-resident BF16 weights, a grow-only
// workspace, batch staging, and the encoder-forward launch sequence.
// Replaces CudaModel (src/cuda/mod.rs) behind the C-ABI of julia1_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/julia1_hip.h"
#include "../../include/julia1_hip_ops.h"
#include "abi_util.hpp"
#include "kernels.hpp"

namespace {

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr; o.bytes = 0; }
    DevBuf& operator=(DevBuf&& o) noexcept {
        if (this != &o) { release(); p = o.p; bytes = o.bytes; o.p = nullptr; o.bytes = 0; }
        return *this;
    }
    ~DevBuf() { release(); }
    void alloc(size_t n) {
        release();
        if (hipMalloc(&p, std::max<size_t>(n, 256)) != hipSuccess) {
            p = nullptr;
            (void)hipGetLastError();
            throw jh_error(JH_ERR_ALLOC, "hipMalloc of " + std::to_string(n) + " bytes failed");
        }
        bytes = n;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    template <class T> T* as() const { return (T*)p; }
};

struct PinnedBuf {
    void* p = nullptr;
    size_t bytes = 0;
    PinnedBuf() = default;
    PinnedBuf(const PinnedBuf&) = delete;
    PinnedBuf& operator=(const PinnedBuf&) = delete;
    ~PinnedBuf() { release(); }
    void alloc(size_t n) {
        release();
        if (hipHostMalloc(&p, std::max<size_t>(n, 256), hipHostMallocDefault) != hipSuccess) {
            p = nullptr;
            (void)hipGetLastError();
            throw jh_error(JH_ERR_ALLOC, "hipHostMalloc of " + std::to_string(n) + " bytes failed");
        }
        bytes = n;
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        bytes = 0;
    }
    template <class T> T* as() const { return (T*)p; }
};

DevBuf upload_bytes(const void* src, size_t bytes) {
    DevBuf b;
    b.alloc(bytes);
    HIP_CHECK(hipMemcpy(b.p, src, bytes, hipMemcpyHostToDevice));
    return b;
}

DevBuf upload_f32(const float* src, size_t n) {
    if (!src) throw jh_error(JH_ERR_INVALID, "missing weight tensor");
    return upload_bytes(src, n * sizeof(float));
}

// FP32 -> BF16 (round to nearest even) on the host, then upload (half::bf16::from_f32, src/cuda/mod.rs:36-39).
DevBuf upload_bf16(const float* src, size_t n) {
    if (!src) throw jh_error(JH_ERR_INVALID, "missing weight tensor");
    std::vector<bf16_t> tmp(n);
    for (size_t i = 0; i < n; ++i) tmp[i] = f2bf_host(src[i]);
    return upload_bytes(tmp.data(), n * sizeof(bf16_t));
}

// The same BF16 matrix [n, k] in the weight-stationary GEMM's fragment order
// (a second copy beside the row-major one, which the other GEMM kernels
// read), or nothing when that kernel does not take the shape (K = 768 with
// n % 256 == 0, or K = 1152 with n % 128 == 0).
DevBuf upload_bf16_ws(const float* src, size_t n, size_t k) {
    if (!((k == 768 && n % 256 == 0) || (k == 1152 && n % 128 == 0))) return DevBuf();
    if (!src) throw jh_error(JH_ERR_INVALID, "missing weight tensor");
    std::vector<bf16_t> tmp(n * k), packed(n * k);
    for (size_t i = 0; i < n * k; ++i) tmp[i] = f2bf_host(src[i]);
    pack_ws(tmp.data(), (int)n, (int)k, packed.data());
    return upload_bytes(packed.data(), n * k * sizeof(bf16_t));
}

struct EncLayer {
    DevBuf attn_norm, wqkv, wo, mlp_norm, wi, wo2;
    DevBuf wqkv_ws, wo_ws, wi_ws, wo2_ws;  // weight-stationary copies (empty where that kernel does not apply)
    int rope = 0;
    bool global = false;
};

struct HeadLayer {
    DevBuf norm1_w, norm1_b, in_w, in_b, out_w, out_b, norm2_w, norm2_b, lin1_w, lin1_b, lin2_w, lin2_b;
    DevBuf in_ws, out_ws, lin1_ws;
};

constexpr int QTILE = 128;  // queries per attention work item (four waves of 32)

// Kernel classes of the launch sequence, for jh_profile_read.
enum KClass {
    K_EMBED, K_LN, K_QKV, K_ATTN_GLOBAL, K_ATTN_LOCAL, K_WO, K_WI, K_WO2, K_FINAL,
    K_HEAD_GEMM, K_HEAD_ATTN, K_HEAD_ROWS, K_SCORER, K_COUNT
};
const char* const kClassNames[K_COUNT] = {
    "embed_ln", "layer_norm", "gemm_qkv_rope", "attn_global", "attn_local", "gemm_wo_resid", "gemm_wi_geglu",
    "gemm_wo2_resid", "final_norm", "head_gemm", "head_attn", "head_rows", "scorer"};

struct ProfRec {
    int cls;
    double flops, bytes;
    hipEvent_t a, b;
};

double gemm_bytes(int epi, double rows, double n, double k) {
    double out = 0;
    switch (epi) {
        case JH_EPI_GEGLU_BF16: out = rows * n / 2 * 2; break;
        case JH_EPI_RESID_F32: out = rows * n * 8; break;
        case JH_EPI_BIAS_F32: out = rows * n * 4; break;
        default: out = rows * n * 2;
    }
    return rows * k * 2 + n * k * 2 + out;
}

// Device and pinned buffers of one staged batch's metadata (ids,
// position|qtype words, attention tiles, marker rows), with the graph captured
// for batches staged in it.  Slot 0 serves jh_stage/jh_forward; the others
// form the jh_submit ring, where a slot stays busy until its ticket is
// collected, so a batch's metadata and scores outlive the next batch's upload.
struct MetaSlot {
    DevBuf dev;
    PinnedBuf host;
    size_t cap = 0;                  // 32-bit words
    hipEvent_t uploaded = nullptr;   // the upload from `host` has completed
    bool upload_pending = false;
    // jh_submit ring only
    PinnedBuf scores;
    size_t cap_scores = 0;           // floats
    hipEvent_t done = nullptr;       // the scores have reached `scores`
    bool busy = false, collecting = false;
    uint64_t ticket = 0;
    size_t markers = 0;
    // graph of the launch sequence for the shape staged in this slot
    hipGraphExec_t graph = nullptr;
    size_t graph_key[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    // shape of the previous execute from this slot: captured only when it repeats
    size_t last_key[8] = {0, 0, 0, 0, 0, 0, 0, 0};
};

}  // namespace

struct jh_model {
    std::mutex mu;
    int device = 0;
    hipStream_t stream = nullptr;
    // configuration
    int h = 0, heads = 0, inter = 0, nlayers = 0, half_window = 0, vocab = 0, max_pos = 0, head_heads = 0, ff = 0;
    float eps = 1e-5f;
    // weights
    DevBuf emb, emb_norm, final_norm, type_emb, s_norm_w, s_norm_b, s_w1, s_b1, s_w2;
    float s_b2 = 0.0f;
    std::vector<EncLayer> layers;
    std::vector<HeadLayer> head;
    std::vector<std::pair<DevBuf, DevBuf>> ropes;
    // workspace (grow-only)
    size_t cap_t = 0, cap_m = 0;
    uint64_t ws_gen = 0;
    DevBuf x, xn, qkv, ctx, hbuf, y, yn, qm, cm, hm, z, scores;
    PinnedBuf scores_host;
    // batch metadata: slot 0 for jh_stage/jh_forward, 1..kSlots-1 for jh_submit
    static constexpr int kSlots = 1 + JH_MAX_INFLIGHT;
    MetaSlot slots[kSlots];
    int cur = 0;  // slot of the staged batch
    uint64_t last_ticket = 0;
    // split-K partial sums of GEMMs whose output has too few tiles (small
    // batches, marker rows): fixed size, allocated with the model
    static constexpr size_t kSplitkBytes = 24u << 20;
    DevBuf splitk;
    // staged batch
    bool staged = false;
    size_t T = 0, S = 0, M = 0, ntiles = 0, nmtiles = 0;
    uint32_t* d_ids = nullptr;
    uint32_t* d_tok = nullptr;
    AttnTile* d_tiles = nullptr;
    AttnTile* d_mtiles = nullptr;
    // Global layers of sequences of kLongSeq tokens or more run 256-query
    // work items of eight waves (d_gtiles[0, nglong)); the other sequences'
    // 128-query tiles follow (d_gtiles[nglong, nglong + ngshort)).  With no
    // long sequence, global layers use d_tiles.
    static constexpr uint32_t kLongSeq = 4096;
    AttnTile* d_gtiles = nullptr;
    size_t nglong = 0, ngshort = 0;
    double pairs_glong = 0, pairs_gshort = 0, rows_glong = 0;
    int32_t* d_markers = nullptr;
    // replay repeated shapes from a captured graph (see jh_set_graph)
    bool use_graph = true;
    // split-K GEMMs for outputs with too few tiles (see jh_set_splitk)
    bool use_splitk = true;
    // debug limit on the bytes of one workspace growth (0 = none; jh_debug_workspace_limit)
    size_t ws_limit = 0;
    std::string name;
    // attention (query, key) pairs of the staged batch, for algorithmic FLOPs
    double pairs_global = 0, pairs_local = 0, pairs_marker = 0;
    // profiling: one event pair per launch, stamped at the dispatch, while enabled
    bool profiling = false;
    std::vector<hipEvent_t> ev_pool;
    size_t ev_next = 0;
    std::vector<ProfRec> recs;
    // profiling: the first GEMM / attention launch of each class, kept by
    // value so jh_profile_replay can repeat it back to back
    std::function<void()> replay[K_COUNT];

    ~jh_model() {
        for (MetaSlot& s : slots) {
            if (s.graph) (void)hipGraphExecDestroy(s.graph);
            if (s.uploaded) (void)hipEventDestroy(s.uploaded);
            if (s.done) (void)hipEventDestroy(s.done);
        }
        for (hipEvent_t e : ev_pool) (void)hipEventDestroy(e);
        if (stream) (void)hipStreamDestroy(stream);
    }

    hipEvent_t next_event() {
        if (ev_next == ev_pool.size()) {
            hipEvent_t e;
            HIP_CHECK(hipEventCreate(&e));
            ev_pool.push_back(e);
        }
        return ev_pool[ev_next++];
    }

    template <class F>
    void timed(int cls, double flops, double bytes, F&& launch) {
        if (!profiling) {
            launch();
            return;
        }
        ProfRec r{cls, flops, bytes, next_event(), next_event()};
        const LaunchEvents ev{r.a, r.b};
        jh_launch_events = &ev;
        try {
            launch();
        } catch (...) {
            jh_launch_events = nullptr;
            throw;
        }
        jh_launch_events = nullptr;
        recs.push_back(r);
    }

    void bind() const { HIP_CHECK(hipSetDevice(device)); }

    // Grows the workspace and the metadata buffers of `slot`.  Submitted
    // forwards may still be running on the old buffers, so growth waits for
    // the stream before it frees them.  Before anything is freed the recorded
    // capacities drop to zero and the generation moves on, so if an
    // allocation fails part way (JH_ERR_ALLOC) no later forward, graph replay
    // or profiling replay can touch a freed or missing buffer: the next batch
    // regrows everything (src/cuda/mod.rs:286-311 clears its buffers the same way).
    void ensure_workspace(size_t t, size_t m, int slot, size_t meta_len) {
        MetaSlot& ms = slots[slot];
        if (t > cap_t || m > cap_m || meta_len > ms.cap) HIP_CHECK(hipStreamSynchronize(stream));
        if (t > cap_t || m > cap_m) {
            size_t ct = 1024, cm_ = 256;
            while (ct < std::max(t, cap_t)) ct <<= 1;
            while (cm_ < std::max(m, cap_m)) cm_ <<= 1;
            cap_t = cap_m = 0;
            ++ws_gen;
            size_t H = h, wide = std::max<size_t>(inter, ff), grown = 0;
            auto grow = [&](DevBuf& b, size_t bytes) {
                grown += bytes;
                if (ws_limit && grown > ws_limit)
                    throw jh_error(JH_ERR_ALLOC, "workspace of " + std::to_string(grown) + " bytes exceeds the debug limit");
                b.alloc(bytes);
            };
            grow(x, ct * H * 4);
            grow(xn, ct * H * 2);
            grow(qkv, ct * 3 * H * 2);
            grow(ctx, ct * H * 2);
            grow(hbuf, ct * wide * 2);
            grow(y, cm_ * H * 4);
            grow(yn, cm_ * H * 2);
            grow(qm, cm_ * H * 2);
            grow(this->cm, cm_ * H * 2);
            grow(hm, cm_ * ff * 2);
            grow(z, cm_ * H * 4);
            grow(scores, cm_ * 4);
            scores_host.alloc(cm_ * 4);
            cap_t = ct;
            cap_m = cm_;
        }
        if (meta_len > ms.cap) {
            size_t n = 4096;
            while (n < meta_len) n <<= 1;
            ms.cap = 0;
            ms.upload_pending = false;
            ++ws_gen;
            ms.dev.alloc(n * 4);
            ms.host.alloc(n * 4);
            ms.cap = n;
        }
        if (!ms.uploaded) HIP_CHECK(hipEventCreateWithFlags(&ms.uploaded, hipEventDisableTiming));
    }

    // Validates a packed batch (Batch, src/model.rs:114-124) and enqueues its
    // upload into metadata slot `slot`; the batch becomes the staged one.
    void stage(int slot, const uint32_t* ids, size_t t, const uint32_t* starts, const uint32_t* lens,
               const uint8_t* qtypes, size_t nseq, const uint32_t* marker_rows, size_t m) {
        // Recorded replays point into the staged batch's metadata and workspace;
        // a batch that fails to stage leaves none staged.
        for (auto& r : replay) r = nullptr;
        staged = false;
        if ((t && !ids) || (nseq && (!starts || !lens || !qtypes)) || (m && !marker_rows))
            throw jh_error(JH_ERR_INVALID, "null batch array");
        if (t > (size_t)0x7fffffff || m > (size_t)0x7fffffff) throw jh_error(JH_ERR_INVALID, "batch too large");
        size_t next = 0;
        for (size_t s = 0; s < nseq; ++s) {
            if (starts[s] != next) throw jh_error(JH_ERR_INVALID, "sequences must be packed back to back in order");
            if (lens[s] > (uint32_t)max_pos)
                throw jh_error(JH_ERR_INVALID, "sequence longer than max_position_embeddings");
            if (qtypes[s] > 2) throw jh_error(JH_ERR_INVALID, "qtype must be 0, 1 or 2");
            next += lens[s];
        }
        if (next != t) throw jh_error(JH_ERR_INVALID, "sequence lengths do not sum to the token count");
        for (size_t i = 0; i < t; ++i)
            if (ids[i] >= (uint32_t)vocab) throw jh_error(JH_ERR_INVALID, "token id out of vocabulary");
        // Attention work items: 128-query tiles per sequence; marker tiles per sequence.
        std::vector<AttnTile> tiles, mtiles;
        for (size_t s = 0; s < nseq; ++s)
            for (uint32_t q0 = 0; q0 < lens[s]; q0 += QTILE)
                tiles.push_back({(int32_t)(starts[s] + q0), (int32_t)std::min<uint32_t>(QTILE, lens[s] - q0),
                                 (int32_t)starts[s], (int32_t)lens[s], (int32_t)q0});
        // Costliest first (queries x keys of a full-attention layer), so the
        // attention kernel dispatches them first and every CU gets a mix of long
        // and short work items; each tile writes only its own rows, so the
        // order does not change results.
        std::stable_sort(tiles.begin(), tiles.end(), [](const AttnTile& x, const AttnTile& y) {
            return (int64_t)x.nq * x.kv_len > (int64_t)y.nq * y.kv_len;
        });
        // Global-layer lists when some sequence is long: its 256-query tiles
        // first (costliest first), then the 128-query tiles of the others, in
        // the order of `tiles`.
        std::vector<AttnTile> gtiles;
        size_t glong = 0;
        bool any_long = false;
        for (size_t s = 0; s < nseq; ++s) any_long |= lens[s] >= kLongSeq;
        if (any_long) {
            for (size_t s = 0; s < nseq; ++s)
                if (lens[s] >= kLongSeq)
                    for (uint32_t q0 = 0; q0 < lens[s]; q0 += 2 * QTILE)
                        gtiles.push_back({(int32_t)(starts[s] + q0), (int32_t)std::min<uint32_t>(2 * QTILE, lens[s] - q0),
                                          (int32_t)starts[s], (int32_t)lens[s], (int32_t)q0});
            std::stable_sort(gtiles.begin(), gtiles.end(), [](const AttnTile& x, const AttnTile& y) {
                return (int64_t)x.nq * x.kv_len > (int64_t)y.nq * y.kv_len;
            });
            glong = gtiles.size();
            for (const AttnTile& tl : tiles)
                if ((uint32_t)tl.kv_len < kLongSeq) gtiles.push_back(tl);
        }
        size_t mi = 0;
        for (size_t s = 0; s < nseq; ++s) {
            size_t first = mi;
            while (mi < m && marker_rows[mi] >= starts[s] && marker_rows[mi] < starts[s] + lens[s]) ++mi;
            for (size_t j = first; j < mi; j += QTILE)
                mtiles.push_back({(int32_t)j, (int32_t)std::min<size_t>(QTILE, mi - j), (int32_t)starts[s],
                                  (int32_t)lens[s], 0});
        }
        if (mi != m) throw jh_error(JH_ERR_INVALID, "marker rows must lie in their sequence, grouped by sequence");
        const size_t meta_len = 2 * t + 5 * (tiles.size() + mtiles.size()) + m + 5 * gtiles.size();
        ensure_workspace(t, m, slot, meta_len);
        MetaSlot& ms = slots[slot];
        // The slot's previous upload may still be reading its pinned staging buffer.
        if (ms.upload_pending) HIP_CHECK(hipEventSynchronize(ms.uploaded));
        ms.upload_pending = false;
        staged = false;
        uint32_t* hm_ = ms.host.as<uint32_t>();
        std::memcpy(hm_, ids, t * 4);
        uint32_t* tok = hm_ + t;
        for (size_t s = 0; s < nseq; ++s)
            for (uint32_t i = 0; i < lens[s]; ++i) tok[starts[s] + i] = i | ((uint32_t)qtypes[s] << 16);
        std::memcpy(hm_ + 2 * t, tiles.data(), tiles.size() * sizeof(AttnTile));
        std::memcpy(hm_ + 2 * t + 5 * tiles.size(), mtiles.data(), mtiles.size() * sizeof(AttnTile));
        std::memcpy(hm_ + 2 * t + 5 * (tiles.size() + mtiles.size()), marker_rows, m * 4);
        std::memcpy(hm_ + 2 * t + 5 * (tiles.size() + mtiles.size()) + m, gtiles.data(), gtiles.size() * sizeof(AttnTile));
        HIP_CHECK(hipMemcpyAsync(ms.dev.p, ms.host.p, meta_len * 4, hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipEventRecord(ms.uploaded, stream));
        ms.upload_pending = true;
        cur = slot;
        uint32_t* dm = ms.dev.as<uint32_t>();
        d_ids = dm;
        d_tok = dm + t;
        d_tiles = (AttnTile*)(dm + 2 * t);
        d_mtiles = (AttnTile*)(dm + 2 * t + 5 * tiles.size());
        d_markers = (int32_t*)(dm + 2 * t + 5 * (tiles.size() + mtiles.size()));
        d_gtiles = (AttnTile*)(dm + 2 * t + 5 * (tiles.size() + mtiles.size()) + m);
        nglong = glong;
        ngshort = gtiles.size() - glong;
        pairs_global = pairs_local = pairs_marker = pairs_glong = pairs_gshort = rows_glong = 0;
        for (size_t sq = 0; sq < nseq; ++sq) {
            const double n = lens[sq];
            pairs_global += n * n;
            if (lens[sq] >= kLongSeq) {
                pairs_glong += n * n;
                rows_glong += n;
            }
            const long w = half_window, len = (long)lens[sq];
            for (long i = 0; i < len; ++i) pairs_local += (double)(std::min(i + w, len - 1) - std::max(i - w, 0L) + 1);
        }
        pairs_gshort = pairs_global - pairs_glong;
        for (const AttnTile& mt : mtiles) pairs_marker += (double)mt.nq * mt.kv_len;
        T = t;
        S = nseq;
        M = m;
        ntiles = tiles.size();
        nmtiles = mtiles.size();
        staged = true;
    }

    void gemm(int cls, int epi, const void* xp, long ldx, const int32_t* gather, size_t rows, const bf16_t* w, int n,
              int k, void* out, long ldo, int col, const float* bias, const float* cos_t = nullptr,
              const float* sin_t = nullptr, int rope_cols = 0, const bf16_t* w_ws = nullptr) {
        GemmArgs a{(const bf16_t*)xp, ldx, gather, (int)rows, w, n, k, out, ldo, col, bias,
                   (const int32_t*)d_tok, cos_t, sin_t, rope_cols};
        a.w_ws = w_ws;
        if (use_splitk) {
            a.partial = splitk.as<float>();
            a.partial_bytes = kSplitkBytes;
        }
        timed(cls, 2.0 * rows * n * k, gemm_bytes(epi, rows, n, k), [&] { launch_gemm(epi, a, stream); });
        if (profiling && !replay[cls]) replay[cls] = [epi, a, st = stream] { launch_gemm(epi, a, st); };
    }

    // RESID_F32 GEMM into xo [rows, H] followed by lo = bf16(LN(xo)).  On the
    // split-K path (small batches) the partial reduction, residual add and
    // LayerNorm are one kernel; otherwise the GEMM epilogue adds the residual
    // and a separate LayerNorm follows.
    void gemm_resid_ln(int cls, int ln_cls, const void* xp, long ldx, size_t rows, const bf16_t* w, int k, float* xo,
                       const float* bias, const float* ln_w, const float* ln_b, float ln_eps, bf16_t* lo,
                       const bf16_t* w_ws = nullptr) {
        const int H = h;
        GemmArgs a{(const bf16_t*)xp, ldx, nullptr, (int)rows, w, H, k, xo, H, 0, bias,
                   (const int32_t*)d_tok, nullptr, nullptr, 0};
        int S = 1;
        if (use_splitk) {
            a.partial = splitk.as<float>();
            a.partial_bytes = kSplitkBytes;
            S = gemm_splitk_count(JH_EPI_RESID_F32, a);
        }
        if (S <= 1) {
            gemm(cls, JH_EPI_RESID_F32, xp, ldx, nullptr, rows, w, H, k, xo, H, 0, bias, nullptr, nullptr, 0, w_ws);
            layer_norm(ln_cls, xo, rows, ln_w, ln_b, ln_eps, lo);
            return;
        }
        timed(cls, 2.0 * rows * H * k, gemm_bytes(JH_EPI_RESID_F32, rows, H, k),
              [&] { launch_gemm_partial(JH_EPI_RESID_F32, a, S, stream); });
        if (profiling && !replay[cls]) replay[cls] = [a, S, st = stream] { launch_gemm_partial(JH_EPI_RESID_F32, a, S, st); };
        timed(ln_cls, 0, (double)rows * H * (4.0 * S + 14), [&] {
            launch_resid_reduce_ln(splitk.as<float>(), S, (int)rows, H, bias, xo, ln_w, ln_b, ln_eps, lo, stream);
        });
    }

    // GEMM whose X operand is bf16(LN(xf row)) with weights ln_w, computed in
    // the small-batch kernel's prologue (K = hidden).
    void gemm_ln(int cls, int epi, const float* xf, size_t rows, const float* ln_w, const bf16_t* w, int n, void* out,
                 long ldo, const float* cos_t = nullptr, const float* sin_t = nullptr, int rope_cols = 0) {
        const int k = h;
        GemmArgs a{nullptr, (long)k, nullptr, (int)rows, w, n, k, out, ldo, 0, nullptr,
                   (const int32_t*)d_tok, cos_t, sin_t, rope_cols};
        a.xf = xf;
        a.ln_w = ln_w;
        a.ln_eps = eps;
        timed(cls, 2.0 * rows * n * k, gemm_bytes(epi, rows, n, k) + 2.0 * rows * k,
              [&] { launch_gemm(epi, a, stream); });
        if (profiling && !replay[cls]) replay[cls] = [epi, a, st = stream] { launch_gemm(epi, a, st); };
    }

    // Whether every encoder GEMM of the staged batch runs as one launch of the
    // small-batch kernel (split-K mode, few tokens).  Then the residual GEMMs
    // add straight into x and the LayerNorms before Wqkv and Wi run in those
    // GEMMs' prologues: five launches per layer instead of seven (a split-K
    // partial pass and a reduce + LayerNorm kernel per residual GEMM).
    bool fused_small_layers() {
        if (!use_splitk || T == 0 || nlayers == 0) return false;
        if (h != 128 && h != 256 && h != 384 && h != 512 && h != 768) return false;
        const EncLayer& L = layers[0];
        auto small = [&](int epi, const void* xp, long ldx, const bf16_t* w, int n, int k, void* out, long ldo) {
            GemmArgs a{(const bf16_t*)xp, ldx, nullptr, (int)T, w, n, k, out, ldo, 0, nullptr, nullptr, nullptr,
                       nullptr, 0};
            a.partial = splitk.as<float>();
            a.partial_bytes = kSplitkBytes;
            return gemm_uses_small(epi, a);
        };
        const int H = h;
        return small(JH_EPI_ROPE_BF16, xn.p, H, L.wqkv.as<bf16_t>(), 3 * H, H, qkv.p, 3 * H) &&
               small(JH_EPI_RESID_F32, ctx.p, H, L.wo.as<bf16_t>(), H, H, x.p, H) &&
               small(JH_EPI_GEGLU_BF16, xn.p, H, L.wi.as<bf16_t>(), 2 * inter, H, hbuf.p, inter) &&
               small(JH_EPI_RESID_F32, hbuf.p, inter, L.wo2.as<bf16_t>(), H, inter, x.p, H);
    }

    void attention(int cls, const bf16_t* q, long ldq, const bf16_t* k, const bf16_t* v, long ldkv, bf16_t* out,
                   long ldo, const AttnTile* tiles, size_t n, int nheads, int window, double pairs, double qrows,
                   int waves = 4) {
        AttnArgs a{q, ldq, k, v, ldkv, out, ldo, tiles, (int)n, nheads, window, 0.125f * 1.4426950408889634f, waves};
        const double hd = 64.0 * nheads;
        timed(cls, 4.0 * hd * pairs, qrows * hd * 2 * 2 + (double)T * hd * 2 * 2, [&] { launch_attention(a, stream); });
        if (profiling && !replay[cls]) replay[cls] = [a, st = stream] { launch_attention(a, st); };
    }

    // Full attention over every staged sequence (encoder global layers, the
    // head's full layer): the long sequences' 256-query items, then the rest.
    void global_attention(int cls, const bf16_t* q, long ldq, const bf16_t* k, const bf16_t* v, long ldkv,
                          bf16_t* out, long ldo, int nheads) {
        if (nglong == 0) {
            attention(cls, q, ldq, k, v, ldkv, out, ldo, d_tiles, ntiles, nheads, -1, pairs_global, (double)T);
            return;
        }
        attention(cls, q, ldq, k, v, ldkv, out, ldo, d_gtiles, nglong, nheads, -1, pairs_glong, rows_glong, 8);
        if (ngshort > 0)
            attention(cls, q, ldq, k, v, ldkv, out, ldo, d_gtiles + nglong, ngshort, nheads, -1, pairs_gshort,
                      (double)T - rows_glong);
    }

    void layer_norm(int cls, const float* xp, size_t rows, const float* w, const float* b, float e, bf16_t* out) {
        timed(cls, 0, (double)rows * h * 6, [&] { launch_layer_norm(xp, (int)rows, w, b, e, h, out, stream); });
    }

    // Embeddings and the first `upto` encoder layers (src/cuda/mod.rs:446-463).
    void run_encoder(int upto) {
        const int H = h;
        const size_t t = T;
        timed(K_EMBED, 0, (double)t * (H * 10 + 4), [&] {
            launch_embed_ln(d_ids, (int)t, emb.as<float>(), emb_norm.as<float>(), eps, H, x.as<float>(),
                            xn.as<bf16_t>(), stream);
        });
        bool xn_ready = false;  // xn already holds this layer's attn_norm(x) (fused into the previous Wo2)
        const bool fused = fused_small_layers();
        for (int l = 0; l < upto; ++l) {
            EncLayer& L = layers[l];
            if (fused) {
                const float* cos_t = ropes[L.rope].first.as<float>();
                const float* sin_t = ropes[L.rope].second.as<float>();
                if (L.attn_norm.p)
                    gemm_ln(K_QKV, JH_EPI_ROPE_BF16, x.as<float>(), t, L.attn_norm.as<float>(), L.wqkv.as<bf16_t>(),
                            3 * H, qkv.p, 3 * H, cos_t, sin_t, 2 * H);
                else
                    gemm(K_QKV, JH_EPI_ROPE_BF16, xn.p, H, nullptr, t, L.wqkv.as<bf16_t>(), 3 * H, H, qkv.p, 3 * H, 0,
                         nullptr, cos_t, sin_t, 2 * H);
                const bf16_t* q = qkv.as<bf16_t>();
                if (L.global)
                    global_attention(K_ATTN_GLOBAL, q, 3 * H, q + H, q + 2 * H, 3 * H, ctx.as<bf16_t>(), H, heads);
                else
                    attention(K_ATTN_LOCAL, q, 3 * H, q + H, q + 2 * H, 3 * H, ctx.as<bf16_t>(), H, d_tiles, ntiles,
                              heads, half_window, pairs_local, (double)t);
                gemm(K_WO, JH_EPI_RESID_F32, ctx.p, H, nullptr, t, L.wo.as<bf16_t>(), H, H, x.p, H, 0, nullptr);
                gemm_ln(K_WI, JH_EPI_GEGLU_BF16, x.as<float>(), t, L.mlp_norm.as<float>(), L.wi.as<bf16_t>(),
                        2 * inter, hbuf.p, inter);
                gemm(K_WO2, JH_EPI_RESID_F32, hbuf.p, inter, nullptr, t, L.wo2.as<bf16_t>(), H, inter, x.p, H, 0,
                     nullptr);
                continue;
            }
            if (L.attn_norm.p && !xn_ready)
                layer_norm(K_LN, x.as<float>(), t, L.attn_norm.as<float>(), nullptr, eps, xn.as<bf16_t>());
            xn_ready = false;
            gemm(K_QKV, JH_EPI_ROPE_BF16, xn.p, H, nullptr, t, L.wqkv.as<bf16_t>(), 3 * H, H, qkv.p, 3 * H, 0, nullptr,
                 ropes[L.rope].first.as<float>(), ropes[L.rope].second.as<float>(), 2 * H, L.wqkv_ws.as<bf16_t>());
            const bf16_t* q = qkv.as<bf16_t>();
            if (L.global)
                global_attention(K_ATTN_GLOBAL, q, 3 * H, q + H, q + 2 * H, 3 * H, ctx.as<bf16_t>(), H, heads);
            else
                attention(K_ATTN_LOCAL, q, 3 * H, q + H, q + 2 * H, 3 * H, ctx.as<bf16_t>(), H, d_tiles, ntiles, heads,
                          half_window, pairs_local, (double)t);
            gemm_resid_ln(K_WO, K_LN, ctx.p, H, t, L.wo.as<bf16_t>(), H, x.as<float>(), nullptr,
                          L.mlp_norm.as<float>(), nullptr, eps, xn.as<bf16_t>(), L.wo_ws.as<bf16_t>());
            gemm(K_WI, JH_EPI_GEGLU_BF16, xn.p, H, nullptr, t, L.wi.as<bf16_t>(), 2 * inter, H, hbuf.p, inter, 0,
                 nullptr, nullptr, nullptr, 0, L.wi_ws.as<bf16_t>());
            if (l + 1 < upto && layers[l + 1].attn_norm.p) {
                gemm_resid_ln(K_WO2, K_LN, hbuf.p, inter, t, L.wo2.as<bf16_t>(), inter, x.as<float>(), nullptr,
                              layers[l + 1].attn_norm.as<float>(), nullptr, eps, xn.as<bf16_t>(), L.wo2_ws.as<bf16_t>());
                xn_ready = true;
            } else {
                gemm(K_WO2, JH_EPI_RESID_F32, hbuf.p, inter, nullptr, t, L.wo2.as<bf16_t>(), H, inter, x.p, H, 0,
                     nullptr, nullptr, nullptr, 0, L.wo2_ws.as<bf16_t>());
            }
        }
    }

    // Final norm, decision head and scorer (src/cuda/mod.rs:464-511; the last head
    // layer computes queries and FFN for markers only, as src/cpu/mod.rs:287-321).
    void run_head() {
        const int H = h;
        const size_t t = T, m = M;
        const int nh = (int)head.size();
        timed(K_FINAL, 0, (double)t * (H * 10 + 4), [&] {
            launch_final_norm(x.as<float>(), (int)t, final_norm.as<float>(), type_emb.as<float>(), d_tok,
                              head[0].norm1_w.as<float>(), head[0].norm1_b.as<float>(), eps, H, xn.as<bf16_t>(),
                              stream);
        });
        for (int j = 0; j + 1 < nh; ++j) {
            HeadLayer& L = head[j];
            gemm(K_HEAD_GEMM, JH_EPI_BIAS_BF16, xn.p, H, nullptr, t, L.in_w.as<bf16_t>(), 3 * H, H, qkv.p, 3 * H, 0,
                 L.in_b.as<float>(), nullptr, nullptr, 0, L.in_ws.as<bf16_t>());
            const bf16_t* q = qkv.as<bf16_t>();
            global_attention(K_HEAD_ATTN, q, 3 * H, q + H, q + 2 * H, 3 * H, ctx.as<bf16_t>(), H, head_heads);
            gemm_resid_ln(K_HEAD_GEMM, K_HEAD_ROWS, ctx.p, H, t, L.out_w.as<bf16_t>(), H, x.as<float>(),
                          L.out_b.as<float>(), L.norm2_w.as<float>(), L.norm2_b.as<float>(), 1e-5f, xn.as<bf16_t>(),
                          L.out_ws.as<bf16_t>());
            gemm(K_HEAD_GEMM, JH_EPI_BIAS_RELU_BF16, xn.p, H, nullptr, t, L.lin1_w.as<bf16_t>(), ff, H, hbuf.p, ff, 0,
                 L.lin1_b.as<float>(), nullptr, nullptr, 0, L.lin1_ws.as<bf16_t>());
            HeadLayer& N = head[j + 1];
            gemm_resid_ln(K_HEAD_GEMM, K_HEAD_ROWS, hbuf.p, ff, t, L.lin2_w.as<bf16_t>(), ff, x.as<float>(),
                          L.lin2_b.as<float>(), N.norm1_w.as<float>(), N.norm1_b.as<float>(), 1e-5f, xn.as<bf16_t>());
        }
        HeadLayer& L = head[nh - 1];
        // Keys/values for every token: in_proj rows [H, 3H) into qkv columns [H, 3H).
        // (In the weight-stationary copy, 256-row slabs are contiguous, so rows [H, 3H) start H·H elements in.)
        gemm(K_HEAD_GEMM, JH_EPI_BIAS_BF16, xn.p, H, nullptr, t, L.in_w.as<bf16_t>() + (size_t)H * H, 2 * H, H, qkv.p,
             3 * H, H, L.in_b.as<float>() + H, nullptr, nullptr, 0,
             L.in_ws.p && H % 256 == 0 ? L.in_ws.as<bf16_t>() + (size_t)H * H : nullptr);
        // Queries for markers only, gathered straight from the normed rows.
        gemm(K_HEAD_GEMM, JH_EPI_BIAS_BF16, xn.p, H, d_markers, m, L.in_w.as<bf16_t>(), H, H, qm.p, H, 0,
             L.in_b.as<float>());
        const bf16_t* kv = qkv.as<bf16_t>();
        attention(K_HEAD_ATTN, qm.as<bf16_t>(), H, kv + H, kv + 2 * H, 3 * H, cm.as<bf16_t>(), H, d_mtiles, nmtiles,
                  head_heads, -1, pairs_marker, (double)m);
        timed(K_HEAD_ROWS, 0, (double)m * H * 8, [&] {
            launch_gather_f32(x.as<float>(), d_markers, (int)m, H, y.as<float>(), stream);
        });
        gemm_resid_ln(K_HEAD_GEMM, K_HEAD_ROWS, cm.p, H, m, L.out_w.as<bf16_t>(), H, y.as<float>(),
                      L.out_b.as<float>(), L.norm2_w.as<float>(), L.norm2_b.as<float>(), 1e-5f, yn.as<bf16_t>());
        gemm(K_HEAD_GEMM, JH_EPI_BIAS_RELU_BF16, yn.p, H, nullptr, m, L.lin1_w.as<bf16_t>(), ff, H, hm.p, ff, 0,
             L.lin1_b.as<float>());
        // Scorer: LayerNorm -> Linear -> GELU -> Linear(.., 1); its LayerNorm follows lin2's residual.
        gemm_resid_ln(K_HEAD_GEMM, K_SCORER, hm.p, ff, m, L.lin2_w.as<bf16_t>(), ff, y.as<float>(),
                      L.lin2_b.as<float>(), s_norm_w.as<float>(), s_norm_b.as<float>(), 1e-5f, yn.as<bf16_t>());
        gemm(K_SCORER, JH_EPI_BIAS_F32, yn.p, H, nullptr, m, s_w1.as<bf16_t>(), H, H, z.p, H, 0, s_b1.as<float>());
        timed(K_SCORER, 4.0 * m * H, (double)m * H * 4 + m * 4.0, [&] {
            launch_scorer(z.as<float>(), (int)m, H, s_w2.as<float>(), s_b2, scores.as<float>(), stream);
        });
    }

    void run_all() {
        if (T == 0 || M == 0) return;
        run_encoder(nlayers);
        run_head();
    }

    void execute() {
        if (!staged) throw jh_error(JH_ERR_INVALID, "no batch staged");
        if (T == 0 || M == 0) return;
        if (!use_graph || profiling) {
            run_all();
            return;
        }
        MetaSlot& ms = slots[cur];
        const size_t key[8] = {T, M, S, ntiles, nmtiles, (size_t)ws_gen, nglong, ngshort};
        if (!ms.graph || !std::equal(key, key + 8, ms.graph_key)) {
            // Capturing and instantiating the ~200-launch forward costs ~0.5 ms
            // on MI355X while replay saves nothing measurable over eager
            // launches, so a shape seen for the first time in a row runs
            // eagerly; the graph is built when the same shape comes again.
            if (!std::equal(key, key + 8, ms.last_key)) {
                std::copy(key, key + 8, ms.last_key);
                run_all();
                return;
            }
            if (ms.graph) {
                // a submitted forward may still be replaying it
                HIP_CHECK(hipStreamSynchronize(stream));
                (void)hipGraphExecDestroy(ms.graph);
                ms.graph = nullptr;
            }
            HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
            try {
                run_all();
            } catch (...) {
                hipGraph_t g = nullptr;
                (void)hipStreamEndCapture(stream, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            hipGraph_t g = nullptr;
            HIP_CHECK(hipStreamEndCapture(stream, &g));
            hipError_t e = hipGraphInstantiate(&ms.graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (e != hipSuccess) {
                ms.graph = nullptr;
                throw jh_error(JH_ERR_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
            }
            std::copy(key, key + 8, ms.graph_key);
        }
        HIP_CHECK(hipGraphLaunch(ms.graph, stream));
    }

    void read_scores(float* out, size_t m) {
        if (!staged) throw jh_error(JH_ERR_INVALID, "no batch staged");
        if (m != M) throw jh_error(JH_ERR_INVALID, "score count does not match the staged markers");
        if (m == 0) {
            HIP_CHECK(hipStreamSynchronize(stream));
            return;
        }
        HIP_CHECK(hipMemcpyAsync(scores_host.p, scores.p, m * 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        std::memcpy(out, scores_host.p, m * 4);
    }

    // jh_submit: stage into a free ring slot, enqueue the forward and the
    // download of its scores, and return without waiting.
    uint64_t submit(const uint32_t* ids, size_t t, const uint32_t* starts, const uint32_t* lens,
                    const uint8_t* qtypes, size_t nseq, const uint32_t* marker_rows, size_t m) {
        int slot = -1;
        for (int i = 1; i < kSlots && slot < 0; ++i)
            if (!slots[i].busy) slot = i;
        if (slot < 0)
            throw jh_error(JH_ERR_INVALID, "too many submitted batches in flight: collect one first");
        MetaSlot& ms = slots[slot];
        if (m > ms.cap_scores) {
            size_t n = 256;
            while (n < m) n <<= 1;
            ms.scores.alloc(n * 4);
            ms.cap_scores = n;
        }
        if (!ms.done) HIP_CHECK(hipEventCreateWithFlags(&ms.done, hipEventDisableTiming));
        stage(slot, ids, t, starts, lens, qtypes, nseq, marker_rows, m);
        execute();
        if (m) HIP_CHECK(hipMemcpyAsync(ms.scores.p, scores.p, m * 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipEventRecord(ms.done, stream));
        ms.busy = true;
        ms.collecting = false;
        ms.markers = m;
        ms.ticket = ++last_ticket;
        return ms.ticket;
    }

    MetaSlot& ticket_slot(uint64_t ticket) {
        for (int i = 1; i < kSlots; ++i)
            if (slots[i].busy && slots[i].ticket == ticket) return slots[i];
        throw jh_error(JH_ERR_INVALID, "unknown or already collected ticket");
    }
};

namespace {

void check_config(const jh_config* c) {
    if (!c) throw jh_error(JH_ERR_INVALID, "null config");
    if (c->head_dim != 64) throw jh_error(JH_ERR_INVALID, "kernels require head_dim 64");
    if (c->hidden == 0 || c->hidden % 64 || c->hidden > 1024 || c->heads * 64 != c->hidden)
        throw jh_error(JH_ERR_INVALID, "hidden must be heads*64 and at most 1024");
    if (c->head_heads * 64 != c->hidden) throw jh_error(JH_ERR_INVALID, "head_heads must be hidden/64");
    if (c->intermediate == 0 || c->intermediate % 64) throw jh_error(JH_ERR_INVALID, "intermediate must be a multiple of 64");
    if (c->head_ff == 0 || c->head_ff % 64) throw jh_error(JH_ERR_INVALID, "head_ff must be a multiple of 64");
    if (c->head_layers < 1) throw jh_error(JH_ERR_INVALID, "at least one head layer is required");
    if (c->layers > 0 && (!c->global || !c->rope_theta)) throw jh_error(JH_ERR_INVALID, "missing per-layer config");
    if (c->max_positions == 0 || c->max_positions > 65535) throw jh_error(JH_ERR_INVALID, "max_positions must be 1..65535");
    if (c->vocab == 0) throw jh_error(JH_ERR_INVALID, "empty vocabulary");
    if (c->half_window > 65535) throw jh_error(JH_ERR_INVALID, "half_window too large");
}

void build_model(jh_model* m, const jh_config* c, const jh_weights* w, int ordinal) {
    check_config(c);
    if (!w || !w->embedding || !w->layers || !w->head) throw jh_error(JH_ERR_INVALID, "null weights");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        throw jh_error(JH_ERR_DEVICE, "HIP device unavailable");
    }
    if (ordinal < 0 || ordinal >= count) throw jh_error(JH_ERR_DEVICE, "HIP device ordinal out of range");
    m->device = ordinal;
    m->bind();
    hipDeviceProp_t prop;
    HIP_CHECK(hipGetDeviceProperties(&prop, ordinal));
    // prop.name can be blank when the marketing-name table is absent; the gfx arch is always set.
    std::string dev_name = prop.name[0] ? prop.name : "AMD GPU";
    std::string arch = prop.gcnArchName;
    arch = arch.substr(0, arch.find(':'));
    m->name = "hip:" + std::to_string(ordinal) + " (" + dev_name + ", " + arch + ")";
    m->splitk.alloc(jh_model::kSplitkBytes);
    HIP_CHECK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    const size_t H = c->hidden, I = c->intermediate, F = c->head_ff;
    m->h = (int)H; m->heads = (int)c->heads; m->inter = (int)I; m->nlayers = (int)c->layers;
    m->half_window = (int)c->half_window; m->vocab = (int)c->vocab; m->max_pos = (int)c->max_positions;
    m->head_heads = (int)c->head_heads; m->ff = (int)F; m->eps = c->norm_eps;
    m->emb = upload_f32(w->embedding, (size_t)c->vocab * H);
    m->emb_norm = upload_f32(w->emb_norm, H);
    std::vector<float> thetas;
    std::vector<float> wi_tmp(2 * I * H);
    for (uint32_t l = 0; l < c->layers; ++l) {
        const jh_encoder_layer& s = w->layers[l];
        EncLayer L;
        if (l > 0 && !s.attn_norm) throw jh_error(JH_ERR_INVALID, "encoder layers after the first need attn_norm");
        if (s.attn_norm) L.attn_norm = upload_f32(s.attn_norm, H);
        L.wqkv = upload_bf16(s.wqkv, 3 * H * H);
        L.wqkv_ws = upload_bf16_ws(s.wqkv, 3 * H, H);
        L.wo = upload_bf16(s.wo, H * H);
        L.wo_ws = upload_bf16_ws(s.wo, H, H);
        L.mlp_norm = upload_f32(s.mlp_norm, H);
        if (!s.wi) throw jh_error(JH_ERR_INVALID, "missing Wi");
        jh_op_interleave_geglu(s.wi, I, H, wi_tmp.data());
        L.wi = upload_bf16(wi_tmp.data(), 2 * I * H);
        L.wi_ws = upload_bf16_ws(wi_tmp.data(), 2 * I, H);
        L.wo2 = upload_bf16(s.wo2, H * I);
        L.wo2_ws = upload_bf16_ws(s.wo2, H, I);
        L.global = c->global[l] != 0;
        const float th = c->rope_theta[l];
        auto it = std::find(thetas.begin(), thetas.end(), th);
        if (it == thetas.end()) {
            std::vector<float> cs((size_t)c->max_positions * 32), sn((size_t)c->max_positions * 32);
            jh_rope_table(th, 64, c->max_positions, cs.data(), sn.data());
            m->ropes.emplace_back(upload_f32(cs.data(), cs.size()), upload_f32(sn.data(), sn.size()));
            thetas.push_back(th);
            L.rope = (int)thetas.size() - 1;
        } else {
            L.rope = (int)(it - thetas.begin());
        }
        m->layers.push_back(std::move(L));
    }
    m->final_norm = upload_f32(w->final_norm, H);
    m->type_emb = upload_f32(w->type_emb, 3 * H);
    for (uint32_t l = 0; l < c->head_layers; ++l) {
        const jh_head_layer& s = w->head[l];
        HeadLayer L;
        L.norm1_w = upload_f32(s.norm1_w, H); L.norm1_b = upload_f32(s.norm1_b, H);
        L.in_w = upload_bf16(s.in_w, 3 * H * H); L.in_b = upload_f32(s.in_b, 3 * H);
        L.out_w = upload_bf16(s.out_w, H * H); L.out_b = upload_f32(s.out_b, H);
        L.in_ws = upload_bf16_ws(s.in_w, 3 * H, H);
        L.out_ws = upload_bf16_ws(s.out_w, H, H);
        L.norm2_w = upload_f32(s.norm2_w, H); L.norm2_b = upload_f32(s.norm2_b, H);
        L.lin1_w = upload_bf16(s.lin1_w, F * H); L.lin1_b = upload_f32(s.lin1_b, F);
        L.lin1_ws = upload_bf16_ws(s.lin1_w, F, H);
        L.lin2_w = upload_bf16(s.lin2_w, H * F); L.lin2_b = upload_f32(s.lin2_b, H);
        m->head.push_back(std::move(L));
    }
    m->s_norm_w = upload_f32(w->scorer_norm_w, H);
    m->s_norm_b = upload_f32(w->scorer_norm_b, H);
    m->s_w1 = upload_bf16(w->scorer_w1, H * H);
    m->s_b1 = upload_f32(w->scorer_b1, H);
    m->s_w2 = upload_f32(w->scorer_w2, H);
    m->s_b2 = w->scorer_b2;
    HIP_CHECK(hipDeviceSynchronize());
}

}  // namespace

extern "C" {

const char* jh_last_error(void) { return jh_error_slot().c_str(); }

void jh_rope_table(float theta, uint32_t head_dim, uint32_t positions, float* cos_out, float* sin_out) {
    // Column by column, so nothing is allocated (no exception can cross the
    // C-ABI) and each inverse frequency is still computed once.
    const uint32_t half = head_dim / 2;
    for (uint32_t i = 0; i < half; ++i) {
        const float inv = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
        for (uint32_t p = 0; p < positions; ++p) {
            const float f = inv * (float)p;
            cos_out[(size_t)p * half + i] = cosf(f);
            sin_out[(size_t)p * half + i] = sinf(f);
        }
    }
}

int jh_debug_workspace_limit(jh_model* model, size_t bytes) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        std::lock_guard<std::mutex> g(model->mu);
        model->ws_limit = bytes;
    });
}

int jh_create(const jh_config* config, const jh_weights* weights, int ordinal, jh_model** out) {
    return jh_guarded([&] {
        if (!out) throw jh_error(JH_ERR_INVALID, "null output handle");
        *out = nullptr;
        auto m = std::make_unique<jh_model>();
        build_model(m.get(), config, weights, ordinal);
        *out = m.release();
    });
}

void jh_destroy(jh_model* model) {
    if (!model) return;
    (void)hipSetDevice(model->device);
    if (model->stream) (void)hipStreamSynchronize(model->stream);
    delete model;
}

const char* jh_name(jh_model* model) { return model ? model->name.c_str() : ""; }

void* jh_stream(jh_model* model) { return model ? (void*)model->stream : nullptr; }

int jh_set_graph(jh_model* model, int enabled) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        std::lock_guard<std::mutex> g(model->mu);
        model->use_graph = enabled != 0;
    });
}

int jh_set_splitk(jh_model* model, int enabled) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        std::lock_guard<std::mutex> g(model->mu);
        if (model->use_splitk != (enabled != 0)) {
            model->use_splitk = enabled != 0;
            ++model->ws_gen;  // the captured graph holds the other launch sequence
        }
    });
}

int jh_profile(jh_model* model, int enabled) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        HIP_CHECK(hipStreamSynchronize(model->stream));
        model->profiling = enabled != 0;
        model->recs.clear();
        model->ev_next = 0;
        for (auto& r : model->replay) r = nullptr;
    });
}

int jh_profile_replay(jh_model* model, const char* kernel_class, size_t reps, double* us_per_launch) {
    return jh_guarded([&] {
        if (!model || !kernel_class || !us_per_launch || reps == 0) throw jh_error(JH_ERR_INVALID, "bad argument");
        std::lock_guard<std::mutex> g(model->mu);
        int cls = -1;
        for (int c = 0; c < K_COUNT; ++c)
            if (std::strcmp(kClassNames[c], kernel_class) == 0) cls = c;
        if (cls < 0 || !model->replay[cls])
            throw jh_error(JH_ERR_INVALID, "no recorded GEMM/attention launch of that class (profile a forward first)");
        model->bind();
        hipEvent_t e0, e1;
        HIP_CHECK(hipEventCreate(&e0));
        HIP_CHECK(hipEventCreate(&e1));
        float ms = 0.0f;
        try {
            model->replay[cls]();  // warm
            HIP_CHECK(hipEventRecord(e0, model->stream));
            for (size_t i = 0; i < reps; ++i) model->replay[cls]();
            HIP_CHECK(hipEventRecord(e1, model->stream));
            HIP_CHECK(hipEventSynchronize(e1));
            HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        } catch (...) {
            (void)hipEventDestroy(e0);
            (void)hipEventDestroy(e1);
            throw;
        }
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        *us_per_launch = 1e3 * (double)ms / (double)reps;
    });
}

int jh_profile_read(jh_model* model, jh_kernel_stat* out, size_t capacity, size_t* count) {
    return jh_guarded([&] {
        if (!model || !count) throw jh_error(JH_ERR_INVALID, "null argument");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        HIP_CHECK(hipStreamSynchronize(model->stream));
        jh_kernel_stat acc[K_COUNT];
        for (int c = 0; c < K_COUNT; ++c) acc[c] = jh_kernel_stat{kClassNames[c], 0, 0.0, 0.0, 0.0};
        for (const ProfRec& r : model->recs) {
            float ms = 0.0f;
            HIP_CHECK(hipEventElapsedTime(&ms, r.a, r.b));
            acc[r.cls].launches += 1;
            acc[r.cls].ms += ms;
            acc[r.cls].flops += r.flops;
            acc[r.cls].bytes += r.bytes;
        }
        model->recs.clear();
        model->ev_next = 0;
        size_t n = 0;
        for (int c = 0; c < K_COUNT; ++c) {
            if (!acc[c].launches) continue;
            if (out && n < capacity) out[n] = acc[c];
            ++n;
        }
        *count = n;
    });
}

int jh_stage(jh_model* model, const uint32_t* ids, size_t tokens, const uint32_t* starts, const uint32_t* lens,
             const uint8_t* qtypes, size_t sequences, const uint32_t* marker_rows, size_t markers) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        model->stage(0, ids, tokens, starts, lens, qtypes, sequences, marker_rows, markers);
    });
}

int jh_execute(jh_model* model) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        model->execute();
    });
}

int jh_scores(jh_model* model, float* scores, size_t markers) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        if (markers && !scores) throw jh_error(JH_ERR_INVALID, "null scores buffer");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        model->read_scores(scores, markers);
    });
}

int jh_forward(jh_model* model, const uint32_t* ids, size_t tokens, const uint32_t* starts, const uint32_t* lens,
               const uint8_t* qtypes, size_t sequences, const uint32_t* marker_rows, size_t markers, float* scores) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        if (markers && !scores) throw jh_error(JH_ERR_INVALID, "null scores buffer");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        model->stage(0, ids, tokens, starts, lens, qtypes, sequences, marker_rows, markers);
        model->execute();
        model->read_scores(scores, markers);
    });
}

int jh_submit(jh_model* model, const uint32_t* ids, size_t tokens, const uint32_t* starts, const uint32_t* lens,
              const uint8_t* qtypes, size_t sequences, const uint32_t* marker_rows, size_t markers,
              uint64_t* ticket) {
    return jh_guarded([&] {
        if (!model || !ticket) throw jh_error(JH_ERR_INVALID, "null argument");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        *ticket = model->submit(ids, tokens, starts, lens, qtypes, sequences, marker_rows, markers);
    });
}

int jh_collect(jh_model* model, uint64_t ticket, float* scores, size_t markers) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        hipEvent_t done;
        {
            std::lock_guard<std::mutex> g(model->mu);
            MetaSlot& ms = model->ticket_slot(ticket);
            if (ms.collecting) throw jh_error(JH_ERR_INVALID, "ticket is being collected by another call");
            if (markers != ms.markers) throw jh_error(JH_ERR_INVALID, "score count does not match the submitted markers");
            if (markers && !scores) throw jh_error(JH_ERR_INVALID, "null scores buffer");
            ms.collecting = true;
            done = ms.done;
        }
        // Wait without the model lock, so other threads can submit meanwhile;
        // the slot stays busy, so its scores buffer and event stay put.
        hipError_t e = hipSetDevice(model->device);
        if (e == hipSuccess) e = hipEventSynchronize(done);
        std::lock_guard<std::mutex> g(model->mu);
        MetaSlot& ms = model->ticket_slot(ticket);
        ms.collecting = false;
        ms.busy = false;
        if (e != hipSuccess) throw jh_error(JH_ERR_DEVICE, std::string("hipEventSynchronize: ") + hipGetErrorString(e));
        if (markers) std::memcpy(scores, ms.scores.p, markers * 4);
    });
}

int jh_forward_padded(jh_model* model, const uint32_t* ids, size_t batch, size_t padded_len, const uint32_t* lens,
                      const uint8_t* qtypes, const uint32_t* markers, const uint32_t* marker_starts, float* scores) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        if (batch && (!ids || !lens || !qtypes || !marker_starts)) throw jh_error(JH_ERR_INVALID, "null batch array");
        const size_t m = batch ? marker_starts[batch] : 0;
        if (m && (!markers || !scores)) throw jh_error(JH_ERR_INVALID, "null marker or score buffer");
        // Pack away the padding on the host: the device only ever sees real tokens.
        std::vector<uint32_t> pids, starts(batch), rows;
        size_t total = 0;
        for (size_t b = 0; b < batch; ++b) {
            if (lens[b] > padded_len) throw jh_error(JH_ERR_INVALID, "row length exceeds the padded length");
            starts[b] = (uint32_t)total;
            total += lens[b];
        }
        pids.reserve(total);
        for (size_t b = 0; b < batch; ++b) {
            pids.insert(pids.end(), ids + b * padded_len, ids + b * padded_len + lens[b]);
            if (marker_starts[b + 1] < marker_starts[b] || marker_starts[b + 1] > m)
                throw jh_error(JH_ERR_INVALID, "marker_starts must be non-decreasing");
            for (uint32_t j = marker_starts[b]; j < marker_starts[b + 1]; ++j) {
                if (markers[j] >= lens[b]) throw jh_error(JH_ERR_INVALID, "marker outside its row");
                rows.push_back(starts[b] + markers[j]);
            }
        }
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        model->stage(0, pids.data(), total, starts.data(), lens, qtypes, batch, rows.data(), rows.size());
        model->execute();
        model->read_scores(scores, m);
    });
}

int jh_debug_tokens(jh_model* model, uint32_t* ids_out, uint32_t* pos_out, size_t tokens) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        if (!model->staged || tokens != model->T) throw jh_error(JH_ERR_INVALID, "token count does not match the staged batch");
        if (!tokens) return;
        std::vector<uint32_t> tok(tokens);
        HIP_CHECK(hipMemcpyAsync(ids_out, model->d_ids, tokens * 4, hipMemcpyDeviceToHost, model->stream));
        HIP_CHECK(hipMemcpyAsync(tok.data(), model->d_tok, tokens * 4, hipMemcpyDeviceToHost, model->stream));
        HIP_CHECK(hipStreamSynchronize(model->stream));
        for (size_t i = 0; i < tokens; ++i) pos_out[i] = tok[i] & 0xffffu;
    });
}

int jh_debug_encode(jh_model* model, uint32_t layers, float* x_out, size_t tokens) {
    return jh_guarded([&] {
        if (!model) throw jh_error(JH_ERR_INVALID, "null model");
        std::lock_guard<std::mutex> g(model->mu);
        model->bind();
        if (!model->staged || tokens != model->T) throw jh_error(JH_ERR_INVALID, "token count does not match the staged batch");
        if (layers > (uint32_t)model->nlayers) throw jh_error(JH_ERR_INVALID, "layer count out of range");
        if (!tokens) return;
        model->run_encoder((int)layers);
        HIP_CHECK(hipMemcpyAsync(x_out, model->x.p, tokens * model->h * 4, hipMemcpyDeviceToHost, model->stream));
        HIP_CHECK(hipStreamSynchronize(model->stream));
    });
}

}  // extern "C"
