// julia1_oracle.cpp — FP32 CPU restatement of the reference's CPU forward.
//
// TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the timed CPU
// baseline for the HIP backend.  Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it, and only as the checker; the
// product library (libjulia1_hip.so) never links or calls it.
//
// What it restates (apiplant/julia1-rs, crate julia1 0.2.1):
//   src/cpu/fastmath.rs:8-49   exp (Cephes), erf (Eigen/XLA rational), gelu
//   src/cpu/gemm.rs:31-55      the five epilogues of `linear`
//   src/cpu/gemm.rs:171-249    linear / linear_geglu (8x32 register tile over all of K)
//   src/cpu/gemm.rs:292-313    the AVX-512 kernel's accumulation order (k-ordered FMA)
//   src/cpu/mod.rs:201-340     forward_packed: op order, head, marker-only last layer, scorer
//   src/cpu/mod.rs:343-360     rope_inplace (rotate-half, pairs (i, i+32))
//   src/cpu/mod.rs:435-576     attention_packed: 32-aligned key band, unscaled QKᵀ,
//                              softmax_range, PV over the whole band
//   src/cpu/mod.rs:579-653     softmax_range, 16-lane sum/max, two-pass layer_norm
//   src/config.rs:99-112       rope_table
// Rust does not contract a*b+c into an FMA; this file is compiled with
// -ffp-contract=off so every expression rounds as the Rust source does, and
// the explicit FMAs of the AVX-512 kernel are explicit here too (std::fma or
// _mm512_fmadd_ps, both single-rounding).  Results therefore do not depend on
// the thread count or on whether the AVX-512 or the scalar kernel runs.
//
// Parity pinning (tests/test_oracle.py): fastmath against libm; linear and
// geglu against f64 brute force (the reference's own unit tests); layer_norm
// against the f64 closed form; rope_table bit-exact against glibc;
// attention against f64 softmax(scale·QKᵀ)·V with window/varlen cases; the
// whole forward against an independent torch/transformers reconstruction
// (tests/golden); batching/permutation invariance.
#include "../include/julia1_hip.h"

#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <string>
#include <vector>

namespace {

// ------------------------------------------------------------ fastmath (fastmath.rs:8-49)
inline float f32_from_bits(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t f32_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

const float kRoundMagic = 12582912.0f;  // 1.5 * 2^23
const float kLog2E = 1.44269504088896340736f;
const float kFrac1Sqrt2 = 0.70710678118654752440f;

inline float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

inline float fm_exp(float x) {
    x = clampf(x, -87.3f, 88.3f);
    float shifted = x * kLog2E + kRoundMagic;
    float n = shifted - kRoundMagic;
    float r = x - n * 0.6933594f - n * -2.1219444e-4f;
    float y = 1.9875691e-4f;
    y = y * r + 1.3982e-3f;
    y = y * r + 8.333452e-3f;
    y = y * r + 4.1665796e-2f;
    y = y * r + 1.6666665e-1f;
    y = y * r + 5e-1f;
    y = y * r * r + r + 1.0f;
    uint32_t n_int = f32_bits(shifted) - f32_bits(kRoundMagic);
    float scale = f32_from_bits((n_int + 127u) << 23);
    return y * scale;
}

inline float fm_erf(float x) {
    x = clampf(x, -4.0f, 4.0f);
    float x2 = x * x;
    float p = -2.7261423e-10f;
    p = p * x2 + 2.7706814e-8f;
    p = p * x2 + -2.101024e-6f;
    p = p * x2 + -5.6925064e-5f;
    p = p * x2 + -7.3499063e-4f;
    p = p * x2 + -2.9546e-3f;
    p = p * x2 + -1.6096033e-2f;
    float q = -1.4566072e-5f;
    q = q * x2 + -2.1337406e-4f;
    q = q * x2 + -1.682827e-3f;
    q = q * x2 + -7.373329e-3f;
    q = q * x2 + -1.426474e-2f;
    return x * p / q;
}

inline float fm_gelu(float x) { return 0.5f * x * (1.0f + fm_erf(x * kFrac1Sqrt2)); }

// ------------------------------------------------------------ reductions (mod.rs:593-617)
float sum_f32(const float* x, size_t n) {
    float acc[16] = {0};
    size_t full = n / 16 * 16;
    for (size_t c = 0; c < full; c += 16)
        for (int i = 0; i < 16; ++i) acc[i] += x[c + i];
    float a = -0.0f;
    for (int i = 0; i < 16; ++i) a += acc[i];
    float r = -0.0f;
    for (size_t i = full; i < n; ++i) r += x[i];
    return a + r;
}

float max_f32(const float* x, size_t n) {
    float acc[16];
    for (int i = 0; i < 16; ++i) acc[i] = -std::numeric_limits<float>::infinity();
    size_t full = n / 16 * 16;
    for (size_t c = 0; c < full; c += 16)
        for (int i = 0; i < 16; ++i) acc[i] = std::fmax(acc[i], x[c + i]);
    float m = -std::numeric_limits<float>::infinity();
    for (int i = 0; i < 16; ++i) m = std::fmax(m, acc[i]);
    for (size_t i = full; i < n; ++i) m = std::fmax(m, x[i]);
    return m;
}

// Planted mistakes for the oracle's own mutation tests (0 = none).
int g_fault = 0;

// Two-pass LayerNorm (mod.rs:620-646).
void layer_norm(const float* x, size_t n, const float* w, const float* b, float eps, float* out) {
    float nf = (float)n;
    float mean = sum_f32(x, n) / nf;
    float acc[16] = {0};
    size_t full = n / 16 * 16;
    for (size_t c = 0; c < full; c += 16)
        for (int i = 0; i < 16; ++i) {
            float d = x[c + i] - mean;
            acc[i] += d * d;
        }
    float a = -0.0f;
    for (int i = 0; i < 16; ++i) a += acc[i];
    float r = -0.0f;
    for (size_t i = full; i < n; ++i) r += (x[i] - mean) * (x[i] - mean);
    float var = (a + r) / nf;
    if (g_fault == 5) var = a / nf;  // planted: drop the variance of the tail (only bites when n % 16 != 0)
    float rstd = 1.0f / std::sqrt(var + eps);
    if (b) {
        for (size_t i = 0; i < n; ++i) out[i] = (x[i] - mean) * rstd * w[i] + b[i];
    } else {
        for (size_t i = 0; i < n; ++i) out[i] = (x[i] - mean) * rstd * w[i];
    }
}

void rows_layer_norm(const float* x, size_t rows, size_t width, const float* w, const float* b, float eps, float* out) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)rows; ++r) layer_norm(x + r * width, width, w, b, eps, out + r * width);
}

// ------------------------------------------------------------ GEMM (gemm.rs)
constexpr int NR = 32;
constexpr int MR = 8;

enum Epi { EPI_STORE = 0, EPI_ADD = 1, EPI_BIAS = 2, EPI_BIAS_RELU = 3, EPI_ADD_BIAS = 4 };

// [n, k] row-major weight packed into 32-column panels [np][k][32], zero padded past n.
struct PackedW {
    std::vector<float> panels;
    size_t n = 0, k = 0;
    PackedW() = default;
    PackedW(const float* w, size_t n_, size_t k_) : n(n_), k(k_) {
        size_t np = (n + NR - 1) / NR;
        panels.assign(np * k * NR, 0.0f);
        for (size_t p = 0; p < np; ++p)
            for (size_t kk = 0; kk < k; ++kk)
                for (int j = 0; j < NR; ++j) {
                    size_t col = p * NR + j;
                    if (col < n) panels[(p * k + kk) * NR + j] = w[col * k + kk];
                }
    }
    const float* panel(size_t p) const { return panels.data() + p * k * NR; }
};

bool g_avx512 = false;

__attribute__((target("avx512f"))) void kernel_avx512(size_t k, const float* a, size_t lda, const float* b, float* tile) {
    __m512 acc[MR][2];
    for (int i = 0; i < MR; ++i) acc[i][0] = acc[i][1] = _mm512_setzero_ps();
    for (size_t kk = 0; kk < k; ++kk) {
        __m512 b0 = _mm512_loadu_ps(b + kk * NR);
        __m512 b1 = _mm512_loadu_ps(b + kk * NR + 16);
        for (int i = 0; i < MR; ++i) {
            __m512 av = _mm512_set1_ps(a[i * lda + kk]);
            acc[i][0] = _mm512_fmadd_ps(av, b0, acc[i][0]);
            acc[i][1] = _mm512_fmadd_ps(av, b1, acc[i][1]);
        }
    }
    for (int i = 0; i < MR; ++i) {
        _mm512_storeu_ps(tile + i * NR, acc[i][0]);
        _mm512_storeu_ps(tile + i * NR + 16, acc[i][1]);
    }
}

void kernel_scalar(size_t k, const float* a, size_t lda, const float* b, float* tile) {
    float acc[MR][NR];
    for (int i = 0; i < MR; ++i)
        for (int j = 0; j < NR; ++j) acc[i][j] = 0.0f;
    for (size_t kk = 0; kk < k; ++kk)
        for (int i = 0; i < MR; ++i) {
            float av = a[i * lda + kk];
            for (int j = 0; j < NR; ++j) acc[i][j] = std::fma(av, b[kk * NR + j], acc[i][j]);
        }
    for (int i = 0; i < MR; ++i)
        for (int j = 0; j < NR; ++j) tile[i * NR + j] = acc[i][j];
}

// tile[8x32] = A[8 x k] (row stride lda) · B[k x 32] (contiguous panel).
inline void tile8x32(size_t k, const float* a, size_t lda, const float* b, float* tile) {
    if (g_avx512) kernel_avx512(k, a, lda, b, tile);
    else kernel_scalar(k, a, lda, b, tile);
}

// tile for rows r..r+mr of x (dense, row stride k); short strips use a zero-padded copy.
inline void tile_product(const float* x, size_t k, size_t r, size_t mr, const float* b, float* tile, std::vector<float>& pad) {
    if (mr == MR) {
        tile8x32(k, x + r * k, k, b, tile);
    } else {
        pad.assign(MR * k, 0.0f);
        std::memcpy(pad.data(), x + r * k, mr * k * sizeof(float));
        tile8x32(k, pad.data(), k, b, tile);
    }
}

inline void apply_epi(int epi, const float* tile, float* out, size_t ncols, const float* bias, size_t col) {
    switch (epi) {
        case EPI_STORE: for (size_t j = 0; j < ncols; ++j) out[j] = tile[j]; break;
        case EPI_ADD: for (size_t j = 0; j < ncols; ++j) out[j] += tile[j]; break;
        case EPI_BIAS: for (size_t j = 0; j < ncols; ++j) out[j] = tile[j] + bias[col + j]; break;
        case EPI_BIAS_RELU: for (size_t j = 0; j < ncols; ++j) out[j] = std::fmax(tile[j] + bias[col + j], 0.0f); break;
        case EPI_ADD_BIAS: for (size_t j = 0; j < ncols; ++j) out[j] += tile[j] + bias[col + j]; break;
    }
}

// out[r, col..col+n] = epi(x[r, :k] · Wᵀ) (gemm.rs:171-206).  Work is split over
// (8-row strip, 32-col panel); each output element is produced by one task.
void linear(const float* x, size_t rows, const PackedW& w, float* out, size_t ldo, size_t col, int epi, const float* bias) {
    if (rows == 0) return;
    size_t np = (w.n + NR - 1) / NR;
    size_t strips = (rows + MR - 1) / MR;
    long tasks = (long)(strips * np);
#pragma omp parallel
    {
        float tile[MR * NR];
        std::vector<float> pad;
#pragma omp for schedule(static)
        for (long t = 0; t < tasks; ++t) {
            size_t s = t / np, p = t % np;
            size_t r = s * MR, mr = std::min<size_t>(MR, rows - r);
            size_t ncols = std::min<size_t>(NR, w.n - p * NR);
            tile_product(x, w.k, r, mr, w.panel(p), tile, pad);
            for (size_t i = 0; i < mr; ++i)
                apply_epi(epi, tile + i * NR, out + (r + i) * ldo + col + p * NR, ncols, bias, p * NR);
        }
    }
}

// g[r, :] = gelu(x·Wᵀ[:, :inter]) * (x·Wᵀ[:, inter:]) (gemm.rs:208-249).
void linear_geglu(const float* x, size_t rows, const PackedW& w, float* g) {
    size_t inter = w.n / 2;
    size_t half = inter / NR;
    size_t strips = (rows + MR - 1) / MR;
    long tasks = (long)(strips * half);
#pragma omp parallel
    {
        float a[MR * NR], b[MR * NR];
        std::vector<float> pad;
#pragma omp for schedule(static)
        for (long t = 0; t < tasks; ++t) {
            size_t s = t / half, p = t % half;
            size_t r = s * MR, mr = std::min<size_t>(MR, rows - r);
            tile_product(x, w.k, r, mr, w.panel(p), a, pad);
            tile_product(x, w.k, r, mr, w.panel(half + p), b, pad);
            for (size_t i = 0; i < mr; ++i) {
                float* dst = g + (r + i) * inter + p * NR;
                for (int j = 0; j < NR; ++j) dst[j] = fm_gelu(a[i * NR + j]) * b[i * NR + j];
            }
        }
    }
}

// ------------------------------------------------------------ attention (mod.rs:435-591)
struct AttnSeq { size_t q_row, nq, kv_row, len; };
constexpr size_t QBLOCK = 64;

void softmax_range(float* row, size_t nk, size_t lo, size_t hi, float scale) {
    for (size_t i = 0; i < lo; ++i) row[i] = 0.0f;
    for (size_t i = hi; i < nk; ++i) row[i] = 0.0f;
    float* r = row + lo;
    size_t n = hi - lo;
    float mx = max_f32(r, n);
    for (size_t i = 0; i < n; ++i) r[i] = fm_exp((r[i] - mx) * scale);
    float inv = 1.0f / sum_f32(r, n);
    for (size_t i = 0; i < n; ++i) r[i] *= inv;
}

// Scaled dot-product attention over packed sequences, one task per (sequence,
// head, 64-query block), in the arithmetic order of attention_packed: Kᵀ and V
// of every (sequence, head) are packed once (zero past len), the key band is
// widened to multiples of 32, S = QKᵀ is accumulated over the 64 head dims with
// FMA, softmax_range scales inside the exponent, and O = P·V runs over the whole
// widened band (zeros outside [lo, hi)).
void attention(const float* q, size_t ldq, size_t q_off, const float* kv, size_t ldkv, size_t k_off, size_t v_off,
               float* out, size_t ldo, const std::vector<AttnSeq>& seqs, size_t heads, long window, float scale) {
    const size_t HD = 64, P = 32;
    // Packed per (sequence, head): Kᵀ [64][npad] then V [npad][64], npad = len rounded up to 32.
    std::vector<size_t> base(seqs.size() * heads + 1, 0);
    for (size_t si = 0; si < seqs.size(); ++si)
        for (size_t h = 0; h < heads; ++h) {
            size_t npad = (seqs[si].len + P - 1) / P * P;
            base[si * heads + h + 1] = base[si * heads + h] + npad * HD * 2;
        }
    std::vector<float> kvp(base.back());
    long nsh = (long)(seqs.size() * heads);
#pragma omp parallel for schedule(dynamic, 1)
    for (long sh = 0; sh < nsh; ++sh) {
        const AttnSeq& s = seqs[sh / heads];
        size_t h = sh % heads, npad = (s.len + P - 1) / P * P;
        float* kt = kvp.data() + base[sh];
        float* vp = kt + npad * HD;
        for (size_t j = 0; j < npad; ++j) {
            const float* row = kv + (s.kv_row + j) * ldkv;
            for (size_t d = 0; d < HD; ++d) {
                kt[d * npad + j] = j < s.len ? row[k_off + h * HD + d] : 0.0f;
                vp[j * HD + d] = j < s.len ? row[v_off + h * HD + d] : 0.0f;
            }
        }
    }
    struct Task { size_t si, head, q0; };
    std::vector<Task> tasks;
    for (size_t si = 0; si < seqs.size(); ++si)
        for (size_t h = 0; h < heads; ++h)
            for (size_t q0 = 0; q0 < seqs[si].nq; q0 += QBLOCK) tasks.push_back({si, h, q0});
    long nt = (long)tasks.size();
#pragma omp parallel
    {
        std::vector<float> sc;
        float o[64];
#pragma omp for schedule(dynamic, 1)
        for (long ti = 0; ti < nt; ++ti) {
            const Task& t = tasks[ti];
            const AttnSeq& s = seqs[t.si];
            size_t npad = (s.len + P - 1) / P * P;
            const float* kt = kvp.data() + base[t.si * heads + t.head];
            const float* vp = kt + npad * HD;
            size_t q1 = std::min(t.q0 + QBLOCK, s.nq), nq = q1 - t.q0;
            size_t k0 = 0, k1 = s.len;
            if (window >= 0) {
                size_t w = (size_t)window;
                k0 = t.q0 > w ? t.q0 - w : 0;
                k1 = std::min(q1 + w, s.len);
            }
            size_t k0a = k0 / P * P, k1a = (k1 + P - 1) / P * P, nk = k1a - k0a;
            sc.assign(nq * nk, 0.0f);
            for (size_t i = 0; i < nq; ++i) {
                const float* qr = q + (s.q_row + t.q0 + i) * ldq + q_off + t.head * HD;
                float* row = sc.data() + i * nk;
                for (size_t d = 0; d < HD; ++d) {
                    float qd = qr[d];
                    const float* kr = kt + d * npad + k0a;
                    for (size_t c = 0; c < nk; ++c) row[c] = std::fma(qd, kr[c], row[c]);
                }
                size_t lo = 0, hi = s.len - k0a;
                if (window >= 0) {
                    size_t w = (size_t)window, qi = t.q0 + i;
                    if (g_fault == 3) w += 1;  // planted: window one wider
                    size_t a = qi > w ? qi - w : 0;
                    lo = std::max(a, k0a) - k0a;
                    hi = std::min(qi + w + 1, s.len) - k0a;
                }
                softmax_range(row, nk, lo, hi, scale);
            }
            for (size_t i = 0; i < nq; ++i) {
                const float* pr = sc.data() + i * nk;
                for (size_t j = 0; j < HD; ++j) o[j] = 0.0f;
                for (size_t c = 0; c < nk; ++c) {
                    float pc = pr[c];
                    const float* vr = vp + (k0a + c) * HD;
                    for (size_t j = 0; j < HD; ++j) o[j] = std::fma(pc, vr[j], o[j]);
                }
                float* orow = out + (s.q_row + t.q0 + i) * ldo + t.head * HD;
                for (size_t j = 0; j < HD; ++j) orow[j] = o[j];
            }
        }
    }
}

// ------------------------------------------------------------ rope (config.rs:99-112)
void rope_table(float theta, uint32_t head_dim, uint32_t positions, float* cos_out, float* sin_out) {
    uint32_t half = head_dim / 2;
    std::vector<float> inv(half);
    for (uint32_t i = 0; i < half; ++i) inv[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
    for (uint32_t p = 0; p < positions; ++p)
        for (uint32_t i = 0; i < half; ++i) {
            float f = inv[i] * (float)p;
            cos_out[(size_t)p * half + i] = cosf(f);
            sin_out[(size_t)p * half + i] = sinf(f);
        }
}

struct Layer {
    std::vector<float> attn_norm, mlp_norm;
    bool has_attn_norm = false;
    PackedW wqkv, wo, wi, wo2;
};

struct Head {
    std::vector<float> norm1_w, norm1_b, in_b, out_b, norm2_w, norm2_b, lin1_b, lin2_b;
    PackedW in_w, q_w, kv_w, out_w, lin1, lin2;
};

}  // namespace

struct jo_model {
    uint32_t h, heads, inter, nlayers, vocab, max_pos, head_heads, ff;
    uint32_t half_window;
    float eps;
    std::vector<uint8_t> global;
    std::vector<float> theta;
    std::vector<float> emb, emb_norm, final_norm, type_emb;
    std::vector<Layer> layers;
    std::vector<Head> head;
    std::vector<float> s_norm_w, s_norm_b, s_b1, s_w2;
    float s_b2;
    PackedW s_w1;
    std::vector<std::pair<float, std::pair<std::vector<float>, std::vector<float>>>> ropes;
    std::vector<int> rope_of_layer;
    int threads = 4;
    std::string err;
};

namespace {

std::vector<float> vec(const float* p, size_t n) { return std::vector<float>(p, p + n); }

// Embeddings + the first `upto` encoder layers (mod.rs:219-250) into x.
void encode_layers(jo_model* m, const uint32_t* ids, size_t t, const uint32_t* starts, const uint32_t* lens, size_t S,
                   uint32_t upto, std::vector<float>& x, std::vector<float>& xn, std::vector<float>& qkv,
                   std::vector<float>& ctx, std::vector<float>& g, std::vector<uint32_t>& pos) {
    const size_t h = m->h, inter = m->inter;
    x.assign(t * h, 0.0f);
    xn.assign(t * h, 0.0f);
    qkv.assign(t * 3 * h, 0.0f);
    ctx.assign(t * h, 0.0f);
    g.assign(t * inter, 0.0f);
    pos.clear();
    for (size_t s = 0; s < S; ++s)
        for (uint32_t i = 0; i < lens[s]; ++i) pos.push_back(i);
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)t; ++r)
        layer_norm(m->emb.data() + (size_t)ids[r] * h, h, m->emb_norm.data(), nullptr, m->eps, x.data() + r * h);
    std::vector<AttnSeq> seqs;
    for (size_t s = 0; s < S; ++s) seqs.push_back({starts[s], lens[s], starts[s], lens[s]});
    for (uint32_t l = 0; l < upto; ++l) {
        const Layer& L = m->layers[l];
        const float* normed = x.data();
        if (L.has_attn_norm) {
            rows_layer_norm(x.data(), t, h, L.attn_norm.data(), nullptr, m->eps, xn.data());
            normed = xn.data();
        }
        linear(normed, t, L.wqkv, qkv.data(), 3 * h, 0, EPI_STORE, nullptr);
        // rope_inplace (mod.rs:343-360)
        const auto& tab = m->ropes[m->rope_of_layer[l]].second;
        const float* cs = tab.first.data();
        const float* sn = tab.second.data();
#pragma omp parallel for schedule(static)
        for (long r = 0; r < (long)t; ++r) {
            float* row = qkv.data() + r * 3 * h;
            const float* c = cs + (size_t)pos[r] * 32;
            const float* s = sn + (size_t)pos[r] * 32;
            for (size_t hd = 0; hd < 2 * h; hd += 64) {
                float* lo = row + hd;
                float* hi = row + hd + 32;
                for (int i = 0; i < 32; ++i) {
                    float a = lo[i], b = hi[i];
                    lo[i] = a * c[i] - b * s[i];
                    hi[i] = g_fault == 2 ? b * c[i] - a * s[i] : b * c[i] + a * s[i];
                }
            }
        }
        long window = m->global[l] ? -1 : (long)m->half_window;
        attention(qkv.data(), 3 * h, 0, qkv.data(), 3 * h, h, 2 * h, ctx.data(), h, seqs, m->heads, window, 0.125f);
        linear(ctx.data(), t, L.wo, x.data(), h, 0, EPI_ADD, nullptr);
        rows_layer_norm(x.data(), t, h, L.mlp_norm.data(), nullptr, m->eps, xn.data());
        linear_geglu(xn.data(), t, L.wi, g.data());
        linear(g.data(), t, L.wo2, x.data(), h, 0, EPI_ADD, nullptr);
    }
}

}  // namespace

extern "C" {

int jo_create(const jh_config* c, const jh_weights* w, int threads, jo_model** out) {
    if (!c || !w || !out || c->head_dim != 64 || c->hidden % 64 || c->hidden > 1024 || c->hidden / 64 != c->heads ||
        c->head_layers < 1 || c->intermediate % 32)
        return JH_ERR_INVALID;
    g_avx512 = __builtin_cpu_supports("avx512f") && !getenv("JULIA_NO_AVX512");
    auto m = std::make_unique<jo_model>();
    size_t h = c->hidden, inter = c->intermediate, ff = c->head_ff;
    m->h = c->hidden; m->heads = c->heads; m->inter = c->intermediate; m->nlayers = c->layers;
    m->vocab = c->vocab; m->max_pos = c->max_positions; m->head_heads = c->head_heads; m->ff = c->head_ff;
    m->half_window = c->half_window; m->eps = c->norm_eps;
    m->threads = threads > 0 ? threads : 4;
    m->global.assign(c->global, c->global + c->layers);
    m->theta.assign(c->rope_theta, c->rope_theta + c->layers);
    m->emb = vec(w->embedding, (size_t)c->vocab * h);
    m->emb_norm = vec(w->emb_norm, h);
    m->final_norm = vec(w->final_norm, h);
    m->type_emb = vec(w->type_emb, 3 * h);
    for (uint32_t l = 0; l < c->layers; ++l) {
        const jh_encoder_layer& s = w->layers[l];
        Layer L;
        L.has_attn_norm = s.attn_norm != nullptr;
        if (L.has_attn_norm) L.attn_norm = vec(s.attn_norm, h);
        L.mlp_norm = vec(s.mlp_norm, h);
        L.wqkv = PackedW(s.wqkv, 3 * h, h);
        L.wo = PackedW(s.wo, h, h);
        L.wi = PackedW(s.wi, 2 * inter, h);
        L.wo2 = PackedW(s.wo2, h, inter);
        m->layers.push_back(std::move(L));
        float th = c->rope_theta[l];
        int found = -1;
        for (size_t i = 0; i < m->ropes.size(); ++i)
            if (m->ropes[i].first == th) found = (int)i;
        if (found < 0) {
            std::vector<float> cs((size_t)c->max_positions * 32), sn((size_t)c->max_positions * 32);
            rope_table(th, 64, c->max_positions, cs.data(), sn.data());
            m->ropes.push_back({th, {std::move(cs), std::move(sn)}});
            found = (int)m->ropes.size() - 1;
        }
        m->rope_of_layer.push_back(found);
    }
    for (uint32_t l = 0; l < c->head_layers; ++l) {
        const jh_head_layer& s = w->head[l];
        Head H;
        H.norm1_w = vec(s.norm1_w, h); H.norm1_b = vec(s.norm1_b, h);
        H.in_b = vec(s.in_b, 3 * h); H.out_b = vec(s.out_b, h);
        H.norm2_w = vec(s.norm2_w, h); H.norm2_b = vec(s.norm2_b, h);
        H.lin1_b = vec(s.lin1_b, ff); H.lin2_b = vec(s.lin2_b, h);
        H.in_w = PackedW(s.in_w, 3 * h, h);
        H.q_w = PackedW(s.in_w, h, h);
        H.kv_w = PackedW(s.in_w + h * h, 2 * h, h);
        H.out_w = PackedW(s.out_w, h, h);
        H.lin1 = PackedW(s.lin1_w, ff, h);
        H.lin2 = PackedW(s.lin2_w, h, ff);
        m->head.push_back(std::move(H));
    }
    m->s_norm_w = vec(w->scorer_norm_w, h);
    m->s_norm_b = vec(w->scorer_norm_b, h);
    m->s_w1 = PackedW(w->scorer_w1, h, h);
    m->s_b1 = vec(w->scorer_b1, h);
    m->s_w2 = vec(w->scorer_w2, h);
    m->s_b2 = w->scorer_b2;
    *out = m.release();
    return JH_OK;
}

void jo_destroy(jo_model* m) { delete m; }

int jo_avx512(void) { return __builtin_cpu_supports("avx512f") ? 1 : 0; }

void jo_set_threads(jo_model* m, int threads) { if (m && threads > 0) m->threads = threads; }

void jo_set_fault(int code) { g_fault = code; }

// Thread count of the op-level entry points (jo_linear, jo_attention, ...).
void jo_omp_threads(int n) { if (n > 0) omp_set_num_threads(n); }

static bool check_batch(jo_model* m, const uint32_t* ids, size_t t, const uint32_t* starts, const uint32_t* lens, size_t S,
                        const uint32_t* marker_rows, size_t M) {
    size_t next = 0;
    for (size_t s = 0; s < S; ++s) {
        if (starts[s] != next || lens[s] > m->max_pos) return false;
        next += lens[s];
    }
    if (next != t) return false;
    for (size_t i = 0; i < t; ++i)
        if (ids[i] >= m->vocab) return false;
    for (size_t i = 0; i < M; ++i)
        if (marker_rows[i] >= t) return false;
    return true;
}

// x after embeddings and the first `upto` encoder layers, [t, hidden].
int jo_encode(jo_model* m, const uint32_t* ids, size_t t, const uint32_t* starts, const uint32_t* lens, size_t S,
              uint32_t upto, float* x_out) {
    if (!check_batch(m, ids, t, starts, lens, S, nullptr, 0) || upto > m->nlayers) return JH_ERR_INVALID;
    omp_set_num_threads(m->threads);
    std::vector<float> x, xn, qkv, ctx, g;
    std::vector<uint32_t> pos;
    encode_layers(m, ids, t, starts, lens, S, upto, x, xn, qkv, ctx, g, pos);
    std::memcpy(x_out, x.data(), x.size() * sizeof(float));
    return JH_OK;
}

// Scores for every marker (forward_packed, mod.rs:201-340).  Marker rows must be
// grouped by sequence in order (as Batch::new builds them).
int jo_forward(jo_model* m, const uint32_t* ids, size_t t, const uint32_t* starts, const uint32_t* lens,
               const uint8_t* qtypes, size_t S, const uint32_t* marker_rows, size_t M, float* scores) {
    if (!check_batch(m, ids, t, starts, lens, S, marker_rows, M)) return JH_ERR_INVALID;
    for (size_t s = 0; s < S; ++s)
        if (qtypes[s] > 2) return JH_ERR_INVALID;
    omp_set_num_threads(m->threads);
    const size_t h = m->h, ff = m->ff;
    const float eps = m->eps;
    std::vector<float> x, xn, qkv, ctx, g;
    std::vector<uint32_t> pos;
    encode_layers(m, ids, t, starts, lens, S, m->nlayers, x, xn, qkv, ctx, g, pos);
    // Final norm + question-type embedding (mod.rs:252-270).
#pragma omp parallel for schedule(dynamic, 1)
    for (long s = 0; s < (long)S; ++s) {
        const float* te = m->type_emb.data() + (size_t)qtypes[s] * h;
        std::vector<float> tmp(h);
        for (size_t r = starts[s]; r < starts[s] + lens[s]; ++r) {
            float* row = x.data() + r * h;
            if (g_fault == 4) std::memcpy(tmp.data(), row, h * sizeof(float));  // planted: skip final norm
            else layer_norm(row, h, m->final_norm.data(), nullptr, eps, tmp.data());
            for (size_t i = 0; i < h; ++i) row[i] = g_fault == 1 ? tmp[i] : tmp[i] + te[i];  // 1: drop type_emb
        }
    }
    std::vector<AttnSeq> seqs;
    for (size_t s = 0; s < S; ++s) seqs.push_back({starts[s], lens[s], starts[s], lens[s]});
    size_t nh = m->head.size();
    std::vector<float> hbuf(t * ff);
    // Decision head: all but the last layer over every token (mod.rs:272-285).
    for (size_t l = 0; l + 1 < nh; ++l) {
        const Head& H = m->head[l];
        rows_layer_norm(x.data(), t, h, H.norm1_w.data(), H.norm1_b.data(), 1e-5f, xn.data());
        linear(xn.data(), t, H.in_w, qkv.data(), 3 * h, 0, EPI_BIAS, H.in_b.data());
        attention(qkv.data(), 3 * h, 0, qkv.data(), 3 * h, h, 2 * h, ctx.data(), h, seqs, m->head_heads, -1, 0.125f);
        linear(ctx.data(), t, H.out_w, x.data(), h, 0, EPI_ADD_BIAS, H.out_b.data());
        rows_layer_norm(x.data(), t, h, H.norm2_w.data(), H.norm2_b.data(), 1e-5f, xn.data());
        linear(xn.data(), t, H.lin1, hbuf.data(), ff, 0, EPI_BIAS_RELU, H.lin1_b.data());
        linear(hbuf.data(), t, H.lin2, x.data(), h, 0, EPI_ADD_BIAS, H.lin2_b.data());
    }
    // Marker rows; the last head layer only computes their queries/FFN (mod.rs:287-321).
    std::vector<float> y(M * h);
    for (size_t i = 0; i < M; ++i) std::memcpy(y.data() + i * h, x.data() + (size_t)marker_rows[i] * h, h * sizeof(float));
    {
        const Head& H = m->head[nh - 1];
        rows_layer_norm(x.data(), t, h, H.norm1_w.data(), H.norm1_b.data(), 1e-5f, xn.data());
        linear(xn.data(), t, H.kv_w, qkv.data(), 3 * h, h, EPI_BIAS, H.in_b.data() + h);
        std::vector<float> xm(M * h), qm(M * h), cm(M * h), yn(M * h), hm(M * ff);
        for (size_t i = 0; i < M; ++i) std::memcpy(xm.data() + i * h, xn.data() + (size_t)marker_rows[i] * h, h * sizeof(float));
        linear(xm.data(), M, H.q_w, qm.data(), h, 0, EPI_BIAS, H.in_b.data());
        // marker_starts: markers are grouped by sequence; sequence s owns the markers inside its rows.
        std::vector<AttnSeq> mseqs;
        size_t mi = 0;
        for (size_t s = 0; s < S; ++s) {
            size_t first = mi;
            while (mi < M && marker_rows[mi] >= starts[s] && marker_rows[mi] < starts[s] + lens[s]) ++mi;
            mseqs.push_back({first, mi - first, starts[s], lens[s]});
        }
        if (mi != M) return JH_ERR_INVALID;
        attention(qm.data(), h, 0, qkv.data(), 3 * h, h, 2 * h, cm.data(), h, mseqs, m->head_heads, -1, 0.125f);
        linear(cm.data(), M, H.out_w, y.data(), h, 0, EPI_ADD_BIAS, H.out_b.data());
        rows_layer_norm(y.data(), M, h, H.norm2_w.data(), H.norm2_b.data(), 1e-5f, yn.data());
        linear(yn.data(), M, H.lin1, hm.data(), ff, 0, EPI_BIAS_RELU, H.lin1_b.data());
        linear(hm.data(), M, H.lin2, y.data(), h, 0, EPI_ADD_BIAS, H.lin2_b.data());
    }
    // Scorer (mod.rs:323-339).
    std::vector<float> yn(M * h), z(M * h);
    rows_layer_norm(y.data(), M, h, m->s_norm_w.data(), m->s_norm_b.data(), 1e-5f, yn.data());
    linear(yn.data(), M, m->s_w1, z.data(), h, 0, EPI_BIAS, m->s_b1.data());
    for (size_t i = 0; i < M; ++i) {
        float acc = 0.0f;
        for (size_t j = 0; j < h; ++j) acc += fm_gelu(z[i * h + j]) * m->s_w2[j];
        scores[i] = acc + m->s_b2;
    }
    return JH_OK;
}

// ---- op-level entry points for the oracle's own tests and for kernel parity tests

void jo_exp(const float* x, size_t n, float* out) { for (size_t i = 0; i < n; ++i) out[i] = fm_exp(x[i]); }
void jo_erf(const float* x, size_t n, float* out) { for (size_t i = 0; i < n; ++i) out[i] = fm_erf(x[i]); }
void jo_gelu(const float* x, size_t n, float* out) { for (size_t i = 0; i < n; ++i) out[i] = fm_gelu(x[i]); }

void jo_layer_norm(const float* x, size_t rows, size_t width, const float* w, const float* b, float eps, float* out) {
    rows_layer_norm(x, rows, width, w, b, eps, out);
}

void jo_linear(const float* x, size_t rows, size_t k, const float* w, size_t n, float* out, size_t ldo, size_t col,
               int epi, const float* bias) {
    g_avx512 = __builtin_cpu_supports("avx512f") && !getenv("JULIA_NO_AVX512");
    PackedW pw(w, n, k);
    linear(x, rows, pw, out, ldo, col, epi, bias);
}

void jo_linear_geglu(const float* x, size_t rows, size_t k, const float* w, size_t n, float* g) {
    g_avx512 = __builtin_cpu_supports("avx512f") && !getenv("JULIA_NO_AVX512");
    PackedW pw(w, n, k);
    linear_geglu(x, rows, pw, g);
}

// seqs: [nseq][4] = {q_row, nq, kv_row, len}; window < 0 = global.
void jo_attention(const float* q, size_t ldq, size_t q_off, const float* kv, size_t ldkv, size_t k_off, size_t v_off,
                  float* out, size_t ldo, const uint32_t* seqs, size_t nseq, size_t heads, long window, float scale) {
    std::vector<AttnSeq> s;
    for (size_t i = 0; i < nseq; ++i) s.push_back({seqs[4 * i], seqs[4 * i + 1], seqs[4 * i + 2], seqs[4 * i + 3]});
    attention(q, ldq, q_off, kv, ldkv, k_off, v_off, out, ldo, s, heads, window, scale);
}

void jo_rope_table(float theta, uint32_t head_dim, uint32_t positions, float* cos_out, float* sin_out) {
    rope_table(theta, head_dim, positions, cos_out, sin_out);
}

}  // extern "C"
