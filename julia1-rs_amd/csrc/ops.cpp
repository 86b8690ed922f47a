// extern "C" op-level entry points of julia1_hip_ops.h: thin guards around the
// launch wrappers, for kernel parity tests and the isolated GEMM sweep.
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/julia1_hip_ops.h"
#include "abi_util.hpp"
#include "kernels.hpp"

namespace {
inline int as_int(size_t v, const char* what) {
    if (v > (size_t)0x7fffffff) throw jh_error(JH_ERR_INVALID, std::string(what) + " too large");
    return (int)v;
}
}  // namespace

extern "C" {

int jh_op_gemm(int epilogue, const void* x, size_t ldx, const int32_t* gather, size_t rows, const void* w, size_t n,
               size_t k, void* out, size_t ldo, size_t col, const float* bias, const int32_t* pos,
               const float* cos_t, const float* sin_t, size_t rope_cols, void* stream) {
    return jh_guarded([&] {
        GemmArgs a{(const bf16_t*)x, (long)ldx, gather, as_int(rows, "rows"), (const bf16_t*)w, as_int(n, "n"),
                   as_int(k, "k"), out, (long)ldo, as_int(col, "col"), bias, pos, cos_t, sin_t,
                   as_int(rope_cols, "rope_cols")};
        launch_gemm(epilogue, a, (hipStream_t)stream);
    });
}

int jh_op_gemm_splitk(int epilogue, const void* x, size_t ldx, const int32_t* gather, size_t rows, const void* w,
                      size_t n, size_t k, void* out, size_t ldo, size_t col, const float* bias, const int32_t* pos,
                      const float* cos_t, const float* sin_t, size_t rope_cols, void* workspace,
                      size_t workspace_bytes, int splits, void* stream) {
    return jh_guarded([&] {
        if (!workspace || ((uintptr_t)workspace & 15)) throw jh_error(1, "gemm: split-K needs a 16-byte aligned workspace");
        GemmArgs a{(const bf16_t*)x, (long)ldx, gather, as_int(rows, "rows"), (const bf16_t*)w, as_int(n, "n"),
                   as_int(k, "k"), out, (long)ldo, as_int(col, "col"), bias, pos, cos_t, sin_t,
                   as_int(rope_cols, "rope_cols")};
        a.partial = (float*)workspace;
        a.partial_bytes = workspace_bytes;
        a.splits = splits;
        launch_gemm(epilogue, a, (hipStream_t)stream);
    });
}

int jh_op_gemm_ln(int epilogue, const float* xf, size_t ldx, size_t rows, const void* w, size_t n, size_t k,
                  void* out, size_t ldo, size_t col, const int32_t* pos, const float* cos_t, const float* sin_t,
                  size_t rope_cols, const float* ln_w, const float* ln_b, float eps, void* stream) {
    return jh_guarded([&] {
        if (!xf) throw jh_error(1, "gemm: null operand");
        GemmArgs a{nullptr, (long)ldx, nullptr, as_int(rows, "rows"), (const bf16_t*)w, as_int(n, "n"),
                   as_int(k, "k"), out, (long)ldo, as_int(col, "col"), nullptr, pos, cos_t, sin_t,
                   as_int(rope_cols, "rope_cols")};
        a.xf = xf;
        a.ln_w = ln_w;
        a.ln_b = ln_b;
        a.ln_eps = eps;
        launch_gemm(epilogue, a, (hipStream_t)stream);
    });
}

int jh_op_gemm_ws(int epilogue, const void* x, size_t ldx, size_t rows, const void* w_packed, size_t n, size_t k,
                  void* out, size_t ldo, size_t col, const float* bias, const int32_t* pos, const float* cos_t,
                  const float* sin_t, size_t rope_cols, void* stream) {
    return jh_guarded([&] {
        GemmArgs a{(const bf16_t*)x, (long)ldx, nullptr, as_int(rows, "rows"), (const bf16_t*)w_packed,
                   as_int(n, "n"), as_int(k, "k"), out, (long)ldo, as_int(col, "col"), bias, pos, cos_t, sin_t,
                   as_int(rope_cols, "rope_cols")};
        a.w_ws = (const bf16_t*)w_packed;
        if (!gemm_ws_supported(epilogue, a))
            throw jh_error(1, "gemm: weight-stationary kernel needs packed W and K = 768 with N % 256 == 0, or K = "
                              "1152 with N % 128 == 0 and the residual epilogue");
        if (!validate_gemm_args(epilogue, a)) return;
        launch_gemm_ws(epilogue, a, (hipStream_t)stream);
    });
}

int jh_op_pack_ws(const void* w, size_t n, size_t k, void* out) {
    return jh_guarded([&] {
        if (!w || !out) throw jh_error(1, "pack_ws: null pointer");
        if (n == 0 || k == 0 || k % 32 || n * k > ((size_t)1 << 31) || n % (k == 1152 ? 128 : 256))
            throw jh_error(1, "pack_ws: need K % 32 == 0 and N % 256 == 0 (N % 128 == 0 at K = 1152)");
        pack_ws((const bf16_t*)w, (int)n, (int)k, (bf16_t*)out);
    });
}

// Gate/up interleave for the GEGLU epilogue (also used by jh_create): 64-row
// block j holds gate rows [32j, 32j+32) then up rows [inter+32j, inter+32j+32).
void jh_op_interleave_geglu(const float* wi, size_t inter, size_t k, float* out) {
    for (size_t j = 0; j < inter / 32; ++j)
        for (size_t r = 0; r < 32; ++r) {
            std::memcpy(out + (64 * j + r) * k, wi + (32 * j + r) * k, k * sizeof(float));
            std::memcpy(out + (64 * j + 32 + r) * k, wi + (inter + 32 * j + r) * k, k * sizeof(float));
        }
}

int jh_op_embed_ln(const uint32_t* ids, size_t rows, const float* table, const float* w, float eps, size_t hidden,
                   float* x, void* xn, void* stream) {
    return jh_guarded([&] {
        launch_embed_ln(ids, as_int(rows, "rows"), table, w, eps, as_int(hidden, "hidden"), x, (bf16_t*)xn,
                        (hipStream_t)stream);
    });
}

int jh_op_layer_norm(const float* x, size_t rows, const float* w, const float* b, float eps, size_t hidden, void* out,
                     void* stream) {
    return jh_guarded([&] {
        launch_layer_norm(x, as_int(rows, "rows"), w, b, eps, as_int(hidden, "hidden"), (bf16_t*)out,
                          (hipStream_t)stream);
    });
}

int jh_op_final_norm(float* x, size_t rows, const float* fw, const float* type_emb, const uint32_t* tok_meta,
                     const float* hw, const float* hb, float eps, size_t hidden, void* out, void* stream) {
    return jh_guarded([&] {
        launch_final_norm(x, as_int(rows, "rows"), fw, type_emb, tok_meta, hw, hb, eps, as_int(hidden, "hidden"),
                          (bf16_t*)out, (hipStream_t)stream);
    });
}

int jh_op_gather_f32(const float* src, const int32_t* idx, size_t rows, size_t hidden, float* dst, void* stream) {
    return jh_guarded([&] {
        launch_gather_f32(src, idx, as_int(rows, "rows"), as_int(hidden, "hidden"), dst, (hipStream_t)stream);
    });
}

int jh_op_scorer(const float* z, size_t rows, size_t hidden, const float* w2, float b2, float* out, void* stream) {
    return jh_guarded([&] {
        launch_scorer(z, as_int(rows, "rows"), as_int(hidden, "hidden"), w2, b2, out, (hipStream_t)stream);
    });
}

int jh_op_attention(const void* q, size_t ldq, const void* k, const void* v, size_t ldkv, void* out, size_t ldo,
                    const jh_attn_tile* tiles, size_t ntiles, size_t heads, int window, float scale, void* stream) {
    return jh_guarded([&] {
        static_assert(sizeof(jh_attn_tile) == sizeof(AttnTile), "tile layout");
        AttnArgs a{(const bf16_t*)q, (long)ldq, (const bf16_t*)k, (const bf16_t*)v, (long)ldkv, (bf16_t*)out,
                   (long)ldo, (const AttnTile*)tiles, as_int(ntiles, "ntiles"), as_int(heads, "heads"), window,
                   scale * 1.4426950408889634f};
        launch_attention(a, (hipStream_t)stream);
    });
}

int jh_op_attention_wide(const void* q, size_t ldq, const void* k, const void* v, size_t ldkv, void* out, size_t ldo,
                         const jh_attn_tile* tiles, size_t ntiles, size_t heads, int window, float scale,
                         void* stream) {
    return jh_guarded([&] {
        AttnArgs a{(const bf16_t*)q, (long)ldq, (const bf16_t*)k, (const bf16_t*)v, (long)ldkv, (bf16_t*)out,
                   (long)ldo, (const AttnTile*)tiles, as_int(ntiles, "ntiles"), as_int(heads, "heads"), window,
                   scale * 1.4426950408889634f, 8};
        launch_attention(a, (hipStream_t)stream);
    });
}

}  // extern "C"
