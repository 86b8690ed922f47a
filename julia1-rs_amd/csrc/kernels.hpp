// Launch wrappers of the gfx950 kernels (implemented in gemm.hip, attention.hip,
// norm.hip).  Each checks the shapes its kernel assumes and throws jh_error
// before launching anything that could read or write out of bounds.
#pragma once

#include <hip/hip_ext.h>

#include "common.hpp"

// Profiling hook: when a launch wrapper runs with a non-null jh_launch_events,
// its kernel is dispatched with hipExtLaunchKernelGGL so the runtime stamps
// the start/stop events at the dispatch itself (the same interval rocprofv3
// reports), instead of separate event packets around it.
struct LaunchEvents {
    hipEvent_t start, stop;
};
inline thread_local const LaunchEvents* jh_launch_events = nullptr;

#define JH_LAUNCH(kernel, grid, block, shm, stream, ...)                                                          \
    do {                                                                                                          \
        if (jh_launch_events)                                                                                     \
            hipExtLaunchKernelGGL(kernel, grid, block, shm, stream, jh_launch_events->start,                      \
                                  jh_launch_events->stop, 0, __VA_ARGS__);                                        \
        else                                                                                                      \
            hipLaunchKernelGGL(kernel, grid, block, shm, stream, __VA_ARGS__);                                    \
    } while (0)

struct GemmArgs {
    const bf16_t* x;        // activations, row stride ldx (elements)
    long ldx;
    const int32_t* gather;  // optional row indirection for x
    int rows;
    const bf16_t* w;        // [n, k] row-major
    int n, k;
    void* out;              // row stride ldo (elements), starting at column col
    long ldo;
    int col;
    const float* bias;      // [n] or null
    const int32_t* pos;     // ROPE: position in the low 16 bits of pos[row]
    const float* cos_t;     // ROPE: [positions, 32]
    const float* sin_t;
    int rope_cols;          // ROPE: columns [0, rope_cols) are rotated
    // Split-K (optional): a device workspace for FP32 partial sums.  When the
    // output has too few tiles to fill the GPU, launch_gemm splits K into
    // chunks written to `partial` and reduces them, in a fixed order, in a
    // second kernel that applies the epilogue.  `splits` > 0 forces that many
    // chunks (tests); 0 chooses automatically; null `partial` disables it.
    float* partial = nullptr;
    size_t partial_bytes = 0;
    int splits = 0;
    // set by launch_gemm for the split-K partial pass
    int kt_chunk = 0;
    // LayerNorm prologue (one-launch small-batch kernel only): when xf is set,
    // x is unused and the X operand is bf16(LN(xf row)) over K = hidden
    // features, computed as layer_norm_kernel does; xf rows have stride ldx
    // floats.  ln_b may be null.
    const float* xf = nullptr;
    const float* ln_w = nullptr;
    const float* ln_b = nullptr;
    float ln_eps = 0.0f;
    // set by launch_gemm for the eight-wave kernel: rows [0, mix_rows) in
    // full-height token tiles, the rest in tiles 32 tokens shorter (0: all full)
    int mix_rows = 0;
    // W pre-packed for the weight-stationary kernel (pack_ws), or null
    const bf16_t* w_ws = nullptr;
};

void launch_gemm(int epilogue, const GemmArgs& a, hipStream_t stream);
// Split count launch_gemm would use for `a` (1 = no split-K), and the split-K
// partial pass alone (FP32 partials [splits][rows][n] into a.partial), for
// callers that fuse the reduction with what follows (launch_resid_reduce_ln).
int gemm_splitk_count(int epilogue, const GemmArgs& a);
// Whether launch_gemm runs `a` as one launch of the small-batch kernel (the
// only kernel with the LayerNorm prologue); false for rows == 0.
bool gemm_uses_small(int epilogue, const GemmArgs& a);
void launch_gemm_partial(int epilogue, const GemmArgs& a, int splits, hipStream_t stream);
// Weight-stationary kernel (gemm_ws.hip): K = 768, N % 256 == 0, a.w_ws set,
// no gather or LayerNorm prologue.  gemm_ws_ranges is the number of token
// ranges each 256-row slab is split into (one workgroup per CU).
bool gemm_ws_supported(int epilogue, const GemmArgs& a);
// The shape, alignment and argument checks of launch_gemm (throws jh_error);
// false when there is nothing to do (rows == 0).
bool validate_gemm_args(int epilogue, const GemmArgs& a);
int gemm_ws_ranges(const GemmArgs& a);
int gemm_ws_block_tokens();
void launch_gemm_ws(int epilogue, const GemmArgs& a, hipStream_t stream);
void pack_ws(const bf16_t* w, int n, int k, bf16_t* out);

struct AttnTile {
    int32_t q_row, nq, kv_row, kv_len, q_pos;
};

struct AttnArgs {
    const bf16_t* q;
    long ldq;
    const bf16_t* k;
    const bf16_t* v;
    long ldkv;
    bf16_t* out;
    long ldo;
    const AttnTile* tiles;
    int ntiles;
    int heads;
    int window;        // < 0: global
    float scale_log2;  // softmax scale · log2(e)
    int waves = 4;     // waves per work item: 4 (tiles of <= 128 queries) or 8 (<= 256 queries)
};

void launch_attention(const AttnArgs& a, hipStream_t stream);

void launch_embed_ln(const uint32_t* ids, int rows, const float* table, const float* w, float eps, int hidden,
                     float* x, bf16_t* xn, hipStream_t stream);
void launch_layer_norm(const float* x, int rows, const float* w, const float* b, float eps, int hidden, bf16_t* out,
                       hipStream_t stream);
void launch_resid_reduce_ln(const float* partial, int splits, int rows, int hidden, const float* bias, float* x,
                            const float* w, const float* b, float eps, bf16_t* out, hipStream_t stream);
void launch_final_norm(float* x, int rows, const float* fw, const float* type_emb, const uint32_t* tok_meta,
                       const float* hw, const float* hb, float eps, int hidden, bf16_t* out, hipStream_t stream);
void launch_gather_f32(const float* src, const int32_t* idx, int rows, int hidden, float* dst, hipStream_t stream);
void launch_scorer(const float* z, int rows, int hidden, const float* w2, float b2, float* out, hipStream_t stream);
