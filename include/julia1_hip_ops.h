/*
 * julia1_hip_ops.h — the individual gfx950 kernels of the encoder forward,
 * callable on caller-owned device memory.
 *
 * These are the launch wrappers jh_forward uses, exported so each kernel can
 * be parity-tested and timed on its own (the GEMM sweep runs through
 * jh_op_gemm).  All pointers are device pointers; `stream` is a hipStream_t
 * (NULL = the null stream).  Calls enqueue work and return; they do not
 * synchronise.  Shape errors return JH_ERR_INVALID before anything is
 * launched.  Element types: f32 = float, bf16 = uint16_t bit patterns.
 *
 * Each entry point names the reference kernel or library call it stands in
 * for; the reference launches its own versions from src/cuda/mod.rs:400-521.
 */
#ifndef JULIA1_HIP_OPS_H
#define JULIA1_HIP_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Epilogues of jh_op_gemm: what happens to each FP32 accumulator tile of out = X · Wᵀ. */
enum {
    JH_EPI_STORE_BF16 = 0,      /* out bf16 = acc                                         */
    JH_EPI_ROPE_BF16 = 1,       /* out bf16 = acc, rotate-half RoPE applied to the columns  */
                                /*   below rope_cols (q and k of a packed qkv row)          */
    JH_EPI_GEGLU_BF16 = 2,      /* W rows interleaved per 32 (see jh_op_interleave_geglu):  */
                                /*   out[:, n/2] bf16 = gelu(gate) * up                     */
    JH_EPI_RESID_F32 = 3,       /* out f32 += acc (+ bias if given)                         */
    JH_EPI_BIAS_BF16 = 4,       /* out bf16 = acc + bias                                    */
    JH_EPI_BIAS_RELU_BF16 = 5,  /* out bf16 = max(acc + bias, 0)                            */
    JH_EPI_BIAS_F32 = 6         /* out f32 = acc + bias                                     */
};

/*
 * out[r, col + n] = epi( Σ_k X[row(r), k] · W[n, k] ) for r < rows, n < N.
 *  X bf16 with row stride ldx; row(r) = gather ? gather[r] : r.
 *  W bf16 [N, K] row-major (PyTorch Linear layout).
 *  out has row stride ldo (elements), written from column `col`.
 *  bias f32 [N] (NULL allowed for RESID_F32).
 *  ROPE: pos[r] is the row's position; cos/sin are [positions, 32] f32 tables;
 *        columns < rope_cols are rotated per 64-wide head.
 * Requirements: K % 64 == 0, N % 64 == 0, K <= 8192; x, w and out 16-byte aligned,
 * and out's rows and column `col` on 16-byte boundaries.  Replaces cuBLAS gemm_ex
 * (src/cuda/mod.rs:347-375) plus the separate geglu/bias_act kernels
 * (src/cuda/kernels.cu:137-172) and the residual add of ln_bf16 (:97-109).
 */
int jh_op_gemm(int epilogue, const void* x, size_t ldx, const int32_t* gather, size_t rows,
               const void* w, size_t n, size_t k, void* out, size_t ldo, size_t col,
               const float* bias, const int32_t* pos, const float* cos_t, const float* sin_t,
               size_t rope_cols, void* stream);

/*
 * jh_op_gemm with split-K: K is cut into `splits` chunks (0 = chosen from the
 * tile count, as the backend does for small batches) whose FP32 partial sums
 * go to `workspace` (splits · rows · N floats must fit `workspace_bytes`;
 * fewer splits are used otherwise), then one more kernel sums them in chunk
 * order and applies the epilogue.  Deterministic.  Same requirements as
 * jh_op_gemm.  No reference counterpart (cuBLAS chooses its own split-K).
 */
int jh_op_gemm_splitk(int epilogue, const void* x, size_t ldx, const int32_t* gather, size_t rows,
                      const void* w, size_t n, size_t k, void* out, size_t ldo, size_t col,
                      const float* bias, const int32_t* pos, const float* cos_t, const float* sin_t,
                      size_t rope_cols, void* workspace, size_t workspace_bytes, int splits, void* stream);

/*
 * jh_op_gemm_splitk without the workspace argument: the FP32 partial sums live
 * in a fixed 16 MiB device array inside the library (one per GPU, held until
 * the process ends), so the call allocates nothing (no hipMalloc, hipFree or
 * allocating library call).  For callers that cannot allocate: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * `splits` as jh_op_gemm_splitk: 0 picks the split count that fits the array,
 * a forced count whose partials (splits x rows x N floats) exceed 16 MiB is
 * rejected with JH_ERR_INVALID.  Calls that overlap on one GPU (two streams,
 * or two threads) share the array and race; serialise them.  Results equal
 * jh_op_gemm_splitk's with the same split count.  No reference counterpart.
 */
int jh_op_gemm_splitk_noalloc(int epilogue, const void* x, size_t ldx, const int32_t* gather,
                              size_t rows, const void* w, size_t n, size_t k, void* out, size_t ldo,
                              size_t col, const float* bias, const int32_t* pos, const float* cos_t,
                              const float* sin_t, size_t rope_cols, int splits, void* stream);

/*
 * jh_op_gemm whose X operand is bf16(LayerNorm(xf[r]; ln_w, ln_b, eps)), the
 * normalisation computed in the small-batch kernel's prologue exactly as
 * jh_op_layer_norm computes it (the same bits).  xf f32 [rows, k] with row
 * stride ldx floats (ldx % 4 == 0, 16-byte aligned); ln_w f32 [k], ln_b f32 [k]
 * or NULL.  k = hidden in {128, 256, 384, 512, 768}; epilogues STORE_BF16,
 * ROPE_BF16 and GEGLU_BF16; one workgroup per 64 x 32 output tile, so it is
 * meant for the few-token batches the backend runs on the small-batch kernel.
 * Replaces ln_bf16 (src/cuda/kernels.cu:97-109) followed by cuBLAS gemm_ex
 * (src/cuda/mod.rs:347-375) for those batches.
 */
int jh_op_gemm_ln(int epilogue, const float* xf, size_t ldx, size_t rows, const void* w, size_t n,
                  size_t k, void* out, size_t ldo, size_t col, const int32_t* pos, const float* cos_t,
                  const float* sin_t, size_t rope_cols, const float* ln_w, const float* ln_b, float eps,
                  void* stream);

/*
 * jh_op_gemm on the weight-stationary kernel: each workgroup (one per CU)
 * keeps a slab of W resident (registers and LDS) and streams 16-token blocks
 * of X through LDS, so only X moves from L2 during the multiply.  w_packed
 * is W (as jh_op_gemm takes it, [n, k] bf16; the GEGLU interleave for Wi) in
 * the fragment order jh_op_pack_ws writes.  Shapes: K == 768 with N % 256 ==
 * 0 (256-row slabs, every epilogue), or K == 1152 with N % 128 == 0 and
 * JH_EPI_RESID_F32 only (128-row slabs, K split between partner waves whose
 * two half sums are added lower half first); no row gather.  Other arguments
 * as jh_op_gemm.  The same bf16 products as jh_op_gemm, summed in FP32 in K
 * order in steps of 32 (jh_op_gemm: 16), so outputs agree to FP32 rounding.
 * jh_forward uses it for the K = 768 GEMMs and the MLP-out projection
 * (K = intermediate = 1152) outside the small-batch path.  Replaces cuBLAS
 * gemm_ex (src/cuda/mod.rs:347-375) for those shapes.
 */
int jh_op_gemm_ws(int epilogue, const void* x, size_t ldx, size_t rows, const void* w_packed, size_t n,
                  size_t k, void* out, size_t ldo, size_t col, const float* bias, const int32_t* pos,
                  const float* cos_t, const float* sin_t, size_t rope_cols, void* stream);

/*
 * Host: reorder a bf16 W [n, k] (row-major) into jh_op_gemm_ws's fragment
 * order (n*k elements; k % 32 == 0 and n % 256 == 0, or n % 128 == 0 at
 * k == 1152, whose layout is the K-split kernel's).  No reference counterpart
 * (a one-time weight layout, as the reference's BF16 conversion at upload,
 * src/cuda/mod.rs:36-39).
 */
int jh_op_pack_ws(const void* w, size_t n, size_t k, void* out);

/* Reorder a host FP32 Wi [2*inter, k] into the gate/up interleave JH_EPI_GEGLU_BF16 expects. */
void jh_op_interleave_geglu(const float* wi, size_t inter, size_t k, float* out);

/*
 * x[t] = LayerNorm(table[ids[t]]; w, no bias, eps) (f32), xn[t] = bf16(x[t]).
 * table f32 [vocab, hidden].  Replaces embed_ln (src/cuda/kernels.cu:66-75).
 */
int jh_op_embed_ln(const uint32_t* ids, size_t rows, const float* table, const float* w,
                   float eps, size_t hidden, float* x, void* xn, void* stream);

/*
 * out[r] = bf16(LayerNorm(x[r]; w, b, eps)), b may be NULL.
 * Replaces ln_bf16 (src/cuda/kernels.cu:97-109) without its residual add,
 * which the producing GEMM's RESID_F32 epilogue performs instead.
 */
int jh_op_layer_norm(const float* x, size_t rows, const float* w, const float* b, float eps,
                     size_t hidden, void* out, void* stream);

/*
 * Encoder final norm fused with the question-type embedding and the first
 * head layer's norm1: x[t] = LN(x[t]; fw, eps) + type_emb[qtype(t)];
 * out[t] = bf16(LN(x[t]; hw, hb, 1e-5)).  tok_meta[t] packs the token's
 * position (bits 0..15) and its sequence's qtype (bits 16..23).
 * Replaces final_norm (src/cuda/kernels.cu:113-132).
 */
int jh_op_final_norm(float* x, size_t rows, const float* fw, const float* type_emb,
                     const uint32_t* tok_meta, const float* hw, const float* hb, float eps,
                     size_t hidden, void* out, void* stream);

/*
 * dst[r] = src[idx[r]] for f32 rows of `hidden`.  Replaces gather_rows
 * (src/cuda/kernels.cu:175-183) for the FP32 residual; bf16 marker gathers
 * are folded into jh_op_gemm's `gather` argument instead.
 */
int jh_op_gather_f32(const float* src, const int32_t* idx, size_t rows, size_t hidden,
                     float* dst, void* stream);

/*
 * score[r] = Σ_i gelu(z[r, i]) · w2[i] + b2 (z already includes scorer.1's bias).
 * Replaces scorer (src/cuda/kernels.cu:186-194).
 */
int jh_op_scorer(const float* z, size_t rows, size_t hidden, const float* w2, float b2,
                 float* out, void* stream);

/*
 * Attention work item: `nq` query rows starting at absolute row `q_row` attend
 * to `kv_len` key/value rows starting at `kv_row`; the first query sits at
 * sequence position `q_pos` (keys are at positions 0..kv_len-1), which is what
 * the sliding window measures against.  nq <= 128.
 */
typedef struct jh_attn_tile {
    int32_t q_row, nq, kv_row, kv_len, q_pos;
} jh_attn_tile;

/*
 * FlashAttention-2 forward, one workgroup per (tile, head): MFMA QKᵀ and PV,
 * K/Vᵀ staged in LDS, online softmax of scale·QKᵀ over keys with
 * |q_pos - k_pos| <= window (window < 0: all keys of the sequence).
 * q/k/v bf16 with row strides ldq/ldkv; head h reads columns [64h, 64h+64)
 * of each; out bf16 row stride ldo.  `tiles` is a device array; work items
 * are dispatched in list order with heads varying fastest, so listing the
 * costliest tiles first (as the backend does) balances the CUs.
 * Replaces attention_rope/attention_plain (src/cuda/kernels.cu:274-391); RoPE
 * is applied by the producing GEMM's ROPE epilogue instead of on every load.
 */
int jh_op_attention(const void* q, size_t ldq, const void* k, const void* v, size_t ldkv,
                    void* out, size_t ldo, const jh_attn_tile* tiles, size_t ntiles,
                    size_t heads, int window, float scale, void* stream);

/*
 * jh_op_attention with work items of up to 256 queries (tiles of nq <= 256):
 * eight waves per (tile, head), each staged K/V tile shared by twice the
 * queries.  The backend uses it for the global layers of sequences of 4096
 * tokens or more.  Same arithmetic per query as jh_op_attention.  No separate
 * counterpart in the reference (part of attention_rope/attention_plain,
 * src/cuda/kernels.cu:274-391).
 */
int jh_op_attention_wide(const void* q, size_t ldq, const void* k, const void* v, size_t ldkv,
                         void* out, size_t ldo, const jh_attn_tile* tiles, size_t ntiles,
                         size_t heads, int window, float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* JULIA1_HIP_OPS_H */
