/*
 * julia1_hip.h — C-ABI of the MI355X (gfx950) encoder-forward backend.
 *
 * This is the device backend that sits behind the reference runtime's
 * `enum Backend { Cpu, Cuda }` (apiplant/julia1-rs src/engine.rs:67-71) as a
 * third arm, `Backend::Hip`.  Every entry point below replaces one member of
 * `CudaModel` (src/cuda/mod.rs); the citation on each says which.
 *
 * Conventions
 *  - Plain C types only: pointers, sizes, fixed-width integers.  No C++
 *    exception crosses this boundary; a failing call returns a nonzero
 *    JH_ERR_* code and leaves a message for jh_last_error() on the calling
 *    thread (the reference returns anyhow::Result with a message).
 *  - Host inputs are borrowed for the duration of the call only.
 *  - A jh_model is thread safe: calls on one model are serialised by an
 *    internal mutex (the reference's workspace Mutex, src/cuda/mod.rs:161,415),
 *    and each entry point makes the model's device current first
 *    (src/cuda/mod.rs:414 binds the context per forward).
 */
#ifndef JULIA1_HIP_H
#define JULIA1_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    JH_OK = 0,
    JH_ERR_INVALID = 1,     /* bad argument, shape or unsupported configuration */
    JH_ERR_DEVICE = 2,      /* no such device, or a HIP runtime call failed      */
    JH_ERR_ALLOC = 3,       /* device or pinned-host allocation failed           */
    JH_ERR_NONFINITE = 4,   /* forward produced a NaN/inf score                  */
    JH_ERR_INTERNAL = 5
};

/*
 * Model configuration: the fields of `ModelConfig` (src/config.rs:6-24) that
 * the forward needs.  `global` and `rope_theta` point at `layers` entries.
 */
typedef struct jh_config {
    uint32_t hidden;         /* d_model; hidden / 64 == heads                    */
    uint32_t heads;
    uint32_t head_dim;       /* must be 64 (src/config.rs:60)                     */
    uint32_t intermediate;   /* GEGLU half width; Wi is [2*intermediate, hidden]  */
    uint32_t layers;
    const uint8_t* global;   /* [layers]: 1 = full attention, 0 = sliding window  */
    uint32_t half_window;    /* |i-j| <= half_window on local layers              */
    const float* rope_theta; /* [layers]: RoPE base per layer                     */
    float norm_eps;          /* encoder LayerNorm eps                            */
    uint32_t vocab;
    uint32_t max_positions;  /* RoPE table length; sequences may not exceed it   */
    uint32_t head_layers;    /* decision-head TransformerEncoderLayers (>= 1)     */
    uint32_t head_heads;     /* hidden / 64                                       */
    uint32_t head_ff;        /* 4 * hidden                                        */
} jh_config;

/* One ModernBERT encoder layer (src/model.rs:6-14); row-major [out, in] FP32. */
typedef struct jh_encoder_layer {
    const float* attn_norm;  /* [hidden], NULL for layer 0 (nn.Identity)          */
    const float* wqkv;       /* [3*hidden, hidden]                                 */
    const float* wo;         /* [hidden, hidden]                                   */
    const float* mlp_norm;   /* [hidden]                                           */
    const float* wi;         /* [2*intermediate, hidden]: rows [0,inter) = gate    */
    const float* wo2;        /* [hidden, intermediate]                             */
} jh_encoder_layer;

/* nn.TransformerEncoderLayer(norm_first, relu) (src/model.rs:16-30). */
typedef struct jh_head_layer {
    const float *norm1_w, *norm1_b;  /* [hidden]                                  */
    const float *in_w, *in_b;        /* [3*hidden, hidden], [3*hidden]             */
    const float *out_w, *out_b;      /* [hidden, hidden], [hidden]                 */
    const float *norm2_w, *norm2_b;  /* [hidden]                                  */
    const float *lin1_w, *lin1_b;    /* [head_ff, hidden], [head_ff]               */
    const float *lin2_w, *lin2_b;    /* [hidden, head_ff], [hidden]                */
} jh_head_layer;

/* All inference weights, borrowed FP32 host pointers (`HostWeights`, src/model.rs:42-50). */
typedef struct jh_weights {
    const float* embedding;          /* [vocab, hidden] tok_embeddings             */
    const float* emb_norm;           /* [hidden]                                   */
    const jh_encoder_layer* layers;  /* [config.layers]                            */
    const float* final_norm;         /* [hidden]                                   */
    const float* type_emb;           /* [3, hidden]                                */
    const jh_head_layer* head;       /* [config.head_layers]                       */
    const float *scorer_norm_w, *scorer_norm_b; /* scorer.0: [hidden]              */
    const float *scorer_w1, *scorer_b1;         /* scorer.1: [hidden,hidden],[hidden] */
    const float* scorer_w2;          /* scorer.3.weight: [hidden]                  */
    float scorer_b2;                 /* scorer.3.bias                              */
} jh_weights;

typedef struct jh_model jh_model;

/*
 * Build the backend on HIP device `ordinal`: convert matrices to BF16
 * (round-to-nearest-even, as half::bf16::from_f32), upload them once, keep
 * norms/biases/embedding FP32, and build one RoPE cos/sin table pair per
 * distinct theta with the same f32 arithmetic as `rope_table`.
 * Replaces `CudaModel::new` (src/cuda/mod.rs:174-276); unlike it, any hidden
 * size that is a multiple of 64 up to 1024 is accepted (384 and 768 are the
 * shapes in use).  Errors: JH_ERR_INVALID (shape), JH_ERR_DEVICE, JH_ERR_ALLOC.
 */
int jh_create(const jh_config* config, const jh_weights* weights, int ordinal, jh_model** out);

/*
 * One forward over a packed varlen batch (`Batch`, src/model.rs:114-124):
 * sequences are packed back to back without padding; sequence s occupies rows
 * [starts[s], starts[s]+lens[s]) of `ids`; `marker_rows` are absolute packed
 * rows, grouped by sequence.  Writes one score per marker into the caller's
 * `scores[M]` and returns after the device-to-host copy has completed.
 * Replaces `CudaModel::forward` (src/cuda/mod.rs:400-521); the caller splits
 * scores per sequence by its marker_starts (src/model.rs:154-156).
 * Errors: JH_ERR_INVALID (ids >= vocab, lens > max_positions, rows out of range,
 * sequences overlapping or out of order), JH_ERR_DEVICE, JH_ERR_ALLOC.
 */
int jh_forward(jh_model* model, const uint32_t* ids, size_t tokens, const uint32_t* starts,
               const uint32_t* lens, const uint8_t* qtypes, size_t sequences,
               const uint32_t* marker_rows, size_t markers, float* scores);

/*
 * Padded-batch form of jh_forward for callers holding a [batch, padded_len]
 * id matrix: row b is real for its first lens[b] ids, the rest is padding
 * that never reaches the device.  markers are positions within the row,
 * grouped by row via marker_starts[batch+1].  The result equals jh_forward on
 * the packed batch.  No reference counterpart (the reference only packs).
 */
int jh_forward_padded(jh_model* model, const uint32_t* ids, size_t batch, size_t padded_len,
                      const uint32_t* lens, const uint8_t* qtypes, const uint32_t* markers,
                      const uint32_t* marker_starts, float* scores);

/*
 * Split form of jh_forward, for callers that time or overlap the forward:
 *  jh_stage   validates the batch and enqueues its upload on the model's stream
 *             (waiting first for its previous upload from the same pinned
 *             staging buffer);
 *  jh_execute enqueues the whole forward on the model's stream, reading the
 *             staged batch (repeatable; does not synchronise);
 *  jh_scores  waits for the stream and copies the M scores to the host.
 * jh_forward == jh_stage + jh_execute + jh_scores.  jh_stream returns the
 * model's hipStream_t (as void*) for event timing.  No reference counterpart.
 */
int jh_stage(jh_model* model, const uint32_t* ids, size_t tokens, const uint32_t* starts,
             const uint32_t* lens, const uint8_t* qtypes, size_t sequences,
             const uint32_t* marker_rows, size_t markers);
int jh_execute(jh_model* model);
int jh_scores(jh_model* model, float* scores, size_t markers);
void* jh_stream(jh_model* model);

/*
 * Pipelined form of jh_forward, for engines that run several micro-batches in
 * a row (`Engine::forward` over `batches`, src/engine.rs:191-223, which calls
 * `CudaModel::forward` once per micro-batch and waits for each):
 *  jh_submit  validates a batch, copies it into pinned staging, enqueues its
 *             upload, the forward and the download of its scores on the
 *             model's stream, and returns at once with a ticket (> 0);
 *  jh_collect waits for that ticket's scores and copies its M scores out.
 * While the GPU runs one batch the caller packs and submits the next, so the
 * GPU does not idle between forwards on host work or on the round trip of a
 * synchronous copy.  Forwards run in submission order on the one stream and
 * give the same scores as jh_forward.  At most JH_MAX_INFLIGHT tickets may be
 * outstanding (submitted, not yet collected); a further jh_submit fails with
 * JH_ERR_INVALID.  Tickets may be collected in any order, each once; a failed
 * jh_submit issues no ticket.  jh_collect waits without holding the model's
 * lock, so another thread may submit meanwhile.  jh_submit also makes its batch
 * the staged one (as jh_stage would) for jh_execute and the debug views.
 * No reference counterpart.
 */
#define JH_MAX_INFLIGHT 2
int jh_submit(jh_model* model, const uint32_t* ids, size_t tokens, const uint32_t* starts,
              const uint32_t* lens, const uint8_t* qtypes, size_t sequences,
              const uint32_t* marker_rows, size_t markers, uint64_t* ticket);
int jh_collect(jh_model* model, uint64_t ticket, float* scores, size_t markers);

/*
 * Use a captured hipGraph for jh_execute, jh_forward and jh_submit (1 = on,
 * 0 = off, default on): when a forward has the same batch shape (tokens,
 * markers, sequences, attention tiles) as the previous one staged in the same
 * staging buffer (one for jh_stage/jh_forward, one per jh_submit slot), its
 * launch sequence is captured once and then replayed while the shape stays
 * unchanged; a shape seen for the first time in a row runs eagerly, because
 * capture and instantiation (~0.5 ms on MI355X) cost more than replay saves.
 * No reference counterpart.
 */
int jh_set_graph(jh_model* model, int enabled);

/*
 * Small-batch GEMM paths (1 = on, default; 0 = off).  When a GEMM's output has
 * too few 128 x 128 tiles to occupy the GPU (small batches, marker rows), K is
 * split: over the four waves of one workgroup (one launch, K <= 768) or into
 * chunks whose FP32 partial sums a second kernel reduces (the residual GEMMs,
 * with the residual add and LayerNorm in that kernel).  Either way the partial
 * sums are added in a fixed order, so results are deterministic, but a row's
 * FP32 summation order then depends on the batch's token count.  Off, every output element is accumulated in the same
 * order whatever the batch, so a row's logits are invariant to what else is
 * batched with it (to FP32 round-off of the bf16 activations, <= 1e-4), at
 * the cost of small-batch latency.  No reference counterpart (cuBLAS picks
 * its own split per shape).
 */
int jh_set_splitk(jh_model* model, int enabled);

/*
 * Per-kernel timing.  While profiling is enabled, jh_execute runs the launch
 * sequence eagerly (no graph) and brackets every launch with a pair of HIP
 * events on the model's stream.  jh_profile_read synchronises, sums the
 * device time, launch count and algorithmic FLOPs/bytes per kernel class
 * ("gemm_qkv_rope", "attn_global", ...) since the last read, and resets.
 * It writes at most `capacity` entries and sets *count to the number of
 * classes with launches.  No reference counterpart (the reference's CPU path
 * has JULIA_PROFILE wall-clock slots, src/cpu/mod.rs:95-128).
 */
typedef struct jh_kernel_stat {
    const char* name;
    uint32_t launches;
    double ms;       /* summed device time of the launches                  */
    double flops;    /* algorithmic FLOPs: 2·M·N·K per GEMM, 4·64·heads per  */
                     /* attended (query, key) pair                          */
    double bytes;    /* algorithmic HBM bytes: operands read once, outputs  */
                     /* written once (FP32 residual read and written)       */
} jh_kernel_stat;

int jh_profile(jh_model* model, int enabled);
int jh_profile_read(jh_model* model, jh_kernel_stat* out, size_t capacity, size_t* count);

/*
 * Device time of one launch of a GEMM or attention kernel class, without
 * per-launch events: the first launch of that class recorded by the last
 * profiled jh_execute is replayed `reps` times back to back between two
 * events on the model's stream, and the mean is written to *us_per_launch.
 * The replay reuses the staged workspace: a residual-epilogue GEMM adds into
 * the residual stream again, so run it after the forward's scores were read
 * (the next jh_execute recomputes everything).  No reference counterpart.
 */
int jh_profile_replay(jh_model* model, const char* kernel_class, size_t reps, double* us_per_launch);

/* "hip:N (<device name>)" — replaces `CudaModel::name` (src/cuda/mod.rs:252,278-280). */
const char* jh_name(jh_model* model);

/* Frees all device and pinned memory — replaces `Drop for DevBuf` (src/cuda/mod.rs:42-49). */
void jh_destroy(jh_model* model);

/* Message of the last failing call on this thread ("" if none). */
const char* jh_last_error(void);

/*
 * RoPE table exactly as `rope_table` (src/config.rs:99-112): f32 inverse
 * frequencies 1/theta^(2i/head_dim), f32 products p*inv[i], f32 cos/sin.
 * cos_out/sin_out are [positions, head_dim/2].  Host-only; used to build the
 * device tables and exported so their bit pattern can be tested.
 */
void jh_rope_table(float theta, uint32_t head_dim, uint32_t positions, float* cos_out, float* sin_out);

/*
 * Debug views of the staged batch, copied back from the device: the token ids
 * and the per-token position within its sequence that the kernels read
 * (ids_out[T], pos_out[T]), and the residual stream x after `layers` encoder
 * layers of jh_execute's launch sequence (x_out[T*hidden], FP32; layers may be
 * 0 for the embedding output, up to config.layers).  No reference counterpart.
 */
int jh_debug_tokens(jh_model* model, uint32_t* ids_out, uint32_t* pos_out, size_t tokens);
int jh_debug_encode(jh_model* model, uint32_t layers, float* x_out, size_t tokens);

/*
 * Test hook: make every later workspace growth fail with JH_ERR_ALLOC once
 * its device buffers would exceed `bytes` (0 = no limit), part way through
 * reallocating them, as a failing hipMalloc would.  The model stays usable:
 * the next batch that fits regrows the workspace.  No reference counterpart.
 */
int jh_debug_workspace_limit(jh_model* model, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* JULIA1_HIP_H */
