/*
 * julia1_engine.h — C++ host mirror of the reference runtime's `Engine`
 * (apiplant/julia1-rs src/engine.rs) on the HIP backend, exported as a C-ABI.
 *
 * It does below the text front end what `Engine` does: parse the checkpoint's
 * julia_config.json + encoder/config.json (`ModelConfig::from_values`,
 * src/config.rs:43-96), memory-map model.safetensors (`SafeTensors`,
 * src/weights.rs:32-94), resolve and shape-check every tensor
 * (`HostWeights::load`, src/model.rs:55-110), build the jh_model backend
 * (`assemble`, src/engine.rs:147-172), then run length-sorted micro-batches
 * (`batches`, src/engine.rs:191-210) through the backend with the nonfinite
 * check of `Engine::forward` (src/engine.rs:212-223).  Micro-batches are
 * pipelined with jh_submit/jh_collect (up to JH_MAX_INFLIGHT ahead), so the
 * host packs the next one while the GPU runs the current one; the logits
 * equal those of one jh_forward per micro-batch.  Text encoding
 * (`Encoder`, src/encode.rs) is not part of this library: callers pass
 * token ids and marker positions, as `logits_encoded` receives them.
 *
 * Checkpoints: julia_config.json's weight_dtype "float32" (the reference's
 * only format: every tensor F32) or "bfloat16" (an extension: any tensor may
 * be BF16; BF16 matrices give the same device weights as the F32 checkpoint
 * they were rounded from, since the backend rounds F32 matrices to BF16 with
 * the same round-to-nearest-even).  A tensor's byte length must match its
 * shape.
 *
 * Errors: nonzero JH_ERR_* codes with the message in jh_last_error(); the
 * messages follow the reference's wording.
 */
#ifndef JULIA1_ENGINE_H
#define JULIA1_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "julia1_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* `EngineOptions` (src/engine.rs:34-65) minus the text front end's fields. */
typedef struct je_options {
    int device_ordinal;         /* Device::Hip(N)                                        */
    uint32_t max_length;        /* 0 = the checkpoint's max_position_embeddings          */
    uint32_t batch_size;        /* rows per forward pass (default 16)                    */
    uint32_t max_batch_tokens;  /* packed tokens per forward pass (default 65536)        */
} je_options;

typedef struct je_engine je_engine;

/* EngineOptions::default() (src/engine.rs:51-65). */
void je_default_options(je_options* out);

/*
 * Device string as `Device::from_str` (src/engine.rs:20-32) with the HIP arm:
 * "hip" -> 0, "hip:N" -> N.  "cpu"/"cuda" are rejected: this library only
 * builds the HIP backend.
 */
int je_parse_device(const char* s, int* ordinal);

/* `Engine::load` (src/engine.rs:89-110) + `assemble` (:147-172) for Device::Hip. */
int je_load(const char* checkpoint_dir, const je_options* options, je_engine** out);

/*
 * `Engine::logits_encoded` (src/engine.rs:225-235): item i has ids
 * ids[id_offsets[i] .. id_offsets[i+1]], option markers (positions within the
 * item) markers[marker_offsets[i] .. marker_offsets[i+1]] and question type
 * qtypes[i] (0 choice, 1 score, 2 noul; src/request.rs:8-12).  Writes the
 * logits of item i to logits[marker_offsets[i] .. marker_offsets[i+1]], in
 * item order.  Items are length-sorted into micro-batches of at most
 * batch_size rows and max_batch_tokens tokens.
 */
int je_logits_encoded(je_engine* engine, size_t items, const uint32_t* ids, const size_t* id_offsets,
                      const uint32_t* markers, const size_t* marker_offsets, const uint8_t* qtypes,
                      float* logits);

/* The parsed configuration; pointers inside stay valid while the engine lives. */
int je_config(je_engine* engine, jh_config* out);

/* The engine's options after je_load resolved them (`Engine::options`,
 * src/engine.rs:174-176): max_length is the effective limit. */
int je_get_options(je_engine* engine, je_options* out);

/* `Engine::device_name` (src/engine.rs:277-283): "hip:N (<device name>)". */
const char* je_device_name(je_engine* engine);

/* Number of forward passes (micro-batches) run so far. */
uint64_t je_forward_count(je_engine* engine);

void je_destroy(je_engine* engine);

/*
 * Host-only checkpoint validation, no device needed: runs the config parser,
 * the safetensors reader and the tensor-name/shape resolution of je_load and
 * writes a one-line JSON summary ({"hidden":..,"layers":..,"tensors":..,
 * "bf16_tensors":..,"bytes":..}) into `summary` (NUL-terminated, truncated to
 * `capacity`).
 */
int je_inspect(const char* checkpoint_dir, char* summary, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* JULIA1_ENGINE_H */
