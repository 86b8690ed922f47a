/*
 * julia1_text.h — text front end and callers above the engine, as a C-ABI.
 *
 * Mirrors what apiplant/julia1-rs runs above `Engine::logits_encoded`:
 *  - request rows and their validation (`Request::from_value`,
 *    src/request.rs:90-130; `parse_rows`, src/engine.rs:298-307);
 *  - `pyjson::dumps` / `float_repr` (src/pyjson.rs:7-118), so JSON states render
 *    byte for byte as Python's json.dumps(value, ensure_ascii=False);
 *  - the marker serialization of `Encoder::sequence` with its token and
 *    encoding LRU caches (src/encode.rs:44-195);
 *  - the legacy list API `Engine::predict` (src/engine.rs:247-258), named
 *    typed questions (`predict_typed`, src/typed.rs) and the hierarchical
 *    `Router` (src/router.rs).
 *
 * The tokenizer itself (`tokenizers::Tokenizer` over tokenizer.json in the
 * reference) is supplied by the caller through jt_tokenizer; the Python
 * package binds the `tokenizers` library to it.  Inference goes through a
 * jt_scorer: the HIP engine (je_engine, julia1_engine.h) or a caller's
 * function (the reference's `Logits` trait, src/engine.rs:287-295).
 *
 * Conventions as in julia1_hip.h: nonzero JH_ERR_* codes with the message in
 * jh_last_error(); messages follow the reference's wording.  Text arguments
 * are UTF-8 (pointer + byte length).  Results that are text are JSON
 * documents allocated by the library: free them with jt_free.  Floats in
 * result documents are printed with the shortest digits that read back to
 * the same value (f32 logits as f32, probabilities as f64).
 */
#ifndef JULIA1_TEXT_H
#define JULIA1_TEXT_H

#include <stddef.h>
#include <stdint.h>

#include "julia1_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

void jt_free(void* p);

/* `pyjson::dumps` (src/pyjson.rs:7-49, 102-118): JSON text -> json.dumps(ensure_ascii=False). */
int jt_pyjson_dumps(const char* json, size_t len, char** out);

/* `pyjson::float_repr` (src/pyjson.rs:56-99): Python's float.__repr__. */
int jt_float_repr(double value, char** out);

/*
 * The tokenizer behind an encoder.  `encode` tokenizes `text` without special
 * tokens (`Tokenizer::encode_fast(text, false)`, src/encode.rs:110): it
 * writes at most `capacity` ids and sets *count to the full count (it is
 * called again with a larger buffer when *count > capacity); `token_to_id`
 * resolves a special token's name (`Tokenizer::token_to_id`).  Both return 0
 * on success.  They may be called from any thread that calls into the
 * encoder.
 */
typedef struct jt_tokenizer {
    void* ctx;
    int (*encode)(void* ctx, const char* text, size_t len, uint32_t* ids, size_t capacity, size_t* count);
    int (*token_to_id)(void* ctx, const char* name, uint32_t* id);
    /* Optional (null: `encode` per text).  Tokenizes n texts in one call, as
     * the reference's parallel row encoding does (rayon over rows with
     * Tokenizer::encode_fast, src/engine.rs:183-188, src/encode.rs:110):
     * counts[i] receives text i's token count and *ids the concatenated ids,
     * in callback-owned memory that stays valid until the calling thread's
     * next encode_batch call on this ctx.  Same ids as `encode`. */
    int (*encode_batch)(void* ctx, size_t n, const char* const* texts, const size_t* lens, size_t* counts,
                        const uint32_t** ids);
} jt_tokenizer;

/* The encoder fields of `EngineOptions` (src/engine.rs:34-65). */
typedef struct jt_encoder_options {
    uint32_t max_length;      /* combined token limit (the engine's max_length)  */
    uint32_t head_length;     /* question + options budget (default 256)         */
    int32_t strict;           /* strict_encoding (default 0)                     */
    uint32_t token_cache;     /* LRU entries of tokenized fragments (8192; 0 off) */
    uint32_t encoding_cache;  /* LRU entries of whole encodings (2048; 0 off)     */
} jt_encoder_options;

/* Defaults of EngineOptions::default(); max_length is left 0 (must be set). */
void jt_default_encoder_options(jt_encoder_options* out);

typedef struct jt_encoder jt_encoder;

/*
 * `Encoder::from_parts` (src/encode.rs:58-93) with the tokenizer abstracted:
 * tokenizer_config.json names mask_token, cls_token, sep_token and pad_token,
 * whose ids come from tok->token_to_id.  `tok` is copied; its ctx must stay
 * valid while the encoder lives.
 */
int jt_encoder_create(const jt_tokenizer* tok, const char* tokenizer_config, size_t len,
                      const jt_encoder_options* options, jt_encoder** out);
void jt_encoder_destroy(jt_encoder* encoder);
/* `Encoder::clear_cache` (src/encode.rs:95-102). */
void jt_encoder_clear_cache(jt_encoder* encoder);
/* mask, cls, sep and pad ids, in that order. */
int jt_encoder_special_ids(jt_encoder* encoder, uint32_t out[4]);

/*
 * `Request::from_value(row, line)` then `Encoder::encode` (src/encode.rs:118-195)
 * of one request object.  Result: {"ids": [..], "markers": [..], "qtype":
 * "choice"|"score"|"noul", "truncated": bool, "option_tokens": [..]}.
 */
int jt_encode(jt_encoder* encoder, const char* row_json, size_t len, size_t line, char** out);

/*
 * `Engine::encoding_info` (src/engine.rs:261-280) over a JSONL document of
 * request rows: [{"tokens", "optionTokens", "headLength", "stateTruncated",
 * "optionsTruncated"}, ..].  Requires strict encoding.
 */
int jt_encoding_info(jt_encoder* encoder, const char* jsonl, size_t len, char** out);

/* Something that scores request rows: the `Logits` trait (src/engine.rs:287-295). */
typedef struct jt_scorer jt_scorer;
/* Sink for a callback scorer's output: one call per row, in row order. */
typedef struct jt_rows jt_rows;
int jt_rows_push(jt_rows* rows, const float* logits, size_t count);

/*
 * A scorer that calls `fn` with the rows as a JSON array of request objects
 * ({"state", "question", "options", "type"}); fn pushes one logits row per
 * request into `out` and returns 0.  Used for model-free tests of the
 * callers below (the reference's test doubles, tests/api.rs:10-26,144-156).
 */
typedef int (*jt_logits_fn)(void* ctx, const char* rows_json, size_t len, jt_rows* out);
int jt_scorer_callback(jt_logits_fn fn, void* ctx, jt_scorer** out);

/*
 * The engine as a scorer: `Engine::logits` (src/engine.rs:238-244) =
 * validate every row, encode every row with `encoder`, then
 * je_logits_encoded.  Engine and encoder must outlive the scorer.
 */
int jt_scorer_engine(je_engine* engine, jt_encoder* encoder, jt_scorer** out);
void jt_scorer_destroy(jt_scorer* scorer);

/* `parse_rows` + `Logits::logits`: JSONL rows -> [[logit, ..], ..] in option order. */
int jt_logits(jt_scorer* scorer, const char* jsonl, size_t len, char** out);

/*
 * `Engine::predict` (src/engine.rs:247-258): [{"index": argmax}, ..], with
 * "probabilities" (display-rounded f32 softmax) when `probabilities` != 0.
 */
int jt_predict(jt_scorer* scorer, const char* jsonl, size_t len, int probabilities, char** out);

/*
 * `predict_typed` (src/typed.rs:134-137) + `answers_to_json` (:59-62):
 * state is a JSON value (text, or an object/array rendered with pyjson),
 * questions maps IDs to {type, instructions, criteria}.  All validation
 * happens before any inference.  Result: {"answers": {id: {"type",
 * "probabilities": {key: p}, "choice"|"score"|"noul", "max_probability"?}}}.
 */
int jt_predict_typed(jt_scorer* scorer, const char* state_json, size_t state_len, const char* questions_json,
                     size_t questions_len, char** out);

/*
 * `Router` (src/router.rs): hierarchical choice routing over more than
 * `width` options.  jt_router_create = `Router::new(engine, width,
 * survivors, batch_size, cache_size, max_options)` (the Python defaults are
 * 20, 2, 16, 0, 4096).  jt_router_route_many takes JSONL rows {"state",
 * "question", "options" (2..max_options strings), "type"?} and returns
 * [RouteResult, ..] with the fields index, candidates, probabilities, rounds,
 * model_rows, cache_hits, hierarchical, probability_scope.
 */
typedef struct jt_router jt_router;
int jt_router_create(jt_scorer* scorer, uint32_t width, uint32_t survivors, uint32_t batch_size, uint32_t cache_size,
                     uint32_t max_options, jt_router** out);
int jt_router_route_many(jt_router* router, const char* jsonl, size_t len, char** out);
void jt_router_clear_cache(jt_router* router);
void jt_router_destroy(jt_router* router);

/* `display_probabilities` (src/request.rs:150-161): out[n]. */
int jt_display_probabilities(const double* values, size_t n, double* out);
/* `Router::confident_winner` (src/router.rs:132-142). */
int jt_confident_winner(const float* scores, size_t n, size_t best, int* out);

#ifdef __cplusplus
}
#endif

#endif /* JULIA1_TEXT_H */
