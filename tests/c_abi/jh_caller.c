/*
 * A plain C99 caller of the HIP backend's C-ABI, linked against the static
 * library libjulia1_hip.a: the same calls a Rust `Backend::Hip` arm makes
 * through its FFI (jh_create / jh_forward / jh_name / jh_destroy, replacing
 * CudaModel::new / forward / name / drop, src/cuda/mod.rs:174-521).
 *
 *   jh_caller WEIGHTS BATCH SCORES_OUT
 *
 * WEIGHTS and BATCH are little-endian files of 4-byte words written by
 * tests/test_gpu_c_abi.py (u32 or f32 per field, see read_weights and
 * read_batch).  The scores of one forward go to SCORES_OUT as raw f32.  The
 * program also checks that a rejected batch (a token id past the vocabulary)
 * returns JH_ERR_INVALID with a message and leaves the model usable: the
 * forward after it must return the same scores bit for bit.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "julia1_hip.h"

typedef struct {
    uint32_t* w;  /* the file as 4-byte words */
    size_t n, at;
} cursor;

static void die(const char* what) {
    fprintf(stderr, "jh_caller: %s\n", what);
    exit(2);
}

static cursor slurp(const char* path) {
    cursor c = {NULL, 0, 0};
    FILE* f = fopen(path, "rb");
    long len;
    if (!f) die("cannot open input");
    if (fseek(f, 0, SEEK_END) != 0 || (len = ftell(f)) < 0 || fseek(f, 0, SEEK_SET) != 0) die("cannot size input");
    if (len % 4) die("input is not a whole number of 4-byte words");
    c.n = (size_t)len / 4;
    c.w = (uint32_t*)malloc(len > 0 ? (size_t)len : 1);
    if (!c.w || fread(c.w, 4, c.n, f) != c.n) die("cannot read input");
    fclose(f);
    return c;
}

static uint32_t u32(cursor* c) {
    if (c->at >= c->n) die("input too short");
    return c->w[c->at++];
}

static float f32(cursor* c) {
    float v;
    uint32_t b = u32(c);
    memcpy(&v, &b, 4);
    return v;
}

/* n floats in place; the pointer stays valid while the buffer lives */
static const float* floats(cursor* c, size_t n) {
    const float* p;
    if (n > c->n - c->at) die("input too short");
    p = (const float*)(c->w + c->at);
    c->at += n;
    return p;
}

static void read_weights(cursor* c, jh_config* cfg, jh_weights* w, uint8_t** global, float** theta,
                         jh_encoder_layer** layers, jh_head_layer** head) {
    uint32_t l, h, i, ff, L, HL;
    if (u32(c) != 0x3157484au) die("bad weights magic"); /* "JHW1" */
    cfg->hidden = u32(c);
    cfg->heads = u32(c);
    cfg->head_dim = u32(c);
    cfg->intermediate = u32(c);
    cfg->layers = u32(c);
    cfg->half_window = u32(c);
    cfg->vocab = u32(c);
    cfg->max_positions = u32(c);
    cfg->head_layers = u32(c);
    cfg->head_heads = u32(c);
    cfg->head_ff = u32(c);
    cfg->norm_eps = f32(c);
    w->scorer_b2 = f32(c);
    h = cfg->hidden, i = cfg->intermediate, ff = cfg->head_ff, L = cfg->layers, HL = cfg->head_layers;
    *global = (uint8_t*)malloc(L ? L : 1);
    *theta = (float*)malloc(sizeof(float) * (L ? L : 1));
    *layers = (jh_encoder_layer*)calloc(L ? L : 1, sizeof(jh_encoder_layer));
    *head = (jh_head_layer*)calloc(HL ? HL : 1, sizeof(jh_head_layer));
    if (!*global || !*theta || !*layers || !*head) die("out of memory");
    for (l = 0; l < L; ++l) (*global)[l] = (uint8_t)u32(c);
    for (l = 0; l < L; ++l) (*theta)[l] = f32(c);
    cfg->global = *global;
    cfg->rope_theta = *theta;
    w->embedding = floats(c, (size_t)cfg->vocab * h);
    w->emb_norm = floats(c, h);
    for (l = 0; l < L; ++l) {
        jh_encoder_layer* e = &(*layers)[l];
        e->attn_norm = u32(c) ? floats(c, h) : NULL;
        e->wqkv = floats(c, (size_t)3 * h * h);
        e->wo = floats(c, (size_t)h * h);
        e->mlp_norm = floats(c, h);
        e->wi = floats(c, (size_t)2 * i * h);
        e->wo2 = floats(c, (size_t)h * i);
    }
    w->layers = *layers;
    w->final_norm = floats(c, h);
    w->type_emb = floats(c, (size_t)3 * h);
    for (l = 0; l < HL; ++l) {
        jh_head_layer* e = &(*head)[l];
        e->norm1_w = floats(c, h);
        e->norm1_b = floats(c, h);
        e->in_w = floats(c, (size_t)3 * h * h);
        e->in_b = floats(c, (size_t)3 * h);
        e->out_w = floats(c, (size_t)h * h);
        e->out_b = floats(c, h);
        e->norm2_w = floats(c, h);
        e->norm2_b = floats(c, h);
        e->lin1_w = floats(c, (size_t)ff * h);
        e->lin1_b = floats(c, ff);
        e->lin2_w = floats(c, (size_t)h * ff);
        e->lin2_b = floats(c, h);
    }
    w->head = *head;
    w->scorer_norm_w = floats(c, h);
    w->scorer_norm_b = floats(c, h);
    w->scorer_w1 = floats(c, (size_t)h * h);
    w->scorer_b1 = floats(c, h);
    w->scorer_w2 = floats(c, h);
    if (c->at != c->n) die("trailing data in weights");
}

typedef struct {
    size_t T, S, M;
    const uint32_t *ids, *starts, *lens, *markers;
    uint8_t* qtypes;
} batch;

static batch read_batch(cursor* c) {
    batch b;
    size_t s;
    if (u32(c) != 0x3142484au) die("bad batch magic"); /* "JHB1" */
    b.T = u32(c);
    b.S = u32(c);
    b.M = u32(c);
    if (b.T > c->n || b.S > c->n || b.M > c->n) die("batch sizes out of range");
    b.ids = (const uint32_t*)floats(c, b.T);
    b.starts = (const uint32_t*)floats(c, b.S);
    b.lens = (const uint32_t*)floats(c, b.S);
    b.qtypes = (uint8_t*)malloc(b.S ? b.S : 1);
    if (!b.qtypes) die("out of memory");
    for (s = 0; s < b.S; ++s) b.qtypes[s] = (uint8_t)u32(c);
    b.markers = (const uint32_t*)floats(c, b.M);
    if (c->at != c->n) die("trailing data in batch");
    return b;
}

int main(int argc, char** argv) {
    cursor cw, cb;
    jh_config cfg;
    jh_weights w;
    uint8_t* global;
    float *theta, *scores, *again;
    jh_encoder_layer* layers;
    jh_head_layer* head;
    jh_model* model = NULL;
    batch b;
    uint32_t* bad_ids;
    FILE* out;
    int rc;

    if (argc != 4) die("usage: jh_caller WEIGHTS BATCH SCORES_OUT");
    memset(&cfg, 0, sizeof cfg);
    memset(&w, 0, sizeof w);
    cw = slurp(argv[1]);
    cb = slurp(argv[2]);
    read_weights(&cw, &cfg, &w, &global, &theta, &layers, &head);
    b = read_batch(&cb);

    rc = jh_create(&cfg, &w, 0, &model);
    if (rc != JH_OK) {
        fprintf(stderr, "jh_create failed (%d): %s\n", rc, jh_last_error());
        return 1;
    }
    printf("name=%s\n", jh_name(model));
    scores = (float*)malloc(sizeof(float) * (b.M ? b.M : 1));
    again = (float*)malloc(sizeof(float) * (b.M ? b.M : 1));
    if (!scores || !again) die("out of memory");
    rc = jh_forward(model, b.ids, b.T, b.starts, b.lens, b.qtypes, b.S, b.markers, b.M, scores);
    if (rc != JH_OK) {
        fprintf(stderr, "jh_forward failed (%d): %s\n", rc, jh_last_error());
        return 1;
    }

    /* A rejected batch: an id past the vocabulary.  The error comes back as a
       code and a message, and the model stays usable. */
    if (b.T) {
        bad_ids = (uint32_t*)malloc(sizeof(uint32_t) * b.T);
        if (!bad_ids) die("out of memory");
        memcpy(bad_ids, b.ids, sizeof(uint32_t) * b.T);
        bad_ids[b.T / 2] = cfg.vocab;
        rc = jh_forward(model, bad_ids, b.T, b.starts, b.lens, b.qtypes, b.S, b.markers, b.M, again);
        if (rc != JH_ERR_INVALID || jh_last_error()[0] == '\0') {
            fprintf(stderr, "bad batch: expected JH_ERR_INVALID with a message, got %d\n", rc);
            return 1;
        }
        printf("rejected=%s\n", jh_last_error());
        free(bad_ids);
        rc = jh_forward(model, b.ids, b.T, b.starts, b.lens, b.qtypes, b.S, b.markers, b.M, again);
        if (rc != JH_OK || memcmp(scores, again, sizeof(float) * b.M) != 0) {
            fprintf(stderr, "forward after a rejected batch differs (%d)\n", rc);
            return 1;
        }
    }
    jh_destroy(model);

    out = fopen(argv[3], "wb");
    if (!out || fwrite(scores, sizeof(float), b.M, out) != b.M) die("cannot write scores");
    fclose(out);
    printf("markers=%zu\n", b.M);
    free(scores);
    free(again);
    free(b.qtypes);
    free(global);
    free(theta);
    free(layers);
    free(head);
    free(cw.w);
    free(cb.w);
    return 0;
}
