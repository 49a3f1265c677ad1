/*
 * ref_probe.c -- a thin driver over the reference's own fast path.
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled together with the reference's sources
 * (read in place from the reference tree by oracle/Makefile) into
 * oracle/_ref/libpickle_ref.so.  It calls only the reference's public API
 * (src/pickle.h, src/pickle_fast.h) and exposes a few flat C entry points
 * that ctypes can drive:
 *
 *   - load a GGUF file, optionally truncating the layer count (the fast
 *     state and the KV cache take n_layers from pickle_arch_t, which is a
 *     plain struct: src/pickle.h:225-249, src/pickle_fast.c:1504,
 *     src/pickle_fast.c:1797);
 *   - run pickle_fast_forward one token at a time (src/pickle_fast.c:1822);
 *   - read and write the KV cache, the RoPE tables and the state's work
 *     buffers (xn, q, k, v, ao: src/pickle_fast.h:105-110), which hold the
 *     last layer's values after a forward call.
 */
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pickle.h"
#include "pickle_fast.h"

/* Defined in src/pickle_host.c:107; the reference declares it only in its CLI. */
int pickle_load_from_file(const char* path, pickle_model_t** out_model);

typedef struct {
    pickle_model_t*     model;
    pickle_arch_t       arch;
    pickle_fast_state_t state;
    pickle_fast_kv_t    kv;
    size_t              kv_pos;
} ref_handle_t;

int ref_open(const char* path, int n_layers_override, void** out) {
    ref_handle_t* h = (ref_handle_t*)calloc(1, sizeof(*h));
    if (!h) return PICKLE_ERR_MEMORY;
    int rc = pickle_load_from_file(path, &h->model);
    if (rc == PICKLE_OK) rc = pickle_arch_detect(h->model, &h->arch);
    if (rc == PICKLE_OK && n_layers_override > 0 &&
        n_layers_override < h->arch.n_layers)
        h->arch.n_layers = n_layers_override;
    if (rc == PICKLE_OK) rc = pickle_fast_state_init(h->model, &h->arch, &h->state);
    if (rc == PICKLE_OK) rc = pickle_fast_kv_alloc(&h->arch, &h->kv);
    if (rc != PICKLE_OK) {
        if (h->model) pickle_free(h->model);
        free(h);
        return rc;
    }
    *out = h;
    return PICKLE_OK;
}

void ref_close(void* p) {
    ref_handle_t* h = (ref_handle_t*)p;
    if (!h) return;
    pickle_fast_kv_free(&h->kv);
    pickle_fast_state_free(&h->state);
    pickle_free(h->model);
    free(h);
}

/* out[0..9] = n_layers, n_heads, n_kv_heads, head_dim, hidden_dim,
 *             intermediate_dim, vocab_size, max_seq, half, rope_filled_upto */
void ref_shape(void* p, int* out) {
    ref_handle_t* h = (ref_handle_t*)p;
    out[0] = h->state.n_layers;
    out[1] = h->state.n_heads;
    out[2] = h->state.n_kv_heads;
    out[3] = h->state.head_dim;
    out[4] = h->state.hidden_dim;
    out[5] = h->state.intermediate_dim;
    out[6] = h->state.vocab_size;
    out[7] = h->state.max_seq;
    out[8] = h->state.half;
    out[9] = h->state.rope_filled_upto;
}

float ref_rope_theta(void* p) { return ((ref_handle_t*)p)->state.rope_theta; }

size_t ref_get_pos(void* p) { return ((ref_handle_t*)p)->kv_pos; }
void   ref_set_pos(void* p, size_t pos) { ((ref_handle_t*)p)->kv_pos = pos; }

/* One token through pickle_fast_forward at the current position. */
int ref_forward1(void* p, int32_t token, float* logits) {
    ref_handle_t* h = (ref_handle_t*)p;
    return pickle_fast_forward(h->model, &h->arch, &h->state, &token, 1,
                               logits, &h->kv, &h->kv_pos);
}

/* n tokens in one pickle_fast_forward call (the reference's prefill form). */
int ref_forward_n(void* p, const int32_t* tokens, size_t n, float* logits) {
    ref_handle_t* h = (ref_handle_t*)p;
    return pickle_fast_forward(h->model, &h->arch, &h->state, tokens, n,
                               logits, &h->kv, &h->kv_pos);
}

/* Stateless forward (kv == NULL). */
int ref_forward_stateless(void* p, int32_t token, float* logits) {
    ref_handle_t* h = (ref_handle_t*)p;
    return pickle_fast_forward(h->model, &h->arch, &h->state, &token, 1,
                               logits, NULL, NULL);
}

/* The handle's fast state and arch, for code that takes the reference's own
 * structs (the seam binding's tests). */
void* ref_state_ptr(void* p) { return &((ref_handle_t*)p)->state; }
void* ref_arch_ptr(void* p) { return &((ref_handle_t*)p)->arch; }

/* which: 1 q, 2 k, 3 v.  Copies n floats into the state's work buffer. */
int ref_write_state(void* p, int which, const float* src, size_t n) {
    ref_handle_t* h = (ref_handle_t*)p;
    float* dst = NULL;
    switch (which) {
        case 1: dst = h->state.q; break;
        case 2: dst = h->state.k; break;
        case 3: dst = h->state.v; break;
        default: return PICKLE_ERR_ARG;
    }
    memcpy(dst, src, n * sizeof(float));
    return PICKLE_OK;
}

/* which: 0 xn, 1 q, 2 k, 3 v, 4 ao.  Copies n floats out. */
int ref_read_state(void* p, int which, float* dst, size_t n) {
    ref_handle_t* h = (ref_handle_t*)p;
    const float* src = NULL;
    switch (which) {
        case 0: src = h->state.xn; break;
        case 1: src = h->state.q;  break;
        case 2: src = h->state.k;  break;
        case 3: src = h->state.v;  break;
        case 4: src = h->state.ao; break;
        default: return PICKLE_ERR_ARG;
    }
    memcpy(dst, src, n * sizeof(float));
    return PICKLE_OK;
}

/* Copy rows [p0, p0+n) of layer L of the K (which=0) or V (which=1) cache
 * in (dir=0: dst <- cache) or out (dir=1: cache <- src). */
int ref_kv_rows(void* p, int which, int layer, size_t p0, size_t n,
                float* buf, int dir) {
    ref_handle_t* h = (ref_handle_t*)p;
    if (layer < 0 || layer >= h->kv.n_layers) return PICKLE_ERR_RANGE;
    if (p0 + n > (size_t)h->kv.max_seq) return PICKLE_ERR_RANGE;
    size_t row = (size_t)h->kv.n_kv_heads * h->kv.head_dim;
    float* base = (which == 0 ? h->kv.k : h->kv.v) +
                  (size_t)layer * h->kv.k_stride_layer + p0 * row;
    if (dir == 0) memcpy(buf, base, n * row * sizeof(float));
    else          memcpy(base, buf, n * row * sizeof(float));
    return PICKLE_OK;
}

/* Copy the inv_freq table (which=0, half floats) or rows [p0, p0+n) of the
 * sin (1) / cos (2) tables.  Extends the tables up to p0+n-1 first, through
 * the reference's own pickle_fast_state_extend_rope. */
int ref_rope(void* p, int which, size_t p0, size_t n, float* dst) {
    ref_handle_t* h = (ref_handle_t*)p;
    int half = h->state.half;
    if (which == 0) {
        memcpy(dst, h->state.rope_inv_freq, (size_t)half * sizeof(float));
        return PICKLE_OK;
    }
    if (n == 0) return PICKLE_OK;
    int rc = pickle_fast_state_extend_rope(&h->state, (int)(p0 + n - 1));
    if (rc != PICKLE_OK) return rc;
    if ((int)(p0 + n) > h->state.rope_filled_upto) return PICKLE_ERR_RANGE;
    const float* src = (which == 1 ? h->state.rope_sin : h->state.rope_cos) +
                       p0 * (size_t)half;
    memcpy(dst, src, n * (size_t)half * sizeof(float));
    return PICKLE_OK;
}

/* OpenMP threads of the reference's parallel loops (its attention runs
 * `omp parallel for` over heads, src/pickle_fast.c:1960). */
void ref_set_threads(int n) { omp_set_num_threads(n); }
int  ref_get_threads(void) { return omp_get_max_threads(); }

int32_t ref_argmax(const float* logits, size_t n) {
    return pickle_fast_argmax(logits, n);
}

int ref_selftest(int32_t* tok) { return pickle_selftest(tok); }
