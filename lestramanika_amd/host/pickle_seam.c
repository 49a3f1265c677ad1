/*
 * pickle_seam.c -- the reference-side binding of the MI355X attention block.
 *
 * This is the code a pickle maintainer adds so that pickle_fast_forward
 * (src/pickle_fast.c:1822-2181) reaches the GPU through libpkh.so.  It is
 * compiled against the reference's own headers (src/pickle.h,
 * src/pickle_fast.h) and is not part of libpkh.so: the reference's Makefile
 * would build it beside src/pickle_fast.c and link -lpkh.
 *
 * The binding keeps the reference's structs as they are and holds the
 * device cache and RoPE table beside them (a pickle_pkh_t next to the
 * pickle_fast_kv_t), so nothing in the reference's headers changes:
 *
 *   pickle_pkh_alloc      after pickle_fast_state_init and
 *                         pickle_fast_kv_alloc (src/pickle_fast.c:1793-1810)
 *   pickle_pkh_attention  in the layer loop in place of the RoPE apply, KV
 *                         append and attention (src/pickle_fast.c:1910-2094)
 *                         when kv != NULL; the stateless branch (:2095-2109)
 *                         stays as it is
 *   pickle_pkh_prefill    a layer-major forward's attention over a whole
 *                         prompt chunk (the token loop of :1881-1898)
 *   pickle_pkh_free       beside pickle_fast_kv_free (:1811-1817)
 *
 * Status codes pass through unchanged: PKH_ERR_* equal PICKLE_ERR_*.
 */
#include <stddef.h>
#include <string.h>

#include "pickle.h"
#include "pickle_fast.h"
#include "pkh_attn.h"

/* pkh_kv_t's first eight fields are pickle_fast_kv_t's (src/pickle_fast.h:
 * 145-154), at the same offsets; k and v are device pointers there. */
_Static_assert(offsetof(pkh_kv_t, n_layers) == offsetof(pickle_fast_kv_t, n_layers), "n_layers");
_Static_assert(offsetof(pkh_kv_t, n_kv_heads) == offsetof(pickle_fast_kv_t, n_kv_heads), "n_kv_heads");
_Static_assert(offsetof(pkh_kv_t, head_dim) == offsetof(pickle_fast_kv_t, head_dim), "head_dim");
_Static_assert(offsetof(pkh_kv_t, max_seq) == offsetof(pickle_fast_kv_t, max_seq), "max_seq");
_Static_assert(offsetof(pkh_kv_t, k_stride_layer) == offsetof(pickle_fast_kv_t, k_stride_layer), "k_stride_layer");
_Static_assert(offsetof(pkh_kv_t, v_stride_layer) == offsetof(pickle_fast_kv_t, v_stride_layer), "v_stride_layer");
_Static_assert(offsetof(pkh_kv_t, k) == offsetof(pickle_fast_kv_t, k), "k");
_Static_assert(offsetof(pkh_kv_t, v) == offsetof(pickle_fast_kv_t, v), "v");

/* The library's status codes are the reference's (src/pickle.h:52-60). */
_Static_assert(PKH_OK == PICKLE_OK, "ok");
_Static_assert(PKH_ERR_MEMORY == PICKLE_ERR_MEMORY, "memory");
_Static_assert(PKH_ERR_IO == PICKLE_ERR_IO, "io");
_Static_assert(PKH_ERR_ARG == PICKLE_ERR_ARG, "arg");
_Static_assert(PKH_ERR_RANGE == PICKLE_ERR_RANGE, "range");

/* The device side of one sequence's cache: the layer-major KV in HBM and the
 * device copy of the state's RoPE tables. */
typedef struct {
    pkh_kv_t   kv;
    pkh_rope_t rope;
} pickle_pkh_t;

/* Allocate the device cache for arch (fp32, max_seq_len positions) and the
 * device RoPE table for state (its max_seq rows of half columns).  On error
 * *p is zeroed and the code returned. */
int pickle_pkh_alloc(const pickle_arch_t* arch, const pickle_fast_state_t* state,
                     pickle_pkh_t* p) {
    if (!arch || !state || !p) return PICKLE_ERR_ARG;
    memset(p, 0, sizeof(*p));
    int rc = pkh_kv_alloc(arch->n_layers, arch->n_kv_heads, arch->head_dim, arch->max_seq_len,
                          PKH_KV_F32, &p->kv);
    if (rc != PICKLE_OK) return rc;
    rc = pkh_rope_alloc(state->max_seq, state->half, &p->rope);
    if (rc != PICKLE_OK) {
        pkh_kv_free(&p->kv);
        return rc;
    }
    return PICKLE_OK;
}

void pickle_pkh_free(pickle_pkh_t* p) {
    if (!p) return;
    pkh_rope_free(&p->rope);
    pkh_kv_free(&p->kv);
}

/* Send the state's table rows not yet on the device.  Called after
 * pickle_fast_state_extend_rope (src/pickle_fast.c:1875-1878); only new rows
 * travel. */
static int pickle_pkh_sync_rope(const pickle_fast_state_t* state, pickle_pkh_t* p) {
    return pkh_rope_upload(&p->rope, state->rope_sin, state->rope_cos, state->rope_filled_upto);
}

/* The attention block of layer `layer` for the token at position pos:
 * state->q [H*D], state->k and state->v [HK*D] as the projections left them
 * (before RoPE); rotates q and k, appends (k_rot, v) to cache row pos,
 * attends rows [0, pos] and writes state->ao [H*D] for the output projection
 * (src/pickle_fast.c:2112).  pos >= max_seq returns PICKLE_ERR_RANGE before
 * any device work (src/pickle_fast.c:1885). */
int pickle_pkh_attention(pickle_fast_state_t* state, pickle_pkh_t* p, int layer, size_t pos) {
    if (!state || !p) return PICKLE_ERR_ARG;
    if (pos >= (size_t)state->max_seq) return PICKLE_ERR_RANGE;
    int rc = pickle_pkh_sync_rope(state, p);
    if (rc != PICKLE_OK) return rc;
    return pkh_attn_decode(&p->kv, &p->rope, layer, (int)pos, state->n_heads, state->q,
                           state->k, state->v, state->ao);
}

/* A layer-major forward's attention for n_tokens consecutive tokens from
 * position pos0 on one layer: q [n][H*D], k and v [n][HK*D] (before RoPE),
 * ao [n][H*D].  Leaves the cache holding the rows the token loop would have
 * appended. */
int pickle_pkh_prefill(pickle_fast_state_t* state, pickle_pkh_t* p, int layer, size_t pos0,
                       size_t n_tokens, const float* q, const float* k, const float* v,
                       float* ao) {
    if (!state || !p || n_tokens == 0) return PICKLE_ERR_ARG;
    if (pos0 + n_tokens > (size_t)state->max_seq) return PICKLE_ERR_RANGE;
    int rc = pickle_fast_state_extend_rope(state, (int)(pos0 + n_tokens - 1));
    if (rc != PICKLE_OK) return rc;
    rc = pickle_pkh_sync_rope(state, p);
    if (rc != PICKLE_OK) return rc;
    return pkh_attn_prefill(&p->kv, &p->rope, layer, (int)pos0, (int)n_tokens, state->n_heads,
                            q, k, v, ao);
}
