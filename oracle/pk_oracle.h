/*
 * pk_oracle.h -- CPU restatement of pickle's fast-path attention block.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle the HIP attention
 * path is checked against: it is linked or loaded only by tests/, by the smoke()
 * entry point and by the CPU-baseline leg of bench.py.  Nothing in the
 * product (lestramanika_amd/) links, loads or calls it.
 *
 * Every function restates one piece of the reference's fast path
 * (src/pickle_fast.c in lee-muriithi-kingori/lestramanika) with the same
 * fp32 arithmetic and the same operation order, so that on an x86-64 host
 * with FMA it reproduces the reference's AVX-512 path bit-for-bit:
 *
 *   pko_rope_half            src/pickle_fast.c:1515-1516
 *   pko_rope_inv_freq        src/pickle_fast.c:1634-1640
 *   pko_rope_fill            src/pickle_fast.c:1772-1788
 *   pko_rope_apply           src/pickle_fast.c:1910-1936
 *   pko_kv_append_f32        src/pickle_fast.c:1938-1944
 *   pko_attend_f32           src/pickle_fast.c:1946-2094
 *   pko_attend_stateless     src/pickle_fast.c:2095-2109
 *   pko_decode_step_f32      RoPE + append + attend for one token
 *   pko_prefill_f32          the token loop of src/pickle_fast.c:1881-1898
 *
 * fp16 KV storage has no counterpart in the reference.  Its oracle
 * (pko_decode_step_f16) is the fp32 attention above run on the fp16 cache
 * widened to fp32, with the appended k/v rounded to fp16 (IEEE binary16,
 * round-to-nearest-even) as they are stored.  The rounding itself is
 * pinned against numpy's float16 conversion in the CPU tests; the
 * attention is pinned against the compiled reference.
 *
 * Status codes reuse the reference's values (src/pickle.h:52-60).
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKO_OK         0
#define PKO_ERR_MEMORY -3
#define PKO_ERR_ARG    -6
#define PKO_ERR_RANGE  -7

/* half = min(head_dim / 2, 64). */
int  pko_rope_half(int head_dim);

/* inv_freq[i] = 1 / theta^((2i) / head_dim), i in [0, half). */
void pko_rope_inv_freq(float* inv_freq, int head_dim, float theta);

/* Fill rows p_begin..p_last (inclusive) of the [pos][half] sin/cos tables. */
void pko_rope_fill(float* sin_tab, float* cos_tab, const float* inv_freq,
                   int half, int p_begin, int p_last);

/* Rotate pairs (x[i], x[i+half]) of each of n_heads rows of head_dim floats
 * by the table row (sin_row, cos_row). */
void pko_rope_apply(float* x, int n_heads, int head_dim, int half,
                    const float* sin_row, const float* cos_row);

/* Copy k[HK*D], v[HK*D] into row pos of one layer's [max_seq][HK][D] cache. */
void pko_kv_append_f32(float* k_layer, float* v_layer, int n_kv_heads,
                       int head_dim, int pos, const float* k, const float* v);

/* Attention of H query heads (already rotated) over cache rows [0, attend_n)
 * of one layer.  Head h reads KV head h*HK/H.  n_threads > 1 runs the heads
 * in an OpenMP team of that size, as the reference does over heads. */
int  pko_attend_f32(const float* k_layer, const float* v_layer, int n_kv_heads,
                    int head_dim, int n_heads, size_t attend_n,
                    const float* q_rot, float* ao, int n_threads);

/* kv == NULL path: out_h = v[kv_head(h)]. */
void pko_attend_stateless(const float* v, int n_kv_heads, int head_dim,
                          int n_heads, float* ao);

/* One decode step on one layer: rotate copies of q and k with table row pos,
 * append (k_rot, v) at pos, attend over [0, pos].  q, k, v are not modified.
 * If q_rot_out / k_rot_out are non-NULL the rotated vectors are copied out. */
int  pko_decode_step_f32(float* k_layer, float* v_layer, int n_kv_heads,
                         int head_dim, int n_heads, int pos,
                         const float* sin_tab, const float* cos_tab, int half,
                         const float* q, const float* k, const float* v,
                         float* ao, float* q_rot_out, float* k_rot_out,
                         int n_threads);

/* Token-loop prefill: row i is a decode step at pos0 + i.
 * q [n][H][D], k/v [n][HK][D], ao [n][H][D]. */
int  pko_prefill_f32(float* k_layer, float* v_layer, int n_kv_heads,
                     int head_dim, int n_heads, int pos0, int n_tokens,
                     const float* sin_tab, const float* cos_tab, int half,
                     const float* q, const float* k, const float* v,
                     float* ao, int n_threads);

/* IEEE binary16 <-> binary32, round-to-nearest-even on the narrowing side. */
uint16_t pko_f32_to_f16(float x);
float    pko_f16_to_f32(uint16_t h);
void     pko_f32_to_f16_n(const float* x, uint16_t* h, size_t n);
void     pko_f16_to_f32_n(const uint16_t* h, float* x, size_t n);

/* fp16-KV decode step: cache rows [0, pos) are fp16; k_rot and v are rounded
 * to fp16 when appended at pos; attention runs in fp32 on the widened cache. */
int  pko_decode_step_f16(uint16_t* k_layer, uint16_t* v_layer, int n_kv_heads,
                         int head_dim, int n_heads, int pos,
                         const float* sin_tab, const float* cos_tab, int half,
                         const float* q, const float* k, const float* v,
                         float* ao, int n_threads);

#ifdef __cplusplus
}
#endif
#endif /* PK_ORACLE_H */
