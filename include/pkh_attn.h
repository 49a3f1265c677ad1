/*
 * pkh_attn.h -- C ABI of the MI355X (gfx950) attention block for pickle's
 * fast path: RoPE on Q/K, KV-cache append and grouped-query attention for
 * single-sequence decode, causal prefill and ragged multi-sequence decode.
 *
 * The reference has no operator seam for attention: it is inline code inside
 * pickle_fast_forward (src/pickle_fast.c:1910-2094).  These entry points are
 * what that inline block calls instead; every declaration names the
 * reference code it replaces.  Plain C types and pointers only.
 *
 * Conventions (the reference's, src/pickle.h:52-60, src/pickle_fast.c:1816):
 *   - functions return PKH_OK (0) or a negative code with the same value as
 *     the matching PICKLE_ERR_* constant, and never abort;
 *   - *_alloc fills a caller-owned struct, *_free releases it and zeroes it;
 *   - one host thread calls in; nothing here is reentrant;
 *   - "_async" entry points take device pointers and a hipStream_t passed as
 *     void* (NULL = the null stream), enqueue work and return; the others
 *     take host pointers and return when the result is in host memory;
 *   - launches on one device must not run concurrently (use one stream, or
 *     order the streams): they share the library's device scratch -- split-K
 *     partials and their ready flags, prefill tiles, host-pointer staging;
 *   - that scratch grows (hipMalloc) when a call needs more than any call
 *     before it, and an outgrown buffer is kept, not freed, until the process
 *     ends, so a HIP graph captured earlier stays valid.  Allocation is not
 *     allowed inside stream capture: make one call at the largest shape
 *     before capturing (the _async launches themselves allocate nothing
 *     once the scratch is large enough, and record no memset), or use
 *     pkh_attn_decode_noalloc_async.
 *
 * Split-K decode within one launch.  A long context is split into work
 * items (chunks of positions); the last item of each (sequence, query-head
 * slot) merges the others' partial results.  Two properties of the hardware
 * are relied on:
 *   - workgroups are dispatched in order of their index, so every item the
 *     merger waits for has already been dispatched and waits on nothing; the
 *     wait is bounded all the same (pkh_tune_decode_wait), and a wait that
 *     runs out yields NaN, never a result merged from missing partials;
 *   - a store with device-scope coherence (the partials) has reached the
 *     device's coherence point once the storing wave's memory counter says it
 *     completed, before the ready flag is set, and the merger's loads of the
 *     partials use device-coherent accesses, issued after it has seen the
 *     flags.  This is the ordering a release/acquire pair gives, without the
 *     whole-L2 writeback a release fence would add.
 *
 * Layouts (fp32 values unless stated):
 *   q   [n_heads][head_dim]           ao  [n_heads][head_dim]
 *   k,v [n_kv_heads][head_dim]        (the reference's state->q/k/v/ao,
 *                                      src/pickle_fast.h:107-110)
 *   KV  layer-major, fp32 or fp16, in device memory; within a layer the
 *       placement is given by strides (pkh_kv_t), head-major by default, the
 *       reference's [pos][kv_head][head_dim] (src/pickle_fast.c:1940-1942)
 *       when described so
 *   query head h reads KV head h * n_kv_heads / n_heads
 *   (src/pickle_fast.c:1963), for any n_heads and n_kv_heads >= 1: groups
 *   need not be equal or powers of two, and when n_heads < n_kv_heads some
 *   KV heads serve no query head (their rows are still appended).
 *
 * Supported shapes: head_dim 1..256 (the kernels run at the next of 16, 32,
 * 64, 128, 256 and mask the rest), any n_heads, n_kv_heads >= 1.  head_dim
 * above 256 and non-positive counts return PKH_ERR_ARG.
 *
 * Size limits (PKH_ERR_ARG beyond them): decode addresses one KV head's
 * rows of one layer (of one sequence, in a batch) with 32-bit offsets, so
 * (attended rows + 1) * stride_pos * element size must stay below 2 GiB --
 * about 2.09M positions for an fp32 cache of head_dim 128 in the default
 * layout.  Prefill covers at most 2,097,088 positions (pos0 + n_tokens),
 * 1,945,184 for head_dim 256.
 */
#ifndef PKH_ATTN_H
#define PKH_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: same values as src/pickle.h:52-60. */
#define PKH_OK          0
#define PKH_ERR_MEMORY -3   /* device allocation failed           */
#define PKH_ERR_IO     -5   /* HIP runtime or launch failure       */
#define PKH_ERR_ARG    -6   /* bad argument or unsupported shape   */
#define PKH_ERR_RANGE  -7   /* position or layer out of range      */

/* KV element types: the ggml_type values of src/pickle.h:85-87. */
#define PKH_KV_F32 0
#define PKH_KV_F16 1

/* ------------------------------------------------------------------ */
/* Library                                                            */
/* ------------------------------------------------------------------ */

/* Select the HIP device used by every later call (default 0).  Optional. */
int pkh_init(int device);

/* Version string of this library. */
const char* pkh_version(void);

/* ------------------------------------------------------------------ */
/* Device KV cache                                                    */
/* ------------------------------------------------------------------ */

/* Device-resident mirror of pickle_fast_kv_t (src/pickle_fast.h:145-154).
 * The first eight fields have the reference's names and meaning; k and v are
 * device pointers of element type dtype, and the placement of element
 * (layer L, position p, KV head g, dim d) is given by strides in elements:
 *     k + L*k_stride_layer + g*stride_head + p*stride_pos + d
 * (v likewise from v + L*v_stride_layer).  pkh_kv_alloc lays each layer out
 * head-major with a position's K and V rows side by side (stride_pos =
 * 2*head_dim, stride_head = max_seq*2*head_dim, v = k + head_dim), so a
 * decode work item streams one contiguous block per KV head.  The
 * reference's own layout [layer][pos][kv_head][dim] is the strides
 * stride_pos = n_kv_heads*head_dim, stride_head = head_dim with separate K
 * and V buffers; the kernels accept either. */
typedef struct {
    int    n_layers;
    int    n_kv_heads;
    int    head_dim;
    int    max_seq;
    size_t k_stride_layer;   /* elements between layers of K */
    size_t v_stride_layer;   /* elements between layers of V */
    void*  k;                /* device; for pkh_kv_alloc the allocation base */
    void*  v;                /* device */
    int    dtype;            /* PKH_KV_F32 or PKH_KV_F16 */
    int    device;
    size_t stride_pos;       /* elements between positions p and p+1 of a head */
    size_t stride_head;      /* elements between KV heads g and g+1 */
} pkh_kv_t;

/* Replaces pickle_fast_kv_alloc (src/pickle_fast.c:1793-1810): one zeroed
 * device allocation holding K and V, n_layers * max_seq * n_kv_heads *
 * head_dim elements each, in the head-major layout above; when head_dim is
 * not a multiple of 8 each row is padded to the next multiple of 8 elements
 * (stride_pos = 2 * that, v = k + that), so every row starts 16-byte
 * aligned.  PKH_ERR_MEMORY if the device cannot hold it (the struct is
 * zeroed). */
int  pkh_kv_alloc(int n_layers, int n_kv_heads, int head_dim, int max_seq,
                  int dtype, pkh_kv_t* kv);

/* Replaces pickle_fast_kv_free (src/pickle_fast.c:1811-1817). */
void pkh_kv_free(pkh_kv_t* kv);

/* Copy n_pos cache rows of one layer between host and device (dir 0:
 * device -> host, 1: host -> device).  Host rows are in the reference's
 * layout [pos][kv_head][head_dim] and the cache's dtype (fp16 as uint16 bit
 * patterns), whatever the device strides.  For callers that seed or inspect
 * a cache; the reference reads kv->k/v directly (src/pickle_fast.h:153). */
int  pkh_kv_copy_rows(const pkh_kv_t* kv, int which_v, int layer, int pos0,
                      int n_pos, void* host, int dir);

/* ------------------------------------------------------------------ */
/* Device RoPE table                                                  */
/* ------------------------------------------------------------------ */

/* Device copy of the fast state's sin/cos tables (src/pickle_fast.h:90-95):
 * [max_seq][half] each, half = min(head_dim / 2, 64). */
typedef struct {
    int    max_seq;
    int    half;
    int    filled_upto;      /* rows [0, filled_upto) are on the device */
    float* sin;              /* device */
    float* cos;              /* device */
    int    device;
} pkh_rope_t;

int  pkh_rope_alloc(int max_seq, int half, pkh_rope_t* rope);
void pkh_rope_free(pkh_rope_t* rope);

/* Upload host rows [rope->filled_upto, filled_upto) of the tables that
 * pickle_fast_state_extend_rope fills (src/pickle_fast.c:1772-1788); call it
 * with state->rope_sin, state->rope_cos, state->rope_filled_upto after each
 * extension.  Rows already on the device are not sent again. */
int  pkh_rope_upload(pkh_rope_t* rope, const float* sin_tab,
                     const float* cos_tab, int filled_upto);

/* Host-side table fill with the reference's formulas (src/pickle_fast.c:
 * 1638-1640 and 1779-1786), for callers that have no pickle_fast_state_t:
 * inv_freq[i] = 1 / theta^((2i)/head_dim); rows p of sin/cos for
 * p in [p_begin, p_last] with angle = inv_freq[i] * (float)p. */
void pkh_rope_host_tables(int head_dim, float theta, int p_begin, int p_last,
                          float* inv_freq, float* sin_tab, float* cos_tab);

/* ------------------------------------------------------------------ */
/* Decode: one token of one sequence on one layer                    */
/* ------------------------------------------------------------------ */

/* Replaces src/pickle_fast.c:1910-2094 for kv != NULL: rotate q and k with
 * table row pos, write (k_rot, v) into cache row pos of `layer`, attend all
 * n_heads query heads over rows [0, pos], write ao.  Host pointers; blocks
 * until ao is written.  pos >= kv->max_seq or pos >= rope->filled_upto
 * returns PKH_ERR_RANGE before any device work (src/pickle_fast.c:1885). */
int pkh_attn_decode(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer,
                    int pos, int n_heads, const float* q, const float* k,
                    const float* v, float* ao);

/* Same with device pointers, enqueued on `stream`. */
int pkh_attn_decode_async(const pkh_kv_t* kv, const pkh_rope_t* rope,
                          int layer, int pos, int n_heads, const float* d_q,
                          const float* d_k, const float* d_v, float* d_ao,
                          void* stream);

/* pkh_attn_decode_async that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory during
 * the call (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, kernels and results as
 * pkh_attn_decode_async; the split-K partials and ready flags live in a
 * fixed 8 MiB device array per device (64 KiB of it flags), set up by
 * pkh_init or by the first call on a device, instead of the library's
 * grow-only scratch.  A call whose split needs more (more than 16,384 work
 * items, or more than 8,323,072 bytes of partials: about 500K positions at
 * the Llama-3-8B shape) returns PKH_ERR_ARG with a line on stderr.  All
 * calls on one device share that array: calls that overlap in time on one
 * device race (order them on one stream). */
int pkh_attn_decode_noalloc_async(const pkh_kv_t* kv, const pkh_rope_t* rope,
                                  int layer, int pos, int n_heads,
                                  const float* d_q, const float* d_k,
                                  const float* d_v, float* d_ao, void* stream);

/* ------------------------------------------------------------------ */
/* Causal prefill: n_tokens consecutive tokens of one sequence        */
/* ------------------------------------------------------------------ */

/* Replaces the token loop of src/pickle_fast.c:1881-1898 for the attention
 * block: row i of q [n][H][D], k/v [n][HK][D] is the token at pos0 + i; its
 * rotated k and v are written into cache rows pos0 + i and it attends rows
 * [0, pos0 + i].  Q.K^T and P.V run on MFMA with fp16 operands and fp32
 * accumulation; softmax is fp32.  Host pointers; blocks until done. */
int pkh_attn_prefill(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer,
                     int pos0, int n_tokens, int n_heads, const float* q,
                     const float* k, const float* v, float* ao);

int pkh_attn_prefill_async(const pkh_kv_t* kv, const pkh_rope_t* rope,
                           int layer, int pos0, int n_tokens, int n_heads,
                           const float* d_q, const float* d_k,
                           const float* d_v, float* d_ao, void* stream);

/* ------------------------------------------------------------------ */
/* Ragged multi-sequence decode                                       */
/* ------------------------------------------------------------------ */

/* Several sequences' caches in one allocation: sequence s owns slots
 * [slot0[s], slot0[s] + max_seq[s]) of every layer and KV head, each slot
 * one head_dim row of K and one of V.  Element (L, s, p, g, d) of K is at
 *     k + L*layer_stride + g*stride_head + (slot0[s] + p)*stride_pos + d
 * (V likewise from v).  pkh_kv_batch_alloc uses the head-major layout of
 * pkh_kv_alloc.  No counterpart in the reference, which keeps one sequence
 * per pickle_fast_kv_t (src/pickle_fast.h:140-157). */
typedef struct {
    int      n_layers;
    int      n_kv_heads;
    int      head_dim;
    int      n_seqs;
    int      dtype;
    int      device;
    size_t   layer_stride;   /* elements between layers */
    int64_t* slot0;          /* host [n_seqs + 1], prefix sum of max_seq */
    int*     max_seq;        /* host [n_seqs] */
    void*    k;              /* device; the allocation base */
    void*    v;              /* device */
    void*    d_slot0;        /* device copy of slot0 */
    size_t   stride_pos;
    size_t   stride_head;
} pkh_kv_batch_t;

int  pkh_kv_batch_alloc(int n_layers, int n_kv_heads, int head_dim,
                        int n_seqs, const int* max_seq, int dtype,
                        pkh_kv_batch_t* kvb);
void pkh_kv_batch_free(pkh_kv_batch_t* kvb);

/* A decode plan: the positions of the next token of every sequence and the
 * split of each sequence's context into work items of a fixed size (chosen
 * from the positions given to pkh_plan_create).  The plan's grid covers each
 * sequence's whole capacity (max_seq[s]), so the same plan -- and a HIP
 * graph captured around the decode calls that use it -- serves every later
 * step: move the positions with pkh_plan_update, which allocates nothing and
 * does not synchronize the device.  pkh_plan_create allocates and copies
 * synchronously; call it once, outside any capture. */
typedef struct pkh_plan pkh_plan_t;

int  pkh_plan_create(const pkh_kv_batch_t* kvb, const int* pos, int n_heads,
                     pkh_plan_t** plan);
void pkh_plan_free(pkh_plan_t* plan);

/* The positions of the next step, pos[s] for each sequence, written into the
 * plan's device copy on `stream` (hipMemcpyAsync; no allocation, no device
 * synchronization).  pos[s] outside [0, max_seq[s]) returns PKH_ERR_RANGE
 * and enqueues nothing.  The copy reads pos when the stream reaches it:
 * pageable memory is read before the call returns; pinned memory is read
 * later, so keep it unchanged until then.  Under stream capture the copy is
 * recorded as a graph node that reads pinned pos on every replay: changing
 * that pinned array between replays advances a captured step (the host
 * cannot check replayed positions; a position past a sequence's capacity
 * gives NaN for that sequence and writes no cache row).  No counterpart in
 * the reference (docs/ROADMAP.md:56-58 plans continuous batching). */
int  pkh_plan_update(pkh_plan_t* plan, const int* pos, void* stream);

/* One decode step of every sequence on one layer: q [n_seqs][H][D],
 * k/v [n_seqs][HK][D], ao [n_seqs][H][D], device pointers. */
int pkh_attn_decode_batch_async(const pkh_kv_batch_t* kvb,
                                const pkh_rope_t* rope, const pkh_plan_t* plan,
                                int layer, const float* d_q, const float* d_k,
                                const float* d_v, float* d_ao, void* stream);

/* Causal prefill of n_tokens tokens of sequence `seq` into its slots of a
 * batch cache, as pkh_attn_prefill_async does for a single cache (the token
 * loop of src/pickle_fast.c:1881-1898 for one sequence): rows pos0 + i of
 * sequence seq receive the rotated k and v, and each token attends that
 * sequence's rows [0, pos0 + i].  Device pointers: q [n][H][D], k/v
 * [n][HK][D], ao [n][H][D]. */
int pkh_attn_prefill_batch_async(const pkh_kv_batch_t* kvb, const pkh_rope_t* rope,
                                 int seq, int layer, int pos0, int n_tokens,
                                 int n_heads, const float* d_q, const float* d_k,
                                 const float* d_v, float* d_ao, void* stream);

/* Copy n_pos rows of sequence `seq` of one layer between host and device
 * (dir 0: device -> host, 1: host -> device); host rows as for
 * pkh_kv_copy_rows. */
int pkh_kv_batch_copy_rows(const pkh_kv_batch_t* kvb, int which_v, int layer,
                           int seq, int pos0, int n_pos, void* host, int dir);

/* ------------------------------------------------------------------ */
/* Tuning                                                             */
/* ------------------------------------------------------------------ */

/* Decode split size: positions per work item (0 = automatic).  Values are
 * rounded up to the kernel's tile.  Returns the previous setting. */
int pkh_tune_decode_chunk(int positions);

/* Bound on the split-K merger's wait for the other work items' partials, in
 * polling rounds (negative = the default, 65,536, which is never reached in
 * a normal launch).  A wait that runs out writes NaN for the heads it merges
 * and leaves no state behind that could affect a later call; 0 makes every
 * multi-chunk decode give up at once, which tests use to force that path
 * from the host.  Returns the previous setting. */
int pkh_tune_decode_wait(int rounds);

#ifdef __cplusplus
}
#endif
#endif /* PKH_ATTN_H */
