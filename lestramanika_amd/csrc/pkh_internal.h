// pkh_internal.h -- shared declarations of the HIP attention library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "pkh_attn.h"

namespace pkh {

// Map a HIP error to a PKH_ERR_* code, with one line on stderr naming the call.
int hip_fail(hipError_t e, const char* what);

#define PKH_HIP(expr)                                                  \
    do {                                                               \
        hipError_t pkh_e_ = (expr);                                    \
        if (pkh_e_ != hipSuccess) return ::pkh::hip_fail(pkh_e_, #expr); \
    } while (0)

// Per-device grow-only scratch owned by the library (split-K partials).
int scratch_get(size_t bytes, void** out);

// Per-device grow-only array of n ints that is zero between launches: it is
// zeroed when (re)allocated, and every kernel that counts in it returns the
// counts it used to zero before it exits.  Kept apart from the scratch so
// that partials of one launch never land where a later launch counts.
int counters_get(size_t n, int** out);

// Per-device grow-only staging buffers for the host-pointer entry points.
int staging_get(int slot, size_t bytes, void** out);

// Per-device grow-only buffer for the fp16 K/V tiles staged by prefill.
int tiles_get(size_t bytes, void** out);

// Current device of the library.
int current_device();

// Largest head_dim the kernels take (rows are processed at a padded width,
// the next of 16, 32, 64, 128, 256).
constexpr int kMaxHeadDim = 256;

// Padded width for head_dim: 16, 32, 64, 128 or 256; 0 if unsupported.
int padded_head_dim(int head_dim);

// Query heads of one launch's workgroup ("head slot"): G in {1, 2, 4, 8}
// heads of one KV head, nsub slots per KV head.  Query head h reads KV head
// h*HK/H (src/pickle_fast.c:1963); gmax bounds G.
struct HeadSlots {
    int G;
    int nsub;
};
HeadSlots head_slots(int n_heads, int n_kv_heads, int gmax);

// True for every shape the decode kernels take: 1 <= head_dim <= 256, any
// n_heads, n_kv_heads >= 1.
bool shape_supported(int head_dim, int n_heads, int n_kv_heads);

// ---- decode ------------------------------------------------------------

// One decode launch: n_seqs sequences (1 for the single-sequence path),
// each with its own position and slot base inside one layer's cache.
struct DecodeArgs {
    const void* k_layer;      // layer base, element type per dtype
    const void* v_layer;
    long long stride_pos;     // elements between positions of one head
    long long stride_head;    // elements between heads
    int dtype;                // PKH_KV_F32 / PKH_KV_F16
    int head_dim, n_heads, n_kv_heads;
    int n_seqs;
    // single sequence (n_seqs == 1 and seq arrays null):
    int pos;
    long long slot0;
    // ragged (device arrays, n_seqs entries; chunk_start has n_seqs + 1):
    const long long* d_seq_slot0;
    const int* d_seq_pos;
    const int* d_chunk_start;
    int total_chunks;         // sum of chunks over sequences
    int max_chunks;           // largest per-sequence chunk count
    int chunk;                // positions per work item
    const float* q;           // [n_seqs][H][D]
    const float* k_new;       // [n_seqs][HK][D]
    const float* v_new;
    float* out;               // [n_seqs][H][D]
    const float* rope_sin;    // [max_seq][half]
    const float* rope_cos;
    int half;
};

// Positions per work item for a context of attend_n rows (tile-aligned).
int decode_chunk_for(int head_dim, int n_heads, int n_kv_heads, int dtype, long long total_rows,
                     int max_attend);
int decode_tile_positions(int head_dim, int dtype);

// no_alloc: take the split-K partials and flags from the library's fixed
// device scratch (PKH_ERR_ARG when they do not fit) instead of the grow-only
// buffers; nothing is allocated.
int launch_decode(const DecodeArgs& a, hipStream_t stream, bool no_alloc = false);

// Set up the fixed no-alloc scratch of `device` (the current device): look up
// its address and clear its flags with a kernel on `stream`.  Once per device.
int noalloc_setup(int device, hipStream_t stream);
int noalloc_workspace(size_t part_bytes, size_t n_flags, hipStream_t stream, void** part,
                      int** flags);

// ---- prefill -----------------------------------------------------------

struct PrefillArgs {
    void* k_layer;            // fp32 or fp16 cache, layer base
    void* v_layer;
    long long stride_pos;
    long long stride_head;
    int dtype;
    int head_dim, n_heads, n_kv_heads;
    int pos0, n_tokens;
    const float* q;           // [n][H][D]
    const float* k_new;       // [n][HK][D]
    const float* v_new;
    float* out;               // [n][H][D]
    const float* rope_sin;
    const float* rope_cos;
    int half;
};

bool prefill_supported(int head_dim, int n_heads, int n_kv_heads, int dtype);
int launch_prefill(const PrefillArgs& a, hipStream_t stream);

}  // namespace pkh
