// pkh_api.hip -- the C ABI of include/pkh_attn.h: device KV caches, the
// device RoPE table, argument checking and the host-pointer entry points.

#include "pkh_internal.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace pkh {

namespace {

constexpr int kMaxDevices = 16;

struct Buf {
    void* ptr = nullptr;
    size_t bytes = 0;
};

int g_device = 0;
Buf g_scratch[kMaxDevices];
Buf g_staging[kMaxDevices][4];
Buf g_tiles[kMaxDevices];
Buf g_counters[kMaxDevices];
Buf g_pinned[kMaxDevices];        // pinned host staging of the host-pointer entry points

// Buffers outgrown by a larger call.  They are never freed: a HIP graph
// captured earlier holds their addresses and may still be replayed.  Growth
// at least doubles, so what is retired stays below the live buffer's size.
std::vector<void*> g_retired;

int grow(Buf& b, size_t bytes, void** out) {
    if (bytes <= b.bytes && b.ptr) {
        *out = b.ptr;
        return PKH_OK;
    }
    size_t want = bytes < 1024 ? 1024 : bytes;
    if (b.ptr && want < 2 * b.bytes) want = 2 * b.bytes;
    void* p = nullptr;
    PKH_HIP(hipMalloc(&p, want));
    if (b.ptr) g_retired.push_back(b.ptr);
    b.ptr = p;
    b.bytes = want;
    *out = b.ptr;
    return PKH_OK;
}

size_t elem_size(int dtype) { return dtype == PKH_KV_F16 ? 2 : 4; }

// Elements per K (or V) row in the library's own cache layouts.
size_t row_pitch(int head_dim) { return ((size_t)head_dim + 7) / 8 * 8; }

bool mul_ok(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > SIZE_MAX / a) return false;
    *out = a * b;
    return true;
}

}  // namespace

int hip_fail(hipError_t e, const char* what) {
    std::fprintf(stderr, "pkh: %s failed: %s\n", what, hipGetErrorString(e));
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();   // clear the sticky-free error state
        return PKH_ERR_MEMORY;
    }
    return PKH_ERR_IO;
}

int current_device() { return g_device; }

int scratch_get(size_t bytes, void** out) { return grow(g_scratch[g_device], bytes, out); }

int counters_get(size_t n, int** out) {
    Buf& b = g_counters[g_device];
    const size_t bytes = n * sizeof(int);
    const bool fresh = !(bytes <= b.bytes && b.ptr);
    void* p = nullptr;
    int rc = grow(b, bytes, &p);
    if (rc != PKH_OK) return rc;
    if (fresh) {
        // A new counter buffer starts zeroed, before any kernel can use it.
        PKH_HIP(hipMemset(b.ptr, 0, b.bytes));
        PKH_HIP(hipDeviceSynchronize());
    }
    *out = static_cast<int*>(p);
    return PKH_OK;
}

int staging_get(int slot, size_t bytes, void** out) {
    return grow(g_staging[g_device][slot], bytes, out);
}

int tiles_get(size_t bytes, void** out) { return grow(g_tiles[g_device], bytes, out); }

// Pinned host staging for the host-pointer entry points.  Nothing captured
// refers to it (those entry points synchronize), so an outgrown buffer is
// freed.
int pinned_get(size_t bytes, void** out) {
    Buf& b = g_pinned[g_device];
    if (bytes <= b.bytes && b.ptr) {
        *out = b.ptr;
        return PKH_OK;
    }
    size_t want = bytes < 65536 ? 65536 : bytes;
    if (b.ptr && want < 2 * b.bytes) want = 2 * b.bytes;
    void* p = nullptr;
    PKH_HIP(hipHostMalloc(&p, want, hipHostMallocDefault));
    if (b.ptr) (void)hipHostFree(b.ptr);
    b.ptr = p;
    b.bytes = want;
    *out = p;
    return PKH_OK;
}

// Host-pointer calls: q, k, v (and ao) in one pinned block and one device
// block, each segment 256-byte aligned, so a call costs one upload and one
// download.
struct HostStage {
    char* host = nullptr;
    char* dev = nullptr;
    size_t off_k = 0, off_v = 0, off_ao = 0, in_bytes = 0, out_bytes = 0;
};

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

int host_stage(size_t q_bytes, size_t kv_bytes, size_t ao_bytes, HostStage* hs) {
    hs->off_k = align256(q_bytes);
    hs->off_v = hs->off_k + align256(kv_bytes);
    hs->in_bytes = hs->off_v + kv_bytes;
    hs->off_ao = align256(hs->in_bytes);
    hs->out_bytes = ao_bytes;
    void *h = nullptr, *d = nullptr;
    int rc = pinned_get(hs->off_ao + ao_bytes, &h);
    if (rc != PKH_OK) return rc;
    rc = staging_get(0, hs->off_ao + ao_bytes, &d);
    if (rc != PKH_OK) return rc;
    hs->host = static_cast<char*>(h);
    hs->dev = static_cast<char*>(d);
    return PKH_OK;
}

}  // namespace pkh

using namespace pkh;

// ---------------------------------------------------------------------------
// Library
// ---------------------------------------------------------------------------

extern "C" int pkh_init(int device) {
    int n = 0;
    PKH_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n || device >= kMaxDevices) return PKH_ERR_ARG;
    PKH_HIP(hipSetDevice(device));
    g_device = device;
    // The no-alloc decode's fixed scratch on this device, set up once.
    int rc = noalloc_setup(device, nullptr);
    if (rc != PKH_OK) return rc;
    PKH_HIP(hipStreamSynchronize(nullptr));
    return PKH_OK;
}

extern "C" const char* pkh_version(void) { return "pkh-attn 0.1.0 (gfx950)"; }

// ---------------------------------------------------------------------------
// KV cache
// ---------------------------------------------------------------------------

extern "C" int pkh_kv_alloc(int n_layers, int n_kv_heads, int head_dim, int max_seq,
                            int dtype, pkh_kv_t* kv) {
    if (!kv) return PKH_ERR_ARG;
    std::memset(kv, 0, sizeof(*kv));
    if (n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_seq <= 0) return PKH_ERR_ARG;
    if (dtype != PKH_KV_F32 && dtype != PKH_KV_F16) return PKH_ERR_ARG;
    // Per layer: [kv_head][pos][K row | V row], each row padded to a multiple
    // of 8 elements (16-byte aligned rows for both element types; the padding
    // stays zero).
    const size_t dp = row_pitch(head_dim);
    size_t head, layer, total, bytes;
    if (!mul_ok((size_t)max_seq, 2 * dp, &head) ||
        !mul_ok(head, (size_t)n_kv_heads, &layer) || !mul_ok(layer, (size_t)n_layers, &total) ||
        !mul_ok(total, elem_size(dtype), &bytes))
        return PKH_ERR_MEMORY;
    PKH_HIP(hipSetDevice(g_device));
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(kv)");
    // The reference's cache is calloc'ed (src/pickle_fast.c:1803-1804).
    e = hipMemset(base, 0, bytes);
    if (e != hipSuccess) {
        (void)hipFree(base);
        return hip_fail(e, "hipMemset(kv)");
    }
    kv->n_layers = n_layers;
    kv->n_kv_heads = n_kv_heads;
    kv->head_dim = head_dim;
    kv->max_seq = max_seq;
    kv->k_stride_layer = layer;
    kv->v_stride_layer = layer;
    kv->k = base;
    kv->v = (char*)base + dp * elem_size(dtype);
    kv->dtype = dtype;
    kv->device = g_device;
    kv->stride_pos = 2 * dp;
    kv->stride_head = head;
    return PKH_OK;
}

extern "C" void pkh_kv_free(pkh_kv_t* kv) {
    if (!kv) return;
    if (kv->k) {
        (void)hipDeviceSynchronize();
        (void)hipFree(kv->k);   // one allocation; v points inside it
    }
    std::memset(kv, 0, sizeof(*kv));
}

namespace {

// Copy rows [pos0, pos0 + n_pos) of every KV head between a host block in the
// reference layout [pos][kv_head][head_dim] and a strided device layer.
int copy_rows_strided(char* dev_layer, size_t stride_pos, size_t stride_head, int n_kv_heads,
                      int head_dim, size_t es, size_t row0, int n_pos, void* host, int dir) {
    if (n_pos == 0) return PKH_OK;
    const size_t width = (size_t)head_dim * es;
    const size_t hpitch = (size_t)n_kv_heads * head_dim * es;
    for (int g = 0; g < n_kv_heads; g++) {
        char* d = dev_layer + ((size_t)g * stride_head + row0 * stride_pos) * es;
        char* h = (char*)host + (size_t)g * width;
        if (dir == 0)
            PKH_HIP(hipMemcpy2D(h, hpitch, d, stride_pos * es, width, (size_t)n_pos,
                                hipMemcpyDeviceToHost));
        else
            PKH_HIP(hipMemcpy2D(d, stride_pos * es, h, hpitch, width, (size_t)n_pos,
                                hipMemcpyHostToDevice));
    }
    return PKH_OK;
}

}  // namespace

extern "C" int pkh_kv_copy_rows(const pkh_kv_t* kv, int which_v, int layer, int pos0,
                                int n_pos, void* host, int dir) {
    if (!kv || !kv->k || !kv->v || !host || n_pos < 0) return PKH_ERR_ARG;
    if (layer < 0 || layer >= kv->n_layers || pos0 < 0 || (long long)pos0 + n_pos > kv->max_seq)
        return PKH_ERR_RANGE;
    const size_t es = elem_size(kv->dtype);
    char* base = (char*)(which_v ? kv->v : kv->k) +
                 (size_t)layer * (which_v ? kv->v_stride_layer : kv->k_stride_layer) * es;
    return copy_rows_strided(base, kv->stride_pos, kv->stride_head, kv->n_kv_heads, kv->head_dim,
                             es, (size_t)pos0, n_pos, host, dir);
}

// ---------------------------------------------------------------------------
// RoPE table
// ---------------------------------------------------------------------------

extern "C" int pkh_rope_alloc(int max_seq, int half, pkh_rope_t* rope) {
    if (!rope) return PKH_ERR_ARG;
    std::memset(rope, 0, sizeof(*rope));
    if (max_seq <= 0 || half < 0 || half > 64) return PKH_ERR_ARG;
    // half == 0 (head_dim 1): a table of no columns; a token allocation.
    const size_t bytes = half ? (size_t)max_seq * half * sizeof(float) : 16;
    PKH_HIP(hipSetDevice(g_device));
    float* s = nullptr;
    float* c = nullptr;
    hipError_t e = hipMalloc(&s, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(rope.sin)");
    e = hipMalloc(&c, bytes);
    if (e != hipSuccess) {
        (void)hipFree(s);
        return hip_fail(e, "hipMalloc(rope.cos)");
    }
    rope->max_seq = max_seq;
    rope->half = half;
    rope->filled_upto = 0;
    rope->sin = s;
    rope->cos = c;
    rope->device = g_device;
    return PKH_OK;
}

extern "C" void pkh_rope_free(pkh_rope_t* rope) {
    if (!rope) return;
    if (rope->sin || rope->cos) {
        (void)hipDeviceSynchronize();
        (void)hipFree(rope->sin);
        (void)hipFree(rope->cos);
    }
    std::memset(rope, 0, sizeof(*rope));
}

extern "C" int pkh_rope_upload(pkh_rope_t* rope, const float* sin_tab, const float* cos_tab,
                               int filled_upto) {
    if (!rope || !rope->sin || !sin_tab || !cos_tab) return PKH_ERR_ARG;
    if (filled_upto > rope->max_seq) return PKH_ERR_RANGE;
    if (filled_upto <= rope->filled_upto) return PKH_OK;
    const size_t off = (size_t)rope->filled_upto * rope->half;
    const size_t n = (size_t)(filled_upto - rope->filled_upto) * rope->half;
    PKH_HIP(hipMemcpy(rope->sin + off, sin_tab + off, n * sizeof(float), hipMemcpyHostToDevice));
    PKH_HIP(hipMemcpy(rope->cos + off, cos_tab + off, n * sizeof(float), hipMemcpyHostToDevice));
    rope->filled_upto = filled_upto;
    return PKH_OK;
}

// ---------------------------------------------------------------------------
// Decode
// ---------------------------------------------------------------------------

namespace {

// The host-pointer entry points' transfers around `launch` (which enqueues
// on the null stream): q, k and v copied into the pinned block and sent in
// one upload, ao returned in one download.
template <typename Launch>
int host_call(size_t q_bytes, size_t kv_bytes, const float* q, const float* k, const float* v,
              float* ao, Launch launch) {
    HostStage hs;
    int rc = host_stage(q_bytes, kv_bytes, q_bytes, &hs);
    if (rc != PKH_OK) return rc;
    std::memcpy(hs.host, q, q_bytes);
    std::memcpy(hs.host + hs.off_k, k, kv_bytes);
    std::memcpy(hs.host + hs.off_v, v, kv_bytes);
    PKH_HIP(hipMemcpyAsync(hs.dev, hs.host, hs.in_bytes, hipMemcpyHostToDevice, nullptr));
    rc = launch(hs.dev, hs);
    if (rc != PKH_OK) {
        (void)hipStreamSynchronize(nullptr);   // the upload still reads the pinned block
        return rc;
    }
    PKH_HIP(hipMemcpyAsync(hs.host + hs.off_ao, hs.dev + hs.off_ao, hs.out_bytes,
                           hipMemcpyDeviceToHost, nullptr));
    PKH_HIP(hipStreamSynchronize(nullptr));
    std::memcpy(ao, hs.host + hs.off_ao, hs.out_bytes);
    return PKH_OK;
}

int check_common(int head_dim, int n_heads, int n_kv_heads, const pkh_rope_t* rope) {
    if (!shape_supported(head_dim, n_heads, n_kv_heads)) return PKH_ERR_ARG;
    if (!rope || !rope->sin || !rope->cos) return PKH_ERR_ARG;
    const int half = head_dim / 2 > 64 ? 64 : head_dim / 2;
    if (rope->half != half) return PKH_ERR_ARG;
    return PKH_OK;
}

int decode_checked(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer, int pos, int n_heads,
                   const float* d_q, const float* d_k, const float* d_v, float* d_ao,
                   hipStream_t st, bool no_alloc = false) {
    const int HK = kv->n_kv_heads, D = kv->head_dim;
    DecodeArgs a{};
    const size_t es = elem_size(kv->dtype);
    a.k_layer = (const char*)kv->k + (size_t)layer * kv->k_stride_layer * es;
    a.v_layer = (const char*)kv->v + (size_t)layer * kv->v_stride_layer * es;
    a.stride_pos = (long long)kv->stride_pos;
    a.stride_head = (long long)kv->stride_head;
    a.dtype = kv->dtype;
    a.head_dim = D;
    a.n_heads = n_heads;
    a.n_kv_heads = HK;
    a.n_seqs = 1;
    a.pos = pos;
    a.slot0 = 0;
    const int attend_n = pos + 1;
    a.chunk = decode_chunk_for(D, n_heads, HK, kv->dtype, attend_n, attend_n);
    a.total_chunks = (attend_n + a.chunk - 1) / a.chunk;
    a.max_chunks = a.total_chunks;
    a.q = d_q;
    a.k_new = d_k;
    a.v_new = d_v;
    a.out = d_ao;
    a.rope_sin = rope->sin;
    a.rope_cos = rope->cos;
    a.half = rope->half;
    return launch_decode(a, st, no_alloc);
}

bool strides_ok(size_t stride_pos, size_t stride_head, int head_dim) {
    return stride_pos >= (size_t)head_dim && stride_head >= (size_t)head_dim &&
           stride_pos % 8 == 0 && stride_head % 8 == 0;
}

int decode_validate(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer, int pos, int n_heads) {
    if (!kv || !kv->k || !kv->v) return PKH_ERR_ARG;
    if (!strides_ok(kv->stride_pos, kv->stride_head, kv->head_dim)) return PKH_ERR_ARG;
    int rc = check_common(kv->head_dim, n_heads, kv->n_kv_heads, rope);
    if (rc != PKH_OK) return rc;
    if (layer < 0 || layer >= kv->n_layers) return PKH_ERR_RANGE;
    if (pos < 0 || pos >= kv->max_seq || pos >= rope->filled_upto) return PKH_ERR_RANGE;
    return PKH_OK;
}

}  // namespace

extern "C" int pkh_attn_decode_async(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer,
                                     int pos, int n_heads, const float* d_q, const float* d_k,
                                     const float* d_v, float* d_ao, void* stream) {
    int rc = decode_validate(kv, rope, layer, pos, n_heads);
    if (rc != PKH_OK) return rc;
    if (!d_q || !d_k || !d_v || !d_ao) return PKH_ERR_ARG;
    return decode_checked(kv, rope, layer, pos, n_heads, d_q, d_k, d_v, d_ao,
                          (hipStream_t)stream);
}

extern "C" int pkh_attn_decode_noalloc_async(const pkh_kv_t* kv, const pkh_rope_t* rope,
                                             int layer, int pos, int n_heads, const float* d_q,
                                             const float* d_k, const float* d_v, float* d_ao,
                                             void* stream) {
    int rc = decode_validate(kv, rope, layer, pos, n_heads);
    if (rc != PKH_OK) return rc;
    if (!d_q || !d_k || !d_v || !d_ao) return PKH_ERR_ARG;
    return decode_checked(kv, rope, layer, pos, n_heads, d_q, d_k, d_v, d_ao,
                          (hipStream_t)stream, true);
}

extern "C" int pkh_attn_decode(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer, int pos,
                               int n_heads, const float* q, const float* k, const float* v,
                               float* ao) {
    int rc = decode_validate(kv, rope, layer, pos, n_heads);
    if (rc != PKH_OK) return rc;
    if (!q || !k || !v || !ao) return PKH_ERR_ARG;
    const size_t qb = (size_t)n_heads * kv->head_dim * sizeof(float);
    const size_t kb = (size_t)kv->n_kv_heads * kv->head_dim * sizeof(float);
    return host_call(qb, kb, q, k, v, ao, [&](const char* d, const HostStage& hs) {
        return decode_checked(kv, rope, layer, pos, n_heads, (const float*)d,
                              (const float*)(d + hs.off_k), (const float*)(d + hs.off_v),
                              (float*)(d + hs.off_ao), nullptr);
    });
}

// ---------------------------------------------------------------------------
// Prefill
// ---------------------------------------------------------------------------

namespace {

int prefill_validate(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer, int pos0,
                     int n_tokens, int n_heads) {
    if (!kv || !kv->k || !kv->v) return PKH_ERR_ARG;
    if (!strides_ok(kv->stride_pos, kv->stride_head, kv->head_dim)) return PKH_ERR_ARG;
    int rc = check_common(kv->head_dim, n_heads, kv->n_kv_heads, rope);
    if (rc != PKH_OK) return rc;
    if (!prefill_supported(kv->head_dim, n_heads, kv->n_kv_heads, kv->dtype)) return PKH_ERR_ARG;
    if (n_tokens <= 0) return PKH_ERR_ARG;
    if (layer < 0 || layer >= kv->n_layers) return PKH_ERR_RANGE;
    const long long last = (long long)pos0 + n_tokens - 1;
    if (pos0 < 0 || last >= kv->max_seq || last >= rope->filled_upto) return PKH_ERR_RANGE;
    return PKH_OK;
}

int prefill_checked(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer, int pos0,
                    int n_tokens, int n_heads, const float* d_q, const float* d_k,
                    const float* d_v, float* d_ao, hipStream_t st) {
    PrefillArgs a{};
    const size_t es = elem_size(kv->dtype);
    a.k_layer = (char*)kv->k + (size_t)layer * kv->k_stride_layer * es;
    a.v_layer = (char*)kv->v + (size_t)layer * kv->v_stride_layer * es;
    a.stride_pos = (long long)kv->stride_pos;
    a.stride_head = (long long)kv->stride_head;
    a.dtype = kv->dtype;
    a.head_dim = kv->head_dim;
    a.n_heads = n_heads;
    a.n_kv_heads = kv->n_kv_heads;
    a.pos0 = pos0;
    a.n_tokens = n_tokens;
    a.q = d_q;
    a.k_new = d_k;
    a.v_new = d_v;
    a.out = d_ao;
    a.rope_sin = rope->sin;
    a.rope_cos = rope->cos;
    a.half = rope->half;
    return launch_prefill(a, st);
}

}  // namespace

extern "C" int pkh_attn_prefill_async(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer,
                                      int pos0, int n_tokens, int n_heads, const float* d_q,
                                      const float* d_k, const float* d_v, float* d_ao,
                                      void* stream) {
    int rc = prefill_validate(kv, rope, layer, pos0, n_tokens, n_heads);
    if (rc != PKH_OK) return rc;
    if (!d_q || !d_k || !d_v || !d_ao) return PKH_ERR_ARG;
    return prefill_checked(kv, rope, layer, pos0, n_tokens, n_heads, d_q, d_k, d_v, d_ao,
                           (hipStream_t)stream);
}

extern "C" int pkh_attn_prefill(const pkh_kv_t* kv, const pkh_rope_t* rope, int layer, int pos0,
                                int n_tokens, int n_heads, const float* q, const float* k,
                                const float* v, float* ao) {
    int rc = prefill_validate(kv, rope, layer, pos0, n_tokens, n_heads);
    if (rc != PKH_OK) return rc;
    if (!q || !k || !v || !ao) return PKH_ERR_ARG;
    const size_t qb = (size_t)n_tokens * n_heads * kv->head_dim * sizeof(float);
    const size_t kb = (size_t)n_tokens * kv->n_kv_heads * kv->head_dim * sizeof(float);
    return host_call(qb, kb, q, k, v, ao, [&](const char* d, const HostStage& hs) {
        return prefill_checked(kv, rope, layer, pos0, n_tokens, n_heads, (const float*)d,
                               (const float*)(d + hs.off_k), (const float*)(d + hs.off_v),
                               (float*)(d + hs.off_ao), nullptr);
    });
}

// ---------------------------------------------------------------------------
// Ragged multi-sequence decode
// ---------------------------------------------------------------------------

struct pkh_plan {
    int n_seqs;
    int n_heads;
    int chunk;
    int total_chunks;
    int max_chunks;
    int max_pos;
    const pkh_kv_batch_t* kvb;
    int* d_pos;
    int* d_chunk_start;
};

extern "C" int pkh_kv_batch_alloc(int n_layers, int n_kv_heads, int head_dim, int n_seqs,
                                  const int* max_seq, int dtype, pkh_kv_batch_t* kvb) {
    if (!kvb) return PKH_ERR_ARG;
    std::memset(kvb, 0, sizeof(*kvb));
    if (n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 || n_seqs <= 0 || !max_seq)
        return PKH_ERR_ARG;
    if (dtype != PKH_KV_F32 && dtype != PKH_KV_F16) return PKH_ERR_ARG;
    int64_t* slot0 = (int64_t*)std::calloc((size_t)n_seqs + 1, sizeof(int64_t));
    int* ms = (int*)std::calloc((size_t)n_seqs, sizeof(int));
    if (!slot0 || !ms) {
        std::free(slot0);
        std::free(ms);
        return PKH_ERR_MEMORY;
    }
    for (int s = 0; s < n_seqs; s++) {
        if (max_seq[s] <= 0) {
            std::free(slot0);
            std::free(ms);
            return PKH_ERR_ARG;
        }
        ms[s] = max_seq[s];
        slot0[s + 1] = slot0[s] + max_seq[s];
    }
    // Per layer: [kv_head][slot][K row | V row], rows padded as in pkh_kv_alloc.
    const size_t slots = (size_t)slot0[n_seqs];
    const size_t dp = row_pitch(head_dim);
    size_t head, stride, total, bytes;
    if (!mul_ok(slots, 2 * dp, &head) || !mul_ok(head, (size_t)n_kv_heads, &stride) ||
        !mul_ok(stride, (size_t)n_layers, &total) || !mul_ok(total, elem_size(dtype), &bytes)) {
        std::free(slot0);
        std::free(ms);
        return PKH_ERR_MEMORY;
    }
    void *k = nullptr, *ds = nullptr;
    hipError_t e = hipSetDevice(g_device);
    if (e == hipSuccess) e = hipMalloc(&k, bytes);
    if (e == hipSuccess) e = hipMalloc(&ds, ((size_t)n_seqs + 1) * sizeof(int64_t));
    if (e == hipSuccess) e = hipMemset(k, 0, bytes);
    if (e == hipSuccess)
        e = hipMemcpy(ds, slot0, ((size_t)n_seqs + 1) * sizeof(int64_t), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(k);
        (void)hipFree(ds);
        std::free(slot0);
        std::free(ms);
        return hip_fail(e, "pkh_kv_batch_alloc");
    }
    kvb->n_layers = n_layers;
    kvb->n_kv_heads = n_kv_heads;
    kvb->head_dim = head_dim;
    kvb->n_seqs = n_seqs;
    kvb->dtype = dtype;
    kvb->device = g_device;
    kvb->layer_stride = stride;
    kvb->slot0 = slot0;
    kvb->max_seq = ms;
    kvb->k = k;
    kvb->v = (char*)k + dp * elem_size(dtype);
    kvb->d_slot0 = ds;
    kvb->stride_pos = 2 * dp;
    kvb->stride_head = head;
    return PKH_OK;
}

extern "C" void pkh_kv_batch_free(pkh_kv_batch_t* kvb) {
    if (!kvb) return;
    if (kvb->k || kvb->d_slot0) {
        (void)hipDeviceSynchronize();
        (void)hipFree(kvb->k);   // one allocation; v points inside it
        (void)hipFree(kvb->d_slot0);
    }
    std::free(kvb->slot0);
    std::free(kvb->max_seq);
    std::memset(kvb, 0, sizeof(*kvb));
}

extern "C" int pkh_attn_prefill_batch_async(const pkh_kv_batch_t* kvb, const pkh_rope_t* rope,
                                            int seq, int layer, int pos0, int n_tokens, int n_heads,
                                            const float* d_q, const float* d_k, const float* d_v,
                                            float* d_ao, void* stream) {
    if (!kvb || !kvb->k || !kvb->v) return PKH_ERR_ARG;
    if (seq < 0 || seq >= kvb->n_seqs) return PKH_ERR_RANGE;
    // Sequence seq's slots as a single-sequence cache: same strides, its
    // own base and capacity.
    pkh_kv_t kv{};
    const size_t es = elem_size(kvb->dtype);
    const size_t base = (size_t)kvb->slot0[seq] * kvb->stride_pos * es;
    kv.n_layers = kvb->n_layers;
    kv.n_kv_heads = kvb->n_kv_heads;
    kv.head_dim = kvb->head_dim;
    kv.max_seq = kvb->max_seq[seq];
    kv.k_stride_layer = kvb->layer_stride;
    kv.v_stride_layer = kvb->layer_stride;
    kv.k = (char*)kvb->k + base;
    kv.v = (char*)kvb->v + base;
    kv.dtype = kvb->dtype;
    kv.device = kvb->device;
    kv.stride_pos = kvb->stride_pos;
    kv.stride_head = kvb->stride_head;
    int rc = prefill_validate(&kv, rope, layer, pos0, n_tokens, n_heads);
    if (rc != PKH_OK) return rc;
    if (!d_q || !d_k || !d_v || !d_ao) return PKH_ERR_ARG;
    return prefill_checked(&kv, rope, layer, pos0, n_tokens, n_heads, d_q, d_k, d_v, d_ao,
                           (hipStream_t)stream);
}

extern "C" int pkh_kv_batch_copy_rows(const pkh_kv_batch_t* kvb, int which_v, int layer, int seq,
                                      int pos0, int n_pos, void* host, int dir) {
    if (!kvb || !kvb->k || !host || n_pos < 0) return PKH_ERR_ARG;
    if (layer < 0 || layer >= kvb->n_layers || seq < 0 || seq >= kvb->n_seqs) return PKH_ERR_RANGE;
    if (pos0 < 0 || (long long)pos0 + n_pos > kvb->max_seq[seq]) return PKH_ERR_RANGE;
    const size_t es = elem_size(kvb->dtype);
    char* base = (char*)(which_v ? kvb->v : kvb->k) + (size_t)layer * kvb->layer_stride * es;
    return copy_rows_strided(base, kvb->stride_pos, kvb->stride_head, kvb->n_kv_heads,
                             kvb->head_dim, es, (size_t)kvb->slot0[seq] + pos0, n_pos, host, dir);
}

extern "C" int pkh_plan_create(const pkh_kv_batch_t* kvb, const int* pos, int n_heads,
                               pkh_plan_t** out) {
    if (!out) return PKH_ERR_ARG;
    *out = nullptr;
    if (!kvb || !kvb->k || !pos) return PKH_ERR_ARG;
    const int HK = kvb->n_kv_heads, D = kvb->head_dim, n = kvb->n_seqs;
    if (!shape_supported(D, n_heads, HK)) return PKH_ERR_ARG;
    long long rows = 0;
    int max_attend = 0, max_pos = 0;
    for (int s = 0; s < n; s++) {
        if (pos[s] < 0 || pos[s] >= kvb->max_seq[s]) return PKH_ERR_RANGE;
        rows += pos[s] + 1;
        if (pos[s] + 1 > max_attend) max_attend = pos[s] + 1;
        if (pos[s] > max_pos) max_pos = pos[s];
    }
    const int chunk = decode_chunk_for(D, n_heads, HK, kvb->dtype, rows, max_attend);
    // Work-item slots for each sequence's whole capacity, so that later
    // positions (pkh_plan_update) fit the same grid; a step uses as many as
    // its position needs.
    std::vector<int> cstart((size_t)n + 1, 0);
    int max_chunks = 0;
    for (int s = 0; s < n; s++) {
        const long long c = ((long long)kvb->max_seq[s] + chunk - 1) / chunk;
        if (cstart[s] + c > 0x7fffffffLL / 64) return PKH_ERR_ARG;   // grid
        cstart[s + 1] = cstart[s] + (int)c;
        if (c > max_chunks) max_chunks = (int)c;
    }
    pkh_plan* p = (pkh_plan*)std::calloc(1, sizeof(pkh_plan));
    if (!p) return PKH_ERR_MEMORY;
    p->n_seqs = n;
    p->n_heads = n_heads;
    p->chunk = chunk;
    p->total_chunks = cstart[n];
    p->max_chunks = max_chunks;
    p->max_pos = max_pos;
    p->kvb = kvb;
    hipError_t e = hipMalloc(&p->d_pos, (size_t)n * sizeof(int));
    if (e == hipSuccess) e = hipMalloc(&p->d_chunk_start, ((size_t)n + 1) * sizeof(int));
    if (e == hipSuccess) e = hipMemcpy(p->d_pos, pos, (size_t)n * sizeof(int), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(p->d_chunk_start, cstart.data(), ((size_t)n + 1) * sizeof(int),
                      hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(p->d_pos);
        (void)hipFree(p->d_chunk_start);
        std::free(p);
        return hip_fail(e, "pkh_plan_create");
    }
    *out = p;
    return PKH_OK;
}

extern "C" int pkh_plan_update(pkh_plan_t* p, const int* pos, void* stream) {
    if (!p || !pos) return PKH_ERR_ARG;
    int max_pos = 0;
    for (int s = 0; s < p->n_seqs; s++) {
        if (pos[s] < 0 || pos[s] >= p->kvb->max_seq[s]) return PKH_ERR_RANGE;
        if (pos[s] > max_pos) max_pos = pos[s];
    }
    PKH_HIP(hipMemcpyAsync(p->d_pos, pos, (size_t)p->n_seqs * sizeof(int), hipMemcpyHostToDevice,
                           (hipStream_t)stream));
    p->max_pos = max_pos;
    return PKH_OK;
}

extern "C" void pkh_plan_free(pkh_plan_t* p) {
    if (!p) return;
    (void)hipDeviceSynchronize();
    (void)hipFree(p->d_pos);
    (void)hipFree(p->d_chunk_start);
    std::free(p);
}

extern "C" int pkh_attn_decode_batch_async(const pkh_kv_batch_t* kvb, const pkh_rope_t* rope,
                                           const pkh_plan_t* plan, int layer, const float* d_q,
                                           const float* d_k, const float* d_v, float* d_ao,
                                           void* stream) {
    if (!kvb || !kvb->k || !plan || plan->kvb != kvb) return PKH_ERR_ARG;
    if (!d_q || !d_k || !d_v || !d_ao) return PKH_ERR_ARG;
    int rc = check_common(kvb->head_dim, plan->n_heads, kvb->n_kv_heads, rope);
    if (rc != PKH_OK) return rc;
    if (layer < 0 || layer >= kvb->n_layers) return PKH_ERR_RANGE;
    if (plan->max_pos >= rope->filled_upto) return PKH_ERR_RANGE;
    DecodeArgs a{};
    const size_t es = elem_size(kvb->dtype);
    a.k_layer = (const char*)kvb->k + (size_t)layer * kvb->layer_stride * es;
    a.v_layer = (const char*)kvb->v + (size_t)layer * kvb->layer_stride * es;
    a.stride_pos = (long long)kvb->stride_pos;
    a.stride_head = (long long)kvb->stride_head;
    a.dtype = kvb->dtype;
    a.head_dim = kvb->head_dim;
    a.n_heads = plan->n_heads;
    a.n_kv_heads = kvb->n_kv_heads;
    a.n_seqs = plan->n_seqs;
    a.d_seq_slot0 = (const long long*)kvb->d_slot0;
    a.d_seq_pos = plan->d_pos;
    a.d_chunk_start = plan->d_chunk_start;
    a.total_chunks = plan->total_chunks;
    a.max_chunks = plan->max_chunks;
    a.chunk = plan->chunk;
    a.q = d_q;
    a.k_new = d_k;
    a.v_new = d_v;
    a.out = d_ao;
    a.rope_sin = rope->sin;
    a.rope_cos = rope->cos;
    a.half = rope->half;
    return launch_decode(a, (hipStream_t)stream);
}
