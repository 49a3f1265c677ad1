// pkh_prefill.hip -- causal prefill of one layer on CDNA4 fp16 MFMA.
//
// The reference prefills by running its decode step once per prompt token
// (src/pickle_fast.c:1881-1898): token i at position p = pos0 + i rotates its
// q/k (:1910-1936), appends k_rot and v at row p (:1938-1944) and attends
// over rows [0, p] (:1946-2094).  The outputs of all tokens therefore equal
// one causal attention of the n queries over the rows [0, pos0 + n), and the
// cache ends up holding the same rows.  That is what is computed here, in
// two launches on the caller's stream:
//
// prefill_stage  one workgroup per (32 rows of a tile of KT rows, KV head),
//                KV head fastest in dispatch order, so that neighbouring
//                workgroups read neighbouring new rows ([n][HK][D]) and the
//                same table rows; KT = 64 keys (32 for head_dim 256).  New
//                rows (p >= pos0) get k rotated in fp32 with the reference's
//                contraction, and k_rot / v are appended to the cache in its
//                element type; rows below pos0 are read back from the cache.  Every row is also written,
//                as fp16, into a tile buffer laid out exactly as the
//                attention kernel keeps it in LDS: K as [key][D + kKPad] and
//                V transposed as [d][KT + kVPad].  Rows past the last
//                position are zero.
//
// prefill_attn   one workgroup per (block of query positions, KV head),
//                dispatched longest-first, with blockIdx % HK == KV head so
//                that on an 8-XCD part each XCD's L2 holds one head's tiles.
//                128 query columns per workgroup: column c is head c % G of
//                the group at token c / G, so the G heads that share a KV
//                head share every K/V tile.  Each wave holds 32 columns and
//                computes S^T = K Q^T and O^T += V^T P^T with
//                v_mfma_f32_32x32x16_f16: keeping the query index on the lane
//                makes the softmax statistics per-lane scalars, and the
//                S^T accumulator registers are, converted to fp16, exactly
//                the B operand of the P^T product once the keys of a 16-key
//                step are taken in the order the accumulator holds them
//                (the V^T reads use the same order).  Softmax runs in fp32,
//                in log2 units (q is pre-scaled by log2(e)/sqrt(D)), with a
//                lazily rescaled running maximum.
//                Query heads are grouped into head slots as in decode: slot
//                y = g*nsub + sub holds up to G heads of KV head g (query
//                head h reads KV head h*HK/H, src/pickle_fast.c:1963), so
//                groups of any size share the tiles; columns of heads past
//                a group's end compute on a clamped query and are not
//                written.  Head dimensions that are not 16, 32, 64, 128 or
//                256 run at the next of those widths (PAD): the tiles and
//                the query are zero past the real width and outputs there
//                are not written; their staging uses prefill_stage_any.
//                Two groups of 4 waves (one wave of each per SIMD) split the
//                key tiles by parity and alternate phases, so that while one
//                group's waves issue MFMAs the other's run the softmax; the
//                groups' (m, l, o) are merged at the end.  Tiles reach LDS
//                through gfx950 direct loads (buffer_load_dwordx4 ... lds) into
//                4-slot K and V rings, issued at the end of the phase before
//                and read two phases later.

#include "pkh_internal.h"

#include <algorithm>
#include <cmath>
#include <utility>

namespace pkh {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kKPad = 8;        // fp16 padding per K row (conflict-free ds_read_b128)
constexpr int kVPad = 4;        // fp16 padding per V^T row (conflict-free ds_read_b64)
constexpr int kThreads = 256;   // staging kernel: 4 waves
constexpr float kTau = 8.0f;    // lazy-rescale threshold, log2 units

constexpr int rope_half_of(int D) { return D / 2 < 64 ? D / 2 : 64; }

// One staged tile of one KV head: KT keys' K rows then V^T rows, fp16.
template <int D>
struct Tile {
    static constexpr int KT = D >= 256 ? 32 : 64;     // keys per tile
    static constexpr int KS = D + kKPad;              // K row stride
    static constexpr int VROWS = D < 32 ? 32 : D;     // V^T rows, zero-padded to a 32-row block
    static constexpr int VS = KT + kVPad;             // V^T row stride
    static constexpr int K_ELEMS = KT * KS;
    static constexpr int V_ELEMS = VROWS * VS;
    static constexpr int ELEMS = K_ELEMS + V_ELEMS;
    static constexpr int BYTES = ELEMS * 2;
    static_assert(BYTES % 16 == 0, "tiles are copied in 16-byte chunks");
};

// ---- element access for the cache types ---------------------------------

__device__ __forceinline__ void load4(const float* p, float (&x)[4]) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
}
// Non-temporal loads for the rows staging reads once per call (the cached
// rows below pos0 and the new rows): measured on a 128-token chunk after
// 8,192 cached rows, 53.3 against 57.0 us per layer call; unchanged on a
// 2048-token prompt.
__device__ __forceinline__ void load4nt(const float* p, float (&x)[4]) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    x[0] = v[0]; x[1] = v[1]; x[2] = v[2]; x[3] = v[3];
}
__device__ __forceinline__ void load4nt(const _Float16* p, float (&x)[4]) {
    const h4 v = __builtin_nontemporal_load(reinterpret_cast<const h4*>(p));
    for (int i = 0; i < 4; i++) x[i] = (float)v[i];
}
__device__ __forceinline__ void load4(const _Float16* p, float (&x)[4]) {
    const h4 v = *reinterpret_cast<const h4*>(p);
    for (int i = 0; i < 4; i++) x[i] = (float)v[i];
}
// Cache rows are stored non-temporally: this launch never reads them back.
__device__ __forceinline__ void store4(float* p, const float (&x)[4]) {
    __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f32x4*>(p));
}
// fp32 -> fp16, round to nearest even, of a value already rounded to fp32.
// The empty asm keeps the compiler from folding the conversion into the
// fused multiply-add that produced x (v_fma_mix*_f16 rounds once, straight
// to fp16, where the reference rounds to fp32 first and then to fp16).
__device__ __forceinline__ _Float16 to_f16(float x) {
    __asm__ volatile("" : "+v"(x));
    return (_Float16)x;
}
__device__ __forceinline__ h4 to_h4(const float (&x)[4]) {
    h4 v;
    for (int i = 0; i < 4; i++) v[i] = to_f16(x[i]);
    return v;
}
__device__ __forceinline__ void store4(_Float16* p, const float (&x)[4]) {
    __builtin_nontemporal_store(to_h4(x), reinterpret_cast<h4*>(p));
}

// ---- stage: append + fp16 tiles -------------------------------------------

struct StageParams {
    void* k_layer;              // cache element type CT
    void* v_layer;
    long long stride_pos, stride_head;
    const float* k_new;         // [n][HK][Dr]
    const float* v_new;
    const float* rope_sin;      // [max_seq][half]
    const float* rope_cos;
    int half, pos0, n, HK;
    int Dr;                     // real head_dim
    int T;                      // tiles per head
    _Float16* tiles;            // [HK][T][Tile::ELEMS]
    // Rows at positions below kExactKeys, computed in fp32 by extra
    // workgroups of this launch (grid rows past the staging ones).
    const float* q;             // [n][H][Dr]
    float* out;                 // [n][H][Dr]
    int H, Gs, nsub;            // query heads; head slots as in prefill_attn
    float qscale;               // log2(e) / sqrt(Dr)
};

// One element d of a head vector x rotated by table row (sn, cs): the two
// fused multiply-adds of src/pickle_fast.c:1917-1922 as compiled, with the
// pair (d, d + half) in either order; elements past 2*half are unrotated.
// Branch-free: the four loads do not depend on which case applies, so a
// caller's unrolled loop issues all of them before any arithmetic.
__device__ __forceinline__ float rope_at(const float* x, int d, int half, const float* sn,
                                         const float* cs) {
    const bool lo = d < half, hi = !lo && d < 2 * half;
    const int pd = lo ? d + half : (hi ? d - half : d);
    const int ti = lo ? d : (hi ? d - half : 0);
    const float xd = x[d], xp = x[pd], s = sn[ti], c = cs[ti];
    const float r_lo = fmaf(c, xd, -(s * xp));
    const float r_hi = fmaf(s, xp, c * xd);
    return lo ? r_lo : (hi ? r_hi : xd);
}

__device__ __forceinline__ float widen(float x) { return x; }
__device__ __forceinline__ float widen(_Float16 x) { return (float)x; }
template <typename CT> __device__ __forceinline__ CT narrow(float x);
template <> __device__ __forceinline__ float narrow<float>(float x) { return x; }
template <> __device__ __forceinline__ _Float16 narrow<_Float16>(float x) { return to_f16(x); }

// Rows at positions below kExactKeys (at most that many keys) are computed
// in fp32 by extra workgroups of prefill_stage, one per (row, head slot),
// which run beside the staging workgroups (the launch is bound by memory
// traffic, not by the VALU); prefill_attn leaves those rows alone.  fp16
// rounding costs such a row
// the most: with one key its output is v rounded to fp16, up to 2^-9 ~ 1.95e-3
// for |v| in [4, 8), while over longer ranges the roundings average out.
// Measured over 20 seeds of a 2048-token Llama-3-8B-shape prompt (fp16 for
// every row): worst 1.94e-3, all in rows 0-11; emulated by number of keys,
// 1.9e-3 below 8 keys, 1.35e-3 for 8-15, 1.1e-3 for 16-31, under 1e-3 above.
constexpr int kExactKeys = 16;

// The reference's decode step (src/pickle_fast.c:1946-2094) for row r and
// the query heads of head slot y, in fp32: q rotated with the reference's
// contraction and scaled, dot products with the row's <= kExactKeys keys,
// exact max, exp2, weighted sum of the values.  Keys below pos0 come from
// the cache; the row's new keys are rotated from the inputs exactly as the
// staging workgroups rotate them (and rounded to the cache type), since
// those are writing the cache concurrently.  Every load is unconditional
// (indices clamped into range, results selected), so each step is one
// memory round trip.  lds: kExactLds floats.
constexpr int kExactSlot = 8;                                 // largest head slot
template <int D> struct ExactLds {
    static constexpr int Q = kExactSlot * D, K = kExactKeys * (D + 1), V = kExactKeys * D,
                         S = kExactSlot * kExactKeys;
    static constexpr int N = Q + K + V + S;
};

template <int D, typename CT, int NT>
__device__ void exact_row(const StageParams& P, int e, float* lds) {
    const int NY = P.HK * P.nsub;
    const int r = e / NY, y = e - (e / NY) * NY;
    const int g = y / P.nsub, ysub = y - g * P.nsub;
    const int head0 = (g * P.H + P.HK - 1) / P.HK + ysub * P.Gs;
    const int gc = min(P.Gs, (g * P.H + P.H + P.HK - 1) / P.HK - head0);
    if (gc <= 0) return;
    float* qs = lds;
    float* ks = qs + ExactLds<D>::Q;
    float* vs = ks + ExactLds<D>::K;
    float* sc = vs + ExactLds<D>::V;
    const int Dr = P.Dr, half = P.half;
    const int pos = P.pos0 + r, nk = pos + 1;
    const int tid = threadIdx.x;
    constexpr int NQ = (kExactSlot * D + NT - 1) / NT, NKV = (kExactKeys * D + NT - 1) / NT;
    float qv[NQ], kl[NKV], vl[NKV];
    {
        const float* sn = P.rope_sin + (size_t)pos * half;
        const float* cs = P.rope_cos + (size_t)pos * half;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const int idx = min(tid + i * NT, P.Gs * D - 1), h = idx / D, d = idx % D;
            const float* qrow = P.q + ((size_t)r * P.H + head0 + min(h, gc - 1)) * Dr;
            qv[i] = rope_at(qrow, min(d, Dr - 1), half, sn, cs) * P.qscale;
        }
    }
    const CT* kc = static_cast<const CT*>(P.k_layer) + (size_t)g * P.stride_head;
    const CT* vc = static_cast<const CT*>(P.v_layer) + (size_t)g * P.stride_head;
    // A prompt from position 0 (the usual case, a uniform branch) has only
    // new keys and skips the cache loads.
    const bool from_cache = P.pos0 > 0;
#pragma unroll
    for (int i = 0; i < NKV; i++) {
        const int idx = min(tid + i * NT, kExactKeys * D - 1), key = min(idx / D, nk - 1);
        const int d = min(idx % D, Dr - 1);
        const int knew = max(key - P.pos0, 0);
        const size_t src = ((size_t)knew * P.HK + g) * Dr;
        const float krot = widen(narrow<CT>(rope_at(P.k_new + src, d, half, P.rope_sin + (size_t)key * half,
                                                    P.rope_cos + (size_t)key * half)));
        const float vin = widen(narrow<CT>(P.v_new[src + d]));
        kl[i] = krot;
        vl[i] = vin;
    }
    if (from_cache) {
#pragma unroll
        for (int i = 0; i < NKV; i++) {
            const int idx = min(tid + i * NT, kExactKeys * D - 1), key = min(idx / D, nk - 1);
            const int d = min(idx % D, Dr - 1);
            const int kold = min(key, P.pos0 - 1);
            const float kcache = widen(kc[(size_t)kold * P.stride_pos + d]);
            const float vcache = widen(vc[(size_t)kold * P.stride_pos + d]);
            if (key < P.pos0) {
                kl[i] = kcache;
                vl[i] = vcache;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int idx = tid + i * NT;
        if (idx < kExactSlot * D) qs[idx] = (idx / D < gc && idx % D < Dr) ? qv[i] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < NKV; i++) {
        const int idx = tid + i * NT, key = idx / D, d = idx % D;
        if (idx < kExactKeys * D) {
            const bool live = key < nk && d < Dr;
            ks[key * (D + 1) + d] = live ? kl[i] : 0.0f;   // zeros: 0 * stale LDS could be NaN
            vs[key * D + d] = live ? vl[i] : 0.0f;
        }
    }
    __syncthreads();
    // Scores: two threads per (head, key), each over half of the width with
    // four independent partial sums, the halves added through a lane swap
    // (short dependency chains: these rows are a latency chain beside the
    // bandwidth-bound staging).
    static_assert(NT == 2 * kExactSlot * kExactKeys, "two threads per (head, key)");
    {
        constexpr int DH = D / 2;
        const int pr = tid >> 1, part = tid & 1;
        const int h = pr / kExactKeys, k = pr % kExactKeys;
        const float* qh = qs + h * D + part * DH;
        const float* kh = ks + k * (D + 1) + part * DH;
        float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int d = 0; d < DH; d++) a4[d & 3] = fmaf(qh[d], kh[d], a4[d & 3]);
        float acc = (a4[0] + a4[1]) + (a4[2] + a4[3]);
        acc += __shfl_xor(acc, 1);
        if (part == 0) sc[pr] = acc;
    }
    __syncthreads();
    // Softmax over keys [0, pos]: one thread per (head, key), the head's 16
    // keys in 16 neighbouring lanes; maximum and sum by lane exchanges.
    if (tid < kExactSlot * kExactKeys) {
        static_assert(kExactKeys == 16, "a head's keys fill a 16-lane group");
        const int k = tid % kExactKeys;
        const float sk = k < nk ? sc[tid] : -INFINITY;
        float m = sk;
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float w = k < nk ? __builtin_amdgcn_exp2f(sk - m) : 0.0f;
        float l = w;
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) l += __shfl_xor(l, o);
        sc[tid] = w * (1.0f / l);
    }
    __syncthreads();
    for (int idx = tid; idx < kExactSlot * D; idx += NT) {
        const int h = idx / D, d = idx % D;
        float o = 0.0f;
#pragma unroll
        for (int k = 0; k < kExactKeys; k++) o = fmaf(sc[h * kExactKeys + k], vs[k * D + d], o);
        if (h < gc && d < Dr) P.out[((size_t)r * P.H + head0 + h) * Dr + d] = o;
    }
}

// Rows of one tile that one staging workgroup covers (two workgroups per
// 64-key tile: 512 workgroups for a 2048-row, 8-head layer).
template <int D> struct StageRows { static constexpr int N = Tile<D>::KT < 32 ? Tile<D>::KT : 32; };

template <int D, typename CT>
__global__ __launch_bounds__(kThreads) void prefill_stage(StageParams P) {
    using TL = Tile<D>;
    constexpr int HALF = rope_half_of(D);
    constexpr int NP = HALF / 4;              // rotated pairs of 4-element groups
    constexpr int NL = (D - 2 * HALF) / 4;    // unrotated 4-element groups (D = 256)
    constexpr int NI = NP + NL;
    constexpr int TPR = NI < 16 ? NI : 16;    // threads per row
    constexpr int RPP = kThreads / TPR;       // rows per pass
    constexpr int RW = StageRows<D>::N;       // rows of this workgroup
    constexpr int NPASS = RW > RPP ? RW / RPP : 1;
    constexpr int NIT = (NI + TPR - 1) / TPR;
    constexpr int NU = NPASS * NIT;           // (row, group) items per thread
    static_assert(RW % RPP == 0 || RPP > RW, "rows split evenly over passes");
    // One LDS buffer: the V rows of a staging workgroup, or an exact row's
    // operands.
    constexpr int kLdsFloats = ExactLds<D>::N > RW * (D + 4) / 2 ? ExactLds<D>::N : RW * (D + 4) / 2;
    __shared__ __attribute__((aligned(16))) float lds[kLdsFloats];
    auto sv = reinterpret_cast<_Float16 (*)[D + 4]>(lds);

    const int tid = threadIdx.x;
    constexpr int SPLIT = TL::KT / RW;
    // The exact rows' grid rows come first, so that their latency chain runs
    // beside the staging instead of after it.
    const int NE = (int)gridDim.y - P.T * SPLIT;
    if ((int)blockIdx.y < NE) {
        exact_row<D, CT, kThreads>(P, (int)blockIdx.y * (int)gridDim.x + (int)blockIdx.x, lds);
        return;
    }
    const int yb = (int)blockIdx.y - NE;
    const int j = yb / SPLIT, r0 = (yb % SPLIT) * RW, g = blockIdx.x;
    _Float16* tk = P.tiles + ((size_t)g * P.T + j) * TL::ELEMS;
    _Float16* tv = tk + TL::K_ELEMS;
    CT* kc = static_cast<CT*>(P.k_layer) + (size_t)g * P.stride_head;
    CT* vc = static_cast<CT*>(P.v_layer) + (size_t)g * P.stride_head;

    // Item u = (pass, i): local row rl = tid / TPR + pass * RPP, 4-element
    // group it = tid % TPR + i * TPR.  All of a thread's loads are issued
    // before any of its stores (a store to the cache may alias an input, so
    // the compiler could not hoist a later item's loads above it).
    float k0[NU][4], k1[NU][4], v0[NU][4], v1[NU][4];
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int rl = tid / TPR + (u / NIT) * RPP, it = tid % TPR + (u % NIT) * TPR;
        const int p = j * TL::KT + r0 + rl;
        const bool pair = it < NP;
        const int d0 = pair ? 4 * it : 2 * HALF + 4 * (it - NP);
#pragma unroll
        for (int i = 0; i < 4; i++) k0[u][i] = k1[u][i] = v0[u][i] = v1[u][i] = 0.0f;
        if (rl >= RW || it >= NI) continue;
        if (p < P.pos0) {
            // Earlier context: already rotated in the cache.
            const size_t row = (size_t)p * P.stride_pos;
            load4nt(kc + row + d0, k0[u]);
            load4nt(vc + row + d0, v0[u]);
            if (pair) {
                load4nt(kc + row + d0 + HALF, k1[u]);
                load4nt(vc + row + d0 + HALF, v1[u]);
            }
        } else if (p < P.pos0 + P.n) {
            const size_t src = ((size_t)(p - P.pos0) * P.HK + g) * D;
            load4nt(P.k_new + src + d0, k0[u]);
            load4nt(P.v_new + src + d0, v0[u]);
            if (pair) {
                load4nt(P.k_new + src + d0 + HALF, k1[u]);
                load4nt(P.v_new + src + d0 + HALF, v1[u]);
            }
        }
    }
    float sn[NU][4], cs[NU][4];
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int rl = tid / TPR + (u / NIT) * RPP, it = tid % TPR + (u % NIT) * TPR;
        const int p = j * TL::KT + r0 + rl;
        if (rl < RW && it < NP && p >= P.pos0 && p < P.pos0 + P.n) {
            load4(P.rope_sin + (size_t)p * P.half + 4 * it, sn[u]);
            load4(P.rope_cos + (size_t)p * P.half + 4 * it, cs[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < NU; u++) {
        const int rl = tid / TPR + (u / NIT) * RPP, it = tid % TPR + (u % NIT) * TPR;
        if (rl >= RW || it >= NI) continue;
        const int p = j * TL::KT + r0 + rl;
        const bool pair = it < NP;
        const int d0 = pair ? 4 * it : 2 * HALF + 4 * (it - NP);
        if (p >= P.pos0 && p < P.pos0 + P.n) {
            if (pair) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // src/pickle_fast.c:1917-1922 as compiled: x0' = c*x0 - s*x1
                    // and x1' = s*x0 + c*x1, each one fused multiply-add.
                    const float a = k0[u][i], b = k1[u][i];
                    k0[u][i] = fmaf(cs[u][i], a, -(sn[u][i] * b));
                    k1[u][i] = fmaf(sn[u][i], a, cs[u][i] * b);
                }
            }
            const size_t row = (size_t)p * P.stride_pos;
            store4(kc + row + d0, k0[u]);
            store4(vc + row + d0, v0[u]);
            if (pair) {
                store4(kc + row + d0 + HALF, k1[u]);
                store4(vc + row + d0 + HALF, v1[u]);
            }
        }
        const int r = r0 + rl;
        *reinterpret_cast<h4*>(tk + r * TL::KS + d0) = to_h4(k0[u]);
        *reinterpret_cast<h4*>(&sv[rl][d0]) = to_h4(v0[u]);
        if (pair) {
            *reinterpret_cast<h4*>(tk + r * TL::KS + d0 + HALF) = to_h4(k1[u]);
            *reinterpret_cast<h4*>(&sv[rl][d0 + HALF]) = to_h4(v1[u]);
        }
    }
    __syncthreads();
    // V^T rows of this workgroup's keys, 8 keys per store (two 8-byte
    // halves: rows are 8-byte aligned).
    for (int u = tid; u < TL::VROWS * (RW / 8); u += kThreads) {
        const int d = u / (RW / 8), c8 = u % (RW / 8);
        h4 lo, hi;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = d < D ? sv[8 * c8 + i][d] : (_Float16)0.0f;
            hi[i] = d < D ? sv[8 * c8 + 4 + i][d] : (_Float16)0.0f;
        }
        _Float16* dst = tv + d * TL::VS + r0 + 8 * c8;
        *reinterpret_cast<h4*>(dst) = lo;
        *reinterpret_cast<h4*>(dst + 4) = hi;
    }
}

// Staging for a real head_dim Dr below the padded width D (any Dr, any
// rotation half): one element per thread and pass, scalar loads and stores,
// the same rotation, cache append and tile layout as prefill_stage, zeros
// past Dr.  Only shapes the vector staging cannot take use it.
template <int D, typename CT>
__global__ __launch_bounds__(kThreads) void prefill_stage_any(StageParams P) {
    using TL = Tile<D>;
    constexpr int RW = StageRows<D>::N;
    constexpr int SPLIT = TL::KT / RW;
    constexpr int kLdsFloats = ExactLds<D>::N > RW * (D + 4) / 2 ? ExactLds<D>::N : RW * (D + 4) / 2;
    __shared__ __attribute__((aligned(16))) float lds[kLdsFloats];
    auto sv = reinterpret_cast<_Float16 (*)[D + 4]>(lds);
    const int tid = threadIdx.x;
    // The exact rows' grid rows come first, so that their latency chain runs
    // beside the staging instead of after it.
    const int NE = (int)gridDim.y - P.T * SPLIT;
    if ((int)blockIdx.y < NE) {
        exact_row<D, CT, kThreads>(P, (int)blockIdx.y * (int)gridDim.x + (int)blockIdx.x, lds);
        return;
    }
    const int yb = (int)blockIdx.y - NE;
    const int j = yb / SPLIT, r0 = (yb % SPLIT) * RW, g = blockIdx.x;
    const int Dr = P.Dr;
    _Float16* tk = P.tiles + ((size_t)g * P.T + j) * TL::ELEMS;
    _Float16* tv = tk + TL::K_ELEMS;
    CT* kc = static_cast<CT*>(P.k_layer) + (size_t)g * P.stride_head;
    CT* vc = static_cast<CT*>(P.v_layer) + (size_t)g * P.stride_head;
    for (int idx = tid; idx < RW * D; idx += kThreads) {
        const int rl = idx / D, d = idx % D;
        const int p = j * TL::KT + r0 + rl;
        float kx = 0.0f, vx = 0.0f;
        if (d < Dr) {
            const size_t row = (size_t)p * P.stride_pos;
            if (p < P.pos0) {
                kx = widen(kc[row + d]);
                vx = widen(vc[row + d]);
            } else if (p < P.pos0 + P.n) {
                const size_t src = ((size_t)(p - P.pos0) * P.HK + g) * Dr;
                kx = rope_at(P.k_new + src, d, P.half, P.rope_sin + (size_t)p * P.half,
                             P.rope_cos + (size_t)p * P.half);
                vx = P.v_new[src + d];
                kc[row + d] = narrow<CT>(kx);
                vc[row + d] = narrow<CT>(vx);
            }
        }
        tk[(r0 + rl) * TL::KS + d] = to_f16(kx);
        sv[rl][d] = to_f16(vx);
    }
    __syncthreads();
    for (int u = tid; u < TL::VROWS * (RW / 8); u += kThreads) {
        const int d = u / (RW / 8), c8 = u % (RW / 8);
        h4 lo, hi;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = d < D ? sv[8 * c8 + i][d] : (_Float16)0.0f;
            hi[i] = d < D ? sv[8 * c8 + 4 + i][d] : (_Float16)0.0f;
        }
        _Float16* dst = tv + d * TL::VS + r0 + 8 * c8;
        *reinterpret_cast<h4*>(dst) = lo;
        *reinterpret_cast<h4*>(dst + 4) = hi;
    }
}

// ---- attention -------------------------------------------------------------

struct AttnParams {
    const _Float16* tiles;      // [HK][T][Tile::ELEMS]
    int T;
    const float* q;             // [n][H][Dr]
    float* out;                 // [n][H][Dr]
    const float* rope_sin;
    const float* rope_cos;
    int half, pos0, n, H, HK, nqb;
    int Dr;                     // real head_dim
    int nsub;                   // head slots per KV head
    float qscale;               // log2(e) / sqrt(Dr)
    // Keys split over workgroups: nsplit workgroups per (query block, head
    // slot), split s taking tiles [s*tps, (s+1)*tps) of its causal range.
    // With nsplit > 1 each writes its unnormalised partial (o, and the
    // column's m and l) to part_o [nsplit][nqb][slot][kCols][D] and part_ml
    // [nsplit][nqb][slot][kCols][2], and prefill_merge finishes the rows.
    int nsplit, tps;
    float* part_o;
    float* part_ml;
};

__device__ __forceinline__ float max_halves(float x) {
    const unsigned u = __float_as_uint(x);
    auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
    const unsigned u = __float_as_uint(x);
    auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Copy BYTES (a multiple of 16) from a buffer to LDS with gfx950 direct
// loads (buffer_load_dwordx4 ... lds): each instruction moves 1 KB, lane l's
// 16 bytes landing at dst + 16*l.  The tile offset goes in the scalar
// offset, the lane's 16-byte chunk in the vector offset.  Instructions are
// dealt round-robin to the waves; the data is visible to the workgroup after
// the issuing waves' s_waitcnt vmcnt and a barrier.  (The MUBUF form, unlike
// global_load_lds, lets the compiler keep counting LDS reads precisely while
// these loads are in flight: it waits lgkmcnt(n) for the one fragment an
// MFMA needs instead of lgkmcnt(0) for all of them.)
template <int BYTES, int WAVES>
__device__ __forceinline__ void copy_to_lds(_Float16* dst, __amdgpu_buffer_rsrc_t rs, unsigned src_bytes, int wave,
                                            int lane) {
    constexpr int CH = BYTES / 16;                 // 16-byte chunks
    constexpr int NI = (CH + 63) / 64;             // wave instructions
#pragma unroll
    for (int i = wave; i < NI; i += WAVES) {
        const int c = 64 * i + lane;
        if (NI * 64 == CH || c < CH)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)(reinterpret_cast<char*>(dst) + 1024 * i), 16,
                16u * (unsigned)c, src_bytes, 0, 0);
    }
}

// The attention workgroup: two groups of 4 waves, one wave of each group on
// every SIMD.  Both groups hold the same 128 query columns (32 per wave);
// group 0 takes the even key tiles and group 1 the odd ones (split-K), and
// the groups alternate phases: while one group's waves run MFMAs the other
// group's run the softmax on the VALU.
// Workgroup barrier with no memory fence.  __syncthreads() is a
// workgroup-scope release, and the compiler completes every direct load
// (they write LDS) before it -- including loads just issued for a later
// phase.  The phase loop waits for its own loads explicitly before this
// barrier; LDS reads are consumed (and so complete) within their phase, long
// before a later direct load reuses their slot.
__device__ __forceinline__ void phase_barrier() { __asm__ volatile("s_barrier" ::: "memory"); }

// Issue order for a run of N MFMAs that each consume one LDS fragment: the
// first kAhead fragment reads, then one MFMA and the next read in turn, so
// every MFMA finds its operand kAhead reads back instead of waiting on its
// own read.  Four reads ahead cover the LDS latency behind four ~39-cycle
// MFMAs; measured on the Llama-3-8B 2048-row layer, 56.0 us for the attention
// kernel against 56.7 us with eight (and 16 fewer VGPRs), 58.6 us with twelve.
constexpr int kAhead = 4;
template <int N>
__device__ __forceinline__ void pipeline_order() {
    constexpr int A = N < kAhead ? N : kAhead;
    __builtin_amdgcn_sched_group_barrier(0x100, A, 0);              // DS read
#pragma unroll
    for (int i = 0; i < N - A; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);          // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, A, 0);              // MFMA
}

// head_dim 256 needs the whole register file for one wave per SIMD: one
// group of 4 waves that runs each tile's QK, softmax and P.V in turn.
template <int D> struct Groups { static constexpr int N = D >= 256 ? 1 : 2; };
constexpr int kSlots = 4;        // K ring and V ring depth
constexpr int kCols = 128;       // query columns per workgroup

template <int D, int G, bool PAD, bool SPLIT>
__global__ __launch_bounds__(256 * Groups<D>::N)
__attribute__((amdgpu_waves_per_eu(Groups<D>::N, Groups<D>::N)))
void prefill_attn(AttnParams P) {
    using TL = Tile<D>;
    constexpr int NG = Groups<D>::N;
    constexpr int kAttnWaves = 4 * NG;
    constexpr int KT = TL::KT;
    constexpr int HALF = rope_half_of(D);
    constexpr int BM = kCols / G;                 // query positions per workgroup
    constexpr int NKS = D / 16;                   // k-steps of S^T = K Q^T
    constexpr int NDB = TL::VROWS / 32;           // 32-row blocks of O^T
    constexpr int NKB = KT / 32;                  // 32-key blocks per tile
    constexpr int NT = KT / 16;                   // 16-key steps per tile
    // Distinct LDS objects per ring slot (not one indexed array), so the
    // compiler can tell a slot being filled by a direct load from the slots
    // being read, and does not wait for the load before those reads.
    __shared__ __attribute__((aligned(16))) _Float16 k0[TL::K_ELEMS], k1[TL::K_ELEMS],
        k2[TL::K_ELEMS], k3[TL::K_ELEMS];
    __shared__ __attribute__((aligned(16))) _Float16 v0[TL::V_ELEMS], v1[TL::V_ELEMS],
        v2[TL::V_ELEMS], v3[TL::V_ELEMS];
    _Float16* const kslot[kSlots] = {k0, k1, k2, k3};
    _Float16* const vslot[kSlots] = {v0, v1, v2, v3};

    const int tid = threadIdx.x;
    const int lane = tid & 63, hh = lane >> 5, l32 = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = w >> 2, sub = w & 3;
    const int NY = P.HK * P.nsub;                             // head slots
    const int y = (int)(blockIdx.x % NY);
    const int g = y / P.nsub;                                 // KV head
    const int ysub = y - g * P.nsub;
    const int head0 = (g * P.H + P.HK - 1) / P.HK + ysub * G;
    const int gc = min(G, (g * P.H + P.H + P.HK - 1) / P.HK - head0);
    if (gc <= 0) return;                                      // a KV head that serves no query head
    const int Dr = PAD ? P.Dr : D;
    const int rest = (int)(blockIdx.x / NY);
    const int split = rest % P.nsplit;                        // key range of this workgroup
    const int qb = P.nqb - 1 - rest / P.nsplit;               // longest first
    const int qmin_wg = P.pos0 + qb * BM;
    const int qmax = P.pos0 + min(qb * BM + BM - 1, P.n - 1);
    const int tbase = split * P.tps;                          // first tile of the range
    const int ntile = min(qmax / KT + 1 - tbase, P.tps);      // tiles in the range
    const size_t pbase = (((size_t)split * P.nqb + qb) * NY + y) * kCols;   // partial rows
    if (SPLIT && ntile <= 0) {
        // A range past this block's causal extent: an empty partial.
        for (int c = threadIdx.x; c < kCols; c += blockDim.x) {
            P.part_ml[(pbase + c) * 2 + 0] = -INFINITY;
            P.part_ml[(pbase + c) * 2 + 1] = 0.0f;
        }
        return;
    }

    // This KV head's tiles as one buffer (reads past its end return zero).
    const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(P.tiles + (size_t)g * P.T * TL::ELEMS), (short)0, P.T * TL::BYTES, 0x00020000);
    // Tile t of the loop below is tile tbase + t of the KV head.
    auto load_k = [&](_Float16* dst, int t) __attribute__((always_inline)) {
        copy_to_lds<TL::K_ELEMS * 2, kAttnWaves>(dst, trs, (unsigned)((tbase + t) * TL::BYTES), w, lane);
    };
    auto load_v = [&](_Float16* dst, int t) __attribute__((always_inline)) {
        copy_to_lds<TL::V_ELEMS * 2, kAttnWaves>(dst, trs, (unsigned)((tbase + t) * TL::BYTES + TL::K_ELEMS * 2),
                                               w, lane);
    };
    // Tiles for the first phases (the loop's phase p issues the loads of
    // phase p + 1 at its end): K(0), K(1), K(2) and V(0) with two groups;
    // K and V of tiles 0, 1, 2 with one.
    load_k(k0, 0);
    if (ntile > 1) load_k(k1, 1);
    if (ntile > 2) load_k(k2, 2);
    load_v(v0, 0);
    if constexpr (NG == 1) {
        if (ntile > 1) load_v(v1, 1);
        if (ntile > 2) load_v(v2, 2);
    }

    // ---- q: load, rotate (same contraction as the reference), scale, fp16.
    // Lane (l32, hh) of wave `sub` holds column 32*sub + l32 and, for k-step
    // ks, elements d = 16ks + 8hh + [0, 8).
    const int col = 32 * sub + l32;
    const int ti = qb * BM + col / G;
    const bool valid = ti < P.n && col % G < gc;
    const int tic = ti < P.n ? ti : P.n - 1;
    const int h = head0 + min(col % G, gc - 1);
    const int qpos = P.pos0 + tic;
    // Every load of q and of its sin/cos rows is issued before any
    // arithmetic: the empty asm statements take all of them at once and hand
    // back opaque values, which the compiler can neither sink below the math
    // nor reload later, so the prologue costs one memory round trip instead
    // of one per batch of loads.
    auto hold = [](float4& v) __attribute__((always_inline)) {
        __asm__ volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
    };
    auto unpack = [](const float4& a, const float4& b, float (&x)[8]) __attribute__((always_inline)) {
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    };
    auto to_qt = [&](const float (&y)[8]) __attribute__((always_inline)) {
        h8 v;
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (_Float16)(y[e] * P.qscale);
        return v;
    };
    const float* qrow = P.q + ((size_t)tic * P.H + h) * Dr;
    const float* srow = P.rope_sin + (size_t)qpos * P.half;
    const float* crow = P.rope_cos + (size_t)qpos * P.half;
    constexpr int KH = HALF % 16 == 0 ? HALF / 16 : 1;    // k-steps holding rotated first halves
    // With two groups, each loads and rotates half of the rotation pairs
    // (k-steps kh and kh + KH for its kh) and hands its fp16 k-steps to the
    // other through LDS: V slots 2 (group 0's) and 3 (group 1's), whose first
    // direct loads are issued at the end of phases 1 and 2, after the phase-0
    // barrier.
    constexpr bool kSplitQ = !PAD && NG == 2 && KH >= 2 && 2 * KH == NKS;
    h8 qt[NKS];
    if constexpr (PAD) {
        // Any width and rotation half: element d = 16ks + 8hh + e, rotated
        // one element at a time, zero past Dr.
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            float y8[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int d = 16 * ks + 8 * hh + e;
                y8[e] = d < Dr ? rope_at(qrow, d, P.half, srow, crow) : 0.0f;
            }
            qt[ks] = to_qt(y8);
        }
    } else if constexpr (kSplitQ) {
        constexpr int KO = KH / 2;
        static_assert(2 * KO * 4 * 64 * 16 <= TL::K_ELEMS * 2 && 2 * KO * 4 * 64 * 16 <= TL::V_ELEMS * 2,
                      "q exchange fits a ring slot");
        const int kh0 = grp * KO;
        float4 xa[2 * KO], xb[2 * KO], sa[KO], sb[KO], ca[KO], cb[KO];
#pragma unroll
        for (int i = 0; i < KO; i++) {
            const int ks = kh0 + i;
            xa[i] = *reinterpret_cast<const float4*>(qrow + 16 * ks + 8 * hh);
            xb[i] = *reinterpret_cast<const float4*>(qrow + 16 * ks + 8 * hh + 4);
            xa[KO + i] = *reinterpret_cast<const float4*>(qrow + 16 * (ks + KH) + 8 * hh);
            xb[KO + i] = *reinterpret_cast<const float4*>(qrow + 16 * (ks + KH) + 8 * hh + 4);
            sa[i] = *reinterpret_cast<const float4*>(srow + 16 * ks + 8 * hh);
            sb[i] = *reinterpret_cast<const float4*>(srow + 16 * ks + 8 * hh + 4);
            ca[i] = *reinterpret_cast<const float4*>(crow + 16 * ks + 8 * hh);
            cb[i] = *reinterpret_cast<const float4*>(crow + 16 * ks + 8 * hh + 4);
        }
#pragma unroll
        for (int i = 0; i < 2 * KO; i++) { hold(xa[i]); hold(xb[i]); }
#pragma unroll
        for (int i = 0; i < KO; i++) { hold(sa[i]); hold(sb[i]); hold(ca[i]); hold(cb[i]); }
        h8* xq = reinterpret_cast<h8*>(grp == 0 ? v2 : v3);
#pragma unroll
        for (int i = 0; i < KO; i++) {
            float x0[8], x1[8], sn[8], cs[8], y0[8], y1[8];
            unpack(xa[i], xb[i], x0);
            unpack(xa[KO + i], xb[KO + i], x1);
            unpack(sa[i], sb[i], sn);
            unpack(ca[i], cb[i], cs);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                y0[e] = fmaf(cs[e], x0[e], -(sn[e] * x1[e]));
                y1[e] = fmaf(sn[e], x0[e], cs[e] * x1[e]);
            }
            xq[(i * 4 + sub) * 64 + lane] = to_qt(y0);
            xq[((KO + i) * 4 + sub) * 64 + lane] = to_qt(y1);
        }
    } else {
        float4 xa[NKS], xb[NKS], sa[KH], sb[KH], ca[KH], cb[KH];
        const int rofs = HALF % 16 == 0 ? 8 * hh : 0;   // D = 16: both halves read [0, 8)
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            xa[ks] = *reinterpret_cast<const float4*>(qrow + 16 * ks + 8 * hh);
            xb[ks] = *reinterpret_cast<const float4*>(qrow + 16 * ks + 8 * hh + 4);
        }
#pragma unroll
        for (int ks = 0; ks < KH; ks++) {
            sa[ks] = *reinterpret_cast<const float4*>(srow + 16 * ks + rofs);
            sb[ks] = *reinterpret_cast<const float4*>(srow + 16 * ks + rofs + 4);
            ca[ks] = *reinterpret_cast<const float4*>(crow + 16 * ks + rofs);
            cb[ks] = *reinterpret_cast<const float4*>(crow + 16 * ks + rofs + 4);
        }
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) { hold(xa[ks]); hold(xb[ks]); }
#pragma unroll
        for (int ks = 0; ks < KH; ks++) { hold(sa[ks]); hold(sb[ks]); hold(ca[ks]); hold(cb[ks]); }
        float x[NKS][8], sn[KH][8], cs[KH][8];
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) unpack(xa[ks], xb[ks], x[ks]);
#pragma unroll
        for (int ks = 0; ks < KH; ks++) {
            unpack(sa[ks], sb[ks], sn[ks]);
            unpack(ca[ks], cb[ks], cs[ks]);
        }
        float y[NKS][8];
        if constexpr (HALF % 16 == 0) {
            // d and d + HALF sit in the same lane, k-steps ks and ks + HALF/16.
#pragma unroll
            for (int ks = 0; ks < KH; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float a = x[ks][e], b = x[ks + KH][e];
                    y[ks][e] = fmaf(cs[ks][e], a, -(sn[ks][e] * b));
                    y[ks + KH][e] = fmaf(sn[ks][e], a, cs[ks][e] * b);
                }
#pragma unroll
            for (int ks = 2 * KH; ks < NKS; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) y[ks][e] = x[ks][e];
        } else {
            // D = 16: HALF = 8, the partner of d is in lane l ^ 32.
            static_assert(NKS == 1 && HALF == 8, "only D = 16 pairs across lanes");
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float other = __shfl_xor(x[0][e], 32);
                const float a = hh ? other : x[0][e];    // element d
                const float b = hh ? x[0][e] : other;    // element d + 8
                y[0][e] = hh ? fmaf(sn[0][e], a, cs[0][e] * b) : fmaf(cs[0][e], a, -(sn[0][e] * b));
            }
        }
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) qt[ks] = to_qt(y[ks]);
    }

    f32x16 acc[NDB];
#pragma unroll
    for (int b = 0; b < NDB; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[b][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    f32x16 S[NKB];                 // scores of this wave's current tile
    h8 pt[NT];                     // its fp16 weights, B operands of P^T

    // S^T block kb: rows = keys kb*32 + 8(r/4) + 4hh + r%4 of the tile,
    // column = l32.  The K fragments of block kb + 1 are read while block
    // kb's MFMAs run, so no MFMA waits on its own LDS read.
    auto qk = [&](const _Float16* sk) __attribute__((always_inline)) {
        h8 a[2][NKS];
        auto fetch = [&](int kb, h8 (&dst)[NKS]) __attribute__((always_inline)) {
            const _Float16* krow = sk + (kb * 32 + l32) * TL::KS + 8 * hh;
#pragma unroll
            for (int ks = 0; ks < NKS; ks++) dst[ks] = *reinterpret_cast<const h8*>(krow + 16 * ks);
        };
        fetch(0, a[0]);
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            if (kb + 1 < NKB) fetch(kb + 1, a[(kb + 1) & 1]);
#pragma unroll
            for (int r = 0; r < 16; r++) S[kb][r] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < NKS; ks++)
                S[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[kb & 1][ks], qt[ks], S[kb], 0, 0, 0);
        }
        pipeline_order<NKB * NKS>();
    };
    // O^T block b += V^T[32b + l32][keys of step t] * P^T[t].  The k index
    // 8hh + c of step t = (kb, tt) is key kb*32 + 16tt + 4hh + c for c < 4 and
    // kb*32 + 16tt + 8 + 4hh + (c - 4) for c >= 4: the order in which the S^T
    // accumulator holds them.  Block b + 1's V^T fragments are read while
    // block b's MFMAs run.
    auto vfetch = [&](const _Float16* sv, int b, h8 (&dst)[NT]) __attribute__((always_inline)) {
        const _Float16* vrow = sv + (32 * b + l32) * TL::VS + 4 * hh;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const h4 lo = *reinterpret_cast<const h4*>(vrow + 16 * t);
            const h4 hi = *reinterpret_cast<const h4*>(vrow + 16 * t + 8);
            dst[t] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };
    // With two groups the first V^T block of a P.V is read at the end of the
    // group's softmax phase before it (the tile is visible from that phase's
    // start, and no direct load targets its slot then), so the MFMA phase
    // does not start by waiting on LDS.
    h8 vpre[NT];
    auto pv = [&](const _Float16* sv) __attribute__((always_inline)) {
        h8 a[2][NT];
        auto fetch = [&](int b, h8 (&dst)[NT]) __attribute__((always_inline)) { vfetch(sv, b, dst); };
        if constexpr (NG == 2) {
#pragma unroll
            for (int t = 0; t < NT; t++) a[0][t] = vpre[t];
        } else {
            fetch(0, a[0]);
        }
#pragma unroll
        for (int b = 0; b < NDB; b++) {
            if (b + 1 < NDB) fetch(b + 1, a[(b + 1) & 1]);
#pragma unroll
            for (int t = 0; t < NT; t++)
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[b & 1][t], pt[t], acc[b], 0, 0, 0);
        }
        pipeline_order<NDB * NT>();
    };
    // Online softmax of tile t's scores: causal mask near the diagonal, lazy
    // running max (the accumulator is rescaled only when the max grows by
    // more than kTau), exp2, row sums of the fp16 weights as P^T uses them.
    auto softmax = [&](int t) __attribute__((always_inline)) {
        const int tg = tbase + t;                  // the KV head's tile index
        if (tg * KT + KT - 1 > qmin_wg) {
#pragma unroll
            for (int kb = 0; kb < NKB; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = tg * KT + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
                    if (key > qpos) S[kb][r] = -INFINITY;
                }
        }
        // Tile max as a tree of four partial maxima (short dependency chain).
        float mp[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) mp[r & 3] = fmaxf(mp[r & 3], S[kb][r]);
        float mt = fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3]));
        mt = max_halves(mt);
        const bool need = mt > m_run + kTau;
        if (__builtin_amdgcn_ballot_w64(need)) {
            const float mn = need ? mt : m_run;
            const float alpha = need ? __builtin_amdgcn_exp2f(m_run - mn) : 1.0f;
#pragma unroll
            for (int b = 0; b < NDB; b++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[b][r] *= alpha;
            l_run *= alpha;
            m_run = mn;
        }
        // A group's first tiles can be fully masked for a column (the odd
        // group starts at keys KT..2KT-1): its max is then still -inf and its
        // weights are exp2(-inf - 0) = 0 rather than exp2(-inf + inf).
        const float msub = m_run == -INFINITY ? 0.0f : m_run;
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
        float lp[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // four independent row-sum chains
#pragma unroll
        for (int t2 = 0; t2 < NT; t2++) {
            h8 v;
#pragma unroll
            for (int c = 0; c < 8; c++)
                v[c] = (_Float16)__builtin_amdgcn_exp2f(S[t2 >> 1][8 * (t2 & 1) + c] - msub);
            pt[t2] = v;
#pragma unroll
            for (int c = 0; c < 8; c += 2) {
                const h2 p2 = {v[c], v[c + 1]};
                lp[c >> 1] = __builtin_amdgcn_fdot2(p2, one, lp[c >> 1], false);
            }
        }
        l_run += (lp[0] + lp[1]) + (lp[2] + lp[3]);
    };

    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if constexpr (kSplitQ) {
        // k-step ks = kh (+ KH) was written by group kh / (KH / 2) at index
        // (kh % (KH / 2)) (+ KH / 2).
        constexpr int KO = KH / 2;
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            const int kh = ks % KH, i = kh % KO + (ks >= KH ? KO : 0);
            const h8* xq = reinterpret_cast<const h8*>(kh / KO == 0 ? v2 : v3);
            qt[ks] = xq[(i * 4 + sub) * 64 + lane];
        }
    }

    // Phase p (p = 0 .. ntile + 1): the group p % 2 runs MFMAs -- P.V of
    // tile p - 2 (its previous tile) and QK of tile p -- while the other
    // group runs tile p - 1's softmax.  Slots: K(t) in kslot[t % 4], V(t) in
    // vslot[t % 4].  Each group runs its own straight-line phase sequence
    // (group 0: M V M V ..., group 1: V M V M ...), unrolled by four so every
    // slot is a fixed LDS object.
    //
    // End of phase p: wait for this wave's direct loads (the ones issued at
    // the end of phase p - 1: K(p + 2) and V(p), read in phase p + 2), issue
    // the loads of phase p + 1 -- K(p + 3) and V(p + 1), into slots last read
    // in phase p - 1 -- and pass the barrier, which makes every wave's
    // completed loads visible.  Only one phase's loads are ever in flight at
    // a wait, so the wait is a plain vmcnt(0) and each load still has a whole
    // phase to land.
    const int nphase = NG == 2 ? ntile + 2 : ntile;
    auto dma = [&](int p, int R) __attribute__((always_inline)) {
        if constexpr (NG == 2) {
            if (p + 2 < ntile) load_k(kslot[(R + 2) % kSlots], p + 2);
            if (p < ntile) load_v(vslot[R], p);
        } else {
            if (p + 2 < ntile) {
                load_k(kslot[(R + 2) % kSlots], p + 2);
                load_v(vslot[(R + 2) % kSlots], p + 2);
            }
        }
    };
    auto end_p = [&](int p, int R) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(0xF70);          // vmcnt(0)
        dma(p + 1, (R + 1) % kSlots);
        phase_barrier();
    };
    auto mphase = [&](int p, int R) __attribute__((always_inline)) {
        if (p >= 2 && p - 2 < ntile) pv(vslot[(R + 2) % kSlots]);
        __builtin_amdgcn_sched_barrier(0);   // P.V's weights die before QK's scores are born
        if (p < ntile) qk(kslot[R]);
    };
    auto vphase = [&](int p, int R) __attribute__((always_inline)) {
        if (p >= 1 && p - 1 < ntile) {
            softmax(p - 1);
            vfetch(vslot[(R + 3) % kSlots], 0, vpre);   // phase p + 1's P.V of tile p - 1
        }
    };
    if constexpr (NG == 2) {
        if (grp == 0) {
            for (int p = 0; p < nphase; p += 4) {
                mphase(p, 0); end_p(p, 0);
                if (p + 1 >= nphase) break;
                vphase(p + 1, 1); end_p(p + 1, 1);
                if (p + 2 >= nphase) break;
                mphase(p + 2, 2); end_p(p + 2, 2);
                if (p + 3 >= nphase) break;
                vphase(p + 3, 3); end_p(p + 3, 3);
            }
        } else {
            for (int p = 0; p < nphase; p += 4) {
                vphase(p, 0); end_p(p, 0);
                if (p + 1 >= nphase) break;
                mphase(p + 1, 1); end_p(p + 1, 1);
                if (p + 2 >= nphase) break;
                vphase(p + 2, 2); end_p(p + 2, 2);
                if (p + 3 >= nphase) break;
                mphase(p + 3, 3); end_p(p + 3, 3);
            }
        }
    } else {
        // One group: phase p runs tile p start to finish.
        auto whole = [&](int p, int R) __attribute__((always_inline)) {
            if (p < ntile) {
                qk(kslot[R]);
                softmax(p);
                pv(vslot[R]);
            }
            end_p(p, R);
        };
        for (int p = 0; p < nphase; p += 4) {
            whole(p, 0);
            if (p + 1 < nphase) whole(p + 1, 1);
            if (p + 2 < nphase) whole(p + 2, 2);
            if (p + 3 < nphase) whole(p + 3, 3);
        }
    }

    // ---- merge the groups' (m, l, o) and write O[d][column] for
    // d = 32b + 8(r/4) + 4hh + r%4.  One exchange: block b of O^T is
    // finished by group owner(b) (the first half of the blocks by group 0,
    // the rest by group 1), and the other group hands its partial block b
    // over through LDS -- the K ring slots, free once the last phase's
    // barrier has passed, when they are large enough, else a dedicated
    // buffer.  Lane (l32, hh) of wave `sub` holds the same (d, column) in
    // both groups, so each lane reads back exactly what its partner wrote.
    constexpr int XBLK = 4 * 16 * 64;                      // floats per exchanged block
    constexpr bool kInRing = TL::K_ELEMS * 2 >= XBLK * 4 && NDB <= kSlots;
    __shared__ __attribute__((aligned(16))) float xm[NG == 2 ? 2 * 4 * 2 * 64 : 1];
    __shared__ __attribute__((aligned(16))) float xo[NG == 2 && !kInRing ? NDB * XBLK : 1];
    auto owner = [&](int b) __attribute__((always_inline)) { return NDB == 1 ? 0 : (b < NDB / 2 ? 0 : 1); };
    auto xbuf = [&](int b) __attribute__((always_inline)) -> float* {
        if constexpr (kInRing) return reinterpret_cast<float*>(kslot[b]);
        else return xo + b * XBLK;
    };
    float fa = 1.0f, fb = 0.0f, inv;
    if constexpr (NG == 2) {
        xm[((grp * 4 + sub) * 2 + 0) * 64 + lane] = m_run;
        xm[((grp * 4 + sub) * 2 + 1) * 64 + lane] = l_run;
#pragma unroll
        for (int b = 0; b < NDB; b++) {
            if (owner(b) != grp) {
                float4* dst = reinterpret_cast<float4*>(xbuf(b));
#pragma unroll
                for (int r4 = 0; r4 < 4; r4++)
                    dst[(sub * 4 + r4) * 64 + lane] = make_float4(acc[b][4 * r4], acc[b][4 * r4 + 1], acc[b][4 * r4 + 2],
                                               acc[b][4 * r4 + 3]);
            }
        }
        __syncthreads();
        const int og = grp ^ 1;
        const float mb = xm[((og * 4 + sub) * 2 + 0) * 64 + lane];
        const float lb = xm[((og * 4 + sub) * 2 + 1) * 64 + lane];
        const float M = fmaxf(m_run, mb);
        fa = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - M);
        fb = mb == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mb - M);
        const float L = sum_halves(l_run * fa + lb * fb);
        inv = 1.0f / L;
        if constexpr (SPLIT) {
            inv = 1.0f;                            // the partial stays unnormalised
            if (grp == 0 && hh == 0) {
                P.part_ml[(pbase + 32 * sub + l32) * 2 + 0] = M;
                P.part_ml[(pbase + 32 * sub + l32) * 2 + 1] = L;
            }
        }
    } else {
        const float L = sum_halves(l_run);
        inv = 1.0f / L;
        if constexpr (SPLIT) {
            inv = 1.0f;
            if (hh == 0) {
                P.part_ml[(pbase + 32 * sub + l32) * 2 + 0] = m_run;
                P.part_ml[(pbase + 32 * sub + l32) * 2 + 1] = L;
            }
        }
    }
    if constexpr (NG == 2) {
        // Owned block b: read the partner's partial (4 KB of xbuf(b) per
        // wave), then restage the finished block in that same region as
        // [column][16-byte unit] with the unit index XORed by column % 8
        // (conflict-free both ways), and write it back row-contiguous: each
        // store instruction covers 8 columns x 128 bytes, whole cache lines
        // of O instead of 32-byte pieces of 32 rows.  The stores are
        // non-temporal: O is not read again here, and streaming it out as it
        // is produced keeps 32 MB of dirty lines (a 2048-token layer) from
        // being written back all at once when the kernel ends.
#pragma unroll
        for (int b = 0; b < NDB; b++) {
            if (owner(b) != grp) continue;
            float4* st = reinterpret_cast<float4*>(xbuf(b)) + sub * 256;
            float4 ob[4];
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) ob[r4] = st[r4 * 64 + lane];
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                float4 o;
                o.x = (acc[b][4 * r4 + 0] * fa + ob[r4].x * fb) * inv;
                o.y = (acc[b][4 * r4 + 1] * fa + ob[r4].y * fb) * inv;
                o.z = (acc[b][4 * r4 + 2] * fa + ob[r4].z * fb) * inv;
                o.w = (acc[b][4 * r4 + 3] * fa + ob[r4].w * fb) * inv;
                const int u = 2 * r4 + hh;
                st[l32 * 8 + (u ^ (l32 & 7))] = o;
            }
            const int u = lane & 7;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = 8 * i + (lane >> 3);
                const float4 o = st[c * 8 + (u ^ (c & 7))];
                const int cg = 32 * sub + c;
                const int tc = qb * BM + cg / G;
                const int d = 32 * b + 4 * u;
                if constexpr (SPLIT) {
                    if (d < D) *reinterpret_cast<float4*>(P.part_o + (pbase + cg) * D + d) = o;
                } else if (tc < P.n && cg % G < gc && d < Dr && P.pos0 + tc >= kExactKeys) {
                    float* orow = P.out + ((size_t)tc * P.H + head0 + cg % G) * Dr;
                    if constexpr (PAD) {
                        const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (d + e < Dr) __builtin_nontemporal_store(ov[e], orow + d + e);
                    } else {
                        __builtin_nontemporal_store(__builtin_bit_cast(f32x4, o),
                                                    reinterpret_cast<f32x4*>(orow + d));
                    }
                }
            }
        }
        return;
    }
    if constexpr (SPLIT) {
        float* prow = P.part_o + (pbase + col) * D;
#pragma unroll
        for (int b = 0; b < NDB; b++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++)
                *reinterpret_cast<float4*>(prow + 32 * b + 8 * r4 + 4 * hh) =
                    make_float4(acc[b][4 * r4 + 0], acc[b][4 * r4 + 1], acc[b][4 * r4 + 2], acc[b][4 * r4 + 3]);
        return;
    }
    if (!valid || P.pos0 + ti < kExactKeys) return;   // rows written by the staging kernel
    float* orow = P.out + ((size_t)ti * P.H + h) * Dr;
#pragma unroll
    for (int b = 0; b < NDB; b++) {
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
            const int d = 32 * b + 8 * r4 + 4 * hh;
            float4 o;
            o.x = acc[b][4 * r4 + 0] * inv;
            o.y = acc[b][4 * r4 + 1] * inv;
            o.z = acc[b][4 * r4 + 2] * inv;
            o.w = acc[b][4 * r4 + 3] * inv;
            if constexpr (PAD) {
                const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (d + e < Dr) orow[d + e] = ov[e];
            } else if (d < D) {
                *reinterpret_cast<float4*>(orow + d) = o;
            }
        }
    }
}

// ---- merge of the key splits -----------------------------------------------

// One thread per (query block, head slot, column, 4 elements of the width):
// the nsplit partials of the column merged with their maxima, normalised,
// written to the column's row (rows below kExactKeys are the staging
// kernel's).  A split with m = -inf (no keys) counts for nothing.
template <int D, int G, bool PAD>
__global__ __launch_bounds__(256) void prefill_merge(AttnParams P) {
    constexpr int BM = kCols / G;
    constexpr int NV = D / 4;
    const int NY = P.HK * P.nsub;
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int v4 = (int)(t % NV);
    long long r = t / NV;
    const int col = (int)(r % kCols);
    r /= kCols;
    const int y = (int)(r % NY);
    const int qb = (int)(r / NY);
    if (qb >= P.nqb) return;
    const int g = y / P.nsub;
    const int ysub = y - g * P.nsub;
    const int head0 = (g * P.H + P.HK - 1) / P.HK + ysub * G;
    const int gc = min(G, (g * P.H + P.H + P.HK - 1) / P.HK - head0);
    const int tc = qb * BM + col / G;
    const int Dr = PAD ? P.Dr : D;
    const int d = 4 * v4;
    if (gc <= 0 || tc >= P.n || col % G >= gc || P.pos0 + tc < kExactKeys || d >= Dr) return;
    const size_t stride = (size_t)P.nqb * NY * kCols;           // one split's rows
    const size_t row = ((size_t)qb * NY + y) * kCols + col;
    // Batches of 8 splits, every load of a batch issued before any is used
    // (one memory round trip per batch), folded online.  The o of an empty
    // split was never written: it is selected away, not multiplied by 0.
    constexpr int NB = 8;
    float M = -INFINITY, L = 0.0f;
    float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = 0; s0 < P.nsplit; s0 += NB) {
        float2 ml[NB];
        float4 o[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const size_t r2 = (size_t)min(s0 + i, P.nsplit - 1) * stride + row;
            ml[i] = *reinterpret_cast<const float2*>(P.part_ml + r2 * 2);
            o[i] = *reinterpret_cast<const float4*>(P.part_o + r2 * D + d);
            if (s0 + i >= P.nsplit) ml[i].x = -INFINITY;
        }
        float mb = M;
#pragma unroll
        for (int i = 0; i < NB; i++) mb = fmaxf(mb, ml[i].x);
        const float a = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - mb);
        L *= a;
        O.x *= a;
        O.y *= a;
        O.z *= a;
        O.w *= a;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const bool live = ml[i].x != -INFINITY;
            const float w = live ? __builtin_amdgcn_exp2f(ml[i].x - mb) : 0.0f;
            L = live ? fmaf(ml[i].y, w, L) : L;
            O.x = live ? fmaf(o[i].x, w, O.x) : O.x;
            O.y = live ? fmaf(o[i].y, w, O.y) : O.y;
            O.z = live ? fmaf(o[i].z, w, O.z) : O.z;
            O.w = live ? fmaf(o[i].w, w, O.w) : O.w;
        }
        M = mb;
    }
    const float inv = 1.0f / L;
    float* orow = P.out + ((size_t)tc * P.H + head0 + col % G) * Dr;
    const float ov[4] = {O.x * inv, O.y * inv, O.z * inv, O.w * inv};
    if constexpr (PAD) {
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (d + e < Dr) orow[d + e] = ov[e];
    } else {
        *reinterpret_cast<float4*>(orow + d) = make_float4(ov[0], ov[1], ov[2], ov[3]);
    }
}

// Key splits per query block: a launch with few query blocks (a prompt chunk
// after a long context) gets about kSplitTarget workgroups, each over at
// least kMinSplitTiles tiles, since a workgroup's fixed cost (q prologue,
// merge, output) is worth several tiles.
constexpr int kSplitTarget = 256;
constexpr int kMinSplitTiles = 8;

// ---- launch ----------------------------------------------------------------

template <int D, int G, typename CT>
int launch_dg(const PrefillArgs& a, int nsub, hipStream_t st) {
    using TL = Tile<D>;
    const long long rows = (long long)a.pos0 + a.n_tokens;
    const int T = (int)((rows + TL::KT - 1) / TL::KT);
    const int HK = a.n_kv_heads;
    // Rows below kExactKeys: n_exact * nsub extra grid rows (the first ones)
    // of HK workgroups, one per (row, head slot).
    const int n_exact = std::max(0, std::min(a.n_tokens, kExactKeys - a.pos0));
    if ((long long)T * (TL::KT / StageRows<D>::N) + (long long)n_exact * nsub > 65535)
        return PKH_ERR_ARG;                                                       // grid y limit
    // A KV head's tiles are addressed with 32-bit signed byte offsets.
    if ((long long)T * TL::BYTES >= (1LL << 31)) return PKH_ERR_ARG;
    constexpr int BM = kCols / G;
    const long long nqb = (a.n_tokens + BM - 1) / BM;
    const long long base_wgs = nqb * HK * nsub;
    int nsplit = 1, tps = T;
    if (base_wgs < kSplitTarget && T >= 2 * kMinSplitTiles) {
        nsplit = (int)std::min<long long>(kSplitTarget / base_wgs, T / kMinSplitTiles);
        tps = (T + nsplit - 1) / nsplit;
        nsplit = (T + tps - 1) / tps;
    }
    if (base_wgs * nsplit > 0x7fffffffLL) return PKH_ERR_ARG;                   // grid x limit
    void* tiles = nullptr;
    int rc = tiles_get((size_t)HK * T * TL::BYTES, &tiles);
    if (rc != PKH_OK) return rc;
    void* parts = nullptr;
    const size_t part_rows = (size_t)nsplit * nqb * HK * nsub * kCols;
    if (nsplit > 1) {
        rc = scratch_get(part_rows * (D + 2) * sizeof(float), &parts);
        if (rc != PKH_OK) return rc;
    }

    // The vector staging needs whole 4-element groups on both sides of the
    // rotation half and 16-byte aligned new rows: the real width D itself.
    const bool pad = a.head_dim != D;
    StageParams S{};
    S.k_layer = a.k_layer;
    S.v_layer = a.v_layer;
    S.stride_pos = a.stride_pos;
    S.stride_head = a.stride_head;
    S.k_new = a.k_new;
    S.v_new = a.v_new;
    S.rope_sin = a.rope_sin;
    S.rope_cos = a.rope_cos;
    S.half = a.half;
    S.pos0 = a.pos0;
    S.n = a.n_tokens;
    S.HK = HK;
    S.Dr = a.head_dim;
    S.T = T;
    S.tiles = static_cast<_Float16*>(tiles);
    S.q = a.q;
    S.out = a.out;
    S.H = a.n_heads;
    S.Gs = G;
    S.nsub = nsub;
    S.qscale = (1.0f / sqrtf((float)a.head_dim)) * 1.4426950408889634f;
    // KV head fastest: measured 9.3 against 10.0 us for the Llama-3-8B
    // 2048-row layer with the tile index fastest.
    const dim3 sgrid(HK, T * (TL::KT / StageRows<D>::N) + n_exact * nsub);
    if (pad)
        hipLaunchKernelGGL((prefill_stage_any<D, CT>), sgrid, dim3(kThreads), 0, st, S);
    else
        hipLaunchKernelGGL((prefill_stage<D, CT>), sgrid, dim3(kThreads), 0, st, S);
    PKH_HIP(hipGetLastError());

    AttnParams A{};
    A.tiles = static_cast<const _Float16*>(tiles);
    A.T = T;
    A.q = a.q;
    A.out = a.out;
    A.rope_sin = a.rope_sin;
    A.rope_cos = a.rope_cos;
    A.half = a.half;
    A.pos0 = a.pos0;
    A.n = a.n_tokens;
    A.H = a.n_heads;
    A.HK = HK;
    A.nqb = (int)nqb;
    A.Dr = a.head_dim;
    A.nsub = nsub;
    A.qscale = (1.0f / sqrtf((float)a.head_dim)) * 1.4426950408889634f;
    A.nsplit = nsplit;
    A.tps = tps;
    A.part_o = static_cast<float*>(parts);
    A.part_ml = A.part_o ? A.part_o + part_rows * D : nullptr;
    const dim3 agrid((unsigned)(base_wgs * nsplit)), ablock(256 * Groups<D>::N);
    if (nsplit > 1) {
        if (pad)
            hipLaunchKernelGGL((prefill_attn<D, G, true, true>), agrid, ablock, 0, st, A);
        else
            hipLaunchKernelGGL((prefill_attn<D, G, false, true>), agrid, ablock, 0, st, A);
    } else {
        if (pad)
            hipLaunchKernelGGL((prefill_attn<D, G, true, false>), agrid, ablock, 0, st, A);
        else
            hipLaunchKernelGGL((prefill_attn<D, G, false, false>), agrid, ablock, 0, st, A);
    }
    PKH_HIP(hipGetLastError());
    if (nsplit > 1) {
        const long long nthreads = base_wgs * kCols * (D / 4);
        const dim3 mgrid((unsigned)((nthreads + 255) / 256));
        if (pad)
            hipLaunchKernelGGL((prefill_merge<D, G, true>), mgrid, dim3(256), 0, st, A);
        else
            hipLaunchKernelGGL((prefill_merge<D, G, false>), mgrid, dim3(256), 0, st, A);
        PKH_HIP(hipGetLastError());
    }

    return PKH_OK;
}

template <int D, typename CT>
int launch_d(const PrefillArgs& a, hipStream_t st) {
    const HeadSlots hs = head_slots(a.n_heads, a.n_kv_heads, 8);
    switch (hs.G) {
        case 1: return launch_dg<D, 1, CT>(a, hs.nsub, st);
        case 2: return launch_dg<D, 2, CT>(a, hs.nsub, st);
        case 4: return launch_dg<D, 4, CT>(a, hs.nsub, st);
        case 8: return launch_dg<D, 8, CT>(a, hs.nsub, st);
        default: return PKH_ERR_ARG;
    }
}

template <typename CT>
int launch_ct(const PrefillArgs& a, hipStream_t st) {
    switch (padded_head_dim(a.head_dim)) {
        case 16: return launch_d<16, CT>(a, st);
        case 32: return launch_d<32, CT>(a, st);
        case 64: return launch_d<64, CT>(a, st);
        case 128: return launch_d<128, CT>(a, st);
        case 256: return launch_d<256, CT>(a, st);
        default: return PKH_ERR_ARG;
    }
}

}  // namespace

bool prefill_supported(int head_dim, int n_heads, int n_kv_heads, int dtype) {
    return padded_head_dim(head_dim) != 0 && n_heads > 0 && n_kv_heads > 0 &&
           (dtype == PKH_KV_F32 || dtype == PKH_KV_F16);
}

int launch_prefill(const PrefillArgs& a, hipStream_t stream) {
    if (!prefill_supported(a.head_dim, a.n_heads, a.n_kv_heads, a.dtype)) return PKH_ERR_ARG;
    if (a.half != rope_half_of(a.head_dim) || a.n_tokens <= 0 || a.pos0 < 0) return PKH_ERR_ARG;
    if (a.dtype == PKH_KV_F32) return launch_ct<float>(a, stream);
    return launch_ct<_Float16>(a, stream);
}

}  // namespace pkh
