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
// prefill_stage  one workgroup per (tile of kKT rows, KV head).  New rows
//                (p >= pos0) get k rotated in fp32 with the reference's
//                contraction, and k_rot / v are appended to the cache in its
//                element type; rows below pos0 are read back from the cache.
//                Every row is also written, as fp16, into a tile buffer laid
//                out exactly as the attention kernel keeps it in LDS:
//                K as [key][D + kKPad] and V transposed as [d][kKT + kVPad].
//                Rows past the last position are zero.
//
// prefill_attn   one workgroup per (block of query positions, KV head),
//                dispatched longest-first, with blockIdx % HK == KV head so
//                that on an 8-XCD part each XCD's L2 holds one head's tiles.
//                The 4 waves hold 128 query columns: column c is head
//                c % G of the group at token c / G, so the G heads that share
//                a KV head share every K/V tile.  Each wave computes
//                S^T = K Q^T and O^T += V^T P^T with
//                v_mfma_f32_32x32x16_f16: keeping the query index on the lane
//                makes the softmax statistics per-lane scalars, and the
//                S^T accumulator registers are, converted to fp16, exactly
//                the B operand of the P^T product once the keys of a 16-key
//                step are taken in the order the accumulator holds them
//                (the V^T reads use the same order).  Softmax runs in fp32,
//                in log2 units (q is pre-scaled by log2(e)/sqrt(D)), with a
//                lazily rescaled running maximum.  Tiles are double-buffered
//                in LDS with a register prefetch one tile ahead.

#include "pkh_internal.h"

#include <cmath>
#include <utility>

namespace pkh {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kKT = 64;         // keys per tile
constexpr int kKPad = 8;        // fp16 padding per K row (conflict-free ds_read_b128)
constexpr int kVPad = 4;        // fp16 padding per V^T row (conflict-free ds_read_b64)
constexpr int kThreads = 256;   // 4 waves
constexpr int kCols = 128;      // query columns per workgroup (32 per wave)
constexpr float kTau = 8.0f;    // lazy-rescale threshold, log2 units

constexpr int rope_half_of(int D) { return D / 2 < 64 ? D / 2 : 64; }

// One staged tile of one KV head: K rows then V^T rows, fp16.
template <int D>
struct Tile {
    static constexpr int KS = D + kKPad;              // K row stride
    static constexpr int VROWS = D < 32 ? 32 : D;     // V^T rows, zero-padded to a 32-row block
    static constexpr int VS = kKT + kVPad;            // V^T row stride
    static constexpr int K_ELEMS = kKT * KS;
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
__device__ __forceinline__ void load4(const _Float16* p, float (&x)[4]) {
    const h4 v = *reinterpret_cast<const h4*>(p);
    for (int i = 0; i < 4; i++) x[i] = (float)v[i];
}
__device__ __forceinline__ void store4(float* p, const float (&x)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
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
    *reinterpret_cast<h4*>(p) = to_h4(x);
}

// ---- stage: append + fp16 tiles -------------------------------------------

struct StageParams {
    void* k_layer;              // cache element type CT
    void* v_layer;
    long long stride_pos, stride_head;
    const float* k_new;         // [n][HK][D]
    const float* v_new;
    const float* rope_sin;      // [max_seq][half]
    const float* rope_cos;
    int half, pos0, n, HK;
    int T;                      // tiles per head
    _Float16* tiles;            // [HK][T][Tile::ELEMS]
};

template <int D, typename CT>
__global__ __launch_bounds__(kThreads) void prefill_stage(StageParams P) {
    using TL = Tile<D>;
    constexpr int HALF = rope_half_of(D);
    constexpr int NP = HALF / 4;              // rotated pairs of 4-element groups
    constexpr int NL = (D - 2 * HALF) / 4;    // unrotated 4-element groups (D = 256)
    constexpr int NI = NP + NL;
    constexpr int TPR = NI < 16 ? NI : 16;    // threads per row
    constexpr int RPP = kThreads / TPR;       // rows per pass
    __shared__ __attribute__((aligned(16))) _Float16 sv[kKT][D + 4];   // 8-byte aligned rows

    const int tid = threadIdx.x;
    const int j = blockIdx.x, g = blockIdx.y;
    _Float16* tk = P.tiles + ((size_t)g * P.T + j) * TL::ELEMS;
    _Float16* tv = tk + TL::K_ELEMS;
    CT* kc = static_cast<CT*>(P.k_layer) + (size_t)g * P.stride_head;
    CT* vc = static_cast<CT*>(P.v_layer) + (size_t)g * P.stride_head;

    for (int r = tid / TPR; r < kKT; r += RPP) {
        const int p = j * kKT + r;
        for (int it = tid % TPR; it < NI; it += TPR) {
            const bool pair = it < NP;
            const int d0 = pair ? 4 * it : 2 * HALF + 4 * (it - NP);
            float k0[4] = {0, 0, 0, 0}, k1[4] = {0, 0, 0, 0};
            float v0[4] = {0, 0, 0, 0}, v1[4] = {0, 0, 0, 0};
            if (p < P.pos0) {
                // Earlier context: already rotated in the cache.
                const size_t row = (size_t)p * P.stride_pos;
                load4(kc + row + d0, k0);
                load4(vc + row + d0, v0);
                if (pair) {
                    load4(kc + row + d0 + HALF, k1);
                    load4(vc + row + d0 + HALF, v1);
                }
            } else if (p < P.pos0 + P.n) {
                const size_t src = ((size_t)(p - P.pos0) * P.HK + g) * D;
                load4(P.k_new + src + d0, k0);
                load4(P.v_new + src + d0, v0);
                if (pair) {
                    load4(P.k_new + src + d0 + HALF, k1);
                    load4(P.v_new + src + d0 + HALF, v1);
                    float s[4], c[4];
                    load4(P.rope_sin + (size_t)p * P.half + d0, s);
                    load4(P.rope_cos + (size_t)p * P.half + d0, c);
                    for (int i = 0; i < 4; i++) {
                        // src/pickle_fast.c:1917-1922 as compiled: x0' = c*x0 - s*x1
                        // and x1' = s*x0 + c*x1, each one fused multiply-add.
                        const float a = k0[i], b = k1[i];
                        k0[i] = fmaf(c[i], a, -(s[i] * b));
                        k1[i] = fmaf(s[i], a, c[i] * b);
                    }
                }
                const size_t row = (size_t)p * P.stride_pos;
                store4(kc + row + d0, k0);
                store4(vc + row + d0, v0);
                if (pair) {
                    store4(kc + row + d0 + HALF, k1);
                    store4(vc + row + d0 + HALF, v1);
                }
            }
            *reinterpret_cast<h4*>(tk + r * TL::KS + d0) = to_h4(k0);
            *reinterpret_cast<h4*>(&sv[r][d0]) = to_h4(v0);
            if (pair) {
                *reinterpret_cast<h4*>(tk + r * TL::KS + d0 + HALF) = to_h4(k1);
                *reinterpret_cast<h4*>(&sv[r][d0 + HALF]) = to_h4(v1);
            }
        }
    }
    __syncthreads();
    // V^T rows, 8 keys per store (two 8-byte halves: rows are 8-byte aligned).
    for (int u = tid; u < TL::VROWS * (kKT / 8); u += kThreads) {
        const int d = u / (kKT / 8), c8 = u % (kKT / 8);
        h4 lo, hi;
        for (int i = 0; i < 4; i++) {
            lo[i] = d < D ? sv[8 * c8 + i][d] : (_Float16)0.0f;
            hi[i] = d < D ? sv[8 * c8 + 4 + i][d] : (_Float16)0.0f;
        }
        _Float16* dst = tv + d * TL::VS + 8 * c8;
        *reinterpret_cast<h4*>(dst) = lo;
        *reinterpret_cast<h4*>(dst + 4) = hi;
    }
}

// ---- attention -------------------------------------------------------------

struct AttnParams {
    const _Float16* tiles;      // [HK][T][Tile::ELEMS]
    int T;
    const float* q;             // [n][H][D]
    float* out;                 // [n][H][D]
    const float* rope_sin;
    const float* rope_cos;
    int half, pos0, n, H, HK, nqb;
    float qscale;               // log2(e) / sqrt(D)
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

// A tile moves HBM/L2 -> registers -> LDS in 16-byte chunks; the register
// copy of the next tile is held across the current tile's compute.
template <int D>
struct TileRegs {
    static constexpr int CH = Tile<D>::BYTES / 16;     // chunks per tile
    static constexpr int FULL = CH / kThreads;         // chunks every thread moves
    static constexpr bool TAIL = CH % kThreads != 0;   // one more for the first threads
    u32x4 r[FULL + 1];

    // Fold expressions keep every index a constant, so r[] stays in VGPRs.
    template <int... I>
    __device__ __forceinline__ void load_full(const u32x4* src, int tid,
                                              std::integer_sequence<int, I...>) {
        ((r[I] = src[tid + kThreads * I]), ...);
    }
    template <int... I>
    __device__ __forceinline__ void store_full(u32x4* dst, int tid,
                                               std::integer_sequence<int, I...>) const {
        ((dst[tid + kThreads * I] = r[I]), ...);
    }
    __device__ __forceinline__ void load(const u32x4* src, int tid) {
        load_full(src, tid, std::make_integer_sequence<int, FULL>{});
        if constexpr (TAIL) {
            if (tid + kThreads * FULL < CH) r[FULL] = src[tid + kThreads * FULL];
        }
    }
    __device__ __forceinline__ void store(_Float16* dst, int tid) const {
        u32x4* d = reinterpret_cast<u32x4*>(dst);
        store_full(d, tid, std::make_integer_sequence<int, FULL>{});
        if constexpr (TAIL) {
            if (tid + kThreads * FULL < CH) d[tid + kThreads * FULL] = r[FULL];
        }
    }
};

template <int D, int G>
__global__ __launch_bounds__(kThreads, D >= 256 ? 1 : 2) void prefill_attn(AttnParams P) {
    using TL = Tile<D>;
    constexpr int HALF = rope_half_of(D);
    constexpr int NKS = D / 16;             // k-steps of S^T = K Q^T
    constexpr int NDB = TL::VROWS / 32;     // 32-row blocks of O^T
    constexpr int NKB = kKT / 32;           // 32-key blocks per tile
    constexpr int BM = kCols / G;           // query positions per workgroup
    constexpr int CH = TL::BYTES / 16;
    __shared__ __attribute__((aligned(16))) _Float16 lds[2][TL::ELEMS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, hh = lane >> 5, l32 = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = blockIdx.x % P.HK;
    const int qb = P.nqb - 1 - (int)(blockIdx.x / P.HK);
    const int col = 32 * w + l32;
    const int ti = qb * BM + col / G;
    const bool valid = ti < P.n;
    const int tic = valid ? ti : P.n - 1;
    const int h = g * G + col % G;
    const int qpos = P.pos0 + tic;
    const int qmin_w = P.pos0 + min(qb * BM + (32 * w) / G, P.n - 1);
    const int qmax = P.pos0 + min(qb * BM + BM - 1, P.n - 1);
    const int ntile = qmax / kKT + 1;

    const u32x4* src = reinterpret_cast<const u32x4*>(P.tiles + (size_t)g * P.T * TL::ELEMS);
    TileRegs<D> pre;
    pre.load(src, tid);

    // ---- q: load, rotate (same contraction as the reference), scale, fp16.
    // Lane (l32, hh) holds, for k-step ks, elements d = 16ks + 8hh + [0, 8).
    h8 qt[NKS];
    {
        const float* qrow = P.q + ((size_t)tic * P.H + h) * D;
        float x[NKS][8];
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            const float4 a = *reinterpret_cast<const float4*>(qrow + 16 * ks + 8 * hh);
            const float4 b = *reinterpret_cast<const float4*>(qrow + 16 * ks + 8 * hh + 4);
            x[ks][0] = a.x; x[ks][1] = a.y; x[ks][2] = a.z; x[ks][3] = a.w;
            x[ks][4] = b.x; x[ks][5] = b.y; x[ks][6] = b.z; x[ks][7] = b.w;
        }
        const float* srow = P.rope_sin + (size_t)qpos * P.half;
        const float* crow = P.rope_cos + (size_t)qpos * P.half;
        float y[NKS][8];
        if constexpr (HALF % 16 == 0) {
            // d and d + HALF sit in the same lane, k-steps ks and ks + HALF/16.
            constexpr int KH = HALF / 16;
#pragma unroll
            for (int ks = 0; ks < KH; ks++) {
                float s[8], c[8];
                const float4 s0 = *reinterpret_cast<const float4*>(srow + 16 * ks + 8 * hh);
                const float4 s1 = *reinterpret_cast<const float4*>(srow + 16 * ks + 8 * hh + 4);
                const float4 c0 = *reinterpret_cast<const float4*>(crow + 16 * ks + 8 * hh);
                const float4 c1 = *reinterpret_cast<const float4*>(crow + 16 * ks + 8 * hh + 4);
                s[0] = s0.x; s[1] = s0.y; s[2] = s0.z; s[3] = s0.w;
                s[4] = s1.x; s[5] = s1.y; s[6] = s1.z; s[7] = s1.w;
                c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w;
                c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float a = x[ks][e], b = x[ks + KH][e];
                    y[ks][e] = fmaf(c[e], a, -(s[e] * b));
                    y[ks + KH][e] = fmaf(s[e], a, c[e] * b);
                }
            }
#pragma unroll
            for (int ks = 2 * KH; ks < NKS; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) y[ks][e] = x[ks][e];
        } else {
            // D = 16: HALF = 8, the partner of d is in lane l ^ 32.
            static_assert(NKS == 1 && HALF == 8, "only D = 16 pairs across lanes");
            const float4 s0 = *reinterpret_cast<const float4*>(srow);
            const float4 s1 = *reinterpret_cast<const float4*>(srow + 4);
            const float4 c0 = *reinterpret_cast<const float4*>(crow);
            const float4 c1 = *reinterpret_cast<const float4*>(crow + 4);
            const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
            const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float other = __shfl_xor(x[0][e], 32);
                const float a = hh ? other : x[0][e];    // element d
                const float b = hh ? x[0][e] : other;    // element d + 8
                y[0][e] = hh ? fmaf(s[e], a, c[e] * b) : fmaf(c[e], a, -(s[e] * b));
            }
        }
#pragma unroll
        for (int ks = 0; ks < NKS; ks++) {
            h8 v;
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = (_Float16)(y[ks][e] * P.qscale);
            qt[ks] = v;
        }
    }

    pre.store(lds[0], tid);
    if (ntile > 1) pre.load(src + CH, tid);
    __syncthreads();

    f32x16 acc[NDB];
#pragma unroll
    for (int b = 0; b < NDB; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[b][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    for (int j = 0; j < ntile; j++) {
        const _Float16* sk = lds[j & 1];
        const _Float16* sv = sk + TL::K_ELEMS;

        // S^T block kb: rows = keys kb*32 + 8(r/4) + 4hh + r%4, column = l32.
        f32x16 s[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
#pragma unroll
            for (int r = 0; r < 16; r++) s[kb][r] = 0.0f;
            const _Float16* krow = sk + (kb * 32 + l32) * TL::KS + 8 * hh;
#pragma unroll
            for (int ks = 0; ks < NKS; ks++) {
                const h8 a = *reinterpret_cast<const h8*>(krow + 16 * ks);
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qt[ks], s[kb], 0, 0, 0);
            }
        }

        const int kbase = j * kKT;
        if (kbase + kKT - 1 > qmin_w) {   // causal mask, only near the diagonal
#pragma unroll
            for (int kb = 0; kb < NKB; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = kbase + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
                    if (key > qpos) s[kb][r] = -INFINITY;
                }
        }

        float mt = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) mt = fmaxf(mt, s[kb][r]);
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

        h8 pt[kKT / 16];
#pragma unroll
        for (int t = 0; t < kKT / 16; t++) {
            h8 v;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const float p = __builtin_amdgcn_exp2f(s[t >> 1][8 * (t & 1) + c] - m_run);
                l_run += p;
                v[c] = (_Float16)p;
            }
            pt[t] = v;
        }

        // O^T block b += V^T[32b + l32][keys of step t] * P^T[step t].  The
        // k index 8hh + c of step t = (kb, tt) is key kb*32 + 16tt + 4hh + c
        // for c < 4 and kb*32 + 16tt + 8 + 4hh + (c - 4) for c >= 4: the
        // order in which the S^T accumulator holds them.
#pragma unroll
        for (int b = 0; b < NDB; b++) {
            const _Float16* vrow = sv + (32 * b + l32) * TL::VS + 4 * hh;
#pragma unroll
            for (int t = 0; t < kKT / 16; t++) {
                const h4 lo = *reinterpret_cast<const h4*>(vrow + 16 * t);
                const h4 hi = *reinterpret_cast<const h4*>(vrow + 16 * t + 8);
                const h8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pt[t], acc[b], 0, 0, 0);
            }
        }

        if (j + 1 < ntile) {
            pre.store(lds[(j + 1) & 1], tid);
            if (j + 2 < ntile) pre.load(src + (size_t)(j + 2) * CH, tid);
        }
        __syncthreads();
    }

    // ---- normalise and write: lane holds O^T[d][l32] for
    // d = 32b + 8(r/4) + 4hh + r%4.
    const float inv = 1.0f / sum_halves(l_run);
    if (valid) {
        float* orow = P.out + ((size_t)ti * P.H + h) * D;
#pragma unroll
        for (int b = 0; b < NDB; b++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const int d = 32 * b + 8 * r4 + 4 * hh;
                if (d < D)
                    *reinterpret_cast<float4*>(orow + d) =
                        make_float4(acc[b][4 * r4] * inv, acc[b][4 * r4 + 1] * inv,
                                    acc[b][4 * r4 + 2] * inv, acc[b][4 * r4 + 3] * inv);
            }
    }
}

// ---- launch ----------------------------------------------------------------

template <int D, int G, typename CT>
int launch_dg(const PrefillArgs& a, hipStream_t st) {
    using TL = Tile<D>;
    const long long rows = (long long)a.pos0 + a.n_tokens;
    const int T = (int)((rows + kKT - 1) / kKT);
    const int HK = a.n_kv_heads;
    void* tiles = nullptr;
    int rc = tiles_get((size_t)HK * T * TL::BYTES, &tiles);
    if (rc != PKH_OK) return rc;

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
    S.T = T;
    S.tiles = static_cast<_Float16*>(tiles);
    hipLaunchKernelGGL((prefill_stage<D, CT>), dim3(T, HK), dim3(kThreads), 0, st, S);
    PKH_HIP(hipGetLastError());

    constexpr int BM = kCols / G;
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
    A.nqb = (a.n_tokens + BM - 1) / BM;
    A.qscale = (1.0f / sqrtf((float)D)) * 1.4426950408889634f;
    hipLaunchKernelGGL((prefill_attn<D, G>), dim3(A.nqb * HK), dim3(kThreads), 0, st, A);
    PKH_HIP(hipGetLastError());
    return PKH_OK;
}

template <int D, typename CT>
int launch_d(const PrefillArgs& a, hipStream_t st) {
    switch (a.n_heads / a.n_kv_heads) {
        case 1: return launch_dg<D, 1, CT>(a, st);
        case 2: return launch_dg<D, 2, CT>(a, st);
        case 4: return launch_dg<D, 4, CT>(a, st);
        case 8: return launch_dg<D, 8, CT>(a, st);
        default: return PKH_ERR_ARG;
    }
}

template <typename CT>
int launch_ct(const PrefillArgs& a, hipStream_t st) {
    switch (a.head_dim) {
        case 16: return launch_d<16, CT>(a, st);
        case 32: return launch_d<32, CT>(a, st);
        case 64: return launch_d<64, CT>(a, st);
        case 128: return launch_d<128, CT>(a, st);
        case 256: return launch_d<256, CT>(a, st);
        default: return PKH_ERR_ARG;
    }
}

}  // namespace

bool prefill_supported(int head_dim, int group, int dtype) {
    const bool d_ok = head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 ||
                      head_dim == 256;
    const bool g_ok = group == 1 || group == 2 || group == 4 || group == 8;
    return d_ok && g_ok && (dtype == PKH_KV_F32 || dtype == PKH_KV_F16);
}

int launch_prefill(const PrefillArgs& a, hipStream_t stream) {
    if (!prefill_supported(a.head_dim, a.n_heads / a.n_kv_heads, a.dtype)) return PKH_ERR_ARG;
    if (a.half != rope_half_of(a.head_dim) || a.n_tokens <= 0 || a.pos0 < 0) return PKH_ERR_ARG;
    if (a.dtype == PKH_KV_F32) return launch_ct<float>(a, stream);
    return launch_ct<_Float16>(a, stream);
}

}  // namespace pkh
