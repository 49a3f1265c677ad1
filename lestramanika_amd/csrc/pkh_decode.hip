// pkh_decode.hip -- split-K flash-decode for gfx950 (CDNA4).
//
// Replaces src/pickle_fast.c:1910-2094 (RoPE apply, KV append, attention of
// one new token over rows [0, pos]) and its multi-sequence generalisation.
//
// Work decomposition.  A work item is (sequence, chunk of `chunk` context
// rows, head slot y); in a ragged batch the items of a (sequence, slot)
// instead take its row tiles round-robin.  One workgroup of WAVES wave64s
// takes one item, so every K/V row it streams from HBM is read once and used
// for all query heads of its slot (the reference re-reads it once per query
// head, one OpenMP thread per head).
//
// Head slots.  Query head h reads KV head h*HK/H (src/pickle_fast.c:1963), so
// KV head g serves heads [ceil(g*H/HK), ceil((g+1)*H/HK)): H/HK of them when
// HK divides H, otherwise floor or ceil of H/HK, and none for some KV heads
// when H < HK.  Slot y = g*nsub + sub takes up to G of those heads, starting
// at the sub-th block of G; nsub = 1 except for groups larger than G (more
// than 8 heads, or 4 at head_dim 256), whose slots each re-read the KV head.
// Heads past the group's end are computed with a zero query and never
// written.  The slot with sub == 0 appends the new row even when its KV head
// serves no query head, as the reference appends every KV head.
//
// Head dimensions.  Rows are processed at a padded width D in {16, 32, 64,
// 128, 256}; with PAD the real width Dr < D: lanes whose 16-byte load starts
// at or past Dr load nothing (an out-of-range buffer offset returns zero
// without a memory access), key elements past Dr are masked to zero, query
// elements past Dr are zero, and outputs past Dr are not written.
//
// Register tiling.  A row of D elements is spread over LPP = D/F lanes, F
// elements per lane, loaded with 16-byte global loads (fp32: 4 elements,
// fp16: 8) at stride EPL*LPP, so a wave reads PPW = 64/LPP whole rows per
// tile with fully coalesced 128-bit accesses.  Scores are lane-partial dot
// products reduced over the LPP lanes of a row with DPP (quad_perm,
// row_half_mirror, row_mirror).  There is no LDS staging of K/V: each tile is
// consumed by the wave that loaded it, straight from VGPRs, while the next
// tile's loads are in flight.
//
// Softmax.  Queries are pre-scaled by log2(e)/sqrt(D), so scores are in log2
// units and exponentials are v_exp_f32.  Each row group keeps its own running
// max m, running sum l and accumulator; m is raised only when a score exceeds
// it by more than kTau (a wave-uniform branch that is rarely taken after the
// first tile), so exp2(s - m) <= 2^kTau and the rescale of the accumulator is
// skipped on almost every tile.  At the end every row group of every wave
// hands its (m, l, o) to LDS, where they are merged per output element, and
// the workgroup's (m, l, o) is either normalised into the output
// (single-chunk sequences) or written as a split-K partial; the last chunk
// of each (sequence, KV head) waits for the others' partial-ready flags and
// merges them in the same launch.
//
// RoPE and append.  Every workgroup rotates its own G query heads from the
// host-computed table row `pos` (the same sin/cos bits as the reference's
// state tables, src/pickle_fast.c:1772-1788).  The workgroup whose chunk
// contains `pos` rotates the new key for its KV head, stores (k_rot, v) into
// cache row pos and uses those registers for that row, so no workgroup reads
// a row another one writes.  The rotation uses the same fused multiply-adds
// as the reference's build of src/pickle_fast.c:1922-1933.

#include "pkh_internal.h"

#include <cmath>
#include <cstdio>

namespace pkh {
namespace {

constexpr float kTau = 8.0f;   // lazy-rescale threshold (log2 units)
constexpr int kCoherent = 16;  // buffer cache policy: sc1, device-coherent access
constexpr int kMaxFlagPolls = 1 << 16;   // default bound on the merger's wait (never reached)
constexpr int kStream = 3;     // buffer cache policy: sc0 | nt, read-once KV stream

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

template <typename KT> struct Elt;
template <> struct Elt<float>    { static constexpr int EPL = 4; };
template <> struct Elt<_Float16> { static constexpr int EPL = 8; };

template <int D, int G, typename KT>
struct Shape {
    static constexpr int EPL = Elt<KT>::EPL;       // elements per 16-byte load
    static constexpr int F   = D >= 256 ? 16 : 8;  // elements per lane per row
    static constexpr int LPP = D / F;              // lanes per row
    static constexpr int PPW = 64 / LPP;           // rows per wave tile
    static constexpr int NLD = F / EPL;            // loads per lane per row
    static constexpr int S   = EPL * LPP;          // element stride between a lane's loads
    // Tiles in flight per wave, enough bytes outstanding to cover HBM
    // latency; MINW is the waves per SIMD the register budget is sized for
    // (the largest query groups hold 2*G*F accumulator and query registers
    // and run one wave per SIMD).
    static constexpr int DEPTH = 4;
    static constexpr int MINW = (G >= 8 || (G >= 4 && D >= 256)) ? 1 : 2;
    static_assert(D % F == 0 && LPP >= 1 && LPP <= 16, "row split");
    static_assert(F % EPL == 0, "whole loads per lane");
};

// ---- cross-lane helpers -----------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over the LPP lanes of a row group (aligned, LPP <= 16); every lane of
// the group receives the sum.
template <int LPP>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (LPP >= 2)  x += dpp<0xB1>(x);    // quad_perm [1,0,3,2]
    if constexpr (LPP >= 4)  x += dpp<0x4E>(x);    // quad_perm [2,3,0,1]
    if constexpr (LPP >= 8)  x += dpp<0x141>(x);   // row_half_mirror
    if constexpr (LPP >= 16) x += dpp<0x140>(x);   // row_mirror
    return x;
}

// ---- element access ---------------------------------------------------

template <typename KT, int NLD>
__device__ __forceinline__ void unpack(const uint4 (&r)[NLD], float (&f)[NLD * Elt<KT>::EPL]) {
    if constexpr (sizeof(KT) == 4) {
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            f[4 * i + 0] = __uint_as_float(r[i].x);
            f[4 * i + 1] = __uint_as_float(r[i].y);
            f[4 * i + 2] = __uint_as_float(r[i].z);
            f[4 * i + 3] = __uint_as_float(r[i].w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            half8_t h = __builtin_bit_cast(half8_t, r[i]);
#pragma unroll
            for (int c = 0; c < 8; c++) f[8 * i + c] = (float)h[c];
        }
    }
}

template <typename KT, int NLD, int EPL, int S>
__device__ __forceinline__ void load_row(uint4 (&r)[NLD], const KT* row, int j) {
#pragma unroll
    for (int i = 0; i < NLD; i++)
        r[i] = *reinterpret_cast<const uint4*>(row + EPL * j + S * i);
}

// Rotate the EPL consecutive elements starting at element b of one head
// vector x (fp32, global) by table row (sn, cs); half = rotation half-width.
// Element i < half becomes fma(c, x[i], -(s*x[i+half])) and element i + half
// becomes fma(s, x[i], c*x[i+half]): the evaluation of
// src/pickle_fast.c:1922-1933 in the reference's default FMA build, so the
// rotated values match it bit for bit.  A block never straddles `half` (both
// are multiples of 4), so the branch-free selects below act per block; all
// loads are 16-byte vectors.
template <int EPL>
__device__ __forceinline__ void rope_block(float (&out)[EPL], const float* x, int b, int half,
                                           const float* sn, const float* cs) {
    const bool lo = b < half;
    const bool hi = !lo && b < 2 * half;
    const int pb = lo ? b + half : b - half;              // partner block
    const int tb = lo ? b : (hi ? b - half : 0);          // table block
#pragma unroll
    for (int c4 = 0; c4 < EPL; c4 += 4) {
        const float4 xv = *reinterpret_cast<const float4*>(x + b + c4);
        const float4 pv = *reinterpret_cast<const float4*>(x + pb + c4);
        const float4 sv = *reinterpret_cast<const float4*>(sn + tb + c4);
        const float4 cv = *reinterpret_cast<const float4*>(cs + tb + c4);
        const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
        const float pa[4] = {pv.x, pv.y, pv.z, pv.w};
        const float sa[4] = {sv.x, sv.y, sv.z, sv.w};
        const float ca[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float r_lo = __builtin_fmaf(ca[c], xa[c], -__fmul_rn(sa[c], pa[c]));
            const float r_hi = __builtin_fmaf(sa[c], pa[c], __fmul_rn(ca[c], xa[c]));
            out[c4 + c] = lo ? r_lo : (hi ? r_hi : xa[c]);
        }
    }
}

// One element d of a head vector x rotated by table row (sn, cs), for rows
// whose width or rotation half is not a multiple of 4: the same two fused
// multiply-adds as rope_block, with scalar loads.
__device__ __forceinline__ float rope_elem(const float* x, int d, int half, const float* sn,
                                           const float* cs) {
    if (d < half) return __builtin_fmaf(cs[d], x[d], -__fmul_rn(sn[d], x[d + half]));
    if (d < 2 * half) return __builtin_fmaf(sn[d - half], x[d - half], __fmul_rn(cs[d - half], x[d]));
    return x[d];
}

// Round the fp32 result into the cache type.  For fp16 the empty asm keeps
// the conversion from being folded into the fused multiply-add that made x
// (a single rounding straight to fp16); the reference rounds to fp32 first.
template <typename KT>
__device__ __forceinline__ KT to_kt(float x) {
    if constexpr (sizeof(KT) == 2) __asm__ volatile("" : "+v"(x));
    return (KT)x;
}

// ---- split kernel -------------------------------------------------------

struct SplitParams {
    const void* k_layer;
    const void* v_layer;
    const float* q;
    const float* k_new;
    const float* v_new;
    float* out;
    float* part_o;            // [total_chunks][H][D]
    float* part_ml;           // [total_chunks][H][2]
    int* counters;            // [HK][total chunks] partial-ready flags; zero between launches
    int max_polls;            // bound on the merger's flag wait, in polling rounds
    const float* rope_sin;
    const float* rope_cos;
    const long long* seq_slot0;
    const int* seq_pos;
    const int* chunk_start;
    long long slot0;
    long long stride_pos;
    long long stride_head;
    int pos;
    int n_seqs;
    int H, HK, half, chunk;
    int Dr;                   // real head_dim (<= the kernel's padded width)
    int nsub;                 // head slots per KV head
    float qscale;
};

template <int D, int G, typename KT, int WAVES, bool RAGGED, bool PAD>
__global__ __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu(Shape<D, G, KT>::MINW))) void decode_split(SplitParams P) {
    using SH = Shape<D, G, KT>;
    constexpr int EPL = SH::EPL, F = SH::F, LPP = SH::LPP, PPW = SH::PPW,
                  NLD = SH::NLD, S = SH::S, DEPTH = SH::DEPTH;

    // Every row group of every wave hands its (m, l, o) to LDS at the end.
    constexpr int NPART = WAVES * PPW;
    static_assert(NPART * G * D * 4 <= 65536, "row-group partials fit in 64 KB of LDS");
    __shared__ __attribute__((aligned(16))) float red_o[NPART][G][D];
    __shared__ __attribute__((aligned(16))) float q_lds[G][D];
    __shared__ float red_m[NPART][G];
    __shared__ float red_l[NPART][G];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane % LPP;        // slot of this lane inside its row group
    const int grp = lane / LPP;      // row of the tile handled by this lane
    const int H = P.H, HK = P.HK, half = P.half;
    const int Dr = PAD ? P.Dr : D;
    // One-dimensional grid, head slot fastest: on an 8-XCD part with 8 head
    // slots each XCD streams one KV head's chunks (workgroups go to XCDs
    // round-robin by index), and a head's merger is still its last item.
    const int ny = P.HK * P.nsub;                        // head slots
    const int y = (int)blockIdx.x % ny;                  // head slot
    const int bx = (int)blockIdx.x / ny;                 // chunk index in the grid
    const int nbx = (int)gridDim.x / ny;                 // chunks in the grid
    const int g = y / P.nsub;        // its KV head
    const int sub = y - g * P.nsub;
    const int head0 = (g * H + HK - 1) / HK + sub * G;               // first query head
    const int gc = min(G, (g * H + H + HK - 1) / HK - head0);        // heads of the slot

    int seq, c, pos, n_chunks, gchunk;
    long long slot0;
    if constexpr (RAGGED) {
        gchunk = bx;
        int lo = 0, hi = P.n_seqs;   // largest s with chunk_start[s] <= gchunk
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (P.chunk_start[mid] <= gchunk) lo = mid; else hi = mid;
        }
        seq = lo;
        c = gchunk - P.chunk_start[seq];
        pos = P.seq_pos[seq];
        slot0 = P.seq_slot0[seq];
        // The plan gives each sequence work-item slots for its whole capacity
        // (so a graph replays with positions that advance); this step uses
        // the first ceil((pos + 1) / chunk) of them and the rest exit.  A
        // position outside the sequence's capacity (one the host could not
        // check, in a replayed graph) yields NaN and writes no cache row.
        const long long cap = P.seq_slot0[seq + 1] - slot0;
        if (pos < 0 || pos >= cap) {
            if (c == 0 && gc > 0)
                for (int i = threadIdx.x; i < gc * Dr; i += 64 * WAVES)
                    P.out[((size_t)seq * H + head0 + i / Dr) * Dr + i % Dr] = __builtin_nanf("");
            return;
        }
        n_chunks = min(P.chunk_start[seq + 1] - P.chunk_start[seq], (pos + P.chunk) / P.chunk);
        if (c >= n_chunks) return;
    } else {
        seq = 0;
        c = bx;
        gchunk = c;
        n_chunks = nbx;
        pos = P.pos;
        slot0 = P.slot0;
    }
    const int attend_n = pos + 1;
    // Which rows a wave streams.  In the loop below a wave's m-th tile of
    // PPW rows is numbered t = w + m*WAVES (w = this wave).
    //  - Single sequence: work item c owns the contiguous chunk
    //    [c*chunk, min((c+1)*chunk, attend_n)); its waves take the chunk's
    //    tiles in turn.
    //  - Ragged batch: the items of a (sequence, KV head) take its tiles
    //    round-robin, one wave at a time (wave w of item c reads tiles
    //    c*WAVES + w + m*n_chunks*WAVES), so the waves of a head sweep one
    //    compact window of rows.  Measured on 16 sequences of 4K-32K rows:
    //    180.8 against 184.6 us; on one 8K-row sequence it is slower (16.6
    //    against 15.9 us), so the single-sequence path keeps chunks.
    constexpr bool kSweep = RAGGED;
    const int p_begin = kSweep ? 0 : c * P.chunk;
    const int p_end = kSweep ? attend_n : min(p_begin + P.chunk, attend_n);
    const int n_tiles_all = (p_end - p_begin + PPW - 1) / PPW;
    const int gw = c * WAVES + wave;                     // round-robin: this wave's first tile
    const int nwh = n_chunks * WAVES;                    // round-robin: waves per (sequence, head)
    const int t_end = kSweep ? wave + (gw < n_tiles_all ? (n_tiles_all - gw + nwh - 1) / nwh : 0) * WAVES
                             : n_tiles_all;
    auto tile_row = [&](int t) {
        return kSweep ? (gw + (t - wave) * n_chunks) * PPW + grp : p_begin + t * PPW + grp;
    };

    // Buffer resources over rows [0, p_end) of this sequence's KV head g:
    // loads past p_end return zeros, so partial tiles need no predicate.
    const unsigned row_bytes = (unsigned)(P.stride_pos * (long long)sizeof(KT));
    const size_t head_off = (size_t)g * P.stride_head + (size_t)slot0 * P.stride_pos;
    KT* kbase = const_cast<KT*>(reinterpret_cast<const KT*>(P.k_layer)) + head_off;
    KT* vbase = const_cast<KT*>(reinterpret_cast<const KT*>(P.v_layer)) + head_off;
    const int extent = (int)((unsigned)p_end * row_bytes);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(kbase, (short)0, extent, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(vbase, (short)0, extent, 0x00020000);
    const float* sn = P.rope_sin + (size_t)pos * half;
    const float* cs = P.rope_cos + (size_t)pos * half;

    float qr[G][F];           // rotated, pre-scaled queries (filled below)
    float m[G], l[G], acc[G][F];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < F; e++) acc[h][e] = 0.0f;
    }

    // Online-softmax update with one row per lane group.
    auto consume = [&](const float (&kf)[F], const float (&vf)[F], bool valid) {
        float s[G];
#pragma unroll
        for (int h = 0; h < G; h++) {
            float d0 = 0.0f;
#pragma unroll
            for (int e = 0; e < F; e++) d0 = fmaf(qr[h][e], kf[e], d0);
            s[h] = group_sum<LPP>(d0);
            if (!valid) s[h] = -INFINITY;
        }
        bool need = false;
#pragma unroll
        for (int h = 0; h < G; h++) need |= s[h] > m[h] + kTau;
        if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
            for (int h = 0; h < G; h++) {
                const bool nh = s[h] > m[h] + kTau;
                const float mn = nh ? s[h] : m[h];
                const float alpha = nh ? __builtin_amdgcn_exp2f(m[h] - mn) : 1.0f;
                l[h] *= alpha;
#pragma unroll
                for (int e = 0; e < F; e++) acc[h][e] *= alpha;
                m[h] = mn;
            }
        }
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float pr = valid ? __builtin_amdgcn_exp2f(s[h] - m[h]) : 0.0f;
            l[h] += pr;
#pragma unroll
            for (int e = 0; e < F; e++) acc[h][e] = fmaf(pr, vf[e], acc[h][e]);
        }
    };

    const unsigned lane_off = (unsigned)(EPL * j * sizeof(KT));
    // With PAD, a load that starts at or past Dr gets an offset beyond every
    // buffer extent (< 2 GiB): it returns zeros and touches no memory.
    unsigned skip[NLD];
#pragma unroll
    for (int i = 0; i < NLD; i++) skip[i] = (PAD && EPL * j + S * i >= Dr) ? 0x80000000u : 0u;
    auto issue = [&](int t, uint4 (&kr)[NLD], uint4 (&vr)[NLD]) {
        const unsigned off = (unsigned)tile_row(t) * row_bytes + lane_off;
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            kr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                        krs, (off + (unsigned)(S * i * sizeof(KT))) | skip[i], 0, kStream));
            vr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                        vrs, (off + (unsigned)(S * i * sizeof(KT))) | skip[i], 0, kStream));
        }
    };
    auto use = [&](int t, const uint4 (&kr)[NLD], const uint4 (&vr)[NLD]) {
        const int p = tile_row(t);
        float kf[F], vf[F];
        unpack<KT, NLD>(kr, kf);
        unpack<KT, NLD>(vr, vf);
        if constexpr (PAD) {
            // Key elements past Dr (a partly valid load) are masked: the
            // zero query there must not meet a non-finite neighbour.
#pragma unroll
            for (int e = 0; e < F; e++)
                if (EPL * j + S * (e / EPL) + e % EPL >= Dr) kf[e] = 0.0f;
        }
        consume(kf, vf, p < p_end && p != pos);
    };

    // The new row: rotate k for KV head g, round to the cache type, store
    // (k_rot, v) into row pos (slot sub 0 only), and, with `fold`, fold it
    // into the owning lane group.
    auto new_row = [&](int r, bool fold) {   // r: row pos relative to the first row of the mapping
        const bool mine = grp == r % PPW;
        const bool store = mine && sub == 0;
        float kf[F], vf[F];
        const float* kh = P.k_new + ((size_t)seq * HK + g) * Dr;
        const float* vh = P.v_new + ((size_t)seq * HK + g) * Dr;
        KT* kdst = kbase + (size_t)pos * P.stride_pos;
        KT* vdst = vbase + (size_t)pos * P.stride_pos;
#pragma unroll
        for (int i = 0; i < NLD; i++) {
            const int b = EPL * j + S * i;
            float blk[EPL];
            if constexpr (PAD) {
#pragma unroll
                for (int e = 0; e < EPL; e++) blk[e] = b + e < Dr ? rope_elem(kh, b + e, half, sn, cs) : 0.0f;
            } else {
                rope_block<EPL>(blk, kh, b, half, sn, cs);
            }
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                const bool live = !PAD || b + e < Dr;
                const KT kq = to_kt<KT>(blk[e]);
                const KT vq = to_kt<KT>(live ? vh[b + e] : 0.0f);
                if (store && live) {
                    kdst[b + e] = kq;
                    vdst[b + e] = vq;
                }
                kf[EPL * i + e] = (float)kq;
                vf[EPL * i + e] = (float)vq;
            }
        }
        if (fold) consume(kf, vf, mine);
    };
    // The wave whose tiles hold row pos.
    bool owns_new;
    if constexpr (kSweep) {
        const int gwp = (pos / PPW) % nwh;
        owns_new = c == gwp / WAVES && wave == gwp % WAVES;
    } else {
        owns_new = pos >= p_begin && pos < p_end && wave == ((pos - p_begin) / PPW) % WAVES;
    }
    // A slot with no query heads only appends the new row (sub 0 does).
    if (gc <= 0) {
        if (owns_new && sub == 0) new_row(kSweep ? pos : pos - p_begin, false);
        return;
    }

    // Main loop over this wave's tiles t = wave, wave + WAVES, ...: a ring
    // of DEPTH tiles is in flight; each consumed slot is refilled with the
    // tile DEPTH steps ahead.  The first DEPTH tiles are issued before the
    // queries are loaded, so their latency overlaps the query prologue.
    // Query prologue.  The workgroup rotates its G query heads once: each
    // thread loads a few elements with their RoPE partners and table entries
    // (issued ahead of the KV ring, so waiting for them does not wait for
    // the ring: loads retire in order), the rotated, pre-scaled rows go to
    // LDS, and every lane then reads its slice from there.
    constexpr int QE = (G * D + 64 * WAVES - 1) / (64 * WAVES);   // elements per thread
    float qx[QE], qp[QE], qs[QE], qc[QE];
#pragma unroll
    for (int u = 0; u < QE; u++) {
        const int idx = min((int)threadIdx.x + u * 64 * WAVES, G * D - 1);
        const int h = idx / D, d = idx % D;
        const bool lo = d < half;
        const bool hi = !lo && d < 2 * half;
        const bool live = h < gc && d < Dr;
        const float* qh = P.q + ((size_t)seq * H + head0 + min(h, gc - 1)) * Dr;
        qx[u] = live ? qh[d] : 0.0f;
        qp[u] = live ? qh[lo ? d + half : (hi ? d - half : d)] : 0.0f;
        const int ti = lo ? d : (hi ? d - half : 0);
        qs[u] = sn[ti];
        qc[u] = cs[ti];
    }
    __builtin_amdgcn_sched_barrier(0);

    uint4 kb[DEPTH][NLD], vb[DEPTH][NLD];
#pragma unroll
    for (int i = 0; i < DEPTH; i++) {
        issue(wave + i * WAVES, kb[i], vb[i]);
        __builtin_amdgcn_sched_barrier(0);   // keep the slots in issue order
    }

    // Same arithmetic as rope_block: fma(c, x, -(s*x_partner)) below half,
    // fma(s, x_partner, c*x) in the upper half, identity past 2*half.
#pragma unroll
    for (int u = 0; u < QE; u++) {
        const int idx = (int)threadIdx.x + u * 64 * WAVES;
        if (idx < G * D) {
            const int d = idx % D;
            const bool lo = d < half;
            const bool hi = !lo && d < 2 * half;
            const float r_lo = __builtin_fmaf(qc[u], qx[u], -__fmul_rn(qs[u], qp[u]));
            const float r_hi = __builtin_fmaf(qs[u], qp[u], __fmul_rn(qc[u], qx[u]));
            q_lds[idx / D][d] = (lo ? r_lo : (hi ? r_hi : qx[u])) * P.qscale;
        }
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int i = 0; i < NLD; i++)
#pragma unroll
            for (int c4 = 0; c4 < EPL; c4 += 4) {
                const float4 t4 = *reinterpret_cast<const float4*>(&q_lds[h][EPL * j + S * i + c4]);
                qr[h][EPL * i + c4 + 0] = t4.x;
                qr[h][EPL * i + c4 + 1] = t4.y;
                qr[h][EPL * i + c4 + 2] = t4.z;
                qr[h][EPL * i + c4 + 3] = t4.w;
            }

    // Loads are unconditional: tiles past the chunk read rows >= p_end,
    // which the buffer resource returns as zeros without touching memory,
    // so the loop has no divergent control flow around its loads and the
    // waits before each use cover only that slot's loads.
    for (int base = wave; base < t_end; base += DEPTH * WAVES) {
#pragma unroll
        for (int i = 0; i < DEPTH; i++) {
            const int t = base + i * WAVES;
            use(t, kb[i], vb[i]);   // rows past the chunk are masked
            issue(t + DEPTH * WAVES, kb[i], vb[i]);
        }
    }

    // Fold the new row into the owning lane group (and append it).
    if constexpr (kSweep) {
        if (owns_new) new_row(pos, true);
    } else if (owns_new) {
        new_row(pos - p_begin, true);
    }

    // Hand each row group's (m, l, o) to LDS: every lane writes its slice of
    // the group's o, the group's first lane m and l.  Merging here, not with
    // cross-lane reductions in registers, costs a few LDS reads per partial
    // instead of three permute steps for each of the G * (F + 2) values a
    // lane holds.
    const int part = wave * PPW + grp;
#pragma unroll
    for (int h = 0; h < G; h++) {
#pragma unroll
        for (int i = 0; i < NLD; i++)
#pragma unroll
            for (int e = 0; e < EPL; e += 4)
                *reinterpret_cast<float4*>(&red_o[part][h][EPL * j + S * i + e]) =
                    make_float4(acc[h][EPL * i + e], acc[h][EPL * i + e + 1], acc[h][EPL * i + e + 2],
                                acc[h][EPL * i + e + 3]);
        if (j == 0) { red_m[part][h] = m[h]; red_l[part][h] = l[h]; }
    }

    __syncthreads();

    // Merge the row groups.  First the per-head max and each partial's
    // weight exp2(m - max), once per (partial, head) rather than once per
    // output; then every output is a weighted sum over the partials.  A
    // sequence that fits one chunk is finished here; otherwise the work
    // item's (max, sum, o) goes to the partial buffer.
    __shared__ float red_f[NPART][G];
    __shared__ float red_M[G];
    for (int t = threadIdx.x; t < NPART * G; t += 64 * WAVES) {
        const int q = t / G, h = t % G;
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < NPART; k++) M = fmaxf(M, red_m[k][h]);
        const float mq = red_m[q][h];
        red_f[q][h] = (mq == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mq - M);
        if (q == 0) red_M[h] = M;
    }
    __syncthreads();
    // Each thread finishes CW consecutive d of one head (CW = 2 where that
    // spreads the G*D outputs over every thread, else 4): one CW*4-byte LDS
    // read per partial, and its head's sum once.  Measured against one
    // scalar output per thread at a stride of 64*WAVES: 16.0 against 16.25
    // us (Llama-3-8B, 8K context), 10.25 against 11.44 us (TinyLlama, 2K);
    // 185.0 against 183.1 us on the 16-sequence ragged fp16 workload.
    constexpr int CW = G * D / 2 <= 64 * WAVES ? 2 : 4;
    constexpr int NCOL = G * D / CW;
    static_assert(NCOL <= 64 * WAVES, "one column per thread");
    const bool has_col = (int)threadIdx.x < NCOL;
    const int ocol = has_col ? (int)threadIdx.x : NCOL - 1;
    const int oh = (CW * ocol) / D, od = (CW * ocol) % D;
    float Ol = 0.0f, Om = 0.0f;
    typedef float fcw_t __attribute__((ext_vector_type(CW)));
    fcw_t Oo = {};
    if (has_col) {   // whole waves past the last column skip it
#pragma unroll
        for (int q = 0; q < NPART; q++) {
            const float f = red_f[q][oh];
            Ol = fmaf(red_l[q][oh], f, Ol);
            const fcw_t x = *reinterpret_cast<const fcw_t*>(&red_o[q][oh][od]);
#pragma unroll
            for (int e = 0; e < CW; e++) Oo[e] = fmaf(x[e], f, Oo[e]);
        }
        Om = red_M[oh];
    }
    if (n_chunks == 1) {
        if (has_col && oh < gc) {
            fcw_t r;
#pragma unroll
            for (int e = 0; e < CW; e++) r[e] = Oo[e] / Ol;
            float* orow = P.out + ((size_t)seq * H + head0 + oh) * Dr;
            if constexpr (PAD) {
#pragma unroll
                for (int e = 0; e < CW; e++)
                    if (od + e < Dr) orow[od + e] = r[e];
            } else {
                *reinterpret_cast<fcw_t*>(orow + od) = r;
            }
        }
        return;
    }
    // Split-K combine, fused.  The last chunk of each (sequence, KV head)
    // merges; the others hand over their partial (max, sum, o).  Partials and
    // flags are written with device-scope atomic stores and read with
    // device-scope atomic loads or loads of the same (sc1) policy, which go
    // through the per-XCD L2 to the device-coherent level, so the merger
    // sees them without a cache writeback or invalidate.  A writer
    // waits for its partial stores to complete and then sets its own flag;
    // the merger, dispatched after every other chunk of its head (workgroups
    // are dispatched in index order, and those chunks wait on nothing), polls
    // the flags, merges, and clears them for the next launch.  One flag per
    // work item replaces a shared ticket counter, whose atomics serialize
    // when all chunks of a head finish together.
    const bool merger = c == n_chunks - 1;
    int* const flags = P.counters + (size_t)y * nbx;
    __shared__ float own_o[G * D];
    __shared__ float own_m[G], own_l[G];
    if (!merger) {
        if (has_col) {
            // 8-byte device-scope atomic stores: (o[d], o[d + 1]) pairs and (m, l).
            // Partials are [chunk][slot][G][D].
            const size_t base = ((size_t)gchunk * ny + y) * G + oh;
            unsigned long long* po = reinterpret_cast<unsigned long long*>(P.part_o + base * D + od);
#pragma unroll
            for (int e = 0; e < CW; e += 2)
                __hip_atomic_store(po + e / 2, __builtin_bit_cast(unsigned long long, make_float2(Oo[e], Oo[e + 1])),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (od == 0)
                __hip_atomic_store(reinterpret_cast<unsigned long long*>(P.part_ml + base * 2),
                                   __builtin_bit_cast(unsigned long long, make_float2(Om, Ol)),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(flags + bx, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // The merger keeps its own partial in LDS.
    if (has_col) {
        *reinterpret_cast<fcw_t*>(&own_o[CW * ocol]) = Oo;
        if (od == 0) { own_m[oh] = Om; own_l[oh] = Ol; }
    }
    // Wait for the other chunks' flags: one batch of flag loads per round.
    // The bound only guarantees that the loop ends (every writer above sets
    // its flag unconditionally); should it ever run out, the head's output
    // is NaN rather than a merge of whatever partials had arrived.  Writers
    // add 1 to their flag and the merger subtracts 1 from every flag it
    // waited on, whether or not the wait ran out: a writer that lands after
    // a timed-out wait brings its flag back to 0, so the next launch (which
    // starts after every workgroup of this one has ended) finds all flags
    // at 0 and never takes a stale flag for its own partial.
    const int cfirst = bx - c;     // this head's first chunk
    bool timed_out = true;
    for (int round = 0; round < P.max_polls; round++) {
        int missing = 0;
        for (int k = threadIdx.x; k < n_chunks - 1; k += 64 * WAVES)
            missing |= __hip_atomic_load(flags + cfirst + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0;
        if (!__syncthreads_or(missing)) {
            timed_out = false;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    const int n_parts = n_chunks - 1;           // partials in memory
    // Final merge: the G*D outputs as float4 columns, the other chunks'
    // partials spread over CGN thread groups; the groups' online
    // (max, sum, o) and the merger's own partial are then merged through LDS.
    constexpr int NV = G * D / 4;                       // float4 columns
    constexpr int CGN = NV >= 64 * WAVES ? 1 : 64 * WAVES / NV;
    constexpr int CPT = NV >= 64 * WAVES ? NV / (64 * WAVES) : 1;   // columns per thread
    static_assert(CPT * 64 * WAVES == NV || CGN * NV == 64 * WAVES, "combine split");
    __shared__ float4 fo[CGN][NV];
    __shared__ float fm[CGN][G], fl[CGN][G];
    const int c0 = RAGGED ? P.chunk_start[seq] : 0;
    const __amdgpu_buffer_rsrc_t pors =
        __builtin_amdgcn_make_buffer_rsrc(P.part_o, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t pmrs =
        __builtin_amdgcn_make_buffer_rsrc(P.part_ml, (short)0, 0x7fffffff, 0x00020000);
    const int cg = (int)threadIdx.x / (NV / CPT < 64 * WAVES ? NV / CPT : 64 * WAVES);
    const int col0 = ((int)threadIdx.x % (NV / CPT)) * CPT;
    // B partials per group and batch.  Each (m, l) pair of the batch is
    // loaded once, by one thread, ahead of the o blocks, and shared through
    // LDS; every thread then loads only its own partials' o blocks, all
    // before any is used, so a batch costs one memory round trip.  Slots
    // past the last chunk reload the last one and get weight 0.  Against a
    // pair load per thread and partial (half the merging CU's loads are
    // then redundant): 16.04 against 16.15 us (Llama-3-8B, 8K context),
    // 9.94 against 10.28 us (TinyLlama, 2K), 185.7 against 186.1 us (ragged).
    constexpr int B = 16;
    static_assert(CPT == 1, "one column per thread in the final merge");
    __shared__ float2 mlb[CGN * B][G];
    const int col = col0;
    const int h = (4 * col) / D;
    float M = -INFINITY, L = 0.0f;
    float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int b0 = 0; b0 < n_parts; b0 += CGN * B) {
        constexpr int NML = (CGN * B * G + 64 * WAVES - 1) / (64 * WAVES);   // pairs per thread
        float2 mlv[NML];
#pragma unroll
        for (int r = 0; r < NML; r++) {
            const int t = min((int)threadIdx.x + r * 64 * WAVES, CGN * B * G - 1);
            const int c = min(b0 + t / G, n_parts - 1);
            mlv[r] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                pmrs, (unsigned)((((size_t)(c0 + c) * ny + y) * G + t % G) * 2 * sizeof(float)), 0,
                kCoherent));
        }
        __builtin_amdgcn_sched_barrier(0);   // the pairs go out first: their wait leaves the o blocks in flight
        float4 oc[B];
#pragma unroll
        for (int i = 0; i < B; i++) {
            const int c = min(b0 + cg + i * CGN, n_parts - 1);
            const size_t base = ((size_t)(c0 + c) * ny + y) * G + h;
            // 16-byte loads with the device-coherent (sc1) policy.
            oc[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                pors, (unsigned)((base * D + (4 * col) % D) * sizeof(float)), 0, kCoherent));
        }
        // Return the flags to 0 for the next launch once the first batch's
        // loads are out: waits for those loads do not cover these younger
        // atomics.
        if (b0 == 0)
            for (int k = threadIdx.x; k < n_chunks - 1; k += 64 * WAVES)
                __hip_atomic_fetch_add(flags + cfirst + k, -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < NML; r++) {
            const int t = (int)threadIdx.x + r * 64 * WAVES;
            if (t < CGN * B * G) mlb[t / G][t % G] = mlv[r];
        }
        __syncthreads();
        float2 ml[B];
#pragma unroll
        for (int i = 0; i < B; i++) ml[i] = mlb[cg + i * CGN][h];
        float mb = M;
#pragma unroll
        for (int i = 0; i < B; i++)
            if (b0 + cg + i * CGN < n_parts) mb = fmaxf(mb, ml[i].x);
        const float a = (M == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(M - mb);
        L *= a;
        O.x *= a;
        O.y *= a;
        O.z *= a;
        O.w *= a;
#pragma unroll
        for (int i = 0; i < B; i++) {
            const float w = b0 + cg + i * CGN < n_parts ? __builtin_amdgcn_exp2f(ml[i].x - mb) : 0.0f;
            L = fmaf(ml[i].y, w, L);
            O.x = fmaf(oc[i].x, w, O.x);
            O.y = fmaf(oc[i].y, w, O.y);
            O.z = fmaf(oc[i].z, w, O.z);
            O.w = fmaf(oc[i].w, w, O.w);
        }
        M = mb;
        __syncthreads();   // mlb is refilled by the next batch
    }
    fo[cg][col] = O;
    if ((4 * col) % D == 0) { fm[cg][h] = M; fl[cg][h] = L; }
    __syncthreads();
    for (int col = threadIdx.x; col < NV; col += 64 * WAVES) {
        const int h = (4 * col) / D;
        float M = own_m[h];
#pragma unroll
        for (int i = 0; i < CGN; i++) M = fmaxf(M, fm[i][h]);
        const float fo_own = (own_m[h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(own_m[h] - M);
        float L = own_l[h] * fo_own;
        const float4 oo = *reinterpret_cast<const float4*>(&own_o[4 * col]);
        float4 O = make_float4(oo.x * fo_own, oo.y * fo_own, oo.z * fo_own, oo.w * fo_own);
#pragma unroll
        for (int i = 0; i < CGN; i++) {
            const float f = (fm[i][h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(fm[i][h] - M);
            L = fmaf(fl[i][h], f, L);
            const float4 oi = fo[i][col];
            O.x = fmaf(oi.x, f, O.x);
            O.y = fmaf(oi.y, f, O.y);
            O.z = fmaf(oi.z, f, O.z);
            O.w = fmaf(oi.w, f, O.w);
        }
        const float inv = timed_out ? __builtin_nanf("") : 1.0f / L;
        if (h < gc) {
            float* orow = P.out + ((size_t)seq * H + head0 + h) * Dr;
            const int d = (4 * col) % D;
            const float4 r = make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
            if constexpr (PAD) {
                if (d + 0 < Dr) orow[d + 0] = r.x;
                if (d + 1 < Dr) orow[d + 1] = r.y;
                if (d + 2 < Dr) orow[d + 2] = r.z;
                if (d + 3 < Dr) orow[d + 3] = r.w;
            } else {
                *reinterpret_cast<float4*>(orow + d) = r;
            }
        }
    }
}

// ---- no-alloc scratch ------------------------------------------------------

__global__ void zero_words(int* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

}  // namespace

// Device scratch of pkh_attn_decode_noalloc_async: the first kNoAllocFlagBytes
// hold the partial-ready flags (zero between launches: cleared at set-up,
// and every launch returns the flags it used to zero), the rest the split-K
// partials.  Each device holds its own copy until the process ends.  In host
// code `scratch` names a host-side stand-in, not device memory: kernels and
// copies use the address hipGetSymbolAddress returns for the current device.
constexpr size_t kNoAllocFlagBytes = 64u << 10;
constexpr size_t kNoAllocBytes = 8u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {

constexpr int kNoAllocDevices = 16;
void* g_noalloc[kNoAllocDevices] = {};   // per device: the address of `scratch` there

}  // namespace

int noalloc_setup(int device, hipStream_t st) {
    if (device < 0 || device >= kNoAllocDevices) return PKH_ERR_ARG;
    if (g_noalloc[device]) return PKH_OK;
    void* p = nullptr;
    PKH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    // A fill kernel rather than a memset, so that a first call under stream
    // capture records nothing a replay could get wrong.
    hipLaunchKernelGGL(zero_words, dim3(16), dim3(256), 0, st, static_cast<int*>(p),
                       (int)(kNoAllocFlagBytes / sizeof(int)));
    PKH_HIP(hipGetLastError());
    g_noalloc[device] = p;
    return PKH_OK;
}

int noalloc_workspace(size_t part_bytes, size_t n_flags, hipStream_t st, void** part, int** flags) {
    int dev = 0;
    PKH_HIP(hipGetDevice(&dev));
    if (n_flags * sizeof(int) > kNoAllocFlagBytes || part_bytes > kNoAllocBytes - kNoAllocFlagBytes) {
        std::fprintf(stderr,
                     "pkh: pkh_attn_decode_noalloc_async needs %zu bytes of partials and %zu flags; "
                     "its fixed scratch holds %zu bytes and %zu flags\n",
                     part_bytes, n_flags, kNoAllocBytes - kNoAllocFlagBytes, kNoAllocFlagBytes / sizeof(int));
        return PKH_ERR_ARG;
    }
    int rc = noalloc_setup(dev, st);
    if (rc != PKH_OK) return rc;
    *flags = static_cast<int*>(g_noalloc[dev]);
    *part = static_cast<char*>(g_noalloc[dev]) + kNoAllocFlagBytes;
    return PKH_OK;
}

namespace {

// ---- dispatch -------------------------------------------------------------

constexpr int kWaves = 4;

template <int D, int G, typename KT>
int launch_typed(const DecodeArgs& a, const SplitParams& P, int total_chunks, int ny, hipStream_t st) {
    dim3 grid((unsigned)total_chunks * (unsigned)ny), block(64 * kWaves);
    const bool ragged = a.d_chunk_start != nullptr;
    const bool pad = P.Dr != D;
#define PKH_GO(R, PD) hipLaunchKernelGGL((decode_split<D, G, KT, kWaves, R, PD>), grid, block, 0, st, P)
    if (ragged) {
        if (pad) PKH_GO(true, true); else PKH_GO(true, false);
    } else {
        if (pad) PKH_GO(false, true); else PKH_GO(false, false);
    }
#undef PKH_GO
    PKH_HIP(hipGetLastError());
    return PKH_OK;
}

template <typename KT>
int launch_kt(const DecodeArgs& a, const SplitParams& P, int tc, int ny, int DP, int G, hipStream_t st) {
#define PKH_CASE(DD, GG) \
    if (DP == DD && G == GG) return launch_typed<DD, GG, KT>(a, P, tc, ny, st);
    PKH_CASE(16, 1) PKH_CASE(16, 2) PKH_CASE(16, 4) PKH_CASE(16, 8)
    PKH_CASE(32, 1) PKH_CASE(32, 2) PKH_CASE(32, 4) PKH_CASE(32, 8)
    PKH_CASE(64, 1) PKH_CASE(64, 2) PKH_CASE(64, 4) PKH_CASE(64, 8)
    PKH_CASE(128, 1) PKH_CASE(128, 2) PKH_CASE(128, 4) PKH_CASE(128, 8)
    PKH_CASE(256, 1) PKH_CASE(256, 2) PKH_CASE(256, 4)
#undef PKH_CASE
    return PKH_ERR_ARG;
}

// Largest head slot of the decode kernel at padded width DP: G = 8 holds
// 2*G*F query and accumulator registers per lane, too many at DP = 256.
int decode_gmax(int DP) { return DP >= 256 ? 4 : 8; }

}  // namespace

int padded_head_dim(int head_dim) {
    if (head_dim < 1 || head_dim > kMaxHeadDim) return 0;
    int dp = 16;
    while (dp < head_dim) dp *= 2;
    return dp;
}

HeadSlots head_slots(int n_heads, int n_kv_heads, int gmax) {
    // KV head g serves query heads [ceil(g*H/HK), ceil((g+1)*H/HK)): at most
    // ceil(H/HK) of them.
    const int maxg = (n_heads + n_kv_heads - 1) / n_kv_heads;
    int G = 1;
    while (G < maxg && G < gmax) G *= 2;
    return HeadSlots{G, (maxg + G - 1) / G};
}

bool shape_supported(int head_dim, int n_heads, int n_kv_heads) {
    if (n_heads <= 0 || n_kv_heads <= 0 || padded_head_dim(head_dim) == 0) return false;
    const int DP = padded_head_dim(head_dim);
    const long long ny = (long long)n_kv_heads * head_slots(n_heads, n_kv_heads, decode_gmax(DP)).nsub;
    return ny <= 65535;   // head slots, kept within one grid dimension
}

int decode_tile_positions(int head_dim, int dtype) {
    (void)dtype;
    const int DP = padded_head_dim(head_dim);
    const int F = DP >= 256 ? 16 : 8;
    const int lpp = DP / F;
    return (64 / lpp) * kWaves;
}

static int g_chunk_override = 0;
static int g_max_polls = kMaxFlagPolls;

int decode_chunk_for(int head_dim, int n_heads, int n_kv_heads, int dtype, long long total_rows,
                     int max_attend) {
    const int tile = decode_tile_positions(head_dim, dtype);
    const int DP = padded_head_dim(head_dim);
    // Workgroups per chunk of rows: one per head slot.
    const long long slots = (long long)n_kv_heads * head_slots(n_heads, n_kv_heads, decode_gmax(DP)).nsub;
    long long chunk;
    if (g_chunk_override > 0) {
        chunk = g_chunk_override;
    } else {
        // About 208 work items, at most one workgroup per CU (a CU that holds
        // two finishes last and sets the launch time): enough resident waves
        // to keep HBM busy (each wave keeps DEPTH tiles in flight) while each
        // (sequence, head slot) has few chunks to merge.  Measured on the
        // Llama-3-8B decode shape at 8K context: 208-216 items 16.7 us/layer,
        // 160 items 17.9, 248-256 items 17.4, 264-520 items 21-23.
        const long long target_items = 208;
        chunk = (total_rows * slots + target_items - 1) / target_items;
        if (chunk < 2LL * tile) chunk = 2LL * tile;
        // Large batches (many sequence x head pairs) finish their merges at
        // different times, hidden behind other items' streaming, so smaller
        // items balance better: measured on 16 sequences of 4K-32K rows,
        // 768-1536-row items stream at 72% of HBM peak against 58% for
        // 13K-row items.
        const long long max_chunk = 1024;
        if (chunk > max_chunk) chunk = max_chunk;
    }
    chunk = (chunk + tile - 1) / tile * tile;
    if (chunk > (long long)max_attend) chunk = ((long long)max_attend + tile - 1) / tile * tile;
    if (chunk < tile) chunk = tile;
    return (int)chunk;
}

int launch_decode(const DecodeArgs& a, hipStream_t st, bool no_alloc) {
    const int H = a.n_heads, HK = a.n_kv_heads;
    const int DP = padded_head_dim(a.head_dim);
    if (!shape_supported(a.head_dim, H, HK)) return PKH_ERR_ARG;
    const HeadSlots hs = head_slots(H, HK, decode_gmax(DP));
    const int ny = HK * hs.nsub;
    SplitParams P{};
    P.k_layer = a.k_layer;
    P.v_layer = a.v_layer;
    P.q = a.q;
    P.k_new = a.k_new;
    P.v_new = a.v_new;
    P.out = a.out;
    P.rope_sin = a.rope_sin;
    P.rope_cos = a.rope_cos;
    P.seq_slot0 = a.d_seq_slot0;
    P.seq_pos = a.d_seq_pos;
    P.chunk_start = a.d_chunk_start;
    P.slot0 = a.slot0;
    P.stride_pos = a.stride_pos;
    P.stride_head = a.stride_head;
    P.pos = a.pos;
    P.n_seqs = a.n_seqs;
    P.H = H;
    P.HK = HK;
    P.half = a.half;
    P.chunk = a.chunk;
    P.Dr = a.head_dim;
    P.nsub = hs.nsub;
    P.qscale = (1.0f / sqrtf((float)a.head_dim)) * 1.4426950408889634f;
    P.max_polls = g_max_polls;

    // Buffer-resource offsets are 32-bit: one sequence's rows of a layer
    // must stay below 2 GiB.
    const long long elem = a.dtype == PKH_KV_F16 ? 2 : 4;
    const long long max_rows = a.n_seqs == 1 && !a.d_chunk_start
                                   ? (long long)a.pos + 1
                                   : (long long)a.max_chunks * a.chunk;
    if ((max_rows + 1) * a.stride_pos * elem >= (1LL << 31)) return PKH_ERR_ARG;

    const int total_chunks = a.total_chunks;
    if ((long long)total_chunks * ny > 0x7fffffffLL) return PKH_ERR_ARG;   // one-dimensional grid
    if (a.max_chunks > 1) {
        // Scratch: [part_o][part_ml], partials indexed [chunk][slot][G][DP];
        // one partial-ready flag per work item (chunk, head slot) in the
        // zero-between-launches flag array.
        const size_t per_chunk = (size_t)ny * hs.G;
        const size_t n_o = (size_t)total_chunks * per_chunk * DP;
        const size_t n_ml = (size_t)total_chunks * per_chunk * 2;
        const size_t n_flags = (size_t)total_chunks * ny;
        void* ws = nullptr;
        int rc = no_alloc ? noalloc_workspace((n_o + n_ml) * sizeof(float), n_flags, st, &ws, &P.counters)
                          : scratch_get((n_o + n_ml) * sizeof(float), &ws);
        if (rc != PKH_OK) return rc;
        if (!no_alloc) {
            rc = counters_get(n_flags, &P.counters);
            if (rc != PKH_OK) return rc;
        }
        P.part_o = reinterpret_cast<float*>(ws);
        P.part_ml = P.part_o + n_o;
    }
    if (a.dtype == PKH_KV_F32) return launch_kt<float>(a, P, total_chunks, ny, DP, hs.G, st);
    if (a.dtype == PKH_KV_F16) return launch_kt<_Float16>(a, P, total_chunks, ny, DP, hs.G, st);
    return PKH_ERR_ARG;
}

}  // namespace pkh

extern "C" int pkh_tune_decode_chunk(int positions) {
    const int prev = pkh::g_chunk_override;
    pkh::g_chunk_override = positions > 0 ? positions : 0;
    return prev;
}

extern "C" int pkh_tune_decode_wait(int rounds) {
    const int prev = pkh::g_max_polls;
    pkh::g_max_polls = rounds >= 0 ? rounds : pkh::kMaxFlagPolls;
    return prev;
}
