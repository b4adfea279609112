// Paged GQA decode attention on gfx950: one query token, H query heads over Hkv KV
// heads (G = H / Hkv query heads share a KV head), bf16 K/V in pages of page_size
// tokens ([Hkv, page_size, D] each: one KV head's keys of a page are page_size x D
// contiguous, 4 KiB at 16 keys of 128 dims), token j in physical page
// page_table[j / page_size] at slot j % page_size.
//
//  * Block (b, g) takes keys [1024 b, 1024 b + 1024) of KV head g; each of its 4 waves 256
//    keys, as pairs of 16-key tiles (a tile is one MFMA tile, inside one page: one
//    contiguous 4 KiB run of K and one of V). K and V of a tile stream once for all G
//    query heads; the next pair's loads are in flight while the current one is reduced.
//    At 32 Ki keys and 8 KV heads that is 256 blocks, one a CU, and 32 partials a KV head
//    for the merge (measured against 64 keys a wave: 29.4 against 31.8 us a step; 128:
//    30.5; 512 keys a wave, or 8-wave blocks, or two and three pairs in flight: slower).
//  * Scores S^T = K . Q^T on bf16 MFMA (v_mfma_f32_16x16x32_bf16; products exact, fp32
//    accumulate): keys are the M side, so K loads need head_dim contiguous per lane
//    (the layout in memory) and each lane ends with 4 keys of one head, which keeps the
//    online-softmax reductions to two lane swaps. fp32 q enters as an exact 3-term bf16
//    split (hi + mid + lo).
//  * P . V on the same bf16 matrix cores, 32 keys (a pair) per MFMA: P enters as an exact
//    3-term bf16 split, so products are exact and accumulate in fp32; V rows load
//    coalesced (16 lanes x 8 head_dim columns a key) and reach the B-operand layout
//    through a per-wave transposed LDS area. (A VALU P . V made the kernel issue-bound:
//    about 650 vector instructions per 16-key tile.)
//  * A block merges its waves' (max, sum, acc) in LDS into one partial; a second kernel
//    merges a KV head's partials weighted by their maxima against the global one and
//    writes out = acc / sum (a KV head with one block writes its result directly).
// The arithmetic follows the reference's fp32 online softmax
// (crates/oominf-cuda/kernels/attention.cu:419-553): dot products, exp and accumulation
// in fp32; only the summation order differs.
#include <algorithm>

#include "common.hpp"

namespace oom {

constexpr int AW = 4;           // waves per block
constexpr int AKW = 256;        // keys per wave
constexpr int AKB = AW * AKW;   // keys per block
constexpr int AG = 8;           // query heads per KV head (at most)
constexpr int A_MAXB = 8192;    // blocks a KV head (8 Mi keys): the merge's weights sit in LDS
constexpr int A_BUF_FLAGS = 0x00020000;
constexpr int A_OOB = 0x7ffffff0;
constexpr int A_BUF_SC1 = 16;

typedef __bf16 abf16x8 __attribute__((ext_vector_type(8)));
typedef float af32x4 __attribute__((ext_vector_type(4)));

struct AttnArgs {
    const void* q;
    const uint16_t* kp;
    const uint16_t* vp;
    const int32_t* pt;
    int n_pages, page_size, kv_len, Hkv, G, bph;
    float scale;
    void* out;
    float* part;        // [Hkv][bph][2 AG + AG D]: each block's max and sum per head, then its acc [AG][D]
};

__device__ __forceinline__ uint4 a_ld16(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Buffer resource over one page, all its KV heads (empty if the page index is bad).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const uint16_t* base, int page, int n_pages,
                                                           int page_bytes) {
    const bool ok = page >= 0 && page < n_pages;
    const uint16_t* p = base + (size_t)(ok ? page : 0) * (page_bytes / 2);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p), (short)0, ok ? page_bytes : 0, A_BUF_FLAGS);
}

// Loads of one 16-key tile (inside one page), keys past kv_len and tiles whose page
// index is out of range reading zeros. Key slot s of KV head g sits at row g * page_size
// + s of the page (D * 2 bytes a row). K in the MFMA A layout of the scores: lane l holds
// key l % 16, head_dim 32 s + 8 (l / 16) .. + 8 (the four instructions of a tile cover its
// 4 KiB run). V: lane l holds head_dim 8 (l % 16) .. + 8 of key 4 q + l / 16 (q < 4): an
// instruction reads 1 KiB contiguous.
template <int D>
__device__ __forceinline__ void k_load(const AttnArgs& a, int g, int key0, int page, int lane, uint4 (&k)[D / 32]) {
    const int ps = a.page_size, page_bytes = ps * a.Hkv * D * 2, row_bytes = D * 2;
    if (key0 >= a.kv_len) page = -1;
    const __amdgpu_buffer_rsrc_t kr = page_rsrc(a.kp, page, a.n_pages, page_bytes);
    const int row0 = g * ps + key0 % ps;
    const int kbase = key0 + (lane & 15) < a.kv_len ? (row0 + (lane & 15)) * row_bytes + 16 * (lane >> 4) : A_OOB;
#pragma unroll
    for (int s = 0; s < D / 32; s++) k[s] = a_ld16(kr, kbase == A_OOB ? A_OOB : kbase + 64 * s);
}

template <int D>
__device__ __forceinline__ void v_load(const AttnArgs& a, int g, int key0, int page, int lane, uint4 (&v)[4]) {
    static_assert(D == 128, "V loads: 16 lanes of 8 head_dim columns a key");
    const int ps = a.page_size, page_bytes = ps * a.Hkv * D * 2, row_bytes = D * 2;
    if (key0 >= a.kv_len) page = -1;
    const __amdgpu_buffer_rsrc_t vr = page_rsrc(a.vp, page, a.n_pages, page_bytes);
    const int row0 = g * ps + key0 % ps;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int kk = 4 * q + (lane >> 4);
        v[q] = a_ld16(vr, key0 + kk < a.kv_len ? (row0 + kk) * row_bytes + (lane & 15) * 16 : A_OOB);
    }
}

// P . V of a 32-key pair of tiles runs on the bf16 matrix cores: O[head, dim] +=
// sum_kappa P[head, kappa] V[kappa, dim] (v_mfma_f32_16x16x32_bf16, heads on M, 16 dims
// on N, the pair's 32 keys on K). Lane l supplies K values 8 (l / 16) .. + 8, and both
// operands order a lane group's 8 keys the same way: position 2 e + t = key 4 (l / 16) + e
// of tile t. That is where the scores leave P (lane l: keys 4 (l / 16) + e of head l % 16),
// so the A operand is built in registers; V reaches that order through a per-wave LDS
// area, written transposed: word e of the 16-byte entry (group q, dim d) holds the bf16
// pair (tile 0, tile 1) of key 4 q + e, at word q VT_GROUP + 4 d + 4 (d / 8) + e. The pad
// of 4 words every 8 dims spreads a write instruction's 64 words (16 dims 8 apart x 4
// keys) over all 64 banks; a B-operand read (16 consecutive dims, 16 bytes each) takes
// 8 lanes' contiguous 128 bytes at a time.
constexpr int VT_GROUP = 128 * 4 + 16 * 4;  // words of one key group (4 keys of both tiles, 128 dims)
constexpr int VT_WORDS = 4 * VT_GROUP;      // one wave's area

__device__ __forceinline__ int vt_word(int q, int d, int e) { return q * VT_GROUP + 4 * d + 4 * (d >> 3) + e; }

// The pair's V (tile t's loads in v[t]) into the wave's transposed area.
__device__ __forceinline__ void v_to_lds(const uint4 (&v)[2][4], uint32_t* vt, int lane) {
    const int e = lane >> 4, dl = lane & 15;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t w0[4] = {v[0][q].x, v[0][q].y, v[0][q].z, v[0][q].w};
        const uint32_t w1[4] = {v[1][q].x, v[1][q].y, v[1][q].z, v[1][q].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int d = 8 * dl + 2 * i;  // word i: dims d (low half) and d + 1 (high half)
            vt[vt_word(q, d, e)] = __builtin_amdgcn_perm(w1[i], w0[i], 0x05040100u);
            vt[vt_word(q, d + 1, e)] = __builtin_amdgcn_perm(w1[i], w0[i], 0x07060302u);
        }
    }
}

// Scores of one 16-key tile for 16 (G real) heads, scaled and masked: lane l holds keys
// key0 + 4 (l / 16) + e of head l % 16.
template <int D, int NQ>
__device__ __forceinline__ void tile_scores(const AttnArgs& a, const uint4 (&k)[D / 32],
                                            const abf16x8 (&qb)[NQ][D / 32], int key0, int lane, float (&s)[4]) {
    af32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int term = 0; term < NQ; term++)
#pragma unroll
        for (int ss = 0; ss < D / 32; ss++)
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(abf16x8, k[ss]), qb[term][ss], c, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; e++) s[e] = key0 + 4 * (lane >> 4) + e < a.kv_len ? c[e] * a.scale : -INFINITY;
}

// max / sum over the four lane groups (the keys of one head)
__device__ __forceinline__ float group_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r2[0]), __uint_as_float(r2[1]));
}
__device__ __forceinline__ float group_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r2[0]) + __uint_as_float(r2[1]);
}

template <int D, int QDT, int ODT>
__global__ void __launch_bounds__(AW * 64) attn_decode_kernel(AttnArgs a) {
    constexpr int NS = D / 32, NP = AKW / 32, NB = D / 16;
    static_assert(D == 128 && AW * VT_WORDS >= AW * AG * D, "the V areas hold the block merge afterwards");
    // the waves' transposed V areas; after the key loop, the block merge's accumulators
    __shared__ __align__(16) uint32_t vts[AW * VT_WORDS];
    __shared__ __align__(16) float clds[AW][16];
    __shared__ float mlds[AW][AG], llds[AW][AG];
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = blockIdx.y, b = blockIdx.x, G = a.G;
    const int kbase = b * AKB + wave * AKW;
    uint32_t* const vt = vts + wave * VT_WORDS;
    // Q^T as the MFMA B operand: column = head l % 16 (zero past G), head_dim 32 s + 8 (l / 16) .. + 8
    constexpr int NQ = QDT == OOM_F32 ? 3 : 1;
    abf16x8 qb[NQ][NS];
    {
        const int head = lane & 15;
        const bool hok = head < G;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const int d0 = 32 * s + 8 * (lane >> 4);
            const size_t qi = (size_t)(g * G + (hok ? head : 0)) * D + d0;
            if constexpr (QDT == OOM_BF16) {
                const uint4 v = hok ? *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.q) + qi)
                                    : make_uint4(0, 0, 0, 0);
                qb[0][s] = __builtin_bit_cast(abf16x8, v);
            } else {
                float f[8];
#pragma unroll
                for (int e = 0; e < 8; e++) f[e] = hok ? reinterpret_cast<const float*>(a.q)[qi + e] : 0.0f;
#pragma unroll
                for (int term = 0; term < 3; term++) {
                    uint16_t hb[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        hb[e] = f32_to_bf16(f[e]);
                        f[e] -= bf16_to_f32(hb[e]);  // exact: the remainder of a round to nearest
                    }
                    uint4 v;
                    v.x = hb[0] | (uint32_t(hb[1]) << 16);
                    v.y = hb[2] | (uint32_t(hb[3]) << 16);
                    v.z = hb[4] | (uint32_t(hb[5]) << 16);
                    v.w = hb[6] | (uint32_t(hb[7]) << 16);
                    qb[term][s] = __builtin_bit_cast(abf16x8, v);
                }
            }
        }
    }
    // running softmax state of head lane % 16 (identical in the four lane groups) and the
    // output accumulator in the MFMA C layout: o[nb][e] = head 4 (l / 16) + e, dim 16 nb + l % 16
    float m = -INFINITY, l = 0.0f;
    af32x4 o[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) o[nb] = af32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // the page of each of this wave's tiles, lane i holding tile i's (one load up front)
    const int pkey = kbase + 16 * lane;
    const int pages = lane < 2 * NP && pkey < a.kv_len ? a.pt[pkey / a.page_size] : -1;
    // software pipeline over pairs: pair j + 1's V loads go out once pair j's V is in LDS,
    // its K loads once pair j's scores are done, so about one pair is always in flight
    uint4 kr[2][NS], vr[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++) v_load<D>(a, g, kbase + 16 * t, __builtin_amdgcn_readlane(pages, t), lane, vr[t]);
#pragma unroll
    for (int t = 0; t < 2; t++) k_load<D>(a, g, kbase + 16 * t, __builtin_amdgcn_readlane(pages, t), lane, kr[t]);
#pragma unroll
    for (int j = 0; j < NP; j++) {
        const int key0 = kbase + 32 * j;
        if (key0 >= a.kv_len) break;  // wave-uniform
        const int nk0 = j + 1 < NP ? key0 + 32 : a.kv_len;  // the next pair (none: every load reads zeros)
        v_to_lds(vr, vt, lane);
#pragma unroll
        for (int t = 0; t < 2; t++)
            v_load<D>(a, g, nk0 + 16 * t, __builtin_amdgcn_readlane(pages, (2 * j + 2 + t) & 63), lane, vr[t]);
        float s[2][4];
#pragma unroll
        for (int t = 0; t < 2; t++) tile_scores<D, NQ>(a, kr[t], qb, key0 + 16 * t, lane, s[t]);
#pragma unroll
        for (int t = 0; t < 2; t++)
            k_load<D>(a, g, nk0 + 16 * t, __builtin_amdgcn_readlane(pages, (2 * j + 2 + t) & 63), lane, kr[t]);
        // ---- online softmax of head lane % 16 over the pair's 32 keys ----
        float tmax = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                           fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
        tmax = group_max(tmax);
        const float mn = fmaxf(m, tmax);  // finite: the pair's first key is visible
        const float corr = expf(m - mn);  // 0 while m is -inf
        float p[2][4], tsum = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                p[t][e] = expf(s[t][e] - mn);
                tsum += p[t][e];
            }
        l = l * corr + group_sum(tsum);
        m = mn;
        // ---- the accumulator rows (heads 4 (l / 16) + e) take their heads' corr ----
        if (lane < 16) clds[wave][lane] = corr;
        wave_lds_order();  // also orders this pair's V writes before the operand reads below
        const float4 cr = *reinterpret_cast<const float4*>(&clds[wave][4 * (lane >> 4)]);
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            o[nb][0] *= cr.x;
            o[nb][1] *= cr.y;
            o[nb][2] *= cr.z;
            o[nb][3] *= cr.w;
        }
        // ---- P as three bf16 terms (hi + mid + lo == p exactly), A operand order 2 e + t ----
        abf16x8 pa[3];
#pragma unroll
        for (int term = 0; term < 3; term++) {
            typedef __bf16 abf16x2 __attribute__((ext_vector_type(2)));
            typedef float af32x2 __attribute__((ext_vector_type(2)));
            uint32_t wv[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const af32x2 pf = {p[0][e], p[1][e]};
                const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(pf, abf16x2));  // RNE
                wv[e] = w;
                p[0][e] -= __uint_as_float(w << 16);  // exact: the remainder of a round to nearest
                p[1][e] -= __uint_as_float(w & 0xffff0000u);
            }
            pa[term] = __builtin_bit_cast(abf16x8, make_uint4(wv[0], wv[1], wv[2], wv[3]));
        }
        // ---- O += P . V, 16 dims at a time ----
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const uint4 vb = *reinterpret_cast<const uint4*>(vt + vt_word(lane >> 4, 16 * nb + (lane & 15), 0));
            const abf16x8 vop = __builtin_bit_cast(abf16x8, vb);
#pragma unroll
            for (int term = 0; term < 3; term++)
                o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[term], vop, o[nb], 0, 0, 0);
        }
        wave_lds_order();  // this pair's reads of the V area are done before the next pair's writes
    }
    __syncthreads();  // every wave is done with its V area: it now holds the block merge
    float (*alds)[AG][D] = reinterpret_cast<float (*)[AG][D]>(vts);
    // ---- block merge in LDS ----
    if (4 * (lane >> 4) < AG)
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
#pragma unroll
            for (int e = 0; e < 4; e++) alds[wave][4 * (lane >> 4) + e][16 * nb + (lane & 15)] = o[nb][e];
    if (lane < AG) {
        mlds[wave][lane] = m;
        llds[wave][lane] = l;
    }
    __syncthreads();
    // thread: head h = tid / (256 / AG), 4 columns
    constexpr int TPH = AW * 64 / AG, CPT = D / TPH;  // threads per head, columns per thread
    static_assert(CPT == 4, "one 16-byte store per thread");
    const int h = tid / TPH, c0 = (tid % TPH) * CPT;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < AW; w++) M = fmaxf(M, mlds[w][h]);
    float L = 0.0f, A[CPT];
#pragma unroll
    for (int j = 0; j < CPT; j++) A[j] = 0.0f;
#pragma unroll
    for (int w = 0; w < AW; w++) {
        const float f = mlds[w][h] == -INFINITY ? 0.0f : expf(mlds[w][h] - M);
        L = fmaf(llds[w][h], f, L);
#pragma unroll
        for (int j = 0; j < CPT; j++) A[j] = fmaf(alds[w][h][c0 + j], f, A[j]);
    }
    if (a.bph == 1) {  // the KV head's only block: its partial is the result
        if (h < G) {
            const size_t oi = (size_t)(g * G + h) * D + c0;
#pragma unroll
            for (int j = 0; j < CPT; j++) store_out<ODT>(a.out, oi + j, A[j] / L);
        }
        return;
    }
    // ---- the block's partial for attn_merge_kernel (plain stores: the kernel boundary
    // publishes them) ----
    float* mine = a.part + ((size_t)g * a.bph + b) * (2 * AG + AG * D);
    if (tid % TPH == 0) {
        mine[h] = M;
        mine[AG + h] = L;
    }
    *reinterpret_cast<float4*>(mine + 2 * AG + h * D + c0) = make_float4(A[0], A[1], A[2], A[3]);
}

// The merge of a KV head's block partials: the global max over the partials, each partial's
// weight exp(M_b - M) (in LDS), the sum, and sum_b w_b acc_b in block order; out = acc / sum.
// A second kernel, not a merge inside the first: a merge there puts three device-scope round
// trips (stores acknowledged, a ticket, the partials' loads) on the last block's path, which
// cost more than a kernel boundary.
//  * Up to 128 partials (32 Ki keys): block (g, h, q) of two waves merges columns 32 q .. 32 q
//    + 31 of head h, so 4 blocks share a head and the grid spreads the partials' loads over 4
//    times as many CUs. Wave w takes partials 64 w .. 64 w + 63: lane l computes partial
//    64 w + l's weight, then loads column 32 q + l % 32 of partials 64 w + 2 j + l / 32
//    (j < 32), every load in flight at once; the two lane halves, then the two waves, add up.
//  * More partials: one wave walks them in rounds of 64 (q = 0 blocks only).
template <int D, int ODT>
__global__ void __launch_bounds__(128) attn_merge_kernel(AttnArgs a) {
    static_assert(D == 128, "four quarters of 32 columns");
    constexpr int PSZ = 2 * AG + AG * D, CH = 64;  // partials a wave covers at once
    __shared__ float wts[A_MAXB];
    __shared__ float part_m[2], part_l[2], part_a[2][32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = blockIdx.x, h = blockIdx.y, n = a.bph;
    const float* hp = a.part + (size_t)g * n * PSZ;
    if (n <= 2 * CH) {
        const int q = blockIdx.z, col = 32 * q + (lane & 31), par = lane >> 5;
        const int p = CH * wave + lane;
        const bool ok = p < n;
        const float mq = ok ? hp[(size_t)p * PSZ + h] : -INFINITY;
        const float lq = ok ? hp[(size_t)p * PSZ + AG + h] : 0.0f;
        float v[CH / 2];
#pragma unroll
        for (int j = 0; j < CH / 2; j++) {
            const int pj = CH * wave + 2 * j + par;
            v[j] = pj < n ? hp[(size_t)pj * PSZ + 2 * AG + h * D + col] : 0.0f;
        }
        const float Mw = wave_max(mq);  // -inf only for a wave with no partial
        const float w = mq == -INFINITY ? 0.0f : expf(mq - Mw);
        const float Lw = wave_sum(lq * w);
        wts[p] = w;
        wave_lds_order();
        float A = 0.0f;
#pragma unroll
        for (int j = 0; j < CH / 2; j++) A = fmaf(v[j], wts[CH * wave + 2 * j + par], A);  // past n: zeros
        A += lane_xor<32>(A, lane);  // the two lane halves (even and odd partials)
        if (lane == 0) {
            part_m[wave] = Mw;
            part_l[wave] = Lw;
        }
        if (lane < 32) part_a[wave][lane] = A;
        __syncthreads();
        if (wave == 1 || lane >= 32) return;
        const float M = fmaxf(part_m[0], part_m[1]);  // finite: every block holds a visible key
        const float f0 = part_m[0] == -INFINITY ? 0.0f : expf(part_m[0] - M);
        const float f1 = part_m[1] == -INFINITY ? 0.0f : expf(part_m[1] - M);
        const float L = fmaf(part_l[1], f1, part_l[0] * f0);
        const float A1 = fmaf(part_a[1][lane], f1, part_a[0][lane] * f0);
        store_out<ODT>(a.out, (size_t)(g * a.G + h) * D + col, A1 / L);
        return;
    }
    if (wave == 1 || blockIdx.z != 0) return;
    const int c0 = 2 * lane;
    float M = -INFINITY, L = 0.0f, A0 = 0.0f, A1 = 0.0f;
    for (int p = lane; p < n; p += 64) M = fmaxf(M, hp[(size_t)p * PSZ + h]);
    M = wave_max(M);
    for (int p0 = 0; p0 < n; p0 += 64) {
        const int p = p0 + lane;
        float w = 0.0f, lq = 0.0f;
        if (p < n) {
            const float mq = hp[(size_t)p * PSZ + h];
            w = mq == -INFINITY ? 0.0f : expf(mq - M);
            lq = hp[(size_t)p * PSZ + AG + h];
            wts[p] = w;
        }
        L += wave_sum(lq * w);
    }
    wave_lds_order();
    for (int p0 = 0; p0 < n; p0 += CH) {
        float2 v[CH];
#pragma unroll
        for (int j = 0; j < CH; j++)
            v[j] = p0 + j < n ? *reinterpret_cast<const float2*>(hp + (size_t)(p0 + j) * PSZ + 2 * AG + h * D + c0)
                              : make_float2(0.0f, 0.0f);
#pragma unroll
        for (int j = 0; j < CH; j++) {
            if (p0 + j >= n) break;
            const float w = wts[p0 + j];
            A0 = fmaf(v[j].x, w, A0);
            A1 = fmaf(v[j].y, w, A1);
        }
    }
    const size_t oi = (size_t)(g * a.G + h) * D + c0;
    store_out<ODT>(a.out, oi, A0 / L);
    store_out<ODT>(a.out, oi + 1, A1 / L);
}

// ---- host side -------------------------------------------------------------------------

static size_t a_al256(size_t v) { return (v + 255) & ~size_t(255); }

struct AttnWs {
    size_t part, total;
};

static AttnWs attn_ws(int kv_len, int kv_heads, int d) {
    AttnWs w;
    const int bph = (int)cdiv(kv_len, AKB);
    w.part = 0;
    w.total = a_al256((size_t)kv_heads * (bph > 1 ? bph : 1) * (2 * AG + AG * (size_t)d) * sizeof(float));
    return w;
}

template <int D, int QDT, int ODT>
static int launch_attn_t(const AttnArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((attn_decode_kernel<D, QDT, ODT>), dim3(a.bph, a.Hkv), dim3(AW * 64), 0, st, a);
    if (a.bph > 1) {
        if (int rc = launched("oom_attn_decode_paged")) return rc;
        hipLaunchKernelGGL((attn_merge_kernel<D, ODT>), dim3(a.Hkv, a.G, a.bph <= 128 ? 4 : 1), dim3(128), 0, st, a);
    }
    return launched("oom_attn_decode_paged");
}

}  // namespace oom

extern "C" size_t oom_attn_decode_workspace_size(int kv_len, int heads, int kv_heads, int d) {
    if (kv_len < 1 || heads < 1 || kv_heads < 1 || d < 1) return 0;
    return oom::attn_ws(kv_len, kv_heads, d).total;
}

extern "C" int oom_attn_decode_paged(const void* q, int q_dtype, const uint16_t* k_pages, const uint16_t* v_pages,
                                     const int32_t* page_table, int n_pages, int page_size, int kv_len, int heads,
                                     int kv_heads, int d, float scale, void* out, int out_dtype, void* ws,
                                     size_t ws_bytes, void* stream) {
    using namespace oom;
    OOM_REQUIRE(d == 128, "oom_attn_decode_paged: head_dim must be 128");
    OOM_REQUIRE(kv_heads >= 1 && heads >= kv_heads && heads % kv_heads == 0 && heads / kv_heads <= AG,
                "oom_attn_decode_paged: heads must be a multiple of kv_heads, at most 8 query heads per KV head");
    OOM_REQUIRE(page_size >= 16 && page_size % 16 == 0, "oom_attn_decode_paged: page_size must be a multiple of 16");
    OOM_REQUIRE(kv_len >= 1 && n_pages >= 1, "oom_attn_decode_paged: kv_len and n_pages must be >= 1");
    OOM_REQUIRE(kv_len <= A_MAXB * AKB, "oom_attn_decode_paged: kv_len above 8 Mi keys");
    OOM_REQUIRE((int64_t)page_size * kv_heads * d * 2 < (1ll << 31), "oom_attn_decode_paged: page too large");
    OOM_REQUIRE(q_dtype == OOM_F32 || q_dtype == OOM_BF16, "oom_attn_decode_paged: q_dtype");
    OOM_REQUIRE(out_dtype == OOM_F32 || out_dtype == OOM_BF16, "oom_attn_decode_paged: out_dtype");
    OOM_REQUIRE(q && k_pages && v_pages && page_table && out, "oom_attn_decode_paged: null buffer");
    OOM_REQUIRE(aligned(q, 16) && aligned(k_pages, 16) && aligned(v_pages, 16),
                "oom_attn_decode_paged: q, k_pages and v_pages must be 16-byte aligned");
    const AttnWs w = attn_ws(kv_len, kv_heads, d);
    if (!ws || ws_bytes < w.total)
        return fail(OOM_ERR_WORKSPACE, "oom_attn_decode_paged: workspace smaller than oom_attn_decode_workspace_size()");
    OOM_REQUIRE(aligned(ws, 256), "oom_attn_decode_paged: workspace must be 256-byte aligned");
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    AttnArgs a;
    a.q = q;
    a.kp = k_pages;
    a.vp = v_pages;
    a.pt = page_table;
    a.n_pages = n_pages;
    a.page_size = page_size;
    a.kv_len = kv_len;
    a.Hkv = kv_heads;
    a.G = heads / kv_heads;
    a.bph = (int)cdiv(kv_len, AKB);
    a.scale = scale;
    a.out = out;
    a.part = reinterpret_cast<float*>(base + w.part);
    hipStream_t st = as_stream(stream);
    if (q_dtype == OOM_BF16)
        return out_dtype == OOM_BF16 ? launch_attn_t<128, OOM_BF16, OOM_BF16>(a, st)
                                     : launch_attn_t<128, OOM_BF16, OOM_F32>(a, st);
    return out_dtype == OOM_BF16 ? launch_attn_t<128, OOM_F32, OOM_BF16>(a, st)
                                 : launch_attn_t<128, OOM_F32, OOM_F32>(a, st);
}
