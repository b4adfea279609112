// Paged GQA decode attention on gfx950: one query token, H query heads over Hkv KV
// heads (G = H / Hkv query heads share a KV head), bf16 K/V in pages of page_size
// tokens ([page_size, Hkv, D] each, token j in physical page page_table[j / page_size]).
//
//  * Block (b, g) takes keys [512 b, 512 b + 512) of KV head g; each of its 4 waves 128
//    keys, in tiles of 16 (one MFMA tile, inside one page). K and V of a tile stream once
//    for all G query heads; the next tile's loads are in flight while the current one
//    is reduced.
//  * Scores S^T = K . Q^T on bf16 MFMA (v_mfma_f32_16x16x32_bf16; products exact, fp32
//    accumulate): keys are the M side, so K loads need head_dim contiguous per lane
//    (the layout in memory) and each lane ends with 4 keys of one head, which keeps the
//    online-softmax reductions to two lane swaps. fp32 q enters as an exact 3-term bf16
//    split (hi + mid + lo).
//  * P . V in fp32 on the VALU: V rows load coalesced (16 lanes x 8 head_dim columns
//    per row) and P reaches every lane through LDS.
//  * A block merges its waves' (max, sum, acc) in LDS into one partial; the partials of
//    a KV head merge in a tree of fan-in 8 (the last block of each group, found by a
//    ticket that its user resets, merges the group's partials rescaled by their maxima),
//    and the block that merges the top level writes out = acc / sum.
// The arithmetic follows the reference's fp32 online softmax
// (crates/oominf-cuda/kernels/attention.cu:419-553): dot products, exp and accumulation
// in fp32; only the summation order differs.
#include <algorithm>

#include "common.hpp"

namespace oom {

constexpr int AW = 4;           // waves per block
constexpr int AKW = 128;        // keys per wave
constexpr int AKB = AW * AKW;   // keys per block
constexpr int AG = 8;           // query heads per KV head (at most)
constexpr int A_TICKET_STRIDE = 64;
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
    int pslots, tslots;  // merge-tree partial slots and tickets per KV head
    float scale;
    void* out;
    float* part;        // [Hkv][pslots][2 AG + AG D]: max, sum, acc per block, then per merge group
    uint32_t* tickets;  // [Hkv][tslots], A_TICKET_STRIDE apart
    uint32_t* status;
};

__device__ __forceinline__ uint4 a_ld16(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Buffer resource over the KV-head slice of one page (empty if the page index is bad).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const uint16_t* base, int page, int n_pages,
                                                           int page_bytes) {
    const bool ok = page >= 0 && page < n_pages;
    const uint16_t* p = base + (size_t)(ok ? page : 0) * (page_bytes / 2);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p), (short)0, ok ? page_bytes : 0, A_BUF_FLAGS);
}

// One 16-key tile (inside one page): K in the MFMA A layout (lane l holds key l % 16,
// head_dim 32 s + 8 (l / 16) .. + 8) and V for the VALU (lane l holds head_dim
// 8 (l % DL) .. + 8 of key KPI q + l / DL). Keys past kv_len, and tiles whose page
// index is out of range, read zeros.
template <int D>
struct KvTile {
    uint4 k[D / 32];
    uint4 v[16 * D / 512];
};

template <int D>
__device__ __forceinline__ void kv_load(const AttnArgs& a, int g, int key0, int page, int lane, KvTile<D>& t) {
    constexpr int DL = D / 8, KPI = 64 / DL, NT = 16 / KPI;
    const int ps = a.page_size, page_bytes = ps * a.Hkv * D * 2, row_bytes = a.Hkv * D * 2;
    if (key0 >= a.kv_len) page = -1;
    const __amdgpu_buffer_rsrc_t kr = page_rsrc(a.kp, page, a.n_pages, page_bytes);
    const __amdgpu_buffer_rsrc_t vr = page_rsrc(a.vp, page, a.n_pages, page_bytes);
    const int slot0 = key0 % ps;
    const int kkey = key0 + (lane & 15);
    const int kbase = kkey < a.kv_len ? (slot0 + (lane & 15)) * row_bytes + g * D * 2 + 16 * (lane >> 4) : A_OOB;
#pragma unroll
    for (int s = 0; s < D / 32; s++) t.k[s] = a_ld16(kr, kbase == A_OOB ? A_OOB : kbase + 64 * s);
#pragma unroll
    for (int q = 0; q < NT; q++) {
        const int kk = KPI * q + lane / DL;
        const int off = key0 + kk < a.kv_len ? (slot0 + kk) * row_bytes + g * D * 2 + (lane % DL) * 16 : A_OOB;
        t.v[q] = a_ld16(vr, off);
    }
}

// One 16-key tile: scores, online softmax update of (m, l) for head lane % 16, and
// acc += P . V. plds / clds are this wave's LDS rows.
template <int D, int NQ>
__device__ __forceinline__ void attn_tile(const AttnArgs& a, const KvTile<D>& cur, int key0, int lane,
                                          const abf16x8 (&qb)[NQ][D / 32], float& m, float& l, float (&acc)[AG][8],
                                          float (*plds)[AG], float* clds) {
    constexpr int NS = D / 32, DL = D / 8, KPI = 64 / DL, NT = 16 / KPI;
    // ---- scores of 16 keys for 16 (G real) heads: lane l holds keys 4 (l / 16) + e of head l % 16 ----
    float s[4];
    {
        af32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int term = 0; term < NQ; term++)
#pragma unroll
            for (int ss = 0; ss < NS; ss++)
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(abf16x8, cur.k[ss]), qb[term][ss], c, 0,
                                                            0, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int key = key0 + 4 * (lane >> 4) + e;
            s[e] = key < a.kv_len ? c[e] * a.scale : -INFINITY;
        }
    }
    // ---- online softmax per head (lane % 16) over the tile's 16 keys ----
    float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
        tmax = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
        const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
        tmax = fmaxf(__uint_as_float(r2[0]), __uint_as_float(r2[1]));
    }
    const float mn = fmaxf(m, tmax);  // finite: the tile holds a visible key
    const float corr = expf(m - mn);  // 0 while m is -inf
    float p[4], tsum = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        p[e] = expf(s[e] - mn);
        tsum += p[e];
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(tsum), __float_as_uint(tsum), false, false);
        tsum = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(tsum), __float_as_uint(tsum), false, false);
        tsum = __uint_as_float(r2[0]) + __uint_as_float(r2[1]);
    }
    l = l * corr + tsum;
    m = mn;
    // P and corr to this wave's LDS, then P . V
    if ((lane & 15) < AG) {
#pragma unroll
        for (int e = 0; e < 4; e++) plds[4 * (lane >> 4) + e][lane & 15] = p[e];
        if (lane < AG) clds[lane] = corr;
    }
    wave_lds_order();
    float cr[AG];
#pragma unroll
    for (int h = 0; h < AG; h++) cr[h] = clds[h];
#pragma unroll
    for (int h = 0; h < AG; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] *= cr[h];
#pragma unroll
    for (int q = 0; q < NT; q++) {
        const int kk = KPI * q + lane / DL;
        float pv[AG];
#pragma unroll
        for (int h = 0; h < AG; h++) pv[h] = plds[kk][h];
        const uint32_t w[4] = {cur.v[q].x, cur.v[q].y, cur.v[q].z, cur.v[q].w};
        float vf[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            vf[2 * e] = __uint_as_float(w[e] << 16);
            vf[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
        }
#pragma unroll
        for (int h = 0; h < AG; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[h][e] = fmaf(pv[h], vf[e], acc[h][e]);
    }
    wave_lds_order();  // this tile's P reads are done before the next tile's writes
}

template <int D, int QDT, int ODT>
__global__ void __launch_bounds__(256) attn_decode_kernel(AttnArgs a) {
    constexpr int NS = D / 32, DL = D / 8, KPI = 64 / DL;
    __shared__ float plds[AW][16][AG];
    __shared__ float clds[AW][AG];
    __shared__ float mlds[AW][AG], llds[AW][AG];
    __shared__ float alds[AW][AG][D];
    __shared__ uint32_t last;
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = blockIdx.y, b = blockIdx.x, G = a.G;
    const int kbase = b * AKB + wave * AKW;
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
    // running softmax state of head lane % 16 (identical in the four lane groups) and
    // this lane's accumulator acc[h][e] = head h, head_dim 8 (lane % DL) + e, over the
    // keys this lane group sees
    float m = -INFINITY, l = 0.0f;
    float acc[AG][8];
#pragma unroll
    for (int h = 0; h < AG; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;
    constexpr int ntile = AKW / 16;
    // the page of each of this wave's tiles, lane i holding tile i's (one load up front)
    const int pkey = kbase + 16 * lane;
    const int pages = lane < ntile && pkey < a.kv_len ? a.pt[pkey / a.page_size] : -1;
    // two tile buffers, fully unrolled (each buffer index is a constant): the next
    // tile's loads are in flight while the current one is reduced
    KvTile<D> tb[2];
    kv_load<D>(a, g, kbase, __builtin_amdgcn_readlane(pages, 0), lane, tb[0]);
#pragma unroll
    for (int i = 0; i < ntile; i++) {
        const int k0 = kbase + 16 * i;
        if (k0 >= a.kv_len) break;  // wave-uniform
        kv_load<D>(a, g, i + 1 < ntile ? k0 + 16 : a.kv_len, __builtin_amdgcn_readlane(pages, (i + 1) & 63), lane,
                   tb[(i + 1) % 2]);
        attn_tile<D, NQ>(a, tb[i % 2], k0, lane, qb, m, l, acc, plds[wave], clds[wave]);
    }
    // ---- the lane groups' accumulators (same columns, different keys) add up ----
#pragma unroll
    for (int h = 0; h < AG; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = acc[h][e];
            if constexpr (KPI >= 4) {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
                v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
            }
            const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            acc[h][e] = __uint_as_float(r2[0]) + __uint_as_float(r2[1]);
        }
    // ---- block merge in LDS ----
    if (lane < DL)
#pragma unroll
        for (int h = 0; h < AG; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) alds[wave][h][8 * lane + e] = acc[h][e];
    if (lane < AG) {
        mlds[wave][lane] = m;
        llds[wave][lane] = l;
    }
    __syncthreads();
    // thread: head h = tid / (256 / AG), 4 columns
    constexpr int TPH = 256 / AG, CPT = D / TPH;  // threads per head, columns per thread
    static_assert(CPT >= 1 && CPT <= 8, "columns per thread");
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
    static_assert(CPT == 4, "one 16-byte store per thread");
    // ---- partials merge in a tree of fan-in AF: a block stores its (M, L, A) at its
    // slot of the level and takes its group's ticket; the group's last block loads the
    // group's partials (all loads in flight together), merges them in slot order and
    // goes up a level with the group's index; the block that merges the last level
    // writes out = A / L ----
    constexpr int PSZ = 2 * AG + AG * D, AF = 8;
    float* const hpart = a.part + (size_t)g * a.pslots * PSZ;
    uint32_t* const htick = a.tickets + (size_t)g * a.tslots * A_TICKET_STRIDE;
    int n = a.bph, idx = b, poff = 0, toff = 0;
    while (n > 1) {
        float* mine = hpart + (size_t)(poff + idx) * PSZ;
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(mine, (short)0, PSZ * 4, A_BUF_FLAGS);
        if (tid % TPH == 0) {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M), wr, h * 4, 0, A_BUF_SC1);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(L), wr, (AG + h) * 4, 0, A_BUF_SC1);
        }
        {
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
            const u32x4 v = {__float_as_uint(A[0]), __float_as_uint(A[1]), __float_as_uint(A[2]), __float_as_uint(A[3])};
            __builtin_amdgcn_raw_buffer_store_b128(v, wr, (2 * AG + h * D + c0) * 4, 0, A_BUF_SC1);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);  // the stores are complete before the ticket
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        const int grp = idx / AF, nin = min(AF, n - grp * AF);
        if (tid == 0) {
            uint32_t* t = htick + (size_t)(toff + grp) * A_TICKET_STRIDE;
            const uint32_t old = __hip_atomic_fetch_add(t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = old == (uint32_t)nin - 1;
            if (last) __hip_atomic_store(t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last) return;
        const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
            hpart + (size_t)(poff + grp * AF) * PSZ, (short)0, nin * PSZ * 4, A_BUF_FLAGS);
        float bm[AF], bl[AF], bv[AF][CPT];
#pragma unroll
        for (int q = 0; q < AF; q++) {
            const bool ok = q < nin;
            const int base = q * PSZ * 4;
            const float mraw =
                __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, ok ? base + h * 4 : A_OOB, 0, A_BUF_SC1));
            bm[q] = ok ? mraw : -INFINITY;
            bl[q] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(pr, ok ? base + (AG + h) * 4 : A_OOB, 0, A_BUF_SC1));
            const auto v =
                __builtin_amdgcn_raw_buffer_load_b128(pr, ok ? base + (2 * AG + h * D + c0) * 4 : A_OOB, 0, A_BUF_SC1);
#pragma unroll
            for (int j = 0; j < CPT; j++) bv[q][j] = __uint_as_float(v[j]);
        }
        M = -INFINITY;
        L = 0.0f;
#pragma unroll
        for (int j = 0; j < CPT; j++) A[j] = 0.0f;
#pragma unroll
        for (int q = 0; q < AF; q++) {
            if (bm[q] == -INFINITY) continue;
            const float nm = fmaxf(M, bm[q]);
            const float fo = expf(M - nm), fb = expf(bm[q] - nm);
            L = L * fo + bl[q] * fb;
#pragma unroll
            for (int j = 0; j < CPT; j++) A[j] = A[j] * fo + bv[q][j] * fb;
            M = nm;
        }
        poff += n;
        toff += (n + AF - 1) / AF;
        n = (n + AF - 1) / AF;
        idx = grp;
    }
    if (h < G) {
        const size_t o = (size_t)(g * G + h) * D + c0;
#pragma unroll
        for (int j = 0; j < CPT; j++) store_out<ODT>(a.out, o + j, A[j] / L);
    }
}

// ---- host side -------------------------------------------------------------------------

static size_t a_al256(size_t v) { return (v + 255) & ~size_t(255); }

// Partial slots and tickets per KV head of the merge tree over bph block partials.
static void merge_tree_slots(int bph, int& pslots, int& tslots) {
    pslots = 0;
    tslots = 0;
    for (int n = bph; n > 1; n = (n + 7) / 8) {
        pslots += n;
        tslots += (n + 7) / 8;
    }
}

struct AttnWs {
    size_t part, tickets, status, total;
    int pslots, tslots;
};

static AttnWs attn_ws(int kv_len, int kv_heads, int d) {
    AttnWs w;
    const int bph = (int)cdiv(kv_len, AKB);
    merge_tree_slots(bph, w.pslots, w.tslots);
    w.part = 0;
    w.tickets = a_al256((size_t)kv_heads * w.pslots * (2 * AG + AG * (size_t)d) * sizeof(float));
    w.status = w.tickets + (size_t)kv_heads * std::max(w.tslots, 1) * A_TICKET_STRIDE * sizeof(uint32_t);
    w.total = w.status + 256;
    return w;
}

template <int D, int QDT, int ODT>
static int launch_attn_t(const AttnArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((attn_decode_kernel<D, QDT, ODT>), dim3(a.bph, a.Hkv), dim3(256), 0, st, a);
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
    a.pslots = w.pslots;
    a.tslots = w.tslots;
    a.scale = scale;
    a.out = out;
    a.part = reinterpret_cast<float*>(base + w.part);
    a.tickets = reinterpret_cast<uint32_t*>(base + w.tickets);
    a.status = reinterpret_cast<uint32_t*>(base + w.status);
    hipStream_t st = as_stream(stream);
    if (q_dtype == OOM_BF16)
        return out_dtype == OOM_BF16 ? launch_attn_t<128, OOM_BF16, OOM_BF16>(a, st)
                                     : launch_attn_t<128, OOM_BF16, OOM_F32>(a, st);
    return out_dtype == OOM_BF16 ? launch_attn_t<128, OOM_F32, OOM_BF16>(a, st)
                                 : launch_attn_t<128, OOM_F32, OOM_F32>(a, st);
}
