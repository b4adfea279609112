// Decode MoE FFN step for a small batch (2..16 tokens, bf16 activations) on bf16 MFMA in
// one persistent kernel: router top-k, routing plan, gate/up + SwiGLU, one grid barrier,
// down projection, a second grid barrier and the slot-order combine (the routed part of
// crates/oominf-models-qwen/src/moe.rs:290-366; arithmetic of
// crates/oominf-cuda/kernels/moe.cu:52-164).
//
// With 16 tokens the routed experts' multiply-adds (16 x 8 x 3 x 4096 x 1536) outgrow the
// vector ALUs, so the products run on v_mfma_f32_16x16x32_bf16: e4m3 weights convert to
// bf16 exactly, bf16 activations are exact, the products are exact in fp32 and sum in
// fp32, as the reference's fp32 multiply-adds do (in another order).
//
//  * Every block routes all tokens (one wave per token) and plans into LDS, and stages
//    the tokens' activations in LDS (bf16 rows, padded so the 16 rows start in different
//    banks). The workspace header's barrier words are the only state kept between calls.
//  * Phase 1: item = (expert, 8 intermediate rows). The MFMA A tile stacks the 8 gate rows
//    over the 8 up rows (lane l: row l % 16, 32 bytes of each 128-column K step), B is the
//    expert's tokens (column n = assignment n of the expert). A K step is 4 MFMAs whose sum
//    is scaled by the rows' 128 x 128 block scale before it joins the accumulator; the
//    wave's next K steps (B_DEPTH of them) are in flight meanwhile. At the item's end a
//    lane swap meets gate and up: h = silu(g) * u, stored per token (16 bytes per lane).
//  * A grid barrier (every block resident).
//  * Phase 2: item = (expert, 16 output rows); with at least 4 blocks an expert, each
//    expert has a contiguous group of blocks that split its row tiles, otherwise block b
//    takes a contiguous share of all items (one or two experts): a block stages its expert's h in LDS as h ~ hi + lo, two
//    bf16 terms (lo = bf16(h - hi): 16 significant bits, relative error <= 2^-16), and its
//    waves take the expert's row tiles. A K step is 8 MFMAs (hi and lo). y rows go out per
//    assignment with no wait; the first K steps of the block's first tiles load before the
//    barrier.
//  * A second grid barrier, then the combine: out[t] = sum over t's slots, in slot order,
//    of w y, one lane per 4 rows of a token.
// h and y move between blocks with device-coherent (sc1) stores and loads.
//
// With a shared expert of the routed geometry (SH, the decode layer's batch step) the plan
// gains one entry after the routed experts: the shared record with all T tokens
// (assignments A .. A + T), so its gate/up rows and down tiles are phase-1 and phase-2
// items like the routed ones. Each block takes the tokens' gate logits x . gate_w from the
// activations in LDS while wave 0 plans, and the combine ends with
// out[t] = routed + sigmoid(gate[t]) * y_shared[t] (Moe::shared and moe_combine,
// crates/oominf-models-qwen/src/moe.rs:498-527, crates/oominf-cuda/kernels/ops.cu:10,310-316).
#include "router.hpp"
#include "stream.hpp"

namespace oom {

constexpr int B_W = 8;             // waves per block: two per SIMD
constexpr int B_T = 16;            // tokens: one MFMA column tile
constexpr int B_KMAX = 8;          // router top-k
constexpr int B_AMAX = B_T * B_KMAX;
constexpr int B_ASH = B_AMAX + B_T;  // with the shared expert's assignments
constexpr int B_HMAX = 4096;
constexpr int B_IMAX = 2048;
constexpr int B_DEPTH = 8;         // K steps in flight per wave (3 loads each)
constexpr int B_XS = B_HMAX + 8;   // LDS row stride (bf16) of the activations
constexpr int B_HS = B_IMAX + 8;   // LDS row stride (bf16) of h
constexpr int B_TILE = 16;         // output rows of a phase-2 item
constexpr int B_Q = 16;            // a wave's queue of claimed items (issue cursor -> consume cursor)

typedef __bf16 bbf16x8 __attribute__((ext_vector_type(8)));
typedef float bf32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t bu32x4 __attribute__((ext_vector_type(4)));

struct BArgs {
    const float* logits;
    const uint16_t* x;  // bf16 [T, H]
    const uint64_t* all_recs;
    int T, E, k, H, I;
    int gw, gs, uw, us, dw, ds;  // record part offsets
    int rec_bytes;               // bytes of a record up to the end of its last part
    int32_t* ids;
    float* weights;
    void* out;
    float* h;  // [A (+ T with the shared expert), I]
    float* y;  // [A (+ T), H]
    // the shared expert (SH): its record address at shared_rec[0] (the routed geometry) and
    // its bf16 gate row [H]
    const uint64_t* shared_rec;
    const uint16_t* gate_w;
    uint32_t* hdr;
    uint32_t* status;  // the device's status word: 1 if a wait gave up (results invalid)
    uint32_t spin;     // polls before a wait gives up
#ifdef OOM_STAMPS
    uint64_t* stamps;  // phase timestamps (profiling build)
#endif
};

// The activation / h rows come first: their 16-byte LDS reads and writes need 16-byte
// aligned addresses (row strides are multiples of 16 bytes).
struct alignas(16) BLds {
    union {
        uint16_t x[B_T * B_XS];       // phase 1: the tokens' activations, bf16
        uint16_t hh[2][B_T * B_HS];   // phase 2: the staged expert's h, hi and lo bf16 terms
    } u;
    uint64_t recs[257];  // entry E: the shared expert's record
    uint64_t keys[B_W][B_KMAX];  // routing scratch of each wave
    float p[B_W][B_KMAX];
    uint32_t mask[256];          // tokens routed to each expert, one bit per token
    int base[256];               // first assignment of each expert
    int ids[B_AMAX];
    float w[B_AMAX];
    int experts[B_AMAX + 1];
    int off[B_AMAX + 2];
    int assign_tok[B_ASH];
    int slot_assign[B_AMAX];
    float gate[B_T];  // the shared expert's gate logits
    int queue[B_W][B_Q];  // each wave's claimed items, from its issue cursor to its consume cursor
    uint32_t claims[2];   // items claimed by the block's waves: phase 1, phase 2
    int n_e;
};
static_assert(offsetof(BLds, u) == 0 && (B_XS * 2) % 16 == 0 && (B_HS * 2) % 16 == 0 &&
                  (B_T * B_HS * 2) % 16 == 0,
              "16-byte LDS accesses need aligned rows");

// One K step of a wave: 32 bytes of this lane's A row and the row's block scale.
struct KStep {
    uint4 w[2];
    float s;
};

// 8 e4m3 weights (two words) as a bf16 MFMA operand, exactly.
__device__ __forceinline__ bbf16x8 e4m3x8_bf16(uint32_t w0, uint32_t w1) {
    const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
    const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
    const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
    const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
    return bbf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ bbf16x8 lds_bf16x8(const uint16_t* p) {
    return __builtin_bit_cast(bbf16x8, *reinterpret_cast<const uint4*>(p));
}

// v, once the accumulator is computed: an empty asm that takes c and hands back v keeps
// whatever uses the result after c's producers.
__device__ __forceinline__ int after(int v, const bf32x4& c) {
    asm volatile("" : "+v"(v) : "v"(c[0]), "v"(c[1]), "v"(c[2]), "v"(c[3]));
    return v;
}

// 16 bytes of four floats with a device-coherent store (zeros-cost resource check).
__device__ __forceinline__ void st_dev16(__amdgpu_buffer_rsrc_t r, int off, const float (&v)[4]) {
    const bu32x4 d = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
    __builtin_amdgcn_raw_buffer_store_b128(d, r, off, 0, BUF_SC1);
}

// ---- phase 1: gate/up ------------------------------------------------------------------

// An item (slot i, intermediate rows j0 .. j0 + 8) as this lane loads it: lane l takes row
// m = l % 16 (gate row j0 + m for m < 8, up row j0 + m - 8 otherwise), bytes 32 (l / 16)
// .. + 32 of each 128-column K step, and the block scale of its output rows (rows
// 4 (l / 16) + e: gate in lanes 0..31, up in 32..63; the 8 rows share a 128-row block).
// Past the wave's items the record's range is 0, so every load reads zeros.
struct GuRow {
    __amdgpu_buffer_rsrc_t r;
    int roff, soff;
    bool ok;  // the lane's row exists
};

__device__ __forceinline__ GuRow gu_row(const BArgs& a, const BLds& L, int it, bool valid, int nrt, int lane) {
    const int i = valid ? it / nrt : 0, j0 = valid ? (it - i * nrt) * 8 : 0;
    const int m = lane & 15, j = j0 + (m & 7), nkb = (a.H + 127) >> 7;
    GuRow g;
    g.r = uniform_rsrc(L.recs[L.experts[i]], valid ? a.rec_bytes : 0);
    g.roff = (m >= 8 ? a.uw : a.gw) + j * a.H + 32 * (lane >> 4);
    g.soff = (lane >= 32 ? a.us : a.gs) + (j0 >> 7) * nkb * 4;
    g.ok = j < a.I;
    return g;
}

// K step ks of an item: zeros past inter and hidden.
// The scale load waits for `dep`, the accumulator that last used the previous scale, so
// the new scale takes the old one's register.
__device__ __forceinline__ void gu_issue(const BArgs& a, const GuRow& g, int ks, int lane, const bf32x4& dep, KStep& t) {
    const int col = ks * 128 + 32 * (lane >> 4), o = g.roff + ks * 128;
    t.w[0] = ld16(g.r, g.ok && col < a.H ? o : OOB);
    t.w[1] = ld16(g.r, g.ok && col + 16 < a.H ? o + 16 : OOB);
    t.s = ldf(g.r, after(g.soff + ks * 4, dep));
}

// c += scale * (A . B) over a K step: 4 MFMAs; B is the tokens' activations at the same
// 32 columns per lane group, from the LDS row offset xo (column n: assignment a0 + n,
// past nb the first one's).
__device__ __forceinline__ void gu_mfma(const BLds& L, const KStep& t, int xo, bf32x4& c) {
    const uint16_t* xr = &L.u.x[xo];
    const uint32_t wd[8] = {t.w[0].x, t.w[0].y, t.w[0].z, t.w[0].w, t.w[1].x, t.w[1].y, t.w[1].z, t.w[1].w};
    bf32x4 cs = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int mm = 0; mm < 4; mm++)
        cs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(e4m3x8_bf16(wd[2 * mm], wd[2 * mm + 1]), lds_bf16x8(xr + 8 * mm),
                                                     cs, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; e++) c[e] = fmaf(cs[e], t.s, c[e]);
}

// End of an item (rows j0 ..): lane l holds rows 4 (l / 16) + e of column n = l % 16;
// rows 0..7 (lanes 0..31) are gate, 8..15 (lanes 32..63) up. h = silu(g) * u in lanes
// 0..31 (v_permlane32_swap brings the up value), 4 consecutive rows per lane.
__device__ __forceinline__ void gu_store(const BArgs& a, __amdgpu_buffer_rsrc_t hr, int j0, int a0, int nb,
                                         int lane, const bf32x4& c) {
    float hv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(c[e]), __float_as_uint(c[e]), false, false);
        hv[e] = siluf(c[e]) * __uint_as_float(r[1]);
    }
    const int n = lane & 15, j = j0 + 4 * (lane >> 4);
    if (lane < 32 && n < nb && j < a.I) st_dev16(hr, ((a0 + n) * a.I + j) * 4, hv);
}

// ---- phase 2: down ---------------------------------------------------------------------

// Output tile `tile` (rows 16 tile ..) of the run's slot as this lane loads it: row
// 16 tile + l % 16, bytes 32 (l / 16) .. + 32 of each K step; the tile's block scale.
struct DnRow {
    int roff, soff;
    bool ok;
};

__device__ __forceinline__ DnRow dn_row(const BArgs& a, int tile, bool valid, int lane) {
    const int row = tile * B_TILE + (lane & 15), nkb = (a.I + 127) >> 7;
    DnRow d;
    d.roff = a.dw + row * a.I + 32 * (lane >> 4);
    d.soff = a.ds + ((tile * B_TILE) >> 7) * nkb * 4;
    d.ok = valid && row < a.H;
    return d;
}

__device__ __forceinline__ void dn_issue(const BArgs& a, __amdgpu_buffer_rsrc_t r, const DnRow& d, int ks, int lane,
                                         const bf32x4& dep, KStep& t) {
    const int col = ks * 128 + 32 * (lane >> 4), o = d.roff + ks * 128;
    t.w[0] = ld16(r, d.ok && col < a.I ? o : OOB);
    t.w[1] = ld16(r, d.ok && col + 16 < a.I ? o + 16 : OOB);
    t.s = ldf(r, after(d.soff + ks * 4, dep));
}

// c += scale * (A . (h_hi + h_lo)) over a K step: 8 MFMAs; ho is the LDS offset of
// column n = l % 16's h row at this lane's 32 columns of the step.
__device__ __forceinline__ void dn_mfma(const BLds& L, const KStep& t, int ho, bf32x4& c) {
    const uint16_t* hi = &L.u.hh[0][ho];
    const uint16_t* lo = &L.u.hh[1][ho];
    const uint32_t wd[8] = {t.w[0].x, t.w[0].y, t.w[0].z, t.w[0].w, t.w[1].x, t.w[1].y, t.w[1].z, t.w[1].w};
    bf32x4 cs = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int mm = 0; mm < 4; mm++) {
        const bbf16x8 av = e4m3x8_bf16(wd[2 * mm], wd[2 * mm + 1]);
        cs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, lds_bf16x8(hi + 8 * mm), cs, 0, 0, 0);
        cs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, lds_bf16x8(lo + 8 * mm), cs, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) c[e] = fmaf(cs[e], t.s, c[e]);
}

// One token's picks from its keys and the k-th key: pick r (in key order) gets ids[r] and
// w[r] = p / (sum of the picks' p in pick order), as the reference renormalises
// (crates/oominf-cuda/kernels/ops.cu:230-294); the token's bit joins each pick's mask.
template <int EQ>
__device__ __forceinline__ void batch_picks(const uint64_t (&key)[EQ], uint64_t kth, int k, int lane, uint64_t* keys,
                                            float* p, int* ids, float* w, uint32_t* mask, int t) {
    int base = 0;
#pragma unroll
    for (int q = 0; q < EQ; q++) {
        const uint64_t sel = __ballot(key[q] >= kth);
        if (key[q] >= kth) {
            const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(sel >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)sel, 0u));
            keys[pos] = key[q];
        }
        base += (int)__builtin_popcountll(sel);
    }
    wave_lds_order();
    const uint64_t mine = lane < k ? keys[lane] : 0ull;
    int rank = 0;
    for (int j = 0; j < k; j++) rank += keys[j] > mine;
    const float pm = __uint_as_float((uint32_t)(mine >> 8) & 0x7fffffffu);
    const int e = 255 - (int)(mine & 255u);
    if (lane < k) {
        ids[rank] = e;
        p[rank] = pm;
        __hip_atomic_fetch_or(&mask[e], 1u << t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    wave_lds_order();
    float picked = 0.0f;
    for (int r = 0; r < k; r++) picked += p[r];
    if (lane < k) w[rank] = pm / picked;
    wave_lds_order();  // keys and p are free for the wave's next token
}

// The shared expert's gate logits L.gate[t] = x[t] . gate_w for tokens t0, t0 + step, ..
// from the activations in LDS (zeros past H): lane l takes columns 8 (l + 64 c) .. + 8.
__device__ __forceinline__ void batch_gate(const BArgs& a, BLds& L, int t0, int step, int lane) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.gate_w), (short)0, a.H * 2, BUF_FLAGS);
    constexpr int NC = B_HMAX / 512;
    uint4 g[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int col = (lane + 64 * c) * 8;
        g[c] = ld16(r, col < a.H ? col * 2 : OOB);
    }
    for (int t = t0; t < a.T; t += step) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const uint4 xv = *reinterpret_cast<const uint4*>(&L.u.x[t * B_XS + (lane + 64 * c) * 8]);
            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, gw[4] = {g[c].x, g[c].y, g[c].z, g[c].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc = fmaf(__uint_as_float(gw[i] << 16), __uint_as_float(xw[i] << 16), acc);
                acc = fmaf(__uint_as_float(gw[i] & 0xffff0000u), __uint_as_float(xw[i] & 0xffff0000u), acc);
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) L.gate[t] = acc;
    }
}

template <int EQ, int ODT, bool SH>
__global__ void __launch_bounds__(64 * B_W) moe_batch_kernel(BArgs a) {
    const uint32_t bbase1 = grid_barrier_base(a.hdr + WS_BAR / 4), bbase2 = grid_barrier_base(a.hdr + WS_BAR2 / 4);
    __shared__ BLds L;
    constexpr int NT = 64 * B_W, TPW = B_T / B_W;  // threads; tokens routed per wave
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int T = a.T, E = a.E, k = a.k, A = T * k, H = a.H, I = a.I;
    OOM_STAMP(a.stamps, B_W, 0);
    OOM_STAMP_WHERE(a.stamps, B_W);
    // ---- set-up: this wave's tokens' logits (t = wave + B_W j) in flight first ----
    float lv[TPW][EQ];
#pragma unroll
    for (int j = 0; j < TPW; j++)
#pragma unroll
        for (int q = 0; q < EQ; q++) {
            const int t = wave + B_W * j, e = lane + 64 * q;
            lv[j][q] = t < T && e < E ? a.logits[(size_t)t * E + e] : -INFINITY;
        }
    if (tid < E) L.recs[tid] = a.all_recs[tid];
    if constexpr (SH) {
        if (tid == E) L.recs[E] = a.shared_rec[0];
    }
    if (tid < 256) L.mask[tid] = 0u;  // (512 threads, 256 masks)
    if (tid == 256) L.claims[0] = L.claims[1] = 0u;
    // activations: thread tid takes columns 8 (tid + NT c) .. + 8 of every token row (zeros
    // past T and H); the loads stay in flight through the routing below and reach LDS after it
    static_assert(B_HMAX / 8 / NT == 1, "one pass of activation loads");
    const int xcol = tid * 8;
    uint4 xv[B_T];
#pragma unroll
    for (int u = 0; u < B_T; u++)
        xv[u] = u < T && xcol < H ? *reinterpret_cast<const uint4*>(a.x + (size_t)u * H + xcol) : make_uint4(0, 0, 0, 0);
    lds_barrier();  // masks are zero (the activation loads stay in flight)
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int t = wave + B_W * j;
        if (t < T) {
            uint64_t key[EQ];
            route_keys<EQ>(lv[j], E, lane, key);
            const uint64_t kth = radix_kth<EQ>(key, k);
            batch_picks<EQ>(key, kth, k, lane, L.keys[wave], L.p[wave], &L.ids[t * k], &L.w[t * k], L.mask, t);
        }
    }
#pragma unroll
    for (int u = 0; u < B_T; u++) *reinterpret_cast<uint4*>(&L.u.x[u * B_XS + xcol]) = xv[u];
    __syncthreads();
    // plan: assignments sorted by (expert, slot); expert e's run starts at the count of
    // assignments to lower ids, and the token order within it is the mask's bit order
    if (wave == 0) {
        uint32_t m[4];
        int c = 0, pr = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = 4 * lane + j;
            m[j] = e < E ? L.mask[e] : 0u;
            c += __builtin_popcount(m[j]);
            pr += m[j] != 0u;
        }
        int ic = c, ip = pr;  // inclusive scans over lanes
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int tc = __shfl_up(ic, o, 64), tp = __shfl_up(ip, o, 64);
            if (lane >= o) {
                ic += tc;
                ip += tp;
            }
        }
        int bc = ic - c, bp = ip - pr;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = 4 * lane + j;
            if (e < E) {
                L.base[e] = bc;
                if (m[j] != 0u) {
                    L.experts[bp] = e;
                    L.off[bp] = bc;
                    bp++;
                }
                bc += __builtin_popcount(m[j]);
            }
        }
        if (lane == 63) {
            L.n_e = ip;
            L.off[ip] = ic;
            if constexpr (SH) {
                // the shared expert after the routed ones: record E, assignments A .. A + T
                L.experts[ip] = E;
                L.off[ip + 1] = ic + T;
                L.n_e = ip + 1;
            }
        }
    } else if constexpr (SH) {
        batch_gate(a, L, wave - 1, B_W - 1, lane);
    }
    __syncthreads();
    for (int s = tid; s < A; s += NT) {
        const int t = s / k, e = L.ids[s];
        const int pos = L.base[e] + __builtin_popcount(L.mask[e] & ((1u << t) - 1u));
        L.slot_assign[s] = pos;
        L.assign_tok[pos] = t;
    }
    if constexpr (SH) {
        if (tid < T) L.assign_tok[A + tid] = tid;
    }
    __syncthreads();
    if (blockIdx.x == 0)
        for (int s = tid; s < A; s += NT) {
            a.ids[s] = L.ids[s];
            a.weights[s] = L.w[s];
        }
    const int n_e = L.n_e;
    OOM_STAMP(a.stamps, B_W, 1);  // routed and planned
    const int NW = gridDim.x * B_W, gw = blockIdx.x * B_W + wave;
    const int nksH = (H + 127) >> 7, nksI = (I + 127) >> 7;
    const int AS = A + (SH ? T : 0);  // rows of h and y
    const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(a.h, (short)0, AS * I * 4, BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(a.y, (short)0, AS * H * 4, BUF_FLAGS);
    const int m16 = lane & 15, kq = lane >> 4;
    // ---- phase 1: block b's items are b, b + G, b + 2 G, ..., so blocks differ by at most
    // one item and the grid's waves stream neighbouring items at any time; its waves claim
    // them in order from a counter in LDS, so every wave streams until the block's items run
    // out. (Items dealt to waves statically, gw + n NW, gave some blocks a third more items
    // than others whenever the routed expert count passed a multiple of the grid's waves,
    // and one 64 KiB item takes a lone wave ~8 us.) K steps in order, an issue cursor
    // B_DEPTH steps ahead of the consume cursor, each claimed item handed from the one to
    // the other through the wave's queue in LDS ----
    int* const queue = L.queue[wave];
    {
        const int nrt = (I + 7) >> 3, NG = n_e * nrt;
        const int hi = NG;
        auto claim = [&]() -> int {
            uint32_t c = 0;
            if (lane == 0) c = __hip_atomic_fetch_add(&L.claims[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            c = __builtin_amdgcn_readfirstlane(c);
            return (int)blockIdx.x + (int)c * (int)gridDim.x;
        };
        int iti = claim(), ni = 0, ksi = 0;  // the issue cursor's item (from hi on: claims stop)
        if (lane == 0) queue[0] = iti;
        GuRow gi = gu_row(a, L, iti, iti < hi, nrt, lane);
        auto issue = [&](KStep& t, const bf32x4& dep) {
            gu_issue(a, gi, ksi, lane, dep, t);
            if (++ksi == nksH) {
                ksi = 0;
                if (iti < hi) iti = claim();
                ++ni;
                if (lane == 0) queue[ni & (B_Q - 1)] = iti;
                gi = gu_row(a, L, iti, iti < hi, nrt, lane);
            }
        };
        KStep ring[B_DEPTH];
#pragma unroll
        for (int d = 0; d < B_DEPTH; d++) issue(ring[d], bf32x4{0.0f, 0.0f, 0.0f, 0.0f});
        int nc = 0, ksc = 0, itc = 0, j0 = 0, a0 = 0, nb = 0, xo = 0;
        auto con_item = [&]() {
            itc = __builtin_amdgcn_readfirstlane(queue[nc & (B_Q - 1)]);
            const int i = itc < hi ? itc / nrt : 0;
            j0 = (itc - i * nrt) * 8;
            a0 = L.off[i];
            nb = L.off[i + 1] - a0;
            xo = L.assign_tok[a0 + (m16 < nb ? m16 : 0)] * B_XS + 32 * kq;
        };
        con_item();
        bf32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
        // every ring slot is consumed and refilled on every step (steps past the last item
        // read zeros and store nothing), so the slots stay in fixed registers across
        // iterations
        while (itc < hi) {
#pragma unroll
            for (int d = 0; d < B_DEPTH; d++) {
                gu_mfma(L, ring[d], xo + ksc * 128, c);
                issue(ring[d], c);
                if (++ksc == nksH) {
                    ksc = 0;
                    if (itc < hi) gu_store(a, hr, j0, a0, nb, lane, c);
                    c = bf32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    ++nc;
                    con_item();
                }
            }
        }
    }
    // ---- phase 2: this block's items (slot, 16-row tile) first .. last, slot-major, in
    // runs of one slot; the first run's first K steps load before the barrier. With at
    // least 4 blocks a slot, slot i has blocks i G / n_e .. (i + 1) G / n_e - 1 to itself
    // and they split its tiles evenly, so every block stages one slot's h once: an even
    // split of all items puts most blocks across two slots, and a second h staging on
    // their path (measured at batch 16, ~32 slots: 141.6 -> 137.4 us a step). With fewer
    // blocks a slot, each block takes an even share of all items: whole-slot groups then
    // leave most blocks a few tiles above the average, which cost more than the second
    // staging (the decode layer at batch 16, ~84 slots: 312.1 us that way, 316.1 us
    // grouped) ----
    const int ntile = (H + B_TILE - 1) / B_TILE, ND = n_e * ntile;
    int first, last;
    if ((int)gridDim.x >= 4 * n_e) {
        const int G = (int)gridDim.x, b = (int)blockIdx.x;
        const int si = ((b + 1) * n_e - 1) / G, b0 = si * G / n_e, nb = (si + 1) * G / n_e - b0, j = b - b0;
        first = si * ntile + j * ntile / nb;
        last = si * ntile + (j + 1) * ntile / nb;
    } else {
        const int per = (ND + gridDim.x - 1) / gridDim.x;
        first = min(ND, (int)blockIdx.x * per);
        last = min(ND, first + per);
    }
    int r0 = first, i = 0, t0 = 0, t1 = 0;
    // the run at r0: slot i, tiles t0 .. t1, which the block's waves claim in order from a
    // counter in LDS; K steps in order, issued B_DEPTH ahead of their use, the claimed tiles
    // handed from the issue cursor to the consume cursor through the wave's queue. Every
    // wave claims each run's tiles until its first claim past t1, so a run takes exactly
    // (t1 - t0) + B_W claims and the next run's claims count from there.
    uint32_t cbase = 0;  // phase-2 claims before this run
    auto claim = [&]() -> int {
        uint32_t c = 0;
        if (lane == 0) c = __hip_atomic_fetch_add(&L.claims[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        c = __builtin_amdgcn_readfirstlane(c);
        return t0 + (int)(c - cbase);
    };
    __amdgpu_buffer_rsrc_t rr = uniform_rsrc(0, 0);
    int ti = 0, ni = 0, ksi = 0;  // the issue cursor's tile (from t1 on: claims stop)
    DnRow di = dn_row(a, 0, false, lane);
    auto issue = [&](KStep& t, const bf32x4& dep) {
        dn_issue(a, rr, di, ksi, lane, dep, t);
        if (++ksi == nksI) {
            ksi = 0;
            if (ti < t1) ti = claim();
            ++ni;
            if (lane == 0) queue[ni & (B_Q - 1)] = ti;
            di = dn_row(a, ti, ti < t1, lane);
        }
    };
    KStep ring[B_DEPTH];
    auto start_run = [&]() {
        const bool any = r0 < last;
        i = any ? r0 / ntile : 0;
        t0 = any ? r0 - i * ntile : 0;
        t1 = any ? min(ntile, t0 + (last - r0)) : 0;
        rr = uniform_rsrc(L.recs[L.experts[i]], any ? a.rec_bytes : 0);
        ni = 0;
        ksi = 0;
        ti = any ? claim() : t1;
        if (lane == 0) queue[0] = ti;
        di = dn_row(a, ti, ti < t1, lane);
#pragma unroll
        for (int d = 0; d < B_DEPTH; d++) issue(ring[d], bf32x4{0.0f, 0.0f, 0.0f, 0.0f});
    };
    start_run();
    OOM_STAMP(a.stamps, B_W, 2);  // gate/up items done (the first run's down loads in flight)
    wait_mem();  // this wave's h stores are complete before its block arrives
    grid_barrier_words(a.hdr + WS_BAR / 4, bbase1, a.status, a.spin);
    OOM_STAMP(a.stamps, B_W, 3);  // the first grid barrier released
    bool staged_once = false;
    while (r0 < last) {
        // stage the slot's h: thread tid takes columns 4 (tid + NT c) .. + 4 of every
        // assignment (zeros past nb and I), 16 loads in flight per pass
        {
            const int a0 = L.off[i], nb = L.off[i + 1] - a0;
#pragma unroll
            for (int c = 0; c < B_IMAX / 4 / NT; c++) {
                const int col = (tid + NT * c) * 4;
                bu32x4 v[B_T];
#pragma unroll
                for (int n = 0; n < B_T; n++)
                    v[n] = __builtin_amdgcn_raw_buffer_load_b128(hr, n < nb && col < I ? ((a0 + n) * I + col) * 4 : OOB,
                                                                 0, BUF_SC1);
#pragma unroll
                for (int n = 0; n < B_T; n++) {
                    uint16_t hi[4], lo[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float f = __uint_as_float(v[n][e]);
                        hi[e] = f32_to_bf16(f);
                        lo[e] = f32_to_bf16(f - bf16_to_f32(hi[e]));
                    }
                    *reinterpret_cast<uint2*>(&L.u.hh[0][n * B_HS + col]) =
                        make_uint2(hi[0] | (uint32_t)hi[1] << 16, hi[2] | (uint32_t)hi[3] << 16);
                    *reinterpret_cast<uint2*>(&L.u.hh[1][n * B_HS + col]) =
                        make_uint2(lo[0] | (uint32_t)lo[1] << 16, lo[2] | (uint32_t)lo[3] << 16);
                }
            }
        }
        __syncthreads();
        if (!staged_once) OOM_STAMP(a.stamps, B_W, 4);  // the first run's h staged
        staged_once = true;
        const int a0 = L.off[i], nb = L.off[i + 1] - a0, ho = m16 * B_HS + 32 * kq;
        int nc = 0, ksc = 0, tc = __builtin_amdgcn_readfirstlane(queue[0]);
        bf32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
        while (tc < t1) {
#pragma unroll
            for (int d = 0; d < B_DEPTH; d++) {
                dn_mfma(L, ring[d], ho + ksc * 128, c);
                issue(ring[d], c);
                if (++ksc == nksI) {
                    // y rows 16 tile + 4 (l / 16) + e of assignment a0 + l % 16
                    ksc = 0;
                    const int row = tc * B_TILE + 4 * kq;
                    const float yv[4] = {c[0], c[1], c[2], c[3]};
                    if (tc < t1 && m16 < nb && row < H) st_dev16(yr, ((a0 + m16) * H + row) * 4, yv);
                    c = bf32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    ++nc;
                    tc = __builtin_amdgcn_readfirstlane(queue[nc & (B_Q - 1)]);
                }
            }
        }
        cbase += (uint32_t)(t1 - t0 + B_W);
        r0 += t1 - t0;
        __syncthreads();  // every wave is done with this run's h before the next is staged
        start_run();
    }
    // ---- combine: out[t][r .. r + 4] = sum over the token's slots, in slot order, of w y;
    // one lane per 4 rows of a token, the slots' y loads all in flight ----
    OOM_STAMP(a.stamps, B_W, 5);  // down tiles done
    wait_mem();
    grid_barrier_words(a.hdr + WS_BAR2 / 4, bbase2, a.status, a.spin);  // the second meeting's own area
    const int nq4 = H >> 2;
    for (int g = gw * 64 + lane; g < T * nq4; g += NW * 64) {
        const int t = g / nq4, r = (g - t * nq4) * 4;
        bu32x4 yv[B_KMAX], ys;
#pragma unroll
        for (int s = 0; s < B_KMAX; s++)
            yv[s] = __builtin_amdgcn_raw_buffer_load_b128(
                yr, s < k ? (L.slot_assign[t * k + s] * H + r) * 4 : OOB, 0, BUF_SC1);
        if constexpr (SH) ys = __builtin_amdgcn_raw_buffer_load_b128(yr, ((A + t) * H + r) * 4, 0, BUF_SC1);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < B_KMAX; s++)
            if (s < k)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = fmaf(L.w[t * k + s], __uint_as_float(yv[s][e]), acc[e]);
        if constexpr (SH) {
            const float sg = 1.0f / (1.0f + expf(-L.gate[t]));  // sigmoid (ops.cu:10)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = acc[e] + sg * __uint_as_float(ys[e]);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) store_out<ODT>(a.out, (size_t)t * H + r + e, acc[e]);
    }
    OOM_STAMP(a.stamps, B_W, 6);  // combined and stored
    grid_barrier_exit(a.hdr + WS_BAR / 4);
    grid_barrier_exit(a.hdr + WS_BAR2 / 4);
}

// ---- host side -----------------------------------------------------------------------

struct BWs {
    size_t h, y, total;
};

// h and y rows: one per assignment, plus one per token for the shared expert (sh).
static BWs batch_ws(int T, int k, const OomFp8Record& g, bool sh = false) {
    const size_t A = (size_t)T * (k + (sh ? 1 : 0));
    BWs w;
    w.h = WS_HEADER;
    w.y = w.h + ((A * g.inter * sizeof(float) + 255) & ~size_t(255));
    w.total = w.y + ((A * g.hidden * sizeof(float) + 255) & ~size_t(255));
    return w;
}

template <int EQ, int ODT, bool SH>
static int batch_grid() {
    static thread_local int cached_dev = -1, cached = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (dev != cached_dev) {
        int cus = 0, per = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, moe_batch_kernel<EQ, ODT, SH>, 64 * B_W, 0) != hipSuccess)
            return 0;
        cached = cus * per;
        cached_dev = dev;
    }
    return cached;
}

template <int EQ, int ODT, bool SH>
static int launch_batch_t(const BArgs& a, hipStream_t st) {
    const char* who = SH ? "oom_moe_layer_decode_fp8" : "oom_moe_decode_fp8";
    const int grid = batch_grid<EQ, ODT, SH>();
    if (grid <= 0) return fail(OOM_ERR_LAUNCH, std::string(who) + ": occupancy query failed");
    hipLaunchKernelGGL((moe_batch_kernel<EQ, ODT, SH>), dim3(grid), dim3(64 * B_W), 0, st, a);
    return launched(who);
}

template <bool SH>
static int launch_batch_any(const BArgs& a, int odt, hipStream_t st) {
    if (a.E <= 128)
        return odt == OOM_BF16 ? launch_batch_t<2, OOM_BF16, SH>(a, st) : launch_batch_t<2, OOM_F32, SH>(a, st);
    return odt == OOM_BF16 ? launch_batch_t<4, OOM_BF16, SH>(a, st) : launch_batch_t<4, OOM_F32, SH>(a, st);
}

// Widths a multiple of 16 keep every 16-byte access inside its row; x 16-byte aligned.
bool batch_supported(int T, int E, int k, const OomFp8Record& g, int xdt, const void* x) {
    return T >= 2 && T <= B_T && k <= B_KMAX && E <= 256 && xdt == OOM_BF16 && g.hidden <= B_HMAX &&
           g.inter <= B_IMAX && g.hidden % 16 == 0 && g.inter % 16 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
           record_span(g) < OOB &&
           (int64_t)T * k * std::max(g.hidden, g.inter) * 4 < OOB;
}

size_t batch_workspace_size(int T, int k, const OomFp8Record& g) { return batch_ws(T, k, g).total; }

// The batch step with a shared expert of the routed geometry as one more plan entry.
bool batch_shared_supported(int T, int E, int k, const OomFp8Record& g, const OomFp8Record& sg, int xdt,
                            const void* x) {
    return batch_supported(T, E, k, g, xdt, x) && (int64_t)T * (k + 1) * std::max(g.hidden, g.inter) * 4 < OOB &&
           g.hidden == sg.hidden && g.inter == sg.inter && g.gate_weight == sg.gate_weight &&
           g.gate_scale == sg.gate_scale && g.up_weight == sg.up_weight && g.up_scale == sg.up_scale &&
           g.down_weight == sg.down_weight && g.down_scale == sg.down_scale;
}

size_t batch_shared_workspace_size(int T, int k, const OomFp8Record& g) { return batch_ws(T, k, g, true).total; }

static BArgs batch_args(const float* logits, const void* x, const uint64_t* all_recs, int T, int E, int k,
                        const OomFp8Record& g, int32_t* ids, float* weights, void* out, void* ws, bool sh) {
    const BWs w = batch_ws(T, k, g, sh);
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    BArgs a;
    a.logits = logits;
    a.x = reinterpret_cast<const uint16_t*>(x);
    a.all_recs = all_recs;
    a.T = T;
    a.E = E;
    a.k = k;
    a.H = (int)g.hidden;
    a.I = (int)g.inter;
    a.gw = (int)g.gate_weight;
    a.gs = (int)g.gate_scale;
    a.uw = (int)g.up_weight;
    a.us = (int)g.up_scale;
    a.dw = (int)g.down_weight;
    a.ds = (int)g.down_scale;
    a.rec_bytes = (int)record_span(g);
    a.ids = ids;
    a.weights = weights;
    a.out = out;
    a.h = reinterpret_cast<float*>(base + w.h);
    a.y = reinterpret_cast<float*>(base + w.y);
    a.hdr = reinterpret_cast<uint32_t*>(base);
    a.status = status_word();
    a.spin = wait_limit();
#ifdef OOM_STAMPS
    a.stamps = stamps_buffer();
#endif
    a.shared_rec = nullptr;
    a.gate_w = nullptr;
    return a;
}

int launch_batch(const float* logits, const void* x, const uint64_t* all_recs, int T, int E, int k,
                 const OomFp8Record& g, int32_t* ids, float* weights, void* out, int odt, void* ws, hipStream_t st) {
    const BArgs a = batch_args(logits, x, all_recs, T, E, k, g, ids, weights, out, ws, false);
    if (!a.status) return fail(OOM_ERR_LAUNCH, "oom_moe_decode_fp8: the device status word has no address");
    return launch_batch_any<false>(a, odt, st);
}

int launch_batch_shared(const float* logits, const void* x, const uint64_t* all_recs, int T, int E, int k,
                        const OomFp8Record& g, const uint64_t* shared_rec, const uint16_t* gate_w, int32_t* ids,
                        float* weights, void* out, int odt, void* ws, hipStream_t st) {
    BArgs a = batch_args(logits, x, all_recs, T, E, k, g, ids, weights, out, ws, true);
    if (!a.status) return fail(OOM_ERR_LAUNCH, "oom_moe_layer_decode_fp8: the device status word has no address");
    a.shared_rec = shared_rec;
    a.gate_w = gate_w;
    return launch_batch_any<true>(a, odt, st);
}

}  // namespace oom
