// One-launch decode MoE FFN step on gfx950: router top-k, routing plan, gate/up + SwiGLU,
// down projection and slot-order weighted combine in a single persistent kernel.
//
//  * Routing is recomputed by every block into LDS (one wave per token, probabilities
//    with the reference's arithmetic, picks by rank), so no block waits for another to
//    route and there is no host round trip (the reference downloads the ids and waits,
//    crates/oominf-models-qwen/src/moe.rs:308-316).
//  * Phase 1: wave-sized gate/up items (expert, intermediate rows), global wave w taking
//    items w, w + NW, ...; each streams its gate and up rows (128-bit loads) for all of
//    the expert's tokens and writes h. With one token the item is one row of each, the
//    token's activations stay in registers for the whole phase, and the loads of the
//    wave's next item are in flight while the current one is reduced.
//  * The weight loads of the wave's down items are issued early (with one token, right
//    after its first gate/up item), and the grid meets at one barrier (one arrival per
//    block): the dependency of down on h costs no HBM idle time. All blocks are
//    resident (the grid never exceeds the occupancy limit), so the barrier completes.
//  * Phase 2: wave-sized down items (expert, 8 output rows) write y. The last expert
//    to finish an output row tile (a ticket per tile, in arrival order, reset by its
//    user) combines the tile over all tokens in slot order, so results do not depend on
//    timing. With one token and at most 8 experts, block b instead takes output tiles
//    b, b + G, ... for every expert (two expert slots per wave), so a tile's expert rows
//    meet in LDS and the slot-order combine needs no y buffer, ticket or second trip
//    to memory.
//  * With a shared expert (one token, the whole decode layer): the shared record is plan
//    slot k, so its gate/up rows are phase-1 items like the routed ones; in phase 2 each
//    wave also takes one row pair of the shared expert's 16-row tile, and the combine adds
//    sigmoid(gate) times the shared row after the routed slot sum. The gate logit
//    x . gate_w is one wave's dot product during routing (x is already in its registers).
// Weights, scales and activations load through buffer resources: a lane or an item
// past the end reads zeros (out-of-range offset, or an empty resource) without a
// branch or a memory access. Counters see one arrival per block (barrier) or per
// (expert, tile) (tickets), and each counter has a 256-byte line of its own: atomics
// on one line serialise at the memory side. The kernel has exactly one grid barrier.
#include <algorithm>

#include "router.hpp"
#include "stream.hpp"

namespace oom {

constexpr int FW = 4;        // waves per block (more than one token)
constexpr int FW1 = 8;       // waves per block with one token: one expert slot each
constexpr int FD1_NP = 8;    // row pairs of a one-token down tile (16 rows)
constexpr int FG_R = 2;      // gate (and up) rows per gate/up item
constexpr int FD_R = 8;      // output rows per down item
constexpr int F_AMAX = 512;  // assignments (T * k) per step
constexpr int F_EMAX = 256;  // experts (register router; larger E takes the multi-launch path)
constexpr int F_HMAX = 4096; // hidden: 4 chunks of 1024 per lane row
constexpr int F_IMAX = 2048; // inter: 2 chunks

struct FusedArgs {
    const float* logits;
    const void* x;
    const uint64_t* all_recs;
    int T, E, k;
    int64_t H, I, gw, gs, uw, us, dw, ds;
    int32_t* ids;
    float* weights;
    void* out;
    float* h;
    float* y;
    uint32_t* tickets;   // [ceil(H / FD_R)] down items finished per row tile, TICKET_STRIDE apart
    uint32_t* bar;       // barrier: group counters, top counter, group flags (256 B apart)
    uint32_t* status;    // the device's status word: 1 if a wait gave up (results invalid)
    uint32_t spin;       // polls before a wait gives up
    int h_bytes;         // bytes of h (bounds of its buffer resource)
    int rec_bytes;       // bytes of a record up to the end of its last part
    // the shared expert (one token, SH): its record address at shared_rec[0] (same geometry
    // as the routed records), the bf16 gate row [H], and where the gate logit is handed over
    const uint64_t* shared_rec;
    const uint16_t* gate_w;
    float* gate;
#ifdef OOM_STAMPS
    uint64_t* stamps;  // phase timestamps of the one-token kernel (profiling build)
#endif
};

// 16 consecutive activations of row `row` starting at column `col`, as fp32.
template <int XDT>
__device__ __forceinline__ void load16(const void* base, size_t off, float* v) {
    if constexpr (XDT == OOM_BF16) {
        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + off);
        uint4 a = p[0], b = p[1];
        uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 a = p[i];
            v[4 * i] = a.x;
            v[4 * i + 1] = a.y;
            v[4 * i + 2] = a.z;
            v[4 * i + 3] = a.w;
        }
    }
}

struct PlanLds {
    uint64_t recs[F_EMAX + 1];  // all_recs, read once per block (+ the shared expert's record)
    uint64_t keys[FW1];     // one-token routing scratch (route_select)
    float p[FW1];
    int n_e;
    uint32_t claims;        // one token: items of this block claimed so far
    int experts[F_AMAX];
    int off[F_AMAX + 1];
    int assign_tok[F_AMAX];
    int slot_assign[F_AMAX];
    int sorted[F_AMAX];
    int ids[F_AMAX];
    float w[F_AMAX];
};

template <int TG, int XDT>
__device__ __forceinline__ void gate_up_item(const FusedArgs& a, const PlanLds& pl, int i, int tile, int lane) {
    const int H = (int)a.H, I = (int)a.I;
    const int CH = (H + 1023) >> 10, nkb = (H + 127) >> 7;
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(pl.recs[pl.experts[i]]);
    const int j0 = tile * FG_R;
    uint4 wg[FG_R][4], wu[FG_R][4];
#pragma unroll
    for (int r = 0; r < FG_R; r++) {
        const size_t row = (size_t)min(j0 + r, I - 1) * H;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int col = c * 1024 + lane * 16;
            const bool ok = c < CH && col < H;
            wg[r][c] = ok ? *reinterpret_cast<const uint4*>(rec + a.gw + row + col) : make_uint4(0, 0, 0, 0);
            wu[r][c] = ok ? *reinterpret_cast<const uint4*>(rec + a.uw + row + col) : make_uint4(0, 0, 0, 0);
        }
    }
    const float* gs = reinterpret_cast<const float*>(rec + a.gs) + (size_t)(j0 >> 7) * nkb;
    const float* us = reinterpret_cast<const float*>(rec + a.us) + (size_t)(j0 >> 7) * nkb;
    const int a_begin = pl.off[i], a_end = pl.off[i + 1];
    for (int a0 = a_begin; a0 < a_end; a0 += TG) {
        const int nb = min(TG, a_end - a0);
        float acc[TG * 2 * FG_R];  // [t][gate r0, gate r1, up r0, up r1]
#pragma unroll
        for (int q = 0; q < TG * 2 * FG_R; q++) acc[q] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            if (c >= CH) break;
            const int col = c * 1024 + lane * 16;
            const bool ok = col < H;
            const float sg = ok ? gs[col >> 7] : 0.0f, su = ok ? us[col >> 7] : 0.0f;
            if constexpr (XDT == OOM_BF16) {
                // bf16 activations: e4m3 pairs -> bf16 pairs, bf16 dot2 into fp32
#pragma unroll
                for (int t = 0; t < TG; t++) {
                    if (t >= nb) break;
                    uint32_t xw[8];
                    if (ok) {
                        const uint4* xp = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.x) +
                                                                         (size_t)pl.assign_tok[a0 + t] * H + col);
                        const uint4 x0 = xp[0], x1 = xp[1];
                        xw[0] = x0.x; xw[1] = x0.y; xw[2] = x0.z; xw[3] = x0.w;
                        xw[4] = x1.x; xw[5] = x1.y; xw[6] = x1.z; xw[7] = x1.w;
                    } else {
#pragma unroll
                        for (int q = 0; q < 8; q++) xw[q] = 0u;
                    }
#pragma unroll
                    for (int r = 0; r < FG_R; r++) {
                        acc[t * 2 * FG_R + r] = fmaf(dot16_e4m3_bf16(wg[r][c], xw), sg, acc[t * 2 * FG_R + r]);
                        acc[t * 2 * FG_R + FG_R + r] =
                            fmaf(dot16_e4m3_bf16(wu[r][c], xw), su, acc[t * 2 * FG_R + FG_R + r]);
                    }
                }
            } else {
                float f[2 * FG_R][16];
#pragma unroll
                for (int r = 0; r < FG_R; r++) {
                    e4m3x16(wg[r][c], f[r]);
                    e4m3x16(wu[r][c], f[FG_R + r]);
                }
#pragma unroll
                for (int t = 0; t < TG; t++) {
                    if (t >= nb) break;
                    float xv[16];
                    if (ok) load16<XDT>(a.x, (size_t)pl.assign_tok[a0 + t] * H + col, xv);
                    else {
#pragma unroll
                        for (int q = 0; q < 16; q++) xv[q] = 0.0f;
                    }
#pragma unroll
                    for (int r = 0; r < 2 * FG_R; r++) {
                        float p = 0.0f;
#pragma unroll
                        for (int q = 0; q < 16; q++) p = fmaf(f[r][q], xv[q], p);
                        acc[t * 2 * FG_R + r] = fmaf(p, r < FG_R ? sg : su, acc[t * 2 * FG_R + r]);
                    }
                }
            }
        }
        // value v = t * 4 + r ends in lane group v (groups of 64 / (4 TG) lanes)
        constexpr int NV = TG * 2 * FG_R, GROUP = 64 / NV;
        float tot = wave_sum_multi<NV>(acc, lane);
        const int v = lane / GROUP;
        float up = __shfl(tot, (lane + FG_R * GROUP) & 63, 64);
        if (lane % GROUP == 0 && (v % (2 * FG_R)) < FG_R) {
            const int t = v / (2 * FG_R), r = v % (2 * FG_R), j = j0 + r;
            if (t < nb && j < I) st_dev(&a.h[(size_t)(a0 + t) * I + j], siluf(tot) * up);
        }
    }
}

// The weights of down item (i, tile): 8 rows x 2 chunks of 1024 columns per lane.
struct DownW {
    uint4 w[FD_R][2];
};

__device__ __forceinline__ void down_load(const FusedArgs& a, const PlanLds& pl, int i, int tile, int lane, DownW& d) {
    const int H = (int)a.H, I = (int)a.I, CH = (I + 1023) >> 10;
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(pl.recs[pl.experts[i]]);
    const int r0 = tile * FD_R;
#pragma unroll
    for (int r = 0; r < FD_R; r++) {
        const size_t row = (size_t)min(r0 + r, H - 1) * I;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int col = c * 1024 + lane * 16;
            d.w[r][c] = (c < CH && col < I) ? *reinterpret_cast<const uint4*>(rec + a.dw + row + col)
                                            : make_uint4(0, 0, 0, 0);
        }
    }
}

// h of assignments a0 .. a0 + nb (zeros past nb) for this lane's 2 chunks of 16
// columns, through device-coherent 128-bit buffer loads.
template <int TG>
__device__ __forceinline__ void down_h_load(const FusedArgs& a, int a0, int nb, int lane, float (&hv)[TG][2][16]) {
    const int I = (int)a.I, CH = (I + 1023) >> 10;
    const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(a.h, (short)0, a.h_bytes, 0x00020000);
#pragma unroll
    for (int t = 0; t < TG; t++)
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int col = c * 1024 + lane * 16;
            if (t < nb && c < CH && col < I) {
                const int off = (int)(((size_t)(a0 + t) * I + col) * sizeof(float));
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b128(hr, off + 16 * q, 0, BUF_SC1);
                    hv[t][c][4 * q] = __uint_as_float(v[0]);
                    hv[t][c][4 * q + 1] = __uint_as_float(v[1]);
                    hv[t][c][4 * q + 2] = __uint_as_float(v[2]);
                    hv[t][c][4 * q + 3] = __uint_as_float(v[3]);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; q++) hv[t][c][q] = 0.0f;
            }
        }
}

// y[a0 + t, r0 .. r0 + FD_R) = h . Wd rows for the token group, from loaded weights and h.
template <int TG>
__device__ __forceinline__ void down_rows(const FusedArgs& a, const PlanLds& pl, int i, int tile, int lane,
                                          const DownW& d, const float (&hv)[TG][2][16], int a0, int nb) {
    const int H = (int)a.H, I = (int)a.I;
    const int CH = (I + 1023) >> 10, nkb = (I + 127) >> 7;
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(pl.recs[pl.experts[i]]);
    const int r0 = tile * FD_R;
    const float* ds = reinterpret_cast<const float*>(rec + a.ds) + (size_t)(r0 >> 7) * nkb;
    float acc[TG * FD_R];
#pragma unroll
    for (int q = 0; q < TG * FD_R; q++) acc[q] = 0.0f;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        if (c >= CH) break;
        const int col = c * 1024 + lane * 16;
        const float sd = col < I ? ds[col >> 7] : 0.0f;
#pragma unroll
        for (int r = 0; r < FD_R; r++) {
            float f[16];
            e4m3x16(d.w[r][c], f);
#pragma unroll
            for (int t = 0; t < TG; t++) {
                float p = 0.0f;
#pragma unroll
                for (int q = 0; q < 16; q++) p = fmaf(f[q], hv[t][c][q], p);
                acc[t * FD_R + r] = fmaf(p, sd, acc[t * FD_R + r]);
            }
        }
    }
    constexpr int NV = TG * FD_R, GROUP = 64 / NV;
    float tot = wave_sum_multi<NV>(acc, lane);
    const int v = lane / GROUP;
    if (lane % GROUP == 0) {
        const int t = v / FD_R, r = r0 + v % FD_R;
        if (t < nb && r < H) st_dev(&a.y[(size_t)(a0 + t) * H + r], tot);
    }
}

// Combine of output row tile `tile` for every token, in slot order, by the wave that
// took the tile's last ticket; it then resets the ticket.
template <int ODT>
__device__ __forceinline__ void combine_tile(const FusedArgs& a, const PlanLds& pl, int tile, int lane) {
    const int H = (int)a.H, r0 = tile * FD_R;
    for (int idx = lane; idx < a.T * FD_R; idx += 64) {
        const int t = idx / FD_R, r = r0 + idx % FD_R;
        if (r >= H) continue;
        float acc = 0.0f;
        for (int s = 0; s < a.k; s++)
            acc = fmaf(pl.w[t * a.k + s], ld_dev(&a.y[(size_t)pl.slot_assign[t * a.k + s] * H + r]), acc);
        store_out<ODT>(a.out, (size_t)t * H + r, acc);
    }
    if (lane == 0) __hip_atomic_store(&a.tickets[tile * TICKET_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Takes a ticket of row tile `tile` (after this wave's y stores completed); true if it
// was the tile's last (every expert's rows of the tile are in y).
__device__ __forceinline__ uint32_t take_ticket(const FusedArgs& a, int tile, int lane) {
    uint32_t old = 0;
    if (lane == 0)
        old = __hip_atomic_fetch_add(&a.tickets[tile * TICKET_STRIDE], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return old;
}

// Down item (i, tile) over all of the expert's tokens, weights already loaded.
template <int TG>
__device__ __forceinline__ void down_item(const FusedArgs& a, const PlanLds& pl, int i, int tile, int lane,
                                          const DownW& d) {
    const int a_begin = pl.off[i], a_end = pl.off[i + 1];
    for (int a0 = a_begin; a0 < a_end; a0 += TG) {
        const int nb = min(TG, a_end - a0);
        float hv[TG][2][16];
        down_h_load<TG>(a, a0, nb, lane, hv);
        down_rows<TG>(a, pl, i, tile, lane, d, hv, a0, nb);
    }
}

// ---- one token (T == 1) ------------------------------------------------------------------

// A record's parts through one buffer resource; an empty resource (bytes 0) reads zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rec_rsrc(const PlanLds& pl, int i, int bytes) {
    const uint64_t r = pl.recs[pl.experts[i]];
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)r), hi = __builtin_amdgcn_readfirstlane((uint32_t)(r >> 32));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, bytes,
                                             BUF_FLAGS);
}

// Gate/up item `it` (plan slot item_slot(it), row it % I): one gate row and one up row,
// 1024 columns per chunk, and their 128 x 128-block scales; an item past NG reads zeros.
// With a shared expert (plan slot k) its rows come first (items 0 .. I - 1: they need no
// routing, so they stream while the token is routed), then routed slot s at (s + 1) I.
struct Gate1 {
    uint4 g[4], u[4];
    float sg[4], su[4];
};

__device__ __forceinline__ int item_slot(const FusedArgs& a, int it, bool shared_first) {
    const int I = (int)a.I;
    return shared_first ? (it < I ? a.k : it / I - 1) : it / I;
}

__device__ __forceinline__ void gate1_load(const FusedArgs& a, const PlanLds& pl, int it, int NG, int lane, Gate1& w,
                                           bool shared_first = false) {
    const int H = (int)a.H, I = (int)a.I, nkb = (H + 127) >> 7;
    const bool valid = it < NG;
    const int i = valid ? item_slot(a, it, shared_first) : 0, j = valid ? it % I : 0;
    const __amdgpu_buffer_rsrc_t r = rec_rsrc(pl, i, valid ? a.rec_bytes : 0);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int col = c * 1024 + lane * 16;
        const bool ok = col < H;
        const int row = j * H + col, sc = ((j >> 7) * nkb + (col >> 7)) * 4;
        w.g[c] = ld16nt(r, ok ? (int)a.gw + row : OOB);
        w.u[c] = ld16nt(r, ok ? (int)a.uw + row : OOB);
        w.sg[c] = ldf(r, ok ? (int)a.gs + sc : OOB);
        w.su[c] = ldf(r, ok ? (int)a.us + sc : OOB);
    }
}

// h[a(it), j(it)] = silu(x . gate row) * (x . up row).
template <int XDT>
__device__ __forceinline__ void gate1_compute(const FusedArgs& a, const PlanLds& pl, int it, int NG, const Gate1& w,
                                              const XRow<XDT>& xr, int lane, bool shared_first = false) {
    float acc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        if constexpr (XDT == OOM_BF16) {
            acc[0] = fmaf(dot16_e4m3_bf16(w.g[c], xr.w[c]), w.sg[c], acc[0]);
            acc[1] = fmaf(dot16_e4m3_bf16(w.u[c], xr.w[c]), w.su[c], acc[1]);
        } else {
            float fg[16], fu[16];
            e4m3x16(w.g[c], fg);
            e4m3x16(w.u[c], fu);
            float pg = 0.0f, pu = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                pg = fmaf(fg[q], xr.v[c][q], pg);
                pu = fmaf(fu[q], xr.v[c][q], pu);
            }
            acc[0] = fmaf(pg, w.sg[c], acc[0]);
            acc[1] = fmaf(pu, w.su[c], acc[1]);
        }
    }
    // gate total in lanes 0..31, up total in lanes 32..63
    const float tot = wave_sum_multi<2>(acc, lane);
    const float up = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot), 32));
    if (lane == 0 && it < NG) {
        const int I = (int)a.I, i = item_slot(a, it, shared_first), j = it % I;
        st_dev(&a.h[(size_t)pl.off[i] * I + j], siluf(tot) * up);
    }
}

// Down item (expert i, output rows 8 t .. 8 t + 8) for one token: lanes 0..31 take rows
// 8 t + 2 p, lanes 32..63 rows 8 t + 2 p + 1 (p < 4), each lane 16 columns of each
// 512-column chunk c < DCH; one scale per chunk (the 8 rows share a 128-row block).
template <int DCH>
struct Down1 {
    uint4 w[FD1_NP][DCH];
    float s[DCH];
};

template <int DCH>
__device__ __forceinline__ void down1_load(const FusedArgs& a, const PlanLds& pl, int i, int tile, bool valid, int lane,
                                           Down1<DCH>& d) {
    const int H = (int)a.H, I = (int)a.I, nkb = (I + 127) >> 7;
    const int r0 = valid ? tile * 2 * FD1_NP : 0;
    const __amdgpu_buffer_rsrc_t r = rec_rsrc(pl, valid ? i : 0, valid ? a.rec_bytes : 0);
    const int half = lane >> 5, l = lane & 31;
#pragma unroll
    for (int c = 0; c < DCH; c++) {
        const int col = c * 512 + l * 16;
#pragma unroll
        for (int p = 0; p < FD1_NP; p++) {
            const int row = r0 + 2 * p + half;
            d.w[p][c] = ld16nt(r, row < H && col < I ? (int)a.dw + row * I + col : OOB);
        }
        d.s[c] = ldf(r, col < I ? (int)a.ds + ((r0 >> 7) * nkb + (col >> 7)) * 4 : OOB);
    }
}

// h of assignment `as` at this lane's 16 columns of each chunk (zeros past inter, or
// everywhere if !valid), through device-coherent loads. The two halves of the wave
// need the same columns: each loads 8 of the 16 and v_permlane32_swap trades them
// (the first result holds the lower half's values in every lane, the second the
// upper half's).
template <int DCH>
__device__ __forceinline__ void down1_h(const FusedArgs& a, int as, bool valid, int lane, float (&hv)[DCH][16]) {
    const int I = (int)a.I, l = lane & 31, half = lane >> 5;
    const __amdgpu_buffer_rsrc_t hr =
        __builtin_amdgcn_make_buffer_rsrc(a.h, (short)0, valid ? a.h_bytes : 0, BUF_FLAGS);
#pragma unroll
    for (int c = 0; c < DCH; c++) {
        const int col = c * 512 + l * 16;
        const int off = col < I ? (as * I + col) * 4 + half * 32 : OOB;
        uint32_t mine[8];
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(hr, off + 16 * q, 0, BUF_SC1);
            mine[4 * q] = v[0];
            mine[4 * q + 1] = v[1];
            mine[4 * q + 2] = v[2];
            mine[4 * q + 3] = v[3];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const auto r = __builtin_amdgcn_permlane32_swap(mine[j], mine[j], false, false);
            hv[c][j] = __uint_as_float(r[0]);
            hv[c][j + 8] = __uint_as_float(r[1]);
        }
    }
}

// The tile's 16 row totals: row pair p's total ends in lanes 4 p .. 4 p + 3 of each half
// (lanes 0..31: row 2 p, lanes 32..63: row 2 p + 1 of the tile).
template <int DCH>
__device__ __forceinline__ float down1_rows(const Down1<DCH>& d, const float (&hv)[DCH][16], int lane) {
    float acc[FD1_NP];
#pragma unroll
    for (int p = 0; p < FD1_NP; p++) {
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < DCH; c++) {
            float f[16];
            e4m3x16(d.w[p][c], f);
            float q0 = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; q++) q0 = fmaf(f[q], hv[c][q], q0);
            s = fmaf(q0, d.s[c], s);
        }
        acc[p] = s;
    }
    return wave_sum_multi<FD1_NP, 16>(acc, lane);
}

// One row pair of the shared expert's down tile: row 16 tile + 2 w + (lane >= 32) for wave
// w, DCH chunks of 512 columns (lane l % 32 takes 16 columns of each), read through the
// record of plan slot `slot` (the shared expert).
template <int DCH>
struct DownPair {
    uint4 w[DCH];
    float s[DCH];
};

template <int DCH>
__device__ __forceinline__ void down_pair_load(const FusedArgs& a, const PlanLds& pl, int slot, int tile, int wave,
                                               bool valid, int lane, DownPair<DCH>& d) {
    const int H = (int)a.H, I = (int)a.I, nkb = (I + 127) >> 7;
    const int row = tile * 2 * FD1_NP + 2 * wave + (lane >> 5), l = lane & 31;
    const bool ok = valid && row < H;
    const __amdgpu_buffer_rsrc_t r = rec_rsrc(pl, slot, ok ? a.rec_bytes : 0);
#pragma unroll
    for (int c = 0; c < DCH; c++) {
        const int col = c * 512 + l * 16;
        d.w[c] = ld16(r, ok && col < I ? (int)a.dw + row * I + col : OOB);
        d.s[c] = ldf(r, ok && col < I ? (int)a.ds + ((row >> 7) * nkb + (col >> 7)) * 4 : OOB);
    }
}

// The pair's row totals: row 2 w in every lane of the lower half, row 2 w + 1 in the upper.
template <int DCH>
__device__ __forceinline__ float down_pair_row(const DownPair<DCH>& d, const float (&hv)[DCH][16], int lane) {
    float s[1] = {0.0f};
#pragma unroll
    for (int c = 0; c < DCH; c++) {
        float f[16];
        e4m3x16(d.w[c], f);
        float q0 = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; q++) q0 = fmaf(f[q], hv[c][q], q0);
        s[0] = fmaf(q0, d.s[c], s[0]);
    }
    return wave_sum_multi<1, 16>(s, lane);
}

// The shared expert's gate logit x . gate_w (bf16 [H]) from the token's activations in
// registers: lane l's 16 columns of each chunk, summed over the wave.
template <int XDT>
__device__ __forceinline__ float gate_dot(const FusedArgs& a, const XRow<XDT>& xr, int lane) {
    const int H = (int)a.H;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.gate_w), (short)0,
                                                                      H * 2, BUF_FLAGS);
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int col = c * 1024 + lane * 16;
        const int off = col < H ? col * 2 : OOB;
        const uint4 g0 = ld16(r, off), g1 = ld16(r, off + 16);
        const uint32_t gw[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float x0, x1;
            if constexpr (XDT == OOM_BF16) {
                x0 = __uint_as_float(xr.w[c][i] << 16);
                x1 = __uint_as_float(xr.w[c][i] & 0xffff0000u);
            } else {
                x0 = xr.v[c][2 * i];
                x1 = xr.v[c][2 * i + 1];
            }
            p = fmaf(__uint_as_float(gw[i] << 16), x0, p);
            p = fmaf(__uint_as_float(gw[i] & 0xffff0000u), x1, p);
        }
        acc += p;
    }
    return wave_sum(acc);
}

// Grid-wide barrier over the workspace header's barrier area (stream.hpp), `base` read at
// the kernel's start. Used once per kernel.
__device__ __forceinline__ void grid_barrier(const FusedArgs& a, uint32_t base) {
    grid_barrier_words(a.bar, base, a.status, a.spin);
}

// The plan of up to 64 slots on one wave, lane s = slot s: ranks by readlane
// broadcast, no LDS round trips. Reads pl.ids, writes slot_assign, assign_tok, experts,
// off and n_e.
__device__ __forceinline__ void plan_wave(PlanLds& pl, int A, int k, int lane) {
    const int e = lane < A ? pl.ids[lane] : 0x7fffffff;
    int pos = 0, below = 0, first = 1;
    for (int j = 0; j < A; j++) {
        const int ej = __builtin_amdgcn_readlane(e, j);
        pos += (ej < e) || (ej == e && j < lane);
        below += ej < e;
        first &= !(ej == e && j < lane);
    }
    const uint64_t firsts = __ballot(lane < A && first);
    if (lane < A) {
        pl.slot_assign[lane] = pos;
        pl.assign_tok[pos] = lane / k;
        if (first) {
            // experts in id order: the rank of this first slot among first slots by id
            int eidx = 0;
            for (int j = 0; j < A; j++) {
                const int ej = __builtin_amdgcn_readlane(e, j);
                const int fj = (int)((firsts >> j) & 1ull);
                eidx += fj && ej < e;
            }
            pl.experts[eidx] = e;
            pl.off[eidx] = below;
        }
    }
    if (lane == 0) {
        const int n = (int)__builtin_popcountll(firsts);
        pl.n_e = n;
        pl.off[n] = A;
    }
}

template <int TG, int DCH, int EQ, int XDT, int ODT, bool SH = false>
__global__ void __launch_bounds__(TG == 1 ? 64 * FW1 : 64 * FW) moe_decode_fused_kernel(FusedArgs a) {
    static_assert(!SH || TG == 1, "the shared expert rides the one-token kernel");
    constexpr int WB = TG == 1 ? FW1 : FW;  // waves per block
    __shared__ PlanLds pl;
    const uint32_t bbase = grid_barrier_base(a.bar);
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if constexpr (TG == 1) {
        OOM_STAMP(a.stamps, WB, 0);
        OOM_STAMP_WHERE(a.stamps, WB);
    }
    const int T = a.T, E = a.E, k = a.k, A = T * k;
    // one token: the routing wave's logits go out first, so its wait for them is one round
    // trip behind nothing else; the record table (copied by the other waves: its LDS
    // stores wait for their loads) and the activations load while the router runs
    float lv0[EQ];
    if constexpr (TG == 1) {
        if (T == 1 && wave == 0) route_logits<EQ>(a.logits, E, lane, lv0);
    }
    constexpr int RT0 = TG == 1 ? 64 : 0;  // first thread of the record-table copy
    static_assert(TG != 1 || 64 * FW1 >= 64 + F_EMAX + 1, "the other waves hold the record table");
    if (tid >= RT0 && tid - RT0 < E) pl.recs[tid - RT0] = a.all_recs[tid - RT0];
    if constexpr (SH) {
        if (tid == RT0 + E) pl.recs[E] = a.shared_rec[0];
        if (tid == 64) {
            // plan slot k, the shared expert (record E of the table, h row k), and the
            // claim counter: set before routing, so the shared rows can stream meanwhile
            pl.experts[k] = E;
            pl.off[k] = k;
            pl.off[k + 1] = k + 1;
            pl.claims = 0u;
        }
    }
    XRow<XDT> xr;
    if constexpr (TG == 1) xrow_load<XDT>(a.x, (int)a.H, lane, xr);
    // one token with a shared expert: the waves other than the router's claim their first
    // item now, and one of the shared expert's rows starts streaming before routing ends
    // (LDS-only block syncs here and after routing: a __syncthreads would wait for those
    // loads)
    int it_pre = 0;
    Gate1 w0, w1;  // one-token phase 1: the wave's current and next gate/up item
    if constexpr (SH) {
        lds_barrier();  // the record table and the shared slot's plan entries
        if (wave != 0) {
            uint32_t c = 0;
            if (lane == 0) c = __hip_atomic_fetch_add(&pl.claims, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            c = __builtin_amdgcn_readfirstlane(c);
            it_pre = (int)(blockIdx.x + c * gridDim.x);
            if (it_pre < (int)a.I) gate1_load(a, pl, it_pre, (int)a.I, lane, w0, true);
        }
    }
    // ---- routing and plan: slots sorted by (expert, slot), experts in id order ----
    if (T == 1) {
        // one token: wave 0 routes it and plans in place, one block-wide sync
        if (wave == 0) {
            // picks and plan in one pass (ballot radix selection); with one token the
            // plan's assignment i is expert slot i
            route_select<EQ>(lv0, E, k, lane, pl.keys, pl.p, pl.experts, pl.ids, pl.w, pl.slot_assign);
            if (lane < k) {
                pl.off[lane] = lane;
                pl.assign_tok[lane] = 0;
            }
            if (lane == 0) {
                pl.n_e = k;
                pl.off[k] = k;
                if constexpr (!SH) pl.claims = 0u;  // with a shared expert: set before routing
            }
        }
        if constexpr (SH) {
            // while wave 0 routes, wave 1 of block 0 takes the shared expert's gate logit
            if (blockIdx.x == 0 && wave == 1) {
                const float g = gate_dot<XDT>(a, xr, lane);
                if (lane == 0) st_dev(a.gate, g);
            }
        }
    } else {
        for (int t = wave; t < T; t += FW) {
            int id = 0;
            float w = 0.0f;
            route_token_regs(a.logits + (size_t)t * E, E, k, lane, id, w);
            if (lane < k) {
                pl.ids[t * k + lane] = id;
                pl.w[t * k + lane] = w;
            }
        }
        __syncthreads();
        if (A <= 64) {
            if (wave == 0) plan_wave(pl, A, k, lane);
        } else {
            for (int s = tid; s < A; s += blockDim.x) {
                const int e = pl.ids[s];
                int pos = 0;
                for (int s2 = 0; s2 < A; s2++) {
                    const int e2 = pl.ids[s2];
                    pos += (e2 < e) || (e2 == e && s2 < s);
                }
                pl.sorted[pos] = e;
                pl.slot_assign[s] = pos;
                pl.assign_tok[pos] = s / k;
            }
            __syncthreads();
            for (int p = tid; p < A; p += blockDim.x) {
                if (p == 0 || pl.sorted[p - 1] != pl.sorted[p]) {
                    int idx = 0;
                    for (int q = 1; q <= p; q++) idx += pl.sorted[q - 1] != pl.sorted[q];
                    pl.experts[idx] = pl.sorted[p];
                    pl.off[idx] = p;
                }
                if (p == A - 1) {
                    int n = 1;
                    for (int q = 1; q < A; q++) n += pl.sorted[q - 1] != pl.sorted[q];
                    pl.n_e = n;
                    pl.off[n] = A;
                }
            }
        }
    }
    if constexpr (SH) lds_barrier();
    else __syncthreads();
    if constexpr (TG == 1) OOM_STAMP(a.stamps, WB, 1);  // routed and planned
    if (blockIdx.x == 0)
        for (int s = tid; s < A; s += blockDim.x) {
            a.ids[s] = pl.ids[s];
            a.weights[s] = pl.w[s];
        }
    const int n_e = pl.n_e;
    const int NW = gridDim.x * WB, gwave = blockIdx.x * WB + wave;
    const int tiles_d = (int)((a.H + FD_R - 1) / FD_R), ND = n_e * tiles_d;
    if constexpr (TG == 1) {
        // ---- phase 1, one token: item it = (expert it / I, row it % I); the next item's
        // loads are in flight while the current one is reduced ----
        const int NG = (n_e + (SH ? 1 : 0)) * (int)a.I;  // the shared expert's rows first
        // Block b owns items b WB + c % WB + (c / WB) NW (c = 0, 1, ...; with the shared
        // expert b + c G, so that every block holds the same number of items to one and
        // starts on shared rows); its waves claim them in that order from a counter in LDS,
        // so a wave that gets fewer issue slots (the second wave of a SIMD) takes fewer
        // items than its partner.
        auto claim = [&]() -> int {
            uint32_t c = 0;
            if (lane == 0) c = __hip_atomic_fetch_add(&pl.claims, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            c = __builtin_amdgcn_readfirstlane(c);
            if constexpr (SH) return (int)(blockIdx.x + c * gridDim.x);
            else return (int)(blockIdx.x * WB + c % WB + (c / WB) * NW);
        };
        int it0;
        if constexpr (SH) {
            // the router's wave claims now; a wave whose first item is a routed row loads it now
            it0 = wave == 0 ? claim() : it_pre;
            if (wave == 0 || it_pre >= (int)a.I) gate1_load(a, pl, it0, NG, lane, w0, true);
        } else {
            it0 = claim();
            gate1_load(a, pl, it0, NG, lane, w0);
        }
        // this block's first 16-row output tile of the wave's expert slot (one slot per
        // wave) streams behind the wave's first gate/up item: block b takes tiles b,
        // b + G, ... for all (<= 8) experts
        const int s0 = wave, tb0 = blockIdx.x, tiles1 = (int)((a.H + 2 * FD1_NP - 1) / (2 * FD1_NP));
        Down1<DCH> d0;
        down1_load<DCH>(a, pl, s0, tb0, s0 < n_e && tb0 < tiles1, lane, d0);
        while (it0 < NG) {
            const int it1 = claim();
            gate1_load(a, pl, it1, NG, lane, w1, SH);
            gate1_compute<XDT>(a, pl, it0, NG, w0, xr, lane, SH);
            if (it1 >= NG) break;
            it0 = claim();
            gate1_load(a, pl, it0, NG, lane, w0, SH);
            gate1_compute<XDT>(a, pl, it1, NG, w1, xr, lane, SH);
        }
        OOM_STAMP(a.stamps, WB, 2);  // gate/up items done, down weights in flight or in
        wait_mem();  // this wave's h stores (and loads) are complete before its block arrives
        grid_barrier(a, bbase);
        OOM_STAMP(a.stamps, WB, 3);  // the grid barrier released
        // ---- phase 2, one token: the slot's h once, then per tile the 16 rows of each
        // expert into LDS and the slot-order combine by wave 0 ----
        __shared__ float ylds[FW1][2 * FD1_NP];
        __shared__ float ysh[2 * FD1_NP];
        float h0[DCH][16];
        down1_h<DCH>(a, pl.off[s0 < n_e ? s0 : 0], s0 < n_e, lane, h0);
        float hs[DCH][16];
        float sg = 0.0f;
        DownPair<DCH> p0;
        if constexpr (SH) {
            // the shared row pair's weights load after the barrier (3 loads a lane), out of
            // phase 1's register budget
            down_pair_load<DCH>(a, pl, k, tb0, wave, tb0 < tiles1, lane, p0);
            down1_h<DCH>(a, k, true, lane, hs);
            if (wave == 0) sg = 1.0f / (1.0f + expf(-ld_dev(a.gate)));  // sigmoid (ops.cu:10)
        }
        const int prow = 2 * ((lane & 31) >> 2) + (lane >> 5);  // this lane group's row in the tile
        for (int tb = tb0; tb < tiles1; tb += gridDim.x) {
            if (tb != tb0) {
                down1_load<DCH>(a, pl, s0, tb, s0 < n_e, lane, d0);
                if constexpr (SH) down_pair_load<DCH>(a, pl, k, tb, wave, true, lane, p0);
            }
            if (tb == tb0) OOM_STAMP_AFTER(a.stamps, WB, 4, h0[DCH - 1][15]);  // the slot's h in
            const float y0 = down1_rows<DCH>(d0, h0, lane);
            if (tb == tb0) OOM_STAMP_AFTER(a.stamps, WB, 5, y0);  // the tile's rows of the wave's slot
            if ((lane & 3) == 0) ylds[s0][prow] = y0;
            if constexpr (SH) {
                const float ys = down_pair_row<DCH>(p0, hs, lane);
                if ((lane & 31) == 0) ysh[2 * wave + (lane >> 5)] = ys;
            }
            __syncthreads();
            // out[r] = sum over slots in order of w[s] * y[slot_assign[s]][r]; with one
            // token, assignment i is expert slot i
            const int r = tb * 2 * FD1_NP + lane;
            if (wave == 0 && lane < 2 * FD1_NP && r < (int)a.H) {
                float acc = 0.0f;
                for (int s = 0; s < k; s++) acc = fmaf(pl.w[s], ylds[pl.slot_assign[s]][lane], acc);
                // the shared expert after the routed sum: routed + sigmoid(gate) * shared
                // (moe_combine, ops.cu:310-316)
                if constexpr (SH) acc = acc + sg * ysh[lane];
                store_out<ODT>(a.out, r, acc);
            }
            __syncthreads();
        }
        OOM_STAMP(a.stamps, WB, 6);  // combined and stored
    } else {
        // ---- phase 1: gate/up + SwiGLU -> h, FG_R rows per item, tokens in groups of TG ----
        const int tiles_g = (int)((a.I + FG_R - 1) / FG_R), NG = n_e * tiles_g;
        for (int it = gwave; it < NG; it += NW) gate_up_item<TG, XDT>(a, pl, it / tiles_g, it % tiles_g, lane);
        wait_mem();  // this wave's h stores are complete before its block arrives
        // ---- the first down item's weights stream while the grid meets ----
        DownW d;
        if (gwave < ND) down_load(a, pl, gwave / tiles_d, gwave % tiles_d, lane, d);
        grid_barrier(a, bbase);
        // ---- phase 2: down projection -> y, then the ticketed slot-order combine ----
        for (int it = gwave; it < ND; it += NW) {
            if (it != gwave) down_load(a, pl, it / tiles_d, it % tiles_d, lane, d);
            down_item<TG>(a, pl, it / tiles_d, it % tiles_d, lane, d);
            wait_mem();
            if ((uint32_t)__builtin_amdgcn_readlane((int)take_ticket(a, it % tiles_d, lane), 0) == (uint32_t)n_e - 1)
                combine_tile<ODT>(a, pl, it % tiles_d, lane);
        }
    }
    grid_barrier_exit(a.bar);
}

// ---- host side -----------------------------------------------------------------------

static size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

// h and y follow the workspace header, which holds the barrier words, the tickets and
// the status word (the state a call leaves for the next).
struct FusedWs {
    size_t h, y, total;
};

static FusedWs fused_ws(int T, int E, int k, const OomFp8Record& g) {
    FusedWs w;
    size_t A = (size_t)T * k;
    w.h = WS_HEADER;
    w.y = w.h + al256((A + 1) * (size_t)g.inter * sizeof(float));  // + a shared expert's h row
    w.total = w.y + al256(A * (size_t)g.hidden * sizeof(float));
    return w;
}

bool fused_supported(int T, int E, int k, const OomFp8Record& g) {
    return (int64_t)T * k <= F_AMAX && E <= F_EMAX && g.hidden <= F_HMAX && g.inter <= F_IMAX && T <= 64 &&
           record_span(g) < OOB && cdiv(g.hidden, FD_R) <= MAX_TILES;
}

size_t fused_workspace_size(int T, int E, int k, const OomFp8Record& g) { return fused_ws(T, E, k, g).total; }

// Blocks of the fused kernel that fit on the device at once (all must be resident).
template <int TG, int DCH, int EQ, int XDT, int ODT, bool SH>
static int resident_blocks(int dev, size_t lds) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, moe_decode_fused_kernel<TG, DCH, EQ, XDT, ODT, SH>,
                                                     TG == 1 ? 64 * FW1 : 64 * FW, lds) !=
        hipSuccess)
        return 0;
    return cus * per;
}

template <int TG, int DCH, int EQ, int XDT, int ODT, bool SH = false>
static int launch_fused_t(const FusedArgs& a, size_t lds, hipStream_t st) {
    static thread_local int cached_dev = -1, cached_blocks = 0;
    static thread_local size_t cached_lds = 0;
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != cached_dev || lds != cached_lds) {
        cached_blocks = resident_blocks<TG, DCH, EQ, XDT, ODT, SH>(dev, lds);
        cached_dev = dev;
        cached_lds = lds;
    }
    if (cached_blocks <= 0) return fail(OOM_ERR_LAUNCH, "oom_moe_decode_fp8: occupancy query failed");
    if (!a.status) return fail(OOM_ERR_LAUNCH, "oom_moe_decode_fp8: the device status word has no address");
    // never more waves than items (at most min(E, A) experts' worth)
    const int wb = TG == 1 ? FW1 : FW;
    const int64_t items =
        ((int64_t)std::min(a.E, a.T * a.k) + (SH ? 1 : 0)) * (cdiv(a.I, TG == 1 ? 1 : FG_R) + cdiv(a.H, FD_R));
    const int blocks = (int)std::max<int64_t>(1, std::min<int64_t>(cached_blocks, cdiv(items, wb)));
    hipLaunchKernelGGL((moe_decode_fused_kernel<TG, DCH, EQ, XDT, ODT, SH>), dim3(blocks), dim3(64 * wb), lds, st, a);
    return launched("oom_moe_decode_fp8");
}

static FusedArgs fused_args(const float* logits, const void* x, const uint64_t* all_recs, int T, int E, int k,
                            const OomFp8Record& g, int32_t* ids, float* weights, void* out, void* ws) {
    FusedWs w = fused_ws(T, E, k, g);
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    FusedArgs a;
    a.logits = logits;
    a.x = x;
    a.all_recs = all_recs;
    a.T = T;
    a.E = E;
    a.k = k;
    a.H = g.hidden;
    a.I = g.inter;
    a.gw = g.gate_weight;
    a.gs = g.gate_scale;
    a.uw = g.up_weight;
    a.us = g.up_scale;
    a.dw = g.down_weight;
    a.ds = g.down_scale;
    a.ids = ids;
    a.weights = weights;
    a.out = out;
    a.h = reinterpret_cast<float*>(base + w.h);
    a.y = reinterpret_cast<float*>(base + w.y);
    a.tickets = reinterpret_cast<uint32_t*>(base + WS_TICKETS);
    a.bar = reinterpret_cast<uint32_t*>(base + WS_BAR);
    a.status = status_word();
    a.spin = wait_limit();
    a.h_bytes = (int)((size_t)T * k * g.inter * sizeof(float));
    a.rec_bytes = (int)record_span(g);
    a.shared_rec = nullptr;
    a.gate_w = nullptr;
    a.gate = nullptr;
#ifdef OOM_STAMPS
    a.stamps = stamps_buffer();
#endif
    return a;
}

int launch_fused(const float* logits, const void* x, int xdt, const uint64_t* all_recs, int T, int E, int k,
                 const OomFp8Record& g, int32_t* ids, float* weights, void* out, int odt, void* ws, hipStream_t st) {
    const FusedArgs a = fused_args(logits, x, all_recs, T, E, k, g, ids, weights, out, ws);
    const size_t lds = 0;
#define FUSED_CASE(TG, DCH, EQ)                                                                               \
    if (xdt == OOM_BF16 && odt == OOM_BF16) return launch_fused_t<TG, DCH, EQ, OOM_BF16, OOM_BF16>(a, lds, st); \
    if (xdt == OOM_BF16 && odt == OOM_F32) return launch_fused_t<TG, DCH, EQ, OOM_BF16, OOM_F32>(a, lds, st);   \
    if (xdt == OOM_F32 && odt == OOM_BF16) return launch_fused_t<TG, DCH, EQ, OOM_F32, OOM_BF16>(a, lds, st);   \
    return launch_fused_t<TG, DCH, EQ, OOM_F32, OOM_F32>(a, lds, st);
    // one token routed to at most FW1 experts: TG 1 with 512-column down chunks for the
    // inter width; otherwise groups of 4 tokens per pass over an item's weights
    if (T == 1 && k <= FW1) {
        if (E <= 128) {
            if (g.inter <= 1024) {
                FUSED_CASE(1, 2, 2)
            } else if (g.inter <= 1536) {
                FUSED_CASE(1, 3, 2)
            } else {
                FUSED_CASE(1, 4, 2)
            }
        } else {
            if (g.inter <= 1024) {
                FUSED_CASE(1, 2, 4)
            } else if (g.inter <= 1536) {
                FUSED_CASE(1, 3, 4)
            } else {
                FUSED_CASE(1, 4, 4)
            }
        }
    } else {
        FUSED_CASE(4, 0, 4)
    }
#undef FUSED_CASE
}

// One token through the one-token kernel with a shared expert of the routed geometry as
// plan slot k: out = sum_s w_s y_s + sigmoid(x . gate_w) * y_shared. The gate logit is
// handed over at `gate` (device memory the caller owns). bf16 activations only.
bool fused_shared_supported(int T, int E, int k, const OomFp8Record& g, const OomFp8Record& sg, int xdt) {
    // inter <= 1536: with 2048 the two h rows and a down tile pass the register budget
    return T == 1 && k <= FW1 && xdt == OOM_BF16 && g.inter <= 1536 && fused_supported(T, E, k, g) &&
           g.hidden == sg.hidden &&
           g.inter == sg.inter && g.gate_weight == sg.gate_weight && g.gate_scale == sg.gate_scale &&
           g.up_weight == sg.up_weight && g.up_scale == sg.up_scale && g.down_weight == sg.down_weight &&
           g.down_scale == sg.down_scale;
}

int launch_fused_shared(const float* logits, const void* x, const uint64_t* all_recs, int E, int k,
                        const OomFp8Record& g, const uint64_t* shared_rec, const uint16_t* gate_w, float* gate,
                        int32_t* ids, float* weights, void* out, int odt, void* ws, hipStream_t st) {
    FusedArgs a = fused_args(logits, x, all_recs, 1, E, k, g, ids, weights, out, ws);
    a.shared_rec = shared_rec;
    a.gate_w = gate_w;
    a.gate = gate;
    a.h_bytes = (int)((size_t)(k + 1) * g.inter * sizeof(float));
    const size_t lds = 0;
#define FUSED_SH_CASE(DCH, EQ)                                                                                  \
    return odt == OOM_BF16 ? launch_fused_t<1, DCH, EQ, OOM_BF16, OOM_BF16, true>(a, lds, st)                  \
                           : launch_fused_t<1, DCH, EQ, OOM_BF16, OOM_F32, true>(a, lds, st);
    if (E <= 128) {
        if (g.inter <= 1024) {
            FUSED_SH_CASE(2, 2)
        } else {
            FUSED_SH_CASE(3, 2)
        }
    } else {
        if (g.inter <= 1024) {
            FUSED_SH_CASE(2, 4)
        } else {
            FUSED_SH_CASE(3, 4)
        }
    }
#undef FUSED_SH_CASE
}

}  // namespace oom
