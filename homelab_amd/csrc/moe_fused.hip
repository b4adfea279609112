// One-launch decode MoE FFN step on gfx950: router top-k, routing plan, gate/up + SwiGLU,
// down projection and slot-order weighted combine in a single persistent kernel.
//
//  * Routing is recomputed by every block into LDS (one wave per token, probabilities
//    with the reference's arithmetic, picks by rank), so no block waits for another to
//    route and there is no host round trip (the reference downloads the ids and waits,
//    crates/oominf-models-qwen/src/moe.rs:308-316).
//  * Phase 1: wave-sized gate/up items (expert, 2 intermediate rows), global wave w
//    taking items w, w + NW, ...; each streams its gate and up rows (128-bit loads, all
//    in flight before use) for all of the expert's tokens and writes h.
//  * Each wave then issues the weight loads of its first down item, and the grid meets
//    at one barrier (one arrival per block, sense-reversing, so it needs no reset): the
//    dependency of down on h costs no HBM idle time. All blocks are resident (the grid
//    never exceeds the occupancy limit), so the barrier always completes.
//  * Phase 2: wave-sized down items (expert, 8 output rows) write y. The last expert
//    to finish an output row tile (a ticket per tile, in arrival order, reset by its
//    user) combines the tile over all tokens in slot order, so results do not depend on
//    timing. With one token, a wave takes both tickets of its two items together.
// Counters see one arrival per block (barrier) or per (expert, tile) (tickets):
// same-address atomics from every wave serialise at the memory side. The kernel has
// exactly one grid barrier.
#include "router.hpp"

namespace oom {

constexpr int FW = 4;        // waves per block
constexpr int FG_R = 2;      // gate (and up) rows per gate/up item
constexpr int FD_R = 8;      // output rows per down item
constexpr int F_AMAX = 512;  // assignments (T * k) per step
constexpr int F_EMAX = 256;  // experts (register router; larger E takes the multi-launch path)
constexpr int F_HMAX = 4096; // hidden: 4 chunks of 1024 per lane row
constexpr int F_IMAX = 2048; // inter: 2 chunks
// down items per wave whose weights load before the barrier (one token per expert: 2)
template <int TG>
constexpr int prefetch_items() { return TG == 1 ? 2 : 1; }
constexpr uint32_t F_SPIN_LIMIT = 1u << 22;
constexpr int BAR_GROUPS = 8;   // barrier groups (one per XCD)
constexpr int BAR_STRIDE = 64;  // u32 words between counters: one 256-byte line each

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
    uint32_t* tickets;   // [ceil(H / FD_R)] down items finished per row tile
    uint32_t* bar;       // barrier: group counters, top counter, group flags (256 B apart)
    uint32_t* status;    // 1 if a wait gave up (results invalid)
    int h_bytes;         // bytes of h (bounds of its buffer resource)
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

// Values handed between waves of different XCDs inside the kernel (h, y) move with
// device-coherent (sc1) dword stores and loads, which skip the per-XCD L2 instead of
// writing it back or invalidating it: an agent-scope fence lowers to buffer_wbl2 /
// buffer_inv of the whole L2, far too costly per work item. A producer waits for its
// stores (s_waitcnt) before it bumps the counter a consumer polls.
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Cache-policy bit of buffer loads for a device-coherent (sc1) access on gfx950.
constexpr int BUF_SC1 = 16;

// All of this wave's memory operations complete (stores acknowledged) before the next.
__device__ __forceinline__ void wait_mem() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

struct PlanLds {
    int n_e;
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
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(a.all_recs[pl.experts[i]]);
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
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(a.all_recs[pl.experts[i]]);
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
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(a.all_recs[pl.experts[i]]);
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
    if (lane == 0) __hip_atomic_store(&a.tickets[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Takes a ticket of row tile `tile` (after this wave's y stores completed); true if it
// was the tile's last (every expert's rows of the tile are in y).
__device__ __forceinline__ uint32_t take_ticket(const FusedArgs& a, int tile, int lane) {
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(&a.tickets[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Grid-wide barrier, one arrival per block, in two levels so no counter sees more
// than 64 arrivals: block b arrives at group b % G (G = 8, one group per XCD under
// round-robin dispatch); the last of a group arrives at the top counter; the last of
// those publishes the next generation in every group's generation word, which that
// group's blocks poll. Counters are reset by their last arrival and generations only
// grow, so nothing needs clearing between calls. Used once per kernel.
__device__ __forceinline__ void grid_barrier(const FusedArgs& a) {
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t G = min(gridDim.x, (uint32_t)BAR_GROUPS), g = blockIdx.x % G;
        const uint32_t n_g = (gridDim.x - g + G - 1) / G;
        uint32_t* cnt = a.bar + g * BAR_STRIDE;
        uint32_t* genw = a.bar + (BAR_GROUPS + 1 + g) * BAR_STRIDE;
        uint32_t* top = a.bar + BAR_GROUPS * BAR_STRIDE;
        // the generation is read before this block arrives, and waited for: memory
        // operations to different addresses may be performed out of order, and a read
        // after the last arrival would see the next generation and wait for one more
        const uint32_t gen = __hip_atomic_load(genw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wait_mem();
        const uint32_t target = gen + 1u;
        bool released = false;
        if (__hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_g - 1) {
            __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wait_mem();
            if (__hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1) {
                __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wait_mem();
                for (uint32_t q = 0; q < G; q++)
                    __hip_atomic_store(a.bar + (BAR_GROUPS + 1 + q) * BAR_STRIDE, target, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                wait_mem();
                released = true;
            }
        }
        if (!released) {
            uint32_t spins = 0;
            while ((int32_t)(__hip_atomic_load(genw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
                __builtin_amdgcn_s_sleep(4);
                if (++spins > F_SPIN_LIMIT) {
                    __hip_atomic_store(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    __syncthreads();
}

template <int TG, int XDT, int ODT>
__global__ void __launch_bounds__(256) moe_decode_fused_kernel(FusedArgs a) {
    __shared__ PlanLds pl;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
    const int T = a.T, E = a.E, k = a.k, A = T * k;
    // ---- routing (every block) ----
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
    // ---- plan: slots sorted by (expert, slot); experts in id order ----
    if (A <= 64) {
        // one wave, lane s = slot s: ranks by readlane broadcast, no LDS round trips
        if (wave == 0) {
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
    __syncthreads();
    if (blockIdx.x == 0)
        for (int s = tid; s < A; s += blockDim.x) {
            a.ids[s] = pl.ids[s];
            a.weights[s] = pl.w[s];
        }
    const int n_e = pl.n_e;
    const int tiles_g = (int)((a.I + FG_R - 1) / FG_R), tiles_d = (int)((a.H + FD_R - 1) / FD_R);
    const int NG = n_e * tiles_g, ND = n_e * tiles_d;
    const int NW = gridDim.x * FW, gwave = blockIdx.x * FW + wave;
    // ---- phase 1: gate/up + SwiGLU -> h ----
    for (int it = gwave; it < NG; it += NW) gate_up_item<TG, XDT>(a, pl, it / tiles_g, it % tiles_g, lane);
    wait_mem();  // this wave's h stores are complete before its block arrives
    // ---- the first down items' weights stream while the grid meets ----
    constexpr int PF = prefetch_items<TG>();
    DownW d[PF];
#pragma unroll
    for (int p = 0; p < PF; p++) {
        const int it = gwave + p * NW;
        if (it < ND) down_load(a, pl, it / tiles_d, it % tiles_d, lane, d[p]);
    }
    grid_barrier(a);
    // ---- phase 2: down projection -> y, then the ticketed slot-order combine ----
    if constexpr (TG == 1) {
        // one token: h of both prefetched items in flight together, tickets taken together
        float hv[PF][1][2][16];
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int it = gwave + p * NW;
            const int i = it < ND ? it / tiles_d : 0;
            down_h_load<1>(a, pl.off[i], it < ND ? 1 : 0, lane, hv[p]);
        }
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int it = gwave + p * NW;
            if (it < ND) down_rows<1>(a, pl, it / tiles_d, it % tiles_d, lane, d[p], hv[p], pl.off[it / tiles_d], 1);
        }
        wait_mem();
        uint32_t old[PF];
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int it = gwave + p * NW;
            old[p] = it < ND ? take_ticket(a, it % tiles_d, lane) : 0u;
        }
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int it = gwave + p * NW;
            if (it < ND && __shfl(old[p], 0, 64) == (uint32_t)n_e - 1) combine_tile<ODT>(a, pl, it % tiles_d, lane);
        }
    } else {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int it = gwave + p * NW;
            if (it < ND) {
                down_item<TG>(a, pl, it / tiles_d, it % tiles_d, lane, d[p]);
                wait_mem();
                if (__shfl(take_ticket(a, it % tiles_d, lane), 0, 64) == (uint32_t)n_e - 1)
                    combine_tile<ODT>(a, pl, it % tiles_d, lane);
            }
        }
    }
    for (int it = gwave + PF * NW; it < ND; it += NW) {
        down_load(a, pl, it / tiles_d, it % tiles_d, lane, d[0]);
        down_item<TG>(a, pl, it / tiles_d, it % tiles_d, lane, d[0]);
        wait_mem();
        if (__shfl(take_ticket(a, it % tiles_d, lane), 0, 64) == (uint32_t)n_e - 1)
            combine_tile<ODT>(a, pl, it % tiles_d, lane);
    }
}

// ---- host side -----------------------------------------------------------------------

static size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

struct FusedWs {
    size_t h, y, tickets, bar, status, total;
};

static FusedWs fused_ws(int T, int E, int k, const OomFp8Record& g) {
    FusedWs w;
    size_t A = (size_t)T * k;
    w.h = 0;
    w.y = al256(A * (size_t)g.inter * sizeof(float));
    w.tickets = w.y + al256(A * (size_t)g.hidden * sizeof(float));
    w.bar = w.tickets + al256((size_t)cdiv(g.hidden, FD_R) * sizeof(uint32_t));
    w.status = w.bar + (2 * BAR_GROUPS + 1) * BAR_STRIDE * sizeof(uint32_t);
    w.total = w.status + 256;
    return w;
}

bool fused_supported(int T, int E, int k, const OomFp8Record& g) {
    return (int64_t)T * k <= F_AMAX && E <= F_EMAX && g.hidden <= F_HMAX && g.inter <= F_IMAX && T <= 64;
}

size_t fused_workspace_size(int T, int E, int k, const OomFp8Record& g) { return fused_ws(T, E, k, g).total; }

// Blocks of the fused kernel that fit on the device at once (all must be resident).
template <int TG, int XDT, int ODT>
static int resident_blocks(int dev, size_t lds) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, moe_decode_fused_kernel<TG, XDT, ODT>, 256, lds) !=
        hipSuccess)
        return 0;
    return cus * per;
}

template <int TG, int XDT, int ODT>
static int launch_fused_t(const FusedArgs& a, size_t lds, hipStream_t st) {
    static thread_local int cached_dev = -1, cached_blocks = 0;
    static thread_local size_t cached_lds = 0;
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != cached_dev || lds != cached_lds) {
        cached_blocks = resident_blocks<TG, XDT, ODT>(dev, lds);
        cached_dev = dev;
        cached_lds = lds;
    }
    if (cached_blocks <= 0) return fail(OOM_ERR_LAUNCH, "oom_moe_decode_fp8: occupancy query failed");
    // never more waves than items (at most min(E, A) experts' worth)
    const int64_t items = (int64_t)std::min(a.E, a.T * a.k) * (cdiv(a.I, FG_R) + cdiv(a.H, FD_R));
    const int blocks = (int)std::max<int64_t>(1, std::min<int64_t>(cached_blocks, cdiv(items, FW)));
    hipLaunchKernelGGL((moe_decode_fused_kernel<TG, XDT, ODT>), dim3(blocks), dim3(256), lds, st, a);
    return launched("oom_moe_decode_fp8");
}

int launch_fused(const float* logits, const void* x, int xdt, const uint64_t* all_recs, int T, int E, int k,
                 const OomFp8Record& g, int32_t* ids, float* weights, void* out, int odt, void* ws, hipStream_t st) {
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
    a.tickets = reinterpret_cast<uint32_t*>(base + w.tickets);
    a.bar = reinterpret_cast<uint32_t*>(base + w.bar);
    a.status = reinterpret_cast<uint32_t*>(base + w.status);
    a.h_bytes = (int)((size_t)T * k * g.inter * sizeof(float));
    const size_t lds = 0;
#define FUSED_CASE(TG)                                                                          \
    if (xdt == OOM_BF16 && odt == OOM_BF16) return launch_fused_t<TG, OOM_BF16, OOM_BF16>(a, lds, st); \
    if (xdt == OOM_BF16 && odt == OOM_F32) return launch_fused_t<TG, OOM_BF16, OOM_F32>(a, lds, st);   \
    if (xdt == OOM_F32 && odt == OOM_BF16) return launch_fused_t<TG, OOM_F32, OOM_BF16>(a, lds, st);   \
    return launch_fused_t<TG, OOM_F32, OOM_F32>(a, lds, st);
    // one token: TG 1; more: groups of 4 tokens per pass over an item's weights
    if (T == 1) {
        FUSED_CASE(1)
    } else {
        FUSED_CASE(4)
    }
#undef FUSED_CASE
}

}  // namespace oom
