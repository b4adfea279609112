// Router top-k and the device routing plan.
#include "router.hpp"

namespace oom {

// Experts up to which the plan ranks slots with ballots and per-wave LDS counts.
constexpr int PLAN_FAST_E = 512;

// One wave per token (grid T, block 64, dynamic LDS E floats).
__global__ void __launch_bounds__(64) router_topk_kernel(const float* __restrict__ logits, int32_t* __restrict__ ids,
                                                         float* __restrict__ weights, int E, int k) {
    extern __shared__ float probs[];
    int t = blockIdx.x, lane = threadIdx.x;
    int id = 0;
    float w = 0.0f;
    if (E <= 256) route_token_regs<4>(logits + (size_t)t * E, E, k, lane, id, w);
    else if (E <= 512) route_token_regs<8>(logits + (size_t)t * E, E, k, lane, id, w);
    else route_token_wave(logits + (size_t)t * E, E, k, probs, lane, id, w);
    if (lane < k) {
        ids[(size_t)t * k + lane] = id;
        weights[(size_t)t * k + lane] = w;
    }
}

// Block-wide exclusive scan of one int per thread (a block of whole waves, at most 16).
__device__ int block_exclusive_scan(int v, int* warp_tot, int& total) {
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int n = __shfl_up(incl, o, 64);
        if (lane >= o) incl += n;
    }
    if (lane == 63) warp_tot[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < nw; w++) {
        int c = warp_tot[w];
        if (w < wave) before += c;
        all += c;
    }
    __syncthreads();
    total = all;
    return before + incl - v;
}

// The routing plan of crates/oominf-models-qwen/src/moe.rs:539-582,638-649 with every
// expert resident: slots grouped by expert in id order, each expert's slots in slot
// order. One block of 1024 threads (16 waves).
//
// E <= PLAN_FAST_E: wave w owns the contiguous slots [w C, w C + C), C = A / 16 rounded up
// to whole rounds of 64. Within a round, the lanes holding the same id find each other by
// ballots over the id's bits (rank = peers below this lane, the lowest peer leads).
// Pass 1 counts each id over the wave's slots into its row of wcnt[16][E] (the leader adds
// the round's count); the column sums are the experts' counts, from which the experts,
// offsets and start[e] follow; one scan down each column turns the rows into each wave's
// first position per id (start[e] plus the waves before); pass 2 walks the slots again and
// places them, the leader advancing the wave's position after the round. A wave's LDS
// accesses run in program order, so the block syncs only between the phases. Ids load
// PB rounds at a time, all in flight together.
// Larger E: counts by LDS atomics, then positions in rounds of 1024 slots (a slot's rank
// among the equal ids before it in the round).
constexpr int PLAN_PB = 16;
__global__ void __launch_bounds__(1024) moe_plan_kernel(const int32_t* __restrict__ ids, int A, int E, int k,
                                                        const uint64_t* __restrict__ all_recs, int32_t* plan_base,
                                                        uint64_t* __restrict__ recs) {
    extern __shared__ int lds[];
    int* count = lds;          // [E]; becomes start[E] in place
    int* start = lds;
    int* wcnt = lds + E;       // [16][E] (E <= PLAN_FAST_E)
    int* round_ids = lds + E;  // [1024] (larger E)
    __shared__ int warp_tot[16];
    __shared__ int bad;
    PlanView plan{plan_base, E, A};
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = (int)blockDim.x >> 6;
    const bool fast = E <= PLAN_FAST_E;
    const int nbits = 32 - __builtin_clz((unsigned)max(E - 1, 1));
    const int chunk = (((A + nw - 1) / nw) + 63) & ~63;
    const int s0 = min(A, wave * chunk), s1 = min(A, s0 + chunk);
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    // peers of this lane's id in the round (e < 0: none), its rank among them and their number
    auto match = [&](int e, int& rank) -> int {
        uint64_t peers = __ballot(e >= 0);
        for (int b = 0; b < nbits; b++) {
            const uint64_t bal = __ballot(e >= 0 && ((e >> b) & 1));
            peers &= ((e >> b) & 1) ? bal : ~bal;
        }
        rank = (int)__builtin_popcountll(peers & below);
        return (int)__builtin_popcountll(peers);
    };
    // this wave's ids of rounds b0 .. b0 + PLAN_PB (-1 past its slots)
    auto load_ids = [&](int b0, int (&eb)[PLAN_PB]) {
#pragma unroll
        for (int r = 0; r < PLAN_PB; r++) {
            const int sl = b0 + 64 * r + lane;
            eb[r] = sl < s1 ? ids[sl] : -1;
        }
    };
    if (tid == 0) bad = 0;
    for (int e = tid; e < E; e += blockDim.x) count[e] = 0;
    if (fast)
        for (int i = lane; i < E; i += 64) wcnt[wave * E + i] = 0;
    __syncthreads();
    if (fast) {
        for (int b0 = s0; b0 < s1; b0 += 64 * PLAN_PB) {
            int eb[PLAN_PB];
            load_ids(b0, eb);
#pragma unroll
            for (int r = 0; r < PLAN_PB; r++) {
                if (b0 + 64 * r >= s1) break;  // wave-uniform
                const bool in = b0 + 64 * r + lane < s1;
                const bool ok = eb[r] >= 0 && eb[r] < E;
                if (in && !ok) bad = 1;
                int rank;
                const int n = match(ok ? eb[r] : -1, rank);
                if (ok && rank == 0) wcnt[wave * E + eb[r]] += n;
                wave_lds_order();
            }
        }
        __syncthreads();
        for (int i = tid; i < E; i += blockDim.x) {
            int c = 0;
            for (int w = 0; w < nw; w++) c += wcnt[w * E + i];
            count[i] = c;
        }
    } else {
        for (int b0 = 0; b0 < A; b0 += (int)blockDim.x * PLAN_PB) {
            int eb[PLAN_PB];
#pragma unroll
            for (int r = 0; r < PLAN_PB; r++) {
                const int sl = b0 + r * (int)blockDim.x + tid;
                eb[r] = sl < A ? ids[sl] : -1;
            }
#pragma unroll
            for (int r = 0; r < PLAN_PB; r++) {
                if (b0 + r * (int)blockDim.x + tid >= A) break;
                const int e = eb[r];
                if (e < 0 || e >= E) bad = 1;
                else atomicAdd(&count[e], 1);
            }
        }
    }
    __syncthreads();
    if (bad) {
        if (tid == 0) *plan.n_e() = -1;
        return;
    }
    // Each thread owns a contiguous run of per = ceil(E / 1024) experts.
    int per = (E + blockDim.x - 1) / blockDim.x;
    int e0 = min(E, tid * per), e1 = min(E, e0 + per);
    int my_assign = 0, my_experts = 0;
    for (int e = e0; e < e1; e++) {
        my_assign += count[e];
        my_experts += count[e] > 0;
    }
    int total_a, n_e;
    int a = block_exclusive_scan(my_assign, warp_tot, total_a);
    int x = block_exclusive_scan(my_experts, warp_tot, n_e);
    for (int e = e0; e < e1; e++) {
        int c = count[e];
        start[e] = a;
        if (c > 0) {
            plan.experts()[x] = e;
            plan.off()[x] = a;
            recs[x] = all_recs[e];
            x++;
        }
        a += c;
    }
    for (int i = n_e + tid; i < E; i += blockDim.x) plan.experts()[i] = -1;
    for (int i = n_e + tid; i <= E; i += blockDim.x) plan.off()[i] = A;
    if (tid == 0) *plan.n_e() = n_e;
    __syncthreads();
    if (fast) {
        for (int i = tid; i < E; i += blockDim.x) {
            int acc = start[i];
            for (int w = 0; w < nw; w++) {
                const int c = wcnt[w * E + i];
                wcnt[w * E + i] = acc;
                acc += c;
            }
        }
        __syncthreads();
        for (int b0 = s0; b0 < s1; b0 += 64 * PLAN_PB) {
            int eb[PLAN_PB];
            load_ids(b0, eb);
#pragma unroll
            for (int r = 0; r < PLAN_PB; r++) {
                if (b0 + 64 * r >= s1) break;  // wave-uniform
                const int sl = b0 + 64 * r + lane, e = eb[r];
                int rank;
                const int n = match(e, rank);
                if (e >= 0) {
                    const int pos = wcnt[wave * E + e] + rank;
                    plan.assign_tok()[pos] = sl / k;
                    plan.slot_assign()[sl] = pos;
                }
                wave_lds_order();  // every lane has read the position before the leader advances it
                if (e >= 0 && rank == 0) wcnt[wave * E + e] += n;
                wave_lds_order();
            }
        }
        return;
    }
    // Positions in rounds of blockDim slots: a slot's rank among the equal ids before it
    // (each round's id loads one round ahead).
    int e_next = tid < A ? ids[tid] : -1;
    for (int base = 0; base < A; base += blockDim.x) {
        int s = base + tid;
        int e = s < A ? e_next : -1;
        e_next = s + (int)blockDim.x < A ? ids[s + blockDim.x] : -1;
        round_ids[tid] = e;
        __syncthreads();
        int pos = 0;
        if (e >= 0) {
            int rank = 0;
            for (int j = 0; j < tid; j++) rank += round_ids[j] == e;
            pos = start[e] + rank;
            plan.assign_tok()[pos] = s / k;
            plan.slot_assign()[s] = pos;
        }
        __syncthreads();
        if (e >= 0) atomicAdd(&start[e], 1);
        __syncthreads();
    }
}

}  // namespace oom
extern "C" int oom_moe_plan(const int32_t* ids, int T, int E, int k, const uint64_t* all_recs, int32_t* plan,
                            uint64_t* recs, void* stream);
namespace oom {

// ---- the plan over many blocks (large steps, E <= PLAN_FAST_E) -------------------------
//
// The same plan in two launches, for steps whose slots would keep one block busy: block b
// of 4 waves owns the slots [b C, b C + C) (C a multiple of 256; wave w the quarter
// [b C + w C / 4, + C / 4)). plan_count_kernel counts each id over the block's slots (the
// ballot matching above, per-wave rows in LDS) and stores the block's counts and an
// invalid-id flag, counts[b][0 .. E) and counts[b][E]. plan_place_kernel reads every
// block's counts: expert e's first position is the assignments of the experts below it,
// block b's first position for e adds the blocks before it, and wave w's the waves before
// it in the block (counted again); block 0 writes the plan's header. Slots keep slot order
// inside each expert, as the single-block kernel's.
constexpr int PM_WAVES = 4;
constexpr int PM_THREADS = 64 * PM_WAVES;

// Peers of this lane's id e in the wave (e < 0: none), its rank among them, their number.
__device__ __forceinline__ int plan_match(int e, int nbits, uint64_t below, int& rank) {
    uint64_t peers = __ballot(e >= 0);
    for (int b = 0; b < nbits; b++) {
        const uint64_t bal = __ballot(e >= 0 && ((e >> b) & 1));
        peers &= ((e >> b) & 1) ? bal : ~bal;
    }
    rank = (int)__builtin_popcountll(peers & below);
    return (int)__builtin_popcountll(peers);
}

// This wave's per-id counts over its slots [s0, s1) into wcnt (E ints); returns whether an
// id was out of range.
__device__ bool plan_wave_count(const int32_t* __restrict__ ids, int s0, int s1, int E, int* wcnt) {
    const int lane = threadIdx.x & 63;
    const int nbits = 32 - __builtin_clz((unsigned)max(E - 1, 1));
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    bool bad = false;
    for (int b0 = s0; b0 < s1; b0 += 64 * PLAN_PB) {
        int eb[PLAN_PB];
#pragma unroll
        for (int r = 0; r < PLAN_PB; r++) {
            const int sl = b0 + 64 * r + lane;
            eb[r] = sl < s1 ? ids[sl] : -1;
        }
#pragma unroll
        for (int r = 0; r < PLAN_PB; r++) {
            if (b0 + 64 * r >= s1) break;  // wave-uniform
            const bool in = b0 + 64 * r + lane < s1;
            const bool ok = eb[r] >= 0 && eb[r] < E;
            bad |= in && !ok;
            int rank;
            const int n = plan_match(ok ? eb[r] : -1, nbits, below, rank);
            if (ok && rank == 0) wcnt[eb[r]] += n;
            wave_lds_order();
        }
    }
    return bad;
}

__global__ void __launch_bounds__(PM_THREADS) plan_count_kernel(const int32_t* __restrict__ ids, int A, int E, int C,
                                                                int32_t* __restrict__ counts) {
    extern __shared__ int lds[];  // wcnt [PM_WAVES][E]
    __shared__ int bad_s;
    const int tid = threadIdx.x, wave = tid >> 6, b = blockIdx.x;
    for (int i = tid; i < PM_WAVES * E; i += PM_THREADS) lds[i] = 0;
    if (tid == 0) bad_s = 0;
    __syncthreads();
    const int q = C / PM_WAVES, s0 = min(A, b * C + wave * q), s1 = min(A, s0 + q);
    if (plan_wave_count(ids, s0, s1, E, lds + wave * E)) bad_s = 1;
    __syncthreads();
    int32_t* row = counts + (size_t)b * (E + 1);
    for (int e = tid; e < E; e += PM_THREADS) {
        int c = 0;
#pragma unroll
        for (int w = 0; w < PM_WAVES; w++) c += lds[w * E + e];
        row[e] = c;
    }
    if (tid == 0) row[E] = bad_s;
}

__global__ void __launch_bounds__(PM_THREADS) plan_place_kernel(const int32_t* __restrict__ ids, int A, int E, int k,
                                                                int C, int NB, const int32_t* __restrict__ counts,
                                                                const uint64_t* __restrict__ all_recs,
                                                                int32_t* plan_base, uint64_t* __restrict__ recs) {
    extern __shared__ int lds[];  // pos [E] (expert e's first position for this block), wcnt [PM_WAVES][E]
    int* pos = lds;
    int* wcnt = lds + E;
    __shared__ int warp_tot[PM_WAVES];
    __shared__ int bad_s;
    PlanView plan{plan_base, E, A};
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, b = blockIdx.x;
    if (tid == 0) bad_s = 0;
    for (int i = tid; i < PM_WAVES * E; i += PM_THREADS) wcnt[i] = 0;
    __syncthreads();
    // expert totals and this block's offsets within them: thread t owns experts
    // [t per, t per + per), per = ceil(E / PM_THREADS)
    const int per = (E + PM_THREADS - 1) / PM_THREADS;
    const int e0 = min(E, tid * per), e1 = min(E, e0 + per);
    int my_assign = 0, my_experts = 0, bad = 0;
    for (int e = e0; e < e1; e++) {
        int tot = 0, before = 0;
        for (int bb = 0; bb < NB; bb++) {
            const int c = counts[(size_t)bb * (E + 1) + e];
            tot += c;
            before += bb < b ? c : 0;
        }
        pos[e] = before;  // the block's offset inside expert e, for now
        wcnt[e] = tot;    // (wave 0's row holds the totals until the scan is done)
        my_assign += tot;
        my_experts += tot > 0;
    }
    for (int bb = tid; bb < NB; bb += PM_THREADS) bad |= counts[(size_t)bb * (E + 1) + E];
    if (bad) bad_s = 1;
    int total_a, n_e;
    int a = block_exclusive_scan(my_assign, warp_tot, total_a);  // (syncs: bad_s is visible after it)
    int x = block_exclusive_scan(my_experts, warp_tot, n_e);
    if (bad_s) {
        if (b == 0 && tid == 0) *plan.n_e() = -1;
        return;
    }
    for (int e = e0; e < e1; e++) {
        const int tot = wcnt[e];
        pos[e] += a;
        if (b == 0 && tot > 0) {
            plan.experts()[x] = e;
            plan.off()[x] = a;
            recs[x] = all_recs[e];
            x++;
        }
        a += tot;
        wcnt[e] = 0;
    }
    if (b == 0) {
        for (int i = n_e + tid; i < E; i += PM_THREADS) plan.experts()[i] = -1;
        for (int i = n_e + tid; i <= E; i += PM_THREADS) plan.off()[i] = A;
        if (tid == 0) *plan.n_e() = n_e;
    }
    __syncthreads();
    // the waves' own counts, then each wave's first position per id
    const int q = C / PM_WAVES, s0 = min(A, b * C + wave * q), s1 = min(A, s0 + q);
    plan_wave_count(ids, s0, s1, E, wcnt + wave * E);
    __syncthreads();
    for (int e = tid; e < E; e += PM_THREADS) {
        int acc = pos[e];
#pragma unroll
        for (int w = 0; w < PM_WAVES; w++) {
            const int c = wcnt[w * E + e];
            wcnt[w * E + e] = acc;
            acc += c;
        }
    }
    __syncthreads();
    // place the wave's slots in order
    const int nbits = 32 - __builtin_clz((unsigned)max(E - 1, 1));
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    int* wpos = wcnt + wave * E;
    for (int b0 = s0; b0 < s1; b0 += 64 * PLAN_PB) {
        int eb[PLAN_PB];
#pragma unroll
        for (int r = 0; r < PLAN_PB; r++) {
            const int sl = b0 + 64 * r + lane;
            eb[r] = sl < s1 ? ids[sl] : -1;
        }
#pragma unroll
        for (int r = 0; r < PLAN_PB; r++) {
            if (b0 + 64 * r >= s1) break;  // wave-uniform
            const int sl = b0 + 64 * r + lane, e = eb[r];
            int rank;
            const int n = plan_match(e, nbits, below, rank);
            if (e >= 0) {
                const int p = wpos[e] + rank;
                plan.assign_tok()[p] = sl / k;
                plan.slot_assign()[sl] = p;
            }
            wave_lds_order();  // every lane has read the position before the leader advances it
            if (e >= 0 && rank == 0) wpos[e] += n;
            wave_lds_order();
        }
    }
}

// Slots a block of the two-launch plan takes, and its block count (at most 64).
static int plan_multi_chunk(int A) { return std::max(1024, (int)((cdiv((int64_t)A, 64) + 255) / 256 * 256)); }
size_t plan_multi_counts(int A, int E) {
    const int C = plan_multi_chunk(A);
    return (size_t)cdiv((int64_t)A, C) * (E + 1);
}
int launch_plan_multi(const int32_t* ids, int T, int E, int k, const uint64_t* all_recs, int32_t* plan, uint64_t* recs,
                      int32_t* counts, hipStream_t st) {
    if (E > PLAN_FAST_E) return oom_moe_plan(ids, T, E, k, all_recs, plan, recs, st);
    const int A = T * k, C = plan_multi_chunk(A), NB = (int)cdiv((int64_t)A, C);
    hipLaunchKernelGGL(plan_count_kernel, dim3(NB), dim3(PM_THREADS), PM_WAVES * E * sizeof(int), st, ids, A, E, C,
                       counts);
    if (int rc = launched("oom_moe_plan")) return rc;
    hipLaunchKernelGGL(plan_place_kernel, dim3(NB), dim3(PM_THREADS), (PM_WAVES + 1) * E * sizeof(int), st, ids, A, E,
                       k, C, NB, counts, all_recs, plan, recs);
    return launched("oom_moe_plan");
}

}  // namespace oom

extern "C" int oom_router_topk(const float* logits, int32_t* ids, float* weights, int T, int E, int k, void* stream) {
    OOM_REQUIRE(T >= 0, "oom_router_topk: T < 0");
    OOM_REQUIRE(k >= 1 && k <= 32 && E >= k && E <= 8192, "oom_router_topk: router top-k > 32 or experts > 8192");
    if (T == 0) return OOM_OK;
    OOM_REQUIRE(logits && ids && weights, "oom_router_topk: null buffer");
    hipLaunchKernelGGL(oom::router_topk_kernel, dim3(T), dim3(64), E * sizeof(float), oom::as_stream(stream), logits,
                       ids, weights, E, k);
    return oom::launched("oom_router_topk");
}

extern "C" size_t oom_moe_plan_size(int T, int E, int k) { return oom::PlanView::size(E, T * k); }

extern "C" int oom_moe_plan(const int32_t* ids, int T, int E, int k, const uint64_t* all_recs, int32_t* plan,
                            uint64_t* recs, void* stream) {
    OOM_REQUIRE(T >= 1 && k >= 1 && E >= 1 && E <= 8192, "oom_moe_plan: shape unsupported");
    OOM_REQUIRE((int64_t)T * k <= (1 << 24), "oom_moe_plan: too many assignments");
    OOM_REQUIRE(ids && all_recs && plan && recs, "oom_moe_plan: null buffer");
    // count / start [E], then the rank rounds' table: per-wave counts [16][E] (E <= PLAN_FAST_E)
    // or the ids of one round [1024]
    size_t lds = ((size_t)E + (E <= oom::PLAN_FAST_E ? 16 * (size_t)E : 1024)) * sizeof(int);
    hipLaunchKernelGGL(oom::moe_plan_kernel, dim3(1), dim3(1024), lds, oom::as_stream(stream), ids, T * k, E, k,
                       all_recs, plan, recs);
    return oom::launched("oom_moe_plan");
}
