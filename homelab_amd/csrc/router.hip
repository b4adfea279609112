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

// Block-wide exclusive scan of one int per thread (blockDim 1024 = 16 waves).
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
// order. One block of 1024 threads; LDS: count[E] (then start[E]), ids of one round.
__global__ void __launch_bounds__(1024) moe_plan_kernel(const int32_t* __restrict__ ids, int A, int E, int k,
                                                        const uint64_t* __restrict__ all_recs, int32_t* plan_base,
                                                        uint64_t* __restrict__ recs) {
    extern __shared__ int lds[];
    int* count = lds;          // [E]; becomes start[E] in place
    int* start = lds;
    int* round_ids = lds + E;  // [1024]
    __shared__ int warp_tot[16];
    __shared__ int bad;
    PlanView plan{plan_base, E, A};
    int tid = threadIdx.x;
    if (tid == 0) bad = 0;
    for (int e = tid; e < E; e += blockDim.x) count[e] = 0;
    __syncthreads();
    for (int s = tid; s < A; s += blockDim.x) {
        int e = ids[s];
        if (e < 0 || e >= E) bad = 1;
        else atomicAdd(&count[e], 1);
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
    if (E <= PLAN_FAST_E) {
        // Positions in rounds of 1024 slots. Within a wave, the lanes holding the same id
        // find each other by ballots over the id's bits (rank = peers below this lane);
        // per-wave counts per id in LDS give the waves before this one.
        int* wcnt = lds + E;  // [16][E]
        const int lane = tid & 63, wave = tid >> 6, nbits = 32 - __builtin_clz((unsigned)max(E - 1, 1));
        for (int base = 0; base < A; base += blockDim.x) {
            for (int i = tid; i < 16 * E; i += blockDim.x) wcnt[i] = 0;
            __syncthreads();
            const int s = base + tid;
            const int e = s < A ? ids[s] : -1;
            uint64_t peers = __ballot(e >= 0);
            for (int b = 0; b < nbits; b++) {
                const uint64_t bal = __ballot(e >= 0 && ((e >> b) & 1));
                peers &= ((e >> b) & 1) ? bal : ~bal;
            }
            const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
            const int rank = (int)__builtin_popcountll(peers & below);
            if (e >= 0 && rank == 0) wcnt[wave * E + e] = (int)__builtin_popcountll(peers);
            __syncthreads();
            if (e >= 0) {
                int pos = start[e] + rank;
                for (int w = 0; w < wave; w++) pos += wcnt[w * E + e];
                plan.assign_tok()[pos] = s / k;
                plan.slot_assign()[s] = pos;
            }
            __syncthreads();
            for (int i = tid; i < E; i += blockDim.x) {
                int c = 0;
                for (int w = 0; w < 16; w++) c += wcnt[w * E + i];
                start[i] += c;
            }
            __syncthreads();
        }
        return;
    }
    // Positions in rounds of blockDim slots: a slot's rank among the equal ids before it.
    for (int base = 0; base < A; base += blockDim.x) {
        int s = base + tid;
        int e = s < A ? ids[s] : -1;
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
