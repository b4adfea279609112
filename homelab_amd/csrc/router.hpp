// Router top-k for one token on one wavefront, and the routing-plan layout.
#pragma once

#include "common.hpp"

namespace oom {

// Softmax over E logits, top k by probability (ties to the lower id), weights
// renormalised over the picks in pick order, for one token on one wave64 whose
// lanes are `lane` = 0..63. `probs` is E floats of LDS owned by this wave.
// The arithmetic is the reference's (crates/oominf-cuda/kernels/ops.cu:230-294):
// p_e = expf(l_e - max) / sum, where sum adds expf(l_e - max) per virtual thread
// t = e mod 256 in e order, then over each 32-thread group by an xor butterfly,
// then over the 8 group totals by the same butterfly: the reference's 256-thread
// block_sum (ops.cu:15-31), so p has the reference's bits given the same expf.
// Lane r < k ends with ids_out = the r-th pick and w_out = its weight.
__device__ __forceinline__ void route_token_wave(const float* __restrict__ l, int E, int k, float* probs, int lane,
                                                 int& id_out, float& w_out) {
    float m = -INFINITY;
    for (int e = lane; e < E; e += 64) m = fmaxf(m, l[e]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    // virtual thread vt = lane + 64 q (q = 0..3) of the reference's 256-thread block
    float part[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float s = 0.0f;
        for (int e = lane + 64 * q; e < E; e += 256) s += expf(l[e] - m);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);  // within each 32-lane half
        part[q] = s;
    }
    // group totals: group 2q is lanes 0..31 of slot q, group 2q + 1 lanes 32..63
    float w8[8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        w8[2 * q] = __shfl(part[q], 0, 64);
        w8[2 * q + 1] = __shfl(part[q], 32, 64);
    }
    // the xor butterfly over lanes 0..7 (zeros above): ((g0+g4)+(g2+g6)) + ((g1+g5)+(g3+g7))
    float sum = ((w8[0] + w8[4]) + (w8[2] + w8[6])) + ((w8[1] + w8[5]) + (w8[3] + w8[7]));
    for (int e = lane; e < E; e += 64) probs[e] = expf(l[e] - m) / sum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    float picked = 0.0f;
    for (int r = 0; r < k; r++) {
        float bv = -3.0f;
        int bi = 0x7fffffff;
        for (int e = lane; e < E; e += 64) {
            float p = probs[e];
            if (p > bv || (p == bv && e < bi)) {
                bv = p;
                bi = e;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            float ov = __shfl_xor(bv, o, 64);
            int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        // every lane holds the winner; picks sit below every probability from now on
        if (lane == (bi & 63)) probs[bi] = -2.0f;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        picked += bv;
        if (lane == r) {
            id_out = bi;
            w_out = bv;
        }
    }
    if (lane < k) w_out = w_out / picked;
}

// Maximum over the wave of a 64-bit unsigned key (every lane ends with it).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v, int lane) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
#define OOM_MAX_U64_STEP(O)                                                                    \
    {                                                                                          \
        const uint32_t plo = __float_as_uint(lane_xor<O>(__uint_as_float(lo), lane));          \
        const uint32_t phi = __float_as_uint(lane_xor<O>(__uint_as_float(hi), lane));          \
        const bool take = ((uint64_t)phi << 32 | plo) > ((uint64_t)hi << 32 | lo);             \
        lo = take ? plo : lo;                                                                  \
        hi = take ? phi : hi;                                                                  \
    }
    OOM_MAX_U64_STEP(1)
    OOM_MAX_U64_STEP(2)
    OOM_MAX_U64_STEP(4)
    OOM_MAX_U64_STEP(8)
    OOM_MAX_U64_STEP(16)
    OOM_MAX_U64_STEP(32)
#undef OOM_MAX_U64_STEP
    return (uint64_t)hi << 32 | lo;
}

// route_token_wave for E <= 64 EQ (EQ = 4: 256, EQ = 8: 512), without LDS round trips:
// lane l holds experts l + 64 q (q < EQ) in registers; sums keep the reference's order
// (virtual thread l + 64 q of its 256-thread block adds experts l + 64 q and l + 64 q + 256
// in id order, then sum32_xor_order).
// The k picks rank experts by one 64-bit key, the probability's bits above the
// complemented id: p >= 0, so a larger key is a larger p, and among equal p the lower
// id, which is the reference's argmax with ties to the lower id. Each round is one wave
// maximum of the lanes' best keys; the winner's lane drops that key (0 is below every
// expert's key) and takes its next best.
template <int EQ = 4>
__device__ __forceinline__ void route_token_regs(const float* __restrict__ l, int E, int k, int lane, int& id_out,
                                                 float& w_out) {
    static_assert(EQ == 4 || EQ == 8, "4 or 8 logits per lane");
    float lv[EQ];
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < EQ; q++) {
        lv[q] = lane + 64 * q < E ? l[lane + 64 * q] : -INFINITY;
        m = fmaxf(m, lv[q]);
    }
    m = wave_max(m);
    // virtual thread vt = lane + 64 q (q < 4) holds experts vt and, with EQ = 8, vt + 256
    float ex[EQ], w8[8];
#pragma unroll
    for (int q = 0; q < EQ; q++) ex[q] = lane + 64 * q < E ? expf(lv[q] - m) : 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float vt = 0.0f + ex[q];
        if constexpr (EQ == 8) vt = vt + ex[q + 4];
        const float s = sum32_xor_order(vt);
        w8[2 * q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
        w8[2 * q + 1] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 32));
    }
    const float sum = ((w8[0] + w8[4]) + (w8[2] + w8[6])) + ((w8[1] + w8[5]) + (w8[3] + w8[7]));
    uint64_t key[EQ], best_mine = 0;
#pragma unroll
    for (int q = 0; q < EQ; q++) {
        const int e = lane + 64 * q;
        key[q] = e < E ? ((uint64_t)__float_as_uint(ex[q] / sum) << 32) | (uint32_t)~(uint32_t)e : 0ull;
        best_mine = key[q] > best_mine ? key[q] : best_mine;
    }
    float picked = 0.0f;
    for (int r = 0; r < k; r++) {
        const uint64_t best = wave_max_u64(best_mine, lane);
        const int e = (int)~(uint32_t)best;
        const float p = __uint_as_float((uint32_t)(best >> 32));
        if ((e & 63) == lane) {
            best_mine = 0;
#pragma unroll
            for (int q = 0; q < EQ; q++) {
                if (key[q] == best) key[q] = 0;
                best_mine = key[q] > best_mine ? key[q] : best_mine;
            }
        }
        picked += p;
        if (lane == r) {
            id_out = e;
            w_out = p;
        }
    }
    if (lane < k) w_out = w_out / picked;
}

// route_token_regs's picks and weights for one token (E <= 64 EQ <= 512, k <= 64) without
// k serial wave maxima: lane r < k ends with pick r's id and weight, bit for bit as
// route_token_regs computes them. The probabilities and their sum follow route_token_regs;
// each expert's key is 1 << 40 | p's bits << 9 | (511 - id) (larger p first, ties to the
// lower id, as the reference's argmax), the k-th largest key comes from a radix descent on
// ballots, the picks go to LDS in id order and rank themselves by key, and the weights
// renormalise by the picks' sum in pick order. ids and p are k-entry LDS scratch, keys
// k entries (EQ = 4) or 64 (EQ = 8: once at most 64 keys reach the descent's candidate, they
// are gathered one a lane through keys, and the descent goes on with one ballot a step
// instead of 8; measured alone, 5500 -> 4850 cycles a call at 512 experts, top-10).
template <int EQ>
__device__ __forceinline__ void route_picks(const float* __restrict__ l, int E, int k, int lane, uint64_t* keys,
                                            int* ids, float* p, int& id_out, float& w_out) {
    static_assert(EQ == 4 || EQ == 8, "4 or 8 logits per lane");
    float lv[EQ];
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < EQ; q++) {
        lv[q] = lane + 64 * q < E ? l[lane + 64 * q] : -INFINITY;
        m = fmaxf(m, lv[q]);
    }
    m = wave_max(m);
    float ex[EQ], w8[8];
#pragma unroll
    for (int q = 0; q < EQ; q++) ex[q] = lane + 64 * q < E ? expf(lv[q] - m) : 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float vt = 0.0f + ex[q];
        if constexpr (EQ == 8) vt = vt + ex[q + 4];
        const float s = sum32_xor_order(vt);
        w8[2 * q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
        w8[2 * q + 1] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 32));
    }
    const float sum = ((w8[0] + w8[4]) + (w8[2] + w8[6])) + ((w8[1] + w8[5]) + (w8[3] + w8[7]));
    uint64_t key[EQ];
#pragma unroll
    for (int q = 0; q < EQ; q++) {
        const int e = lane + 64 * q;
        key[q] = e < E ? (1ull << 40) | ((uint64_t)__float_as_uint(ex[q] / sum) << 9) | (uint64_t)(511 - e) : 0ull;
    }
    // keys are distinct (the id bits), so the descent ends with exactly k keys >= kth
    uint64_t kth = 1ull << 40;
    int b = 39, cnt = 0;
    bool gathered = false;
    for (; b >= 0; b--) {
        const uint64_t cand = kth | (1ull << b);
        int c = 0;
#pragma unroll
        for (int q = 0; q < EQ; q++) c += (int)__builtin_popcountll(__ballot(key[q] >= cand));
        if (c >= k) {
            kth = cand;
            cnt = c;
            if (c == k) break;
            if (EQ == 8 && c <= 64) {
                gathered = true;
                b--;
                break;
            }
        }
    }
    // the keys >= kth in lane order, to LDS (the picks, or the cnt <= 64 left in the race)
    const auto gather = [&](const auto& ks, int n) {
        int base = 0;
#pragma unroll
        for (int q = 0; q < n; q++) {
            const uint64_t sel = __ballot(ks[q] >= kth);
            if (ks[q] >= kth)
                keys[base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(sel >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)sel, 0u))] = ks[q];
            base += (int)__builtin_popcountll(sel);
        }
        wave_lds_order();
    };
    if (gathered) {
        gather(key, EQ);
        uint64_t one[1] = {lane < cnt ? keys[lane] : 0ull};
        for (; b >= 0; b--) {
            const uint64_t cand = kth | (1ull << b);
            const int c = (int)__builtin_popcountll(__ballot(one[0] >= cand));
            if (c >= k) {
                kth = cand;
                if (c == k) break;
            }
        }
        gather(one, 1);
    } else {
        gather(key, EQ);
    }
    const uint64_t mine = lane < k ? keys[lane] : 0ull;
    int rank = 0;
    for (int j = 0; j < k; j++) rank += keys[j] > mine;
    if (lane < k) {
        ids[rank] = 511 - (int)(mine & 511u);
        p[rank] = __uint_as_float((uint32_t)(mine >> 9) & 0x7fffffffu);
    }
    wave_lds_order();
    float picked = 0.0f;
    for (int r = 0; r < k; r++) picked += p[r];
    if (lane < k) {
        id_out = ids[lane];
        w_out = p[lane] / picked;
    }
}

// route_token_regs's routing of one token (E <= 64 EQ <= 256, k <= 8) without k serial
// rounds, with the one-token plan in the same pass. Every expert gets a key that orders
// as the reference's argmax does (larger p first, ties to the lower id): bit 39 set for
// a real expert, p's bits in 38..8, 255 - id in 7..0. The k-th largest key K comes from
// a radix descent on ballots: each step keeps a candidate bit if at least k keys reach
// the candidate, and the descent stops when exactly k do. The picks are the keys >= K:
// their ballot bits in lane order are the experts in id order (the plan's order), and a
// pick's rank among the k picks is its pick order. Weights are p / (sum of the picks' p
// in pick order), as the reference renormalises (crates/oominf-cuda/kernels/ops.cu:230-294).
// Written to LDS: experts[i] (ids ascending), ids[r] and w[r] (pick order) and
// slot_assign[r] (the id-order position of pick r). keys and p are k-entry LDS scratch.
// Keys of one token's experts from its logits (lane l holds expert l + 64 q in lv[q]):
// the softmax with the reference's 256-thread block sum (virtual thread lane + 64 q holds
// expert lane + 64 q; groups of 32 threads absent here (q >= EQ) add zeros, which leaves
// the sum's bits as route_token_regs computes them), then key = 1 << 39 | p's bits << 8 |
// (255 - id) for a real expert, 0 past E.
template <int EQ>
__device__ __forceinline__ void route_keys(const float (&lv)[EQ], int E, int lane, uint64_t (&key)[EQ]) {
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < EQ; q++) m = fmaxf(m, lv[q]);
    m = wave_max(m);
    float ex[EQ], w8[8];
#pragma unroll
    for (int g = 0; g < 8; g++) w8[g] = 0.0f;
#pragma unroll
    for (int q = 0; q < EQ; q++) {
        ex[q] = lane + 64 * q < E ? expf(lv[q] - m) : 0.0f;
        const float s = sum32_xor_order(0.0f + ex[q]);
        w8[2 * q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
        w8[2 * q + 1] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 32));
    }
    const float sum = ((w8[0] + w8[4]) + (w8[2] + w8[6])) + ((w8[1] + w8[5]) + (w8[3] + w8[7]));
#pragma unroll
    for (int q = 0; q < EQ; q++) {
        const int e = lane + 64 * q;
        key[q] = e < E ? (1ull << 39) | ((uint64_t)__float_as_uint(ex[q] / sum) << 8) | (uint64_t)(255 - e) : 0ull;
    }
}

// The k-th largest of the wave's keys (k <= the number of real keys) by a radix descent
// on ballots: each step keeps a candidate bit if at least k keys reach the candidate, and
// the descent stops when exactly k do. Every real key reaches 1 << 39.
template <int EQ>
__device__ __forceinline__ uint64_t radix_kth(const uint64_t (&key)[EQ], int k) {
    uint64_t kth = 1ull << 39;
    for (int b = 38; b >= 0; b--) {
        const uint64_t cand = kth | (1ull << b);
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < EQ; q++) cnt += (int)__builtin_popcountll(__ballot(key[q] >= cand));
        if (cnt >= k) {
            kth = cand;
            if (cnt == k) break;
        }
    }
    return kth;
}

// The token's logits as route_select reads them: lane l holds expert l + 64 q in lv[q]
// (-inf past E). Issued apart from route_select so a caller can put them in flight first.
template <int EQ>
__device__ __forceinline__ void route_logits(const float* __restrict__ l, int E, int lane, float (&lv)[EQ]) {
#pragma unroll
    for (int q = 0; q < EQ; q++) lv[q] = lane + 64 * q < E ? l[lane + 64 * q] : -INFINITY;
}

template <int EQ>
__device__ __forceinline__ void route_select(const float (&lv)[EQ], int E, int k, int lane, uint64_t* keys,
                                             float* p, int* experts, int* ids, float* w, int* slot_assign) {
    uint64_t key[EQ];
    route_keys<EQ>(lv, E, lane, key);
    const uint64_t kth = radix_kth<EQ>(key, k);
    // the picks in id order: lane order within q, q ascending (expert lane + 64 q)
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
    if (lane < k) {
        const int e = 255 - (int)(mine & 255u);
        experts[lane] = e;
        ids[rank] = e;
        slot_assign[rank] = lane;
        p[rank] = pm;
    }
    wave_lds_order();
    float picked = 0.0f;
    for (int r = 0; r < k; r++) picked += p[r];
    if (lane < k) w[rank] = pm / picked;
}

// Routing-plan buffer (i32) of a step with T tokens, E experts and top k:
//   [0]                     n_e, the number of distinct experts
//   [1, 1 + E)              experts: distinct ids ascending, then -1
//   [1 + E, 2 + 2E)         off: off[i] = first assignment of expert i; A past n_e
//   [2 + 2E, 2 + 2E + A)    assign_tok: token of each assignment
//   [2 + 2E + A, 2 + 2E + 2A) slot_assign: assignment of slot t * k + s
struct PlanView {
    int32_t* base;
    int E, A;
    __host__ __device__ int32_t* n_e() const { return base; }
    __host__ __device__ int32_t* experts() const { return base + 1; }
    __host__ __device__ int32_t* off() const { return base + 1 + E; }
    __host__ __device__ int32_t* assign_tok() const { return base + 2 + 2 * E; }
    __host__ __device__ int32_t* slot_assign() const { return base + 2 + 2 * E + A; }
    static size_t size(int E, int A) { return size_t(2 + 2 * E + 2 * A); }
};

}  // namespace oom
