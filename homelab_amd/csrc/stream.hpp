// Shared pieces of the one-launch decode kernels: buffer-resource loads, the token's
// activations in registers, device-coherent hand-offs between waves, and the fixed
// header of a decode workspace (the state a decode call leaves for the next one).
#pragma once

#include <algorithm>

#include "common.hpp"

namespace oom {

constexpr int BUF_FLAGS = 0x00020000;  // buffer resource word 3: 32-bit data format
constexpr int OOB = 0x7ffffff0;        // an offset past every resource: loads read 0
constexpr int BUF_SC1 = 16;            // cache-policy bit of a device-coherent (sc1) buffer load on gfx950

// ---- decode workspace header ---------------------------------------------------------
// Every decode workspace starts with this header at fixed offsets, whatever the step's
// shape, so a workspace shared by steps of different shapes (batch 1 and batch 16 of one
// model) never reads another layout's data as its state. Each word or counter has a
// 256-byte line of its own: atomics and polls on one line serialise at the memory side.
constexpr size_t WS_EPOCH = 0;          // u32: the one-token kernel's call epoch
constexpr size_t WS_STATUS = 256;       // u32: 1 if a wait of a decode kernel gave up
constexpr int D1_MAX_BLOCKS = 1024;     // blocks of the one-token kernel
constexpr size_t WS_STARTED = 512;      // u32[D1_MAX_BLOCKS]: the epoch each block of the last call saw
constexpr int BAR_GROUPS = 8;           // barrier groups of the multi-token kernel
constexpr int BAR_STRIDE = 64;          // u32 words between its counters
constexpr size_t WS_BAR = WS_STARTED + D1_MAX_BLOCKS * 4;        // (2 BAR_GROUPS + 1) lines
constexpr int TICKET_STRIDE = 64;
constexpr int MAX_TILES = 4096 / 8;     // row tiles of 8 rows for hidden <= 4096
constexpr size_t WS_TICKETS = WS_BAR + (2 * BAR_GROUPS + 1) * BAR_STRIDE * 4;  // MAX_TILES lines
constexpr size_t WS_HEADER = (WS_TICKETS + (size_t)MAX_TILES * TICKET_STRIDE * 4 + 4095) & ~size_t(4095);

// ---- loads ----------------------------------------------------------------------------

__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float ldf(__amdgpu_buffer_rsrc_t r, int off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// A buffer resource over `bytes` at `p` whose address is uniform (kept in SGPRs).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(uint64_t p, int bytes) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p), hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, bytes,
                                             BUF_FLAGS);
}

// The token's activations: lane l holds columns 1024 c + 16 l .. + 16 (c < 4), zeros
// past hidden.
template <int XDT>
struct XRow;
template <>
struct XRow<OOM_BF16> {
    uint32_t w[4][8];
};
template <>
struct XRow<OOM_F32> {
    float v[4][16];
};

template <int XDT>
__device__ __forceinline__ void xrow_load(const void* x, int H, int lane, XRow<XDT>& xr) {
    constexpr int ES = XDT == OOM_BF16 ? 2 : 4;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(x), (short)0, H * ES, BUF_FLAGS);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int col = c * 1024 + lane * 16;
        const int off = col < H ? col * ES : OOB;
        if constexpr (XDT == OOM_BF16) {
            const uint4 a0 = ld16(r, off), a1 = ld16(r, off + 16);
            xr.w[c][0] = a0.x; xr.w[c][1] = a0.y; xr.w[c][2] = a0.z; xr.w[c][3] = a0.w;
            xr.w[c][4] = a1.x; xr.w[c][5] = a1.y; xr.w[c][6] = a1.z; xr.w[c][7] = a1.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint4 v = ld16(r, off + 16 * q);
                xr.v[c][4 * q] = __uint_as_float(v.x);
                xr.v[c][4 * q + 1] = __uint_as_float(v.y);
                xr.v[c][4 * q + 2] = __uint_as_float(v.z);
                xr.v[c][4 * q + 3] = __uint_as_float(v.w);
            }
        }
    }
}

// ---- hand-offs between waves ----------------------------------------------------------
// Values handed between waves of different XCDs inside a kernel move with
// device-coherent (sc1) stores and loads, which skip the per-XCD L2 instead of writing
// it back or invalidating it: an agent-scope fence lowers to buffer_wbl2 / buffer_inv of
// the whole L2, far too costly per work item.
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All of this wave's memory operations complete (stores acknowledged) before the next.
__device__ __forceinline__ void wait_mem() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// This wave's LDS operations complete, then the block meets; outstanding global loads
// stay in flight (a __syncthreads() fence would wait for them too).
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- grid barrier -------------------------------------------------------------------------
// One arrival per block, in two levels so no counter sees more than 64 arrivals: block b
// arrives at group b % G (G = 8, one group per XCD under round-robin dispatch); the last
// of a group arrives at the top counter; the last of those publishes the next generation
// in every group's generation word, which that group's blocks poll. Counters are reset by
// their last arrival and generations only grow, so nothing needs clearing between calls.
// `bar` is the workspace header's barrier area; a wait that gives up sets *status = 1.
// Every block of the grid must be resident.
__device__ __forceinline__ void grid_barrier_words(uint32_t* bar, uint32_t* status, uint32_t spin_limit) {
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t G = min(gridDim.x, (uint32_t)BAR_GROUPS), g = blockIdx.x % G;
        const uint32_t n_g = (gridDim.x - g + G - 1) / G;
        uint32_t* cnt = bar + g * BAR_STRIDE;
        uint32_t* genw = bar + (BAR_GROUPS + 1 + g) * BAR_STRIDE;
        uint32_t* top = bar + BAR_GROUPS * BAR_STRIDE;
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
                    __hip_atomic_store(bar + (BAR_GROUPS + 1 + q) * BAR_STRIDE, target, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                wait_mem();
                released = true;
            }
        }
        if (!released) {
            uint32_t spins = 0;
            while ((int32_t)(__hip_atomic_load(genw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
                __builtin_amdgcn_s_sleep(4);
                if (++spins > spin_limit) {
                    __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    __syncthreads();
}

// ---- host -------------------------------------------------------------------------------

// Bytes of a record up to the end of its last part (the span a buffer resource covers).
inline int64_t record_span(const OomFp8Record& g) {
    const int64_t nbg = cdiv(g.inter, 128) * cdiv(g.hidden, 128) * 4;
    int64_t m = g.gate_weight + g.inter * g.hidden;
    m = std::max(m, g.gate_scale + nbg);
    m = std::max(m, g.up_weight + g.inter * g.hidden);
    m = std::max(m, g.up_scale + nbg);
    m = std::max(m, g.down_weight + g.hidden * g.inter);
    return std::max(m, g.down_scale + nbg);
}

}  // namespace oom
