// Shared pieces of the one-launch decode kernels: buffer-resource loads, the token's
// activations in registers, device-coherent hand-offs between waves, and the fixed
// header of a decode workspace (the state a decode call leaves for the next one).
#pragma once

#include <algorithm>

#include "common.hpp"
#include "grid_barrier.hpp"

namespace oom {

constexpr int BUF_FLAGS = 0x00020000;  // buffer resource word 3: 32-bit data format
constexpr int OOB = 0x7ffffff0;        // an offset past every resource: loads read 0
constexpr int BUF_SC1 = 16;            // cache-policy bit of a device-coherent (sc1) buffer load on gfx950

// ---- decode workspace header ---------------------------------------------------------
// Every decode workspace starts with this header at fixed offsets, whatever the step's
// shape, so a workspace shared by steps of different shapes (batch 1 and batch 16 of one
// model) never reads another layout's data as its state. Each counter has a 256-byte line
// of its own: atomics and polls on one line serialise at the memory side. A barrier area's
// counters only grow and agree again whenever a call ends (grid_barrier.hpp), and tickets
// are reset by their users, so only a new workspace needs clearing (oom_workspace_init).
constexpr size_t WS_BAR = 0;                                      // barrier area of a kernel's first grid meeting
constexpr size_t WS_BAR2 = WS_BAR + BAR_WORDS * 4;                // ... and of its second
constexpr int TICKET_STRIDE = 64;
constexpr int MAX_TILES = 4096 / 8;     // row tiles of 8 rows for hidden <= 4096
constexpr size_t WS_TICKETS = WS_BAR2 + BAR_WORDS * 4;            // MAX_TILES lines
constexpr size_t WS_HEADER = (WS_TICKETS + (size_t)MAX_TILES * TICKET_STRIDE * 4 + 4095) & ~size_t(4095);

// ---- phase timestamps (a profiling build only) -----------------------------------------
// Built with -DOOM_STAMPS (a profiling library made apart from liboom_hip.so:
// homelab_amd.build.build(build_dir=..., lib=..., defines=("OOM_STAMPS",))), the one-launch
// decode kernels record the device's 100 MHz real-time clock
// per wave at their phase boundaries: wave w of block b writes point p to
// stamps[(b * waves + w) * STAMP_POINTS + p] (stamps: the buffer last handed to
// oom_debug_set_stamps; none: nothing is written). The default build compiles none of it.
constexpr int STAMP_POINTS = 8;
#ifdef OOM_STAMPS
uint64_t* stamps_buffer();
#define OOM_STAMP(buf, waves, p)                                                                         \
    do {                                                                                                 \
        __builtin_amdgcn_sched_barrier(0);                                                               \
        const uint64_t t_ = wall_clock64();                                                              \
        if ((buf) && (threadIdx.x & 63) == 0)                                                            \
            (buf)[((size_t)blockIdx.x * (waves) + (threadIdx.x >> 6)) * STAMP_POINTS + (p)] = t_;        \
        __builtin_amdgcn_sched_barrier(0);                                                               \
    } while (0)
// the stamp after v is computed (v's producers complete first)
#define OOM_STAMP_AFTER(buf, waves, p, v)      \
    do {                                       \
        asm volatile("" ::"v"(v));             \
        OOM_STAMP(buf, waves, p);              \
    } while (0)
// where the wave runs, in the last point: XCC_ID (hardware register 20, bits 3:0) in bits
// 32..35, HW_ID (register 4: wave 3:0, SIMD 5:4, CU 11:8, SH 12, SE 15:13) in bits 0..31
#define OOM_STAMP_WHERE(buf, waves)                                                                      \
    do {                                                                                                 \
        const uint64_t x_ = (uint32_t)__builtin_amdgcn_s_getreg(20 | (15 << 11));                       \
        const uint64_t h_ = (uint32_t)__builtin_amdgcn_s_getreg(4 | (31 << 11));                         \
        if ((buf) && (threadIdx.x & 63) == 0)                                                            \
            (buf)[((size_t)blockIdx.x * (waves) + (threadIdx.x >> 6)) * STAMP_POINTS + STAMP_POINTS - 1] = \
                (x_ << 32) | h_;                                                                         \
    } while (0)
#else
#define OOM_STAMP_WHERE(buf, waves) \
    do {                            \
    } while (0)
#define OOM_STAMP(buf, waves, p) \
    do {                         \
    } while (0)
#define OOM_STAMP_AFTER(buf, waves, p, v) \
    do {                                  \
    } while (0)
#endif

// ---- loads ----------------------------------------------------------------------------

__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
// A streamed (read-once) 16 bytes: nontemporal, so weights that are read once do not evict
// lines that are reused (measured on the one-token decode step: 8 % faster streaming).
constexpr int BUF_NT = 2;  // cache-policy bit of a nontemporal buffer load on gfx950
__device__ __forceinline__ uint4 ld16nt(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, BUF_NT);
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
// The protocol is grid_barrier.hpp's over relaxed agent-scope atomics, which are performed
// at the device's point of coherence (not in one XCD's L2): lane q < BAR_GROUPS of the
// block's first wave handles group counter q.

// The bases of barrier area `bar`: lane q < BAR_GROUPS of the first wave reads group q's
// exit counter (every other thread returns 0). Called at kernel start by every thread;
// the value is used by the block's first wave at the barrier.
__device__ __forceinline__ uint32_t grid_barrier_base(uint32_t* bar) {
    return threadIdx.x < (unsigned)BAR_GROUPS
               ? __hip_atomic_load(bar + BAR_EXIT + threadIdx.x * BAR_STRIDE, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT)
               : 0u;
}

// The block's exit from barrier area `bar`: its last action on the area, after its wait
// (every block of the grid, exactly once per call, on every path).
__device__ __forceinline__ void grid_barrier_exit(uint32_t* bar) {
    if (threadIdx.x == 0)
        (void)__hip_atomic_fetch_add(bar + BAR_EXIT + bar_group_of(blockIdx.x, gridDim.x) * BAR_STRIDE, 1u,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The grid meets at barrier area `bar` (one area per meeting of a kernel), `base` from
// grid_barrier_base at the kernel's start; every block calls grid_barrier_exit(bar) after
// it. Every wave's earlier stores must be complete
// (wait_mem) before it reaches the barrier. A wait that gives up after `spin_limit` polls
// sets the device's status word (*status = 1, read by oom_status) and lets the block go
// on: the kernel still ends, its outputs are invalid. The launchers size the grid by the
// occupancy limit so it is resident at once; when it is not, the bounded wait turns that
// into a reported error, not a hang.
__device__ __forceinline__ void grid_barrier_words(uint32_t* bar, uint32_t base, uint32_t* status,
                                                   uint32_t spin_limit) {
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        wait_mem();  // the bases have been read before this block arrives
        if (lane == 0)
            (void)__hip_atomic_fetch_add(bar + bar_group_of(blockIdx.x, gridDim.x) * BAR_STRIDE, 1u,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t need = lane < BAR_GROUPS ? bar_target(base, 0u, (uint32_t)lane, gridDim.x) : 0u;
        uint32_t* mine = bar + (lane < BAR_GROUPS ? lane : 0) * BAR_STRIDE;
        for (uint32_t spins = 0;;) {
            const bool met = lane >= BAR_GROUPS ||
                             (int32_t)(__hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - need) >= 0;
            if (__ballot(!met) == 0) break;
            __builtin_amdgcn_s_sleep(2);
            if (++spins > spin_limit) {
                if (lane == 0) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
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
