// Shared device helpers and C-ABI plumbing for the gfx950 (MI355X) hot-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/oom_hip.h"

namespace oom {

// ---- errors (C ABI) --------------------------------------------------------------

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Maps a HIP launch status to OOM_OK / OOM_ERR_LAUNCH with the runtime's message.
int launched(const char* what);

// Polls of a bounded wait before it gives up (oom_set_wait_limit changes it).
constexpr uint32_t DEFAULT_WAIT_LIMIT = 1u << 22;
// The current device's status word (set by a kernel whose bounded wait gave up), or
// nullptr if the runtime gives it no address; the spin limit of bounded waits.
uint32_t* status_word();
uint32_t wait_limit();

#define OOM_REQUIRE(cond, msg)                                 \
    do {                                                       \
        if (!(cond)) return ::oom::fail(OOM_ERR_ARG, (msg));   \
    } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- number formats ---------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Round to nearest even; NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7fffffffu) > 0x7f800000u) return uint16_t((b >> 16) | 0x40);
    return uint16_t((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

// Four e4m3fn codes (one 32-bit word, byte 0 first) to fp32, exactly, with the
// gfx950 OCP-FP8 conversion (v_cvt_pk_f32_fp8): S.1111.111 reads as NaN.
__device__ __forceinline__ void e4m3x4(uint32_t w, float* out) {
    auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(int(w), false);
    auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(int(w), true);
    out[0] = lo[0];
    out[1] = lo[1];
    out[2] = hi[0];
    out[3] = hi[1];
}

// Sixteen e4m3 codes of a 128-bit load to fp32.
__device__ __forceinline__ void e4m3x16(const uint4& v, float* out) {
    e4m3x4(v.x, out);
    e4m3x4(v.y, out + 4);
    e4m3x4(v.z, out + 8);
    e4m3x4(v.w, out + 12);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// sum_i w[i] * x[i] over 16 e4m3 weights (one 128-bit load) and 16 bf16 activations
// (8 packed words), fp32 accumulate: each weight pair converts exactly to a bf16 pair
// (v_cvt_scalef32_pk_bf16_fp8, scale 1) and meets its activation pair in one
// v_dot2c_f32_bf16 (bf16 products are exact in fp32).
__device__ __forceinline__ float dot16_e4m3_bf16(const uint4& w, const uint32_t* xw) {
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const bf16x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(ww[i], 1.0f, false);
        const bf16x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(ww[i], 1.0f, true);
        p = __builtin_amdgcn_fdot2_f32_bf16(lo, __builtin_bit_cast(bf16x2_t, xw[2 * i]), p, false);
        p = __builtin_amdgcn_fdot2_f32_bf16(hi, __builtin_bit_cast(bf16x2_t, xw[2 * i + 1]), p, false);
    }
    return p;
}

// Activations in either element type.
template <int DT>
__device__ __forceinline__ float load_act(const void* p, size_t i) {
    if constexpr (DT == OOM_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    else return reinterpret_cast<const float*>(p)[i];
}

template <int DT>
__device__ __forceinline__ void store_out(void* p, size_t i, float v) {
    if constexpr (DT == OOM_BF16) reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
    else reinterpret_cast<float*>(p)[i] = v;
}

__device__ __forceinline__ float siluf(float v) { return v / (1.0f + expf(-v)); }

// Compiler-only ordering for an exchange through LDS inside one wave: a wave's LDS
// operations complete in issue order, so another lane's ds_write is visible to a later
// ds_read of the same wave; no wait on outstanding global memory operations is needed.
__device__ __forceinline__ void wave_lds_order() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- wavefront reductions (wave64) -----------------------------------------------

// v of another lane through DPP (no LDS): CTRL is a gfx9 dpp_ctrl code.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_XOR3 = 0x1B;         // quad_perm [3,2,1,0]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <-> 7 - i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <-> 15 - i within 16
constexpr int DPP_ROR8 = 0x128;        // row_ror:8, lane i <- i ^ 8 within 16

// The value of lane ^ O for every lane of a fully active wave, without the LDS
// crossbar: O = 1, 2 by quad permutes; 4 by a half-row mirror (i ^ 7) then a quad
// reversal (^ 3); 8 by a row rotation; 16 and 32 by v_permlane16_swap /
// v_permlane32_swap of the value with itself, which leaves the two rows (halves) of
// each pair in the two results: a lane in an even row (lower half) finds its partner
// in the second result, a lane in an odd row (upper half) in the first.
template <int O>
__device__ __forceinline__ float lane_xor(float v, int lane) {
    if constexpr (O == 1) return dpp_f32<DPP_XOR1>(v);
    else if constexpr (O == 2) return dpp_f32<DPP_XOR2>(v);
    else if constexpr (O == 4) return dpp_f32<DPP_XOR3>(dpp_f32<DPP_HALF_MIRROR>(v));
    else if constexpr (O == 8) return dpp_f32<DPP_ROR8>(v);
    else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float((lane & 16) ? r[0] : r[1]);
    } else {
        static_assert(O == 32, "lane_xor: O is a power of two <= 32");
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float((lane & 32) ? r[0] : r[1]);
    }
}

// lane_xor with the offset as a value (folds to one case once loops over o unroll).
__device__ __forceinline__ float lane_xor_n(float v, int o, int lane) {
    switch (o) {
        case 1: return lane_xor<1>(v, lane);
        case 2: return lane_xor<2>(v, lane);
        case 4: return lane_xor<4>(v, lane);
        case 8: return lane_xor<8>(v, lane);
        case 16: return lane_xor<16>(v, lane);
        default: return lane_xor<32>(v, lane);
    }
}

// Sum over each 32-lane half with the pairing of a 32-lane xor butterfly (partners
// lane ^ 1, ^ 2, ^ 4, ^ 8, ^ 16), so the total has the butterfly's rounding. Steps
// 3 and 4 use DPP mirrors: after the previous steps every lane of a quad (of a group
// of 8) holds the same value, so the mirror partner's value is the xor partner's.
// Step 5 adds the two rows of each pair (v_permlane16_swap), own + partner.
__device__ __forceinline__ float sum32_xor_order(float v) {
    v += dpp_f32<DPP_XOR1>(v);
    v += dpp_f32<DPP_XOR2>(v);
    v += dpp_f32<DPP_HALF_MIRROR>(v);
    v += dpp_f32<DPP_MIRROR>(v);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Maximum over the wave (order-free).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f32<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f32<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f32<DPP_MIRROR>(v));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// Sum over all 64 lanes; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
    v = sum32_xor_order(v);
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Sums N per-lane values v[0..N) over groups of 2 TOP lanes (TOP = 32: the whole wave;
// 16: each half) with N - 1 + log2(2 TOP / N) exchanges instead of N log2(2 TOP). Each
// round (lane offset o = TOP, TOP / 2, ...) halves the values a lane holds: a lane with
// bit o set keeps the upper half and sends the lower half to its partner lane ^ o,
// which keeps the lower half. When one value is left the rest of the rounds are a
// plain butterfly. Value g's total ends in every lane of sub-group g of 2 TOP / N
// lanes, g = (lane % (2 TOP)) / (2 TOP / N). N is a power of two <= 2 TOP.
template <int N, int TOP = 32>
__device__ __forceinline__ float wave_sum_multi(float (&v)[N], int lane) {
    static_assert(N >= 1 && N <= 2 * TOP && (N & (N - 1)) == 0, "N must be a power of two <= 2 TOP");
    int count = N;
#pragma unroll
    for (int o = TOP; o >= 1; o >>= 1) {
        if (count > 1) {
            const int half = count / 2;
            // lanes with bit o set send the lower half; the choice is a bit blend through a
            // mask the compiler cannot see through: written as `upper ? v[i] : v[i + half]`
            // it becomes one read of v at a lane-varying index, lowered to a compare and
            // select over every element of v
            uint32_t m = (lane & o) ? ~0u : 0u;
            asm("" : "+v"(m));
#pragma unroll
            for (int i = 0; i < half; i++) {
                const uint32_t lo = __float_as_uint(v[i]), hi = __float_as_uint(v[i + half]);
                const float send = __uint_as_float((lo & m) | (hi & ~m));
                const float keep = __uint_as_float((hi & m) | (lo & ~m));
                v[i] = keep + lane_xor_n(send, o, lane);
            }
            count = half;
        } else {
            v[0] += lane_xor_n(v[0], o, lane);
        }
    }
    return v[0];
}

}  // namespace oom
