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

// ---- wavefront reductions (wave64) -----------------------------------------------

// Sum over all 64 lanes; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sums N per-lane values v[0..N) over the wave with N - 1 + log2(64/N) exchanges
// instead of 6 N. Each round (lane offset o = 32, 16, ...) halves the values a lane
// holds: a lane with bit o set keeps the upper half and sends the lower half to its
// partner lane ^ o, which keeps the lower half. When one value is left the rest of
// the rounds are a plain butterfly. Returns the total of value lane / (64 / N),
// which every lane of that group of 64 / N lanes holds. N is a power of two <= 64.
template <int N>
__device__ __forceinline__ float wave_sum_multi(float (&v)[N], int lane) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two <= 64");
    int count = N;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        if (count > 1) {
            const int half = count / 2;
            const bool upper = (lane & o) != 0;
#pragma unroll
            for (int i = 0; i < half; i++) {
                float send = upper ? v[i] : v[i + half];
                float keep = upper ? v[i + half] : v[i];
                v[i] = keep + __shfl_xor(send, o, 64);
            }
            count = half;
        } else {
            v[0] += __shfl_xor(v[0], o, 64);
        }
    }
    return v[0];
}

}  // namespace oom
