// Turbo KV cache rows and the D = 256, G = 12 decode attention over them, on gfx950.
//
// A cache row holds one head vector of D coordinates (KvFormat, crates/oominf-core/src/
// backend.rs:571-635): bits == 0: D fp32 values; bits 2..8 (Turbo): the vector rotated by
// a fixed randomized Walsh-Hadamard transform, then per block of 32 coordinates an fp16
// scale (the block's RMS; the D/32 scales padded to 16 bytes) and `bits` 32-bit words,
// word j holding bit j of the 32 coordinates' codebook indices. A coordinate decodes as
// level[idx] * scale with the Lloyd-Max levels of a unit Gaussian (the table of
// oom_kv_codebooks, levels for b bits starting at 2^b - 4).
//
// The row codec (rotate, append, read) is one block of D threads per row, with the
// butterfly order, the block RMS and the nearest-level search of
// crates/oominf-cuda/kernels/attention.cu:9-131, so codes and scales are bit-exact against
// the oracle. The decode attention (attention.cu:584-686, flash_decode in
// crates/oominf-cuda/src/attention.rs:365-447) lists the visible keys (mask_compact,
// attention.cu:363-374), splits the list evenly over P partials (each a 32-lane half of a
// wave, lane l owning coordinates l, l + 32, ...: the reference's per-warp layout), keeps
// an online-softmax partial per (partial, query head) in fp32, and merges the partials
// per head; a rotated cache gets rotated queries and its output rotated back.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include <hip/hip_fp16.h>

#include "common.hpp"

namespace oom {

constexpr int TQ_MAXD = 256;          // coordinates a row (one block of D threads)
constexpr int TQ_LEVELS = 508;        // levels for 2..8 bits: 4 + 8 + ... + 256
constexpr int TQ_MASK_THREADS = 1024; // mask_compact's block
constexpr int TQ_G = 12;              // query heads a KV head (the decode kernel's instance)
constexpr int TQ_D = 256;             // head_dim of the decode kernel
constexpr int TQ_HW = 8;              // partials (32-lane halves) a block

__host__ __device__ inline int kv_scale_bytes(int D) { return ((D / 32) * 2 + 15) & ~15; }
__host__ __device__ inline int kv_row_bytes(int D, int bits) {
    return bits ? kv_scale_bytes(D) + (D / 32) * bits * 4 : D * 4;
}
__host__ __device__ inline int codebook_offset(int bits) { return (1 << bits) - 4; }

// The fixed random sign of coordinate i in the rotation (Knuth's multiplicative hash,
// top bit).
__device__ __forceinline__ float kv_sign(int i) { return (((unsigned)i * 2654435761u) >> 31) ? -1.0f : 1.0f; }

// Unnormalised Walsh-Hadamard transform of s[0 .. D) in LDS by the block's D threads:
// stages h = 1, 2, 4, ..., thread i < D with (i & h) == 0 forming (s[i] + s[i + h],
// s[i] - s[i + h]). Synchronises before each stage and after the last.
__device__ void tq_wht(float* s, int D) {
    for (int h = 1; h < D; h <<= 1) {
        __syncthreads();
        const int i = threadIdx.x;
        if (i < D && (i & h) == 0) {
            const float a = s[i], b = s[i + h];
            s[i] = a + b;
            s[i + h] = a - b;
        }
    }
    __syncthreads();
}

// Sum of v over the 32 lanes of this lane's half-wave by the xor butterfly 16, 8, 4, 2,
// 1 (every lane ends with the same bits).
__device__ __forceinline__ float half_xor_sum(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 32);
    return v;
}

// Coordinate d of a cache row (rotated space for Turbo rows); lv is the row's codebook.
__device__ __forceinline__ float kv_value(const uint8_t* row, int d, int D, int bits, const float* lv) {
    if (!bits) return reinterpret_cast<const float*>(row)[d];
    const int b = d >> 5, lane = d & 31;
    const float sc = __half2float(reinterpret_cast<const __half*>(row)[b]);
    const uint32_t* w = reinterpret_cast<const uint32_t*>(row + kv_scale_bytes(D)) + b * bits;
    int idx = 0;
    for (int j = 0; j < bits; j++) idx |= ((w[j] >> lane) & 1) << j;
    return lv[idx] * sc;
}

// Rotates rows of D coordinates in place: forward y = H (s . x) / sqrt(D), inverse
// x = s . (H y) / sqrt(D) (H symmetric, H H = D I). Grid: one block of D threads a row.
__global__ void __launch_bounds__(TQ_MAXD) kv_rotate_kernel(float* __restrict__ x, int D, int inverse) {
    __shared__ float s[TQ_MAXD];
    float* r = x + (size_t)blockIdx.x * D;
    const int i = threadIdx.x;
    const float norm = 1.0f / sqrtf((float)D);
    s[i] = inverse ? r[i] : r[i] * kv_sign(i);
    tq_wht(s, D);
    r[i] = inverse ? s[i] * kv_sign(i) * norm : s[i] * norm;
}

// Appends rows (src [n, D]) at cache row row0, rotated and quantised for bits 2..8 (fp32
// copies for bits 0). Grid: one block of D threads a row.
__global__ void __launch_bounds__(TQ_MAXD) kv_append_kernel(const float* __restrict__ src, uint8_t* __restrict__ cache,
                                                           int64_t row0, int D, int bits,
                                                           const float* __restrict__ levels) {
    __shared__ float s[TQ_MAXD];
    __shared__ float lv[256];
    const size_t r = blockIdx.x;
    const int i = threadIdx.x;
    const float* x = src + r * D;
    uint8_t* row = cache + ((size_t)row0 + r) * kv_row_bytes(D, bits);
    if (!bits) {
        reinterpret_cast<float*>(row)[i] = x[i];
        return;
    }
    for (int t = i; t < (1 << bits); t += blockDim.x) lv[t] = levels[codebook_offset(bits) + t];
    s[i] = x[i] * kv_sign(i);
    tq_wht(s, D);  // (its first synchronisation also publishes lv)
    const float y = s[i] / sqrtf((float)D);
    const float ss = half_xor_sum(y * y);
    const __half hs = __float2half(sqrtf(ss / 32.0f));  // round to nearest even
    const float sc = __half2float(hs);
    const float u = sc > 0.0f ? y / sc : 0.0f;
    // nearest level: bisection of the ascending codebook, then the closer neighbour
    // (ties to the lower level)
    int lo = 0, hi = (1 << bits) - 1;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (lv[mid] <= u) lo = mid;
        else hi = mid;
    }
    const int idx = fabsf(u - lv[lo]) <= fabsf(u - lv[hi]) ? lo : hi;
    const int lane = i & 31, b = i >> 5;
    if (lane == 0) reinterpret_cast<__half*>(row)[b] = hs;
    uint32_t* w = reinterpret_cast<uint32_t*>(row + kv_scale_bytes(D)) + b * bits;
    const uint64_t sh = (threadIdx.x & 32) ? 32 : 0;  // this lane's half of the wave
    for (int j = 0; j < bits; j++) {
        const uint32_t m = (uint32_t)(__ballot((idx >> j) & 1) >> sh);
        if (lane == j) w[j] = m;
    }
}

// Reads rows back as fp32 [n, D], decoded and un-rotated for bits 2..8. Grid: one block
// of D threads a row.
__global__ void __launch_bounds__(TQ_MAXD) kv_read_kernel(const uint8_t* __restrict__ cache, float* __restrict__ dst,
                                                         int D, int bits, const float* __restrict__ levels) {
    __shared__ float s[TQ_MAXD];
    __shared__ float lv[256];
    const size_t r = blockIdx.x;
    const int i = threadIdx.x;
    const uint8_t* row = cache + r * kv_row_bytes(D, bits);
    float* out = dst + r * D;
    if (!bits) {
        out[i] = reinterpret_cast<const float*>(row)[i];
        return;
    }
    for (int t = i; t < (1 << bits); t += blockDim.x) lv[t] = levels[codebook_offset(bits) + t];
    __syncthreads();
    s[i] = kv_value(row, i, D, bits, lv);
    tq_wht(s, D);
    out[i] = s[i] * kv_sign(i) / sqrtf((float)D);
}

// Inclusive prefix sum of v over the block (blockDim a multiple of 64, at most 1024):
// wave scans, then the waves' totals.
__device__ unsigned block_scan(unsigned v, unsigned* wsum) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    unsigned x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    unsigned before = 0;
    for (int w = 0; w < nw; w++)
        if (w < wave) before += wsum[w];
    __syncthreads();
    return before + x;
}

// The positions j < n with mask[j] set, in order: sel[0] = count, sel[1 ..] = positions.
// One block of TQ_MASK_THREADS; each thread takes a contiguous slice and a prefix count
// places its positions.
__global__ void __launch_bounds__(TQ_MASK_THREADS) mask_compact_kernel(const uint8_t* __restrict__ mask,
                                                                       int32_t* __restrict__ sel, int n) {
    __shared__ unsigned wsum[TQ_MASK_THREADS / 64];
    const int per = (n + (int)blockDim.x - 1) / (int)blockDim.x;
    const int lo = min(n, (int)threadIdx.x * per), hi = min(n, lo + per);
    unsigned c = 0;
    for (int j = lo; j < hi; j++) c += mask[j] != 0;
    const unsigned incl = block_scan(c, wsum);
    unsigned at = incl - c;
    for (int j = lo; j < hi; j++)
        if (mask[j]) sel[1 + at++] = j;
    if (threadIdx.x == blockDim.x - 1) sel[0] = (int32_t)incl;
}

struct TurboArgs {
    const float* q;       // [H, D] (rotated for a Turbo cache)
    const uint8_t* k;     // rows [kv_len, Hkv] of kv_row_bytes(D, kb)
    const uint8_t* v;     // rows [kv_len, Hkv] of kv_row_bytes(D, vb)
    const int32_t* sel;   // count, then the visible positions
    const float* levels;  // the codebook table (null for fp32 rows)
    float* part;          // [Hkv, P, G, D + 2]: acc[D], m, l
    float* out;           // [H, D]
    int Hkv, P, kb, vb;
    float scale;
};

// Flash-decode partials of one query token: partial p = 8 blockIdx.x + half-wave takes an
// even share of the visible positions and all G query heads of KV head blockIdx.y.
template <int G>
__global__ void __launch_bounds__(256) attn_turbo_partial_kernel(TurboArgs a) {
    constexpr int D = TQ_D, E = D / 32;  // coordinates a lane
    __shared__ float qs[G][32][E];       // qs[g][lane][e] = q[g][32 e + lane]
    __shared__ float lvk[256], lvv[256];
    const int tid = threadIdx.x, lane = tid & 31, hw = tid >> 5;
    const int kvh = blockIdx.y, p = blockIdx.x * TQ_HW + hw;
    if (a.kb)
        for (int t = tid; t < (1 << a.kb); t += blockDim.x) lvk[t] = a.levels[codebook_offset(a.kb) + t];
    if (a.vb)
        for (int t = tid; t < (1 << a.vb); t += blockDim.x) lvv[t] = a.levels[codebook_offset(a.vb) + t];
    for (int t = tid; t < G * D; t += blockDim.x) {
        const int g = t / D, d = t % D;
        qs[g][d & 31][d >> 5] = a.q[(size_t)kvh * G * D + t];
    }
    __syncthreads();
    const int krow = kv_row_bytes(D, a.kb), vrow = kv_row_bytes(D, a.vb);
    float acc[G][E], m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < E; e++) acc[g][e] = 0.0f;
    }
    const int count = a.sel[0];
    const int chunk = (count + a.P - 1) / a.P;
    const int i0 = min(count, p * chunk), i1 = min(count, i0 + chunk);
    for (int i = i0; i < i1; i++) {
        const int j = a.sel[1 + i];
        const uint8_t* kr = a.k + ((size_t)j * a.Hkv + kvh) * krow;
        const uint8_t* vr = a.v + ((size_t)j * a.Hkv + kvh) * vrow;
        float kk[E], vv[E];
#pragma unroll
        for (int e = 0; e < E; e++) {
            kk[e] = kv_value(kr, 32 * e + lane, D, a.kb, lvk);
            vv[e] = kv_value(vr, 32 * e + lane, D, a.vb, lvv);
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float dot = 0.0f;
#pragma unroll
            for (int e = 0; e < E; e++) dot = fmaf(qs[g][lane][e], kk[e], dot);
            dot = half_xor_sum(dot);
            const float s = dot * a.scale;
            const float mn = fmaxf(m[g], s);
            const float corr = expf(m[g] - mn);
            const float w = expf(s - mn);
            l[g] = l[g] * corr + w;
#pragma unroll
            for (int e = 0; e < E; e++) acc[g][e] = fmaf(acc[g][e], corr, w * vv[e]);
            m[g] = mn;
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        float* o = a.part + (((size_t)kvh * a.P + p) * G + g) * (D + 2);
#pragma unroll
        for (int e = 0; e < E; e++) o[32 * e + lane] = acc[g][e];
        if (lane == 0) {
            o[D] = m[g];
            o[D + 1] = l[g];
        }
    }
}

// out[h, d] = sum_p e^(m_p - M) acc_p[d] / sum_p e^(m_p - M) l_p over the partials of head
// h (a partial with no keys has m = -inf and weight 0). One block per head, one thread per d.
template <int G>
__global__ void __launch_bounds__(TQ_D) attn_turbo_combine_kernel(TurboArgs a) {
    constexpr int D = TQ_D;
    const int h = blockIdx.x, d = threadIdx.x, kvh = h / G, g = h % G;
    float M = -INFINITY;
    for (int p = 0; p < a.P; p++) M = fmaxf(M, a.part[(((size_t)kvh * a.P + p) * G + g) * (D + 2) + D]);
    float num = 0.0f, den = 0.0f;
    for (int p = 0; p < a.P; p++) {
        const float* pr = a.part + (((size_t)kvh * a.P + p) * G + g) * (D + 2);
        const float mp = pr[D];
        if (mp == -INFINITY) continue;
        const float w = expf(mp - M);
        num = fmaf(w, pr[d], num);
        den = fmaf(w, pr[D + 1], den);
    }
    a.out[(size_t)h * D + d] = num / den;
}

// ---- host ---------------------------------------------------------------------------

// The 2^bits Lloyd-Max levels of a unit Gaussian (KvFormat::codebooks,
// crates/oominf-core/src/backend.rs:637-700): levels start evenly over +-(4 + bits / 4);
// each round puts the cell edges halfway between levels and moves every level to its
// cell's conditional mean (pdf(a) - pdf(b)) / (Q(a) - Q(b)), with the upper tail Q from
// the Numerical Recipes erfc approximation (erfcc, fractional error below 1.2e-7),
// until no level moves by 1e-12 (at most 200000 rounds); f64 throughout, f32 out.
static std::vector<float> lloyd_max_gaussian(int bits) {
    const int n = 1 << bits;
    const double SQRT_2 = 1.4142135623730951, TWO_PI = 6.283185307179586;
    auto pdf = [&](double x) { return std::exp(-0.5 * x * x) / std::sqrt(TWO_PI); };
    auto q = [&](double x) {
        const double z = std::fabs(x) / SQRT_2;
        const double t = 1.0 / (1.0 + 0.5 * z);
        const double erfc =
            t * std::exp(-z * z - 1.26551223 +
                         t * (1.00002368 +
                              t * (0.37409196 +
                                   t * (0.09678418 +
                                        t * (-0.18628806 +
                                             t * (0.27886807 +
                                                  t * (-1.13520398 +
                                                       t * (1.48851587 + t * (-0.82215223 + t * 0.17087277)))))))));
        return x >= 0.0 ? 0.5 * erfc : 1.0 - 0.5 * erfc;
    };
    const double span = 4.0 + bits * 0.25;
    std::vector<double> c(n), next(n);
    for (int i = 0; i < n; i++) c[i] = -span + 2.0 * span * (i + 0.5) / n;
    for (int round = 0; round < 200000; round++) {
        double moved = 0.0;
        for (int i = 0; i < n; i++) {
            const double a = i == 0 ? -INFINITY : 0.5 * (c[i - 1] + c[i]);
            const double b = i + 1 == n ? INFINITY : 0.5 * (c[i] + c[i + 1]);
            const double pa = std::isfinite(a) ? pdf(a) : 0.0, pb = std::isfinite(b) ? pdf(b) : 0.0;
            const double mass = q(a) - q(b);
            const double mv = mass > 0.0 ? (pa - pb) / mass : c[i];
            moved = std::max(moved, std::fabs(mv - c[i]));
            next[i] = mv;
        }
        c.swap(next);
        if (moved < 1e-12) break;
    }
    std::vector<float> out(n);
    for (int i = 0; i < n; i++) out[i] = (float)c[i];
    return out;
}

static const std::vector<float>& codebooks() {
    static std::once_flag once;
    static std::vector<float> table;
    std::call_once(once, [] {
        for (int b = 2; b <= 8; b++) {
            const std::vector<float> l = lloyd_max_gaussian(b);
            table.insert(table.end(), l.begin(), l.end());
        }
    });
    return table;
}

// Rows of d coordinates stored at `bits` (0: fp32): one block of d threads a row, and a
// power-of-two d for the rotation (kv_row_shape, crates/oominf-cuda/src/attention.rs:351-356).
static bool kv_row_shape(int d, int bits) {
    return d >= 32 && d % 32 == 0 && d <= TQ_MAXD && (bits == 0 || ((d & (d - 1)) == 0 && bits >= 2 && bits <= 8));
}

// Partials of the decode attention: about 16 visible keys each, at most 4096 keys
// counted, a multiple of the block's 8 (attention.rs:417-419).
static int turbo_partials(int kv_len) {
    const int p = (std::min(kv_len, 4096) + 15) / 16;
    return (p + TQ_HW - 1) / TQ_HW * TQ_HW;
}

struct TurboWs {
    size_t sel, qrot, part, total;
};

static size_t t_al256(size_t v) { return (v + 255) & ~size_t(255); }

static TurboWs turbo_ws(int heads, int kv_heads, int d, int kv_len) {
    TurboWs w;
    w.sel = 0;
    w.qrot = t_al256((size_t)(kv_len + 1) * 4);
    w.part = w.qrot + t_al256((size_t)heads * d * 4);
    w.total = w.part + t_al256((size_t)kv_heads * turbo_partials(kv_len) * (heads / kv_heads) * (d + 2) * 4);
    return w;
}

}  // namespace oom

// ---- C ABI ------------------------------------------------------------------------------

extern "C" size_t oom_kv_codebook_size(void) { return oom::TQ_LEVELS; }

extern "C" int oom_kv_codebooks(float* levels, size_t n) {
    using namespace oom;
    OOM_REQUIRE(levels && n >= (size_t)TQ_LEVELS, "oom_kv_codebooks: room for 508 levels");
    const std::vector<float>& t = codebooks();
    std::copy(t.begin(), t.end(), levels);
    return OOM_OK;
}

extern "C" size_t oom_kv_row_bytes(int d, int bits) {
    if (!oom::kv_row_shape(d, bits)) return 0;
    return (size_t)oom::kv_row_bytes(d, bits);
}

extern "C" int oom_kv_rotate(float* x, int rows, int d, int inverse, void* stream) {
    using namespace oom;
    OOM_REQUIRE(kv_row_shape(d, 4) && rows >= 0, "oom_kv_rotate: d must be a power of two, 32..256");
    if (rows == 0) return OOM_OK;
    OOM_REQUIRE(x, "oom_kv_rotate: null buffer");
    hipLaunchKernelGGL(kv_rotate_kernel, dim3((unsigned)rows), dim3(d), 0, as_stream(stream), x, d, inverse ? 1 : 0);
    return launched("oom_kv_rotate");
}

extern "C" int oom_kv_append(const float* src, uint8_t* cache, int64_t start, int t, int kv_heads, int d, int bits,
                             const float* levels, void* stream) {
    using namespace oom;
    OOM_REQUIRE(kv_row_shape(d, bits), "oom_kv_append: d a multiple of 32 up to 256 (a power of two for bits 2..8)");
    OOM_REQUIRE(t >= 0 && kv_heads >= 1 && start >= 0, "oom_kv_append: shape");
    const int64_t rows = (int64_t)t * kv_heads;
    if (rows == 0) return OOM_OK;
    OOM_REQUIRE(rows < (1ll << 31), "oom_kv_append: too many rows");
    OOM_REQUIRE(src && cache && (bits == 0 || levels), "oom_kv_append: null buffer");
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)rows), dim3(d), 0, as_stream(stream), src, cache,
                       start * kv_heads, d, bits, levels);
    return launched("oom_kv_append");
}

extern "C" int oom_kv_read(const uint8_t* cache, float* dst, int len, int kv_heads, int d, int bits,
                           const float* levels, void* stream) {
    using namespace oom;
    OOM_REQUIRE(kv_row_shape(d, bits), "oom_kv_read: d a multiple of 32 up to 256 (a power of two for bits 2..8)");
    OOM_REQUIRE(len >= 0 && kv_heads >= 1, "oom_kv_read: shape");
    const int64_t rows = (int64_t)len * kv_heads;
    if (rows == 0) return OOM_OK;
    OOM_REQUIRE(rows < (1ll << 31), "oom_kv_read: too many rows");
    OOM_REQUIRE(cache && dst && (bits == 0 || levels), "oom_kv_read: null buffer");
    hipLaunchKernelGGL(kv_read_kernel, dim3((unsigned)rows), dim3(d), 0, as_stream(stream), cache, dst, d, bits,
                       levels);
    return launched("oom_kv_read");
}

extern "C" int oom_mask_compact(const uint8_t* mask, int32_t* sel, int n, void* stream) {
    using namespace oom;
    OOM_REQUIRE(n >= 0 && mask && sel, "oom_mask_compact: null buffer or negative length");
    hipLaunchKernelGGL(mask_compact_kernel, dim3(1), dim3(TQ_MASK_THREADS), 0, as_stream(stream), mask, sel, n);
    return launched("oom_mask_compact");
}

extern "C" size_t oom_attn_decode_turbo_workspace_size(int heads, int kv_heads, int d, int kv_len) {
    if (heads < 1 || kv_heads < 1 || d < 1 || kv_len < 1 || heads % kv_heads) return 0;
    return oom::turbo_ws(heads, kv_heads, d, kv_len).total;
}

extern "C" int oom_attn_decode_turbo(const float* q, const uint8_t* k, const uint8_t* v, int k_bits, int v_bits,
                                     const float* levels, const uint8_t* mask, int heads, int kv_heads, int d,
                                     int kv_len, float scale, float* out, void* ws, size_t ws_bytes, void* stream) {
    using namespace oom;
    OOM_REQUIRE(d == TQ_D && kv_heads >= 1 && heads == TQ_G * kv_heads,
                "oom_attn_decode_turbo: head_dim 256 and 12 query heads a KV head");
    OOM_REQUIRE(kv_row_shape(d, k_bits) && kv_row_shape(d, v_bits) && (k_bits == 0) == (v_bits == 0),
                "oom_attn_decode_turbo: k_bits and v_bits both 0 (fp32) or both 2..8");
    OOM_REQUIRE(kv_len >= 1, "oom_attn_decode_turbo: kv_len must be >= 1");
    OOM_REQUIRE((int64_t)kv_len * kv_heads * kv_row_bytes(d, std::max(k_bits, v_bits)) < (1ll << 40),
                "oom_attn_decode_turbo: cache too large");
    OOM_REQUIRE(q && k && v && mask && out && (k_bits == 0 || levels), "oom_attn_decode_turbo: null buffer");
    const TurboWs w = turbo_ws(heads, kv_heads, d, kv_len);
    if (!ws || ws_bytes < w.total)
        return fail(OOM_ERR_WORKSPACE,
                    "oom_attn_decode_turbo: workspace smaller than oom_attn_decode_turbo_workspace_size()");
    OOM_REQUIRE(aligned(ws, 256), "oom_attn_decode_turbo: workspace must be 256-byte aligned");
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    hipStream_t st = as_stream(stream);
    const bool rotated = k_bits != 0;
    TurboArgs a{};
    a.q = q;
    if (rotated) {
        float* qr = reinterpret_cast<float*>(base + w.qrot);
        if (hipMemcpyAsync(qr, q, (size_t)heads * d * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
            return launched("oom_attn_decode_turbo");
        hipLaunchKernelGGL(kv_rotate_kernel, dim3((unsigned)heads), dim3(d), 0, st, qr, d, 0);
        if (int rc = launched("oom_attn_decode_turbo")) return rc;
        a.q = qr;
    }
    int32_t* sel = reinterpret_cast<int32_t*>(base + w.sel);
    hipLaunchKernelGGL(mask_compact_kernel, dim3(1), dim3(TQ_MASK_THREADS), 0, st, mask, sel, kv_len);
    if (int rc = launched("oom_attn_decode_turbo")) return rc;
    a.k = k;
    a.v = v;
    a.sel = sel;
    a.levels = levels;
    a.part = reinterpret_cast<float*>(base + w.part);
    a.out = out;
    a.Hkv = kv_heads;
    a.P = turbo_partials(kv_len);
    a.kb = k_bits;
    a.vb = v_bits;
    a.scale = scale;
    hipLaunchKernelGGL(attn_turbo_partial_kernel<TQ_G>, dim3((unsigned)(a.P / TQ_HW), (unsigned)kv_heads), dim3(256), 0,
                       st, a);
    if (int rc = launched("oom_attn_decode_turbo")) return rc;
    hipLaunchKernelGGL(attn_turbo_combine_kernel<TQ_G>, dim3((unsigned)heads), dim3(TQ_D), 0, st, a);
    if (int rc = launched("oom_attn_decode_turbo")) return rc;
    if (rotated) hipLaunchKernelGGL(kv_rotate_kernel, dim3((unsigned)heads), dim3(d), 0, st, out, d, 1);
    return launched("oom_attn_decode_turbo");
}
