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
// The row codec (rotate, append, read) keeps a row in registers across D / 4 lanes of one
// wave (four coordinates a lane, 256 / D rows a wave): the butterflies run in the lane and
// across lanes by DPP and permlane moves, the block RMS by an 8-lane exchange, and the
// codes are packed by OR-ing the lanes' nibbles. The arithmetic is the format's, fixed by
// crates/oominf-cuda/kernels/attention.cu:9-131 (stage order, 1/sqrt(D) after the
// butterflies, the 32-way xor pairing of the RMS sum, fp16 scales rounded to nearest even,
// nearest level by bisection with ties to the lower level), so codes and scales are
// bit-exact against the oracle. The decode attention (attention.cu:584-686, flash_decode in
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

#include "stream.hpp"

namespace oom {

constexpr int TQ_MAXD = 256;          // coordinates a row
constexpr int TQ_LEVELS = 508;        // levels for 2..8 bits: 4 + 8 + ... + 256
constexpr int TQ_MASK_THREADS = 1024; // mask_compact's block
constexpr int TQ_G = 12;              // query heads a KV head (the decode kernel's instance)
constexpr int TQ_D = 256;             // head_dim of the decode kernel

__host__ __device__ inline int kv_scale_bytes(int D) { return ((D / 32) * 2 + 15) & ~15; }
__host__ __device__ inline int kv_row_bytes(int D, int bits) {
    return bits ? kv_scale_bytes(D) + (D / 32) * bits * 4 : D * 4;
}
__host__ __device__ inline int codebook_offset(int bits) { return (1 << bits) - 4; }

// The rotation's sign of coordinate i: the top bit of Knuth's multiplicative hash of i
// (the cache format fixes it, so it is computed, not stored).
__device__ __forceinline__ float kv_sign(int i) { return (((unsigned)i * 2654435761u) >> 31) ? -1.0f : 1.0f; }

// ---- rows, one wave per 256 / D rows ------------------------------------------------
// A row of D coordinates (D = 32, 64, 128 or 256) sits in D / 4 consecutive lanes of a
// wave: lane l of the row (l = lane % (D / 4)) holds coordinates 4 l .. 4 l + 3 in
// registers, one 16-byte load of an fp32 row, and a 32-coordinate block of the row is 8
// neighbouring lanes. Every lane stays active through the cross-lane steps (DPP and
// permlane read whole rows of lanes); only memory operations are predicated. No multiply
// and add fuse here (fp contract off): the format's arithmetic rounds each product (a
// decoded level times its scale, a square) before it enters a butterfly or a sum.
constexpr int TR_WAVES = 4;  // waves a block of the row kernels

// Walsh-Hadamard butterflies over the row in the format's stage order h = 1, 2, ..., D / 2,
// each pair (i, i + h) becoming (s_i + s_{i+h}, s_i - s_{i+h}): stages 1 and 2 inside the
// lane, stage 4 o with the lane l ^ o (the lane whose bit o is clear keeps the sum, the
// other the lower coordinate's value minus its own).
template <int D>
__device__ __forceinline__ void row_wht(float (&x)[4], int lane) {
#pragma clang fp contract(off)
    const float a0 = x[0] + x[1], a1 = x[0] - x[1], a2 = x[2] + x[3], a3 = x[2] - x[3];
    x[0] = a0 + a2;
    x[2] = a0 - a2;
    x[1] = a1 + a3;
    x[3] = a1 - a3;
#pragma unroll
    for (int o = 1; 4 * o < D; o <<= 1) {
        const bool upper = (lane & o) != 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = lane_xor_n(x[i], o, lane);
            x[i] = upper ? p - x[i] : x[i] + p;
        }
    }
}

// The sum of a 32-coordinate block's values v (this lane's four of them) with the pairing
// of a 32-way xor butterfly over the coordinates, partner offsets 16, 8, 4, 2, 1 in that
// order: offsets 16, 8 and 4 are the lanes l ^ 4, l ^ 2, l ^ 1 of the block's 8, offsets 2
// and 1 the lane's own coordinates. Every lane of the block ends with the same bits.
__device__ __forceinline__ float block_xor_sum(float (&v)[4], int lane) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = v[i] + lane_xor<4>(v[i], lane);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = v[i] + lane_xor<2>(v[i], lane);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = v[i] + lane_xor<1>(v[i], lane);
    const float p0 = v[0] + v[2], p1 = v[1] + v[3];
    return p0 + p1;
}

// OR of a 32-bit value over the 8 lanes of a block (every lane ends with it).
__device__ __forceinline__ uint32_t block_or(uint32_t v, int lane) {
    v |= __float_as_uint(lane_xor<1>(__uint_as_float(v), lane));
    v |= __float_as_uint(lane_xor<2>(__uint_as_float(v), lane));
    v |= __float_as_uint(lane_xor<4>(__uint_as_float(v), lane));
    return v;
}

// The row this lane serves (rows past n: memory operations skipped) and its lane in the row.
template <int D>
__device__ __forceinline__ int64_t row_of(int lane, int& l) {
    constexpr int LPR = D / 4;
    l = lane % LPR;
    return ((int64_t)blockIdx.x * TR_WAVES + (threadIdx.x >> 6)) * (64 / LPR) + lane / LPR;
}

// Rotates rows of D coordinates in place: forward y = H (s . x) / sqrt(D), inverse
// x = s . (H y) / sqrt(D) (H symmetric, H H = D I).
template <int D>
__global__ void __launch_bounds__(64 * TR_WAVES) kv_rotate_kernel(float* __restrict__ x, int64_t rows, int inverse) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    int l;
    const int64_t r = row_of<D>(lane, l);
    const bool ok = r < rows;
    float* p = x + r * D + 4 * l;  // four fp32 accesses a lane: the ABI asks 4-byte alignment only
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = ok ? p[i] : 0.0f;
    const float norm = 1.0f / sqrtf((float)D);
    if (!inverse) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] *= kv_sign(4 * l + i);
    }
    row_wht<D>(v, lane);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = inverse ? v[i] * kv_sign(4 * l + i) * norm : v[i] * norm;
    if (ok) {
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = v[i];
    }
}

// Appends rows (src [n, D] fp32) as Turbo rows of `bits` at cache row row0: rotated
// (y = H (s . x) / sqrt(D)), per block of 32 the fp16 RMS scale (round to nearest even),
// each coordinate the nearest codebook level of y / scale (bisection of the ascending
// levels, then the closer neighbour, ties to the lower level), and the codes as `bits`
// bit-plane words per block. lv_all: the 508-level table of oom_kv_codebooks.
template <int D>
__global__ void __launch_bounds__(64 * TR_WAVES) kv_append_kernel(const float* __restrict__ src,
                                                                 uint8_t* __restrict__ cache, int64_t row0,
                                                                 int64_t rows, int bits,
                                                                 const float* __restrict__ lv_all) {
#pragma clang fp contract(off)
    __shared__ float lv[256];
    const int lane = threadIdx.x & 63, n = 1 << bits;
    for (int t = threadIdx.x; t < n; t += blockDim.x) lv[t] = lv_all[codebook_offset(bits) + t];
    int l;
    const int64_t r = row_of<D>(lane, l);
    const bool ok = r < rows;
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = ok ? src[r * D + 4 * l + i] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] *= kv_sign(4 * l + i);
    row_wht<D>(y, lane);
    float sq[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        y[i] = y[i] / sqrtf((float)D);
        sq[i] = y[i] * y[i];
    }
    const float ss = block_xor_sum(sq, lane);
    const __half hs = __float2half(sqrtf(ss / 32.0f));  // round to nearest even
    const float sc = __half2float(hs);
    __syncthreads();  // the levels are in LDS
    int idx[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float u = sc > 0.0f ? y[i] / sc : 0.0f;
        int lo = 0, hi = n - 1;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (lv[mid] <= u) lo = mid;
            else hi = mid;
        }
        idx[i] = fabsf(u - lv[lo]) <= fabsf(u - lv[hi]) ? lo : hi;
    }
    // word j of the block: bit t = 4 (l % 8) + i is bit j of coordinate t's code; the 8
    // lanes OR their nibbles together and lane l % 8 == j keeps word j
    const int lb = l & 7, b = l >> 3;
    uint32_t mine = 0;
    for (int j = 0; j < bits; j++) {
        uint32_t nib = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) nib |= (uint32_t)((idx[i] >> j) & 1) << i;
        const uint32_t w = block_or(nib << (4 * lb), lane);
        mine = lb == j ? w : mine;
    }
    if (ok) {
        uint8_t* row = cache + (row0 + r) * kv_row_bytes(D, bits);
        if (lb == 0) reinterpret_cast<__half*>(row)[b] = hs;
        if (lb < bits) reinterpret_cast<uint32_t*>(row + kv_scale_bytes(D))[b * bits + lb] = mine;
    }
}

// Reads Turbo rows of `bits` back as fp32 [n, D]: each coordinate level[code] * scale of its
// block, then un-rotated: x = s . (H y) / sqrt(D).
template <int D>
__global__ void __launch_bounds__(64 * TR_WAVES) kv_read_kernel(const uint8_t* __restrict__ cache,
                                                               float* __restrict__ dst, int64_t rows, int bits,
                                                               const float* __restrict__ lv_all) {
#pragma clang fp contract(off)
    __shared__ float lv[256];
    const int lane = threadIdx.x & 63, n = 1 << bits;
    for (int t = threadIdx.x; t < n; t += blockDim.x) lv[t] = lv_all[codebook_offset(bits) + t];
    int l;
    const int64_t r = row_of<D>(lane, l);
    const bool ok = r < rows;
    const int lb = l & 7, b = l >> 3;
    const uint8_t* row = cache + (ok ? r : 0) * kv_row_bytes(D, bits);
    const float sc = ok ? __half2float(reinterpret_cast<const __half*>(row)[b]) : 0.0f;
    const uint32_t* wd = reinterpret_cast<const uint32_t*>(row + kv_scale_bytes(D)) + b * bits;
    int idx[4] = {0, 0, 0, 0};
    for (int j = 0; j < bits; j++) {
        const uint32_t w = ok ? wd[j] : 0u;
#pragma unroll
        for (int i = 0; i < 4; i++) idx[i] |= (int)((w >> (4 * lb + i)) & 1u) << j;
    }
    __syncthreads();  // the levels are in LDS
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = lv[idx[i]] * sc;
    row_wht<D>(v, lane);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = v[i] * kv_sign(4 * l + i) / sqrtf((float)D);
    if (ok) {
#pragma unroll
        for (int i = 0; i < 4; i++) dst[r * D + 4 * l + i] = v[i];
    }
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

// Nonzero bytes of a dword: each byte's bits or-ed down to its bit 0, then counted.
__device__ __forceinline__ unsigned nonzero_bytes(uint32_t x) {
    x |= x >> 4;
    x |= x >> 2;
    x |= x >> 1;
    return __popc(x & 0x01010101u);
}

// Mask bytes 16 q .. 16 q + 15 (zeros past n): one 16-byte load, or byte loads for a last
// chunk that ends past n (the buffer's bounds check works on whole dwords).
__device__ __forceinline__ uint4 mask_chunk(__amdgpu_buffer_rsrc_t mr, int q, int n) {
    if (16 * q + 16 <= n) return ld16(mr, 16 * q);
    uint32_t w[4] = {0, 0, 0, 0};
    for (int j = 0; 16 * q + j < n; j++)
        w[j >> 2] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(mr, 16 * q + j, 0, 0) << (8 * (j & 3));
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// The positions j < n with mask[j] set, in order: sel[0] = count, sel[1 ..] = positions.
// One block of TQ_MASK_THREADS; each thread takes a contiguous run of 16-byte chunks
// (one buffer load each, zeros past n), counts its visible bytes, and a block prefix sum
// places its positions.
__global__ void __launch_bounds__(TQ_MASK_THREADS) mask_compact_kernel(const uint8_t* __restrict__ mask,
                                                                       int32_t* __restrict__ sel, int n) {
    __shared__ unsigned wsum[TQ_MASK_THREADS / 64];
    const __amdgpu_buffer_rsrc_t mr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(mask), (short)0, n,
                                                                        BUF_FLAGS);
    const int nchunks = (n + 15) / 16;
    const int per = (nchunks + (int)blockDim.x - 1) / (int)blockDim.x;
    const int lo = min(nchunks, (int)threadIdx.x * per), hi = min(nchunks, lo + per);
    unsigned c = 0;
    for (int q = lo; q < hi; q++) {
        const uint4 x = mask_chunk(mr, q, n);
        c += nonzero_bytes(x.x) + nonzero_bytes(x.y) + nonzero_bytes(x.z) + nonzero_bytes(x.w);
    }
    const unsigned incl = block_scan(c, wsum);
    unsigned at = incl - c;
    for (int q = lo; q < hi; q++) {
        const uint4 x = mask_chunk(mr, q, n);
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int j = 0; j < 16; j++)
            if ((w[j >> 2] >> (8 * (j & 3))) & 0xff) sel[1 + at++] = 16 * q + j;
    }
    if (threadIdx.x == blockDim.x - 1) sel[0] = (int32_t)incl;
}

// ---- decode attention (d = 256, 12 query heads a KV head) ------------------------------
//
// Work split: keys go in groups of 16 consecutive positions; wave w of a KV head's W waves
// takes groups w, w + W, w + 2 W, ..., one a round, so a block-sparse mask
// spreads over the waves. A key that is masked (or past kv_len) gets probability exactly 0
// and its rows are not read: the result is the softmax over the visible keys with no
// compaction pass. Each block merges its waves' online-softmax states in LDS and writes
// one partial a head; attn_turbo_combine_kernel merges the blocks' partials by
// max-rescale and rotates the result back.
//
// Matrix layout (v_mfma_f32_16x16x4f32, fp32 products and sums; lane l = 16 r + m):
// scores are formed transposed, S^T[key][head] = K Q^T over 16 keys and 16 head rows (12
// used), four coordinates a step. Lane (m, r) supplies key m's coordinates 64 r .. 64 r +
// 63 (Turbo blocks 2 r and 2 r + 1) and head m's same coordinates, and ends holding
// S^T[4 r + e][m] -- already the A operand P[m][4 r + e] of O = P V. There lane (m, r)
// supplies V[4 r + e][16 m + t] (half block 16 m .. 16 m + 15) and holds
// O[4 r + e][16 m + t], t < 16.
//
// Decoding: a lane takes a block's bit planes (word j holds bit j of the 32 codes) and
// transposes them to one code a byte with three field swaps between plane pairs (about
// 1.5 VALU operations a coordinate), then looks the level up in an LDS copy of the
// codebook and multiplies by the block's scale -- the same f32 product as the reference's
// per-coordinate decode.
constexpr int TT_WAVES = 8;  // waves a block: two a SIMD, so one wave's MFMAs overlap the other's decoding
constexpr int TT_GPW = 2;    // groups of 16 keys a wave is sized for (one a round)
constexpr int TT_QS = 260;   // LDS row stride (floats) of a query head
constexpr int TQ_OOB = 0x70000000;  // an offset past every buffer here: loads read 0
constexpr int TC_THREADS = 1024;    // combine block: 4 slices of the partials x 256 coordinates
constexpr int TC_BATCH = 32;        // partials a combine thread loads at once

typedef float tq_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t tq_u2 __attribute__((ext_vector_type(2)));

struct TurboArgs {
    const float* q;       // [Hkv * 12, 256] as given
    const uint8_t* k;     // rows [kv_len, Hkv] of kv_row_bytes(256, kb)
    const uint8_t* v;     // rows [kv_len, Hkv] of kv_row_bytes(256, vb)
    const uint8_t* mask;  // [kv_len], nonzero = visible
    const float* levels;  // the codebook table (Turbo rows)
    float* part;          // [Hkv, nblk, 12, 256]: a block's un-normalised output
    float* ml;            // [Hkv, nblk, 12, 2]: its max and sum of exponentials
    float* out;           // [Hkv * 12, 256]
    int Hkv, kv_len, nblk, kb, vb;
    float scale;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tq_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, BUF_FLAGS);
}

// Position (in the order the score steps read) of coordinate c of a query head: within
// each 32-coordinate block, column 8 i + k is read at step 4 k + i.
__device__ __forceinline__ int tq_qperm(int c) { return (c & ~31) + 4 * (c & 7) + ((c >> 3) & 3); }

// Swaps S-bit fields between two bit-plane words (the three stages of tq_codes).
template <int S>
__device__ __forceinline__ void tq_swap(uint32_t& a, uint32_t& b) {
    constexpr uint32_t M = S == 1 ? 0x55555555u : S == 2 ? 0x33333333u : 0x0F0F0F0Fu;
    const uint32_t na = (a & ~(M << S)) | ((b << S) & (M << S));
    const uint32_t nb = (b & ~M) | ((a >> S) & M);
    a = na;
    b = nb;
}
// Bit-matrix transpose: on entry bit c of w[j] is bit j of column c's code; on exit byte
// i of w[k] is the code of column 8 i + k.
__device__ __forceinline__ void tq_codes(uint32_t (&w)[8]) {
    tq_swap<1>(w[0], w[1]);
    tq_swap<1>(w[2], w[3]);
    tq_swap<1>(w[4], w[5]);
    tq_swap<1>(w[6], w[7]);
    tq_swap<2>(w[0], w[2]);
    tq_swap<2>(w[1], w[3]);
    tq_swap<2>(w[4], w[6]);
    tq_swap<2>(w[5], w[7]);
    tq_swap<4>(w[0], w[4]);
    tq_swap<4>(w[1], w[5]);
    tq_swap<4>(w[2], w[6]);
    tq_swap<4>(w[3], w[7]);
}

// The N bit planes of a block at byte `off` (N < 0: `rn` planes, read as 8 words with the
// surplus cleared); planes N .. 7 are zero.
template <int N>
__device__ __forceinline__ void tq_planes(__amdgpu_buffer_rsrc_t r, int off, int rn, uint32_t (&w)[8]) {
    static_assert(N < 0 || N == 6 || N == 8, "plane counts with a load pattern");
    const uint4 a = ld16(r, off);
    w[0] = a.x;
    w[1] = a.y;
    w[2] = a.z;
    w[3] = a.w;
    if constexpr (N == 6) {
        const tq_u2 b = __builtin_amdgcn_raw_buffer_load_b64(r, off + 16, 0, 0);
        w[4] = b[0];
        w[5] = b[1];
        w[6] = 0;
        w[7] = 0;
    } else {
        const uint4 b = ld16(r, off + 16);
        w[4] = b.x;
        w[5] = b.y;
        w[6] = b.z;
        w[7] = b.w;
        if constexpr (N < 0) {
#pragma unroll
            for (int j = 2; j < 8; j++)
                if (j >= rn) w[j] = 0;
        }
    }
}

__device__ __forceinline__ float tq_half(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffff)));
}

// A group's K rows as this lane needs them (see the layout above) ...
template <int KB>
struct TqK {
    uint32_t w[2][8];  // bit planes of key m's blocks 2 r, 2 r + 1
    uint32_t s;        // their fp16 scales
};
template <>
struct TqK<0> {
    float k[64];  // key m, coordinates 64 r ..
};
// ... and its V rows.
template <int VB>
struct TqV {
    uint32_t w[4][8];  // bit planes of block m / 2 of keys 4 r + e
    uint32_t s[4];     // that block's fp16 scale
};
template <>
struct TqV<0> {
    float v[4][16];  // keys 4 r + e, coordinates 16 m ..
};

// Issues this lane's loads of one group's K rows (tv: the group's visibility bits;
// invisible keys read nothing).
template <int KB>
__device__ __forceinline__ void tq_load_k(TqK<KB>& t, const TurboArgs& a, __amdgpu_buffer_rsrc_t kr, int grp,
                                          uint32_t tv, int m, int r, int kvh, int kb, int krb) {
    const int kpos = 16 * grp + m;
    const int krow = (tv >> m) & 1 ? (kpos * a.Hkv + kvh) * krb : TQ_OOB;
    if constexpr (KB == 0) {
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const uint4 x = ld16(kr, krow + 256 * r + 16 * q);
            t.k[4 * q] = __uint_as_float(x.x);
            t.k[4 * q + 1] = __uint_as_float(x.y);
            t.k[4 * q + 2] = __uint_as_float(x.z);
            t.k[4 * q + 3] = __uint_as_float(x.w);
        }
    } else {
        t.s = __builtin_amdgcn_raw_buffer_load_b32(kr, krow + 4 * r, 0, 0);
#pragma unroll
        for (int b = 0; b < 2; b++) tq_planes<KB>(kr, krow + 16 + (2 * r + b) * kb * 4, kb, t.w[b]);
    }
}

// ... and of its V rows.
template <int VB>
__device__ __forceinline__ void tq_load_v(TqV<VB>& t, const TurboArgs& a, __amdgpu_buffer_rsrc_t vr, int grp,
                                          uint32_t tv, int m, int r, int kvh, int vb, int vrb) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int vpos = 16 * grp + 4 * r + e;
        const int vrow = (tv >> (4 * r + e)) & 1 ? (vpos * a.Hkv + kvh) * vrb : TQ_OOB;
        if constexpr (VB == 0) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint4 x = ld16(vr, vrow + 64 * m + 16 * q);
                t.v[e][4 * q] = __uint_as_float(x.x);
                t.v[e][4 * q + 1] = __uint_as_float(x.y);
                t.v[e][4 * q + 2] = __uint_as_float(x.z);
                t.v[e][4 * q + 3] = __uint_as_float(x.w);
            }
        } else {
            t.s[e] = __builtin_amdgcn_raw_buffer_load_b16(vr, vrow + 2 * (m >> 1), 0, 0);
            tq_planes<VB>(vr, vrow + 16 + (m >> 1) * vb * 4, vb, t.w[e]);
        }
    }
}

// The level of the code in byte i of w: one SDWA shift (byte select and times 4) forms
// the byte offset into the codebook's LDS copy.
__device__ __forceinline__ float tq_level(const float* tab, uint32_t w, int i) {
    uint32_t off;
    if (i == 0)
        asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
            : "=v"(off) : "v"(w));
    else if (i == 1)
        asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
            : "=v"(off) : "v"(w));
    else if (i == 2)
        asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
            : "=v"(off) : "v"(w));
    else
        asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
            : "=v"(off) : "v"(w));
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(tab) + off);
}

// S^T[4 r + e][m] of one group: 64 steps of four coordinates. A block's 32 levels are
// looked up together before its 32 steps, so the LDS latency is paid once a block.
template <int KB>
__device__ __forceinline__ tq_f4 tq_scores(const TqK<KB>& t, const float (*qsp)[TT_QS], const float* lvk, int m,
                                           int r) {
    tq_f4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int b = 0; b < 2; b++) {
        float kv[32];
        if constexpr (KB == 0) {
#pragma unroll
            for (int k = 0; k < 8; k++)
#pragma unroll
                for (int i = 0; i < 4; i++) kv[4 * k + i] = t.k[32 * b + 8 * i + k];
        } else {
            uint32_t w[8];
#pragma unroll
            for (int j = 0; j < 8; j++) w[j] = t.w[b][j];
            tq_codes(w);
#pragma unroll
            for (int k = 0; k < 8; k++)
#pragma unroll
                for (int i = 0; i < 4; i++) kv[4 * k + i] = tq_level(lvk, w[k], i);
            const float sc = tq_half(t.s >> (16 * b));
#pragma unroll
            for (int j = 0; j < 32; j++) kv[j] *= sc;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const tq_f4 q4 = *reinterpret_cast<const tq_f4*>(&qsp[m][64 * r + 32 * b + 4 * k]);
#pragma unroll
            for (int i = 0; i < 4; i++) c = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[4 * k + i], q4[i], c, 0, 0, 0);
        }
    }
    return c;
}

// o[t] += P V over one group: p[e] = P[m][4 r + e]. A key pair's 32 levels are looked up
// together before its 32 steps.
template <int VB>
__device__ __forceinline__ void tq_pv(const TqV<VB>& t, const float (&p)[4], tq_f4 (&o)[16], const float* lvv, int m) {
    const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;  // this lane's 16-bit half of each plane
#pragma unroll
    for (int pr = 0; pr < 2; pr++) {
        const int e0 = 2 * pr, e1 = e0 + 1;
        float v0[16], v1[16];
        if constexpr (VB == 0) {
#pragma unroll
            for (int c = 0; c < 16; c++) {
                v0[c] = t.v[e0][c];
                v1[c] = t.v[e1][c];
            }
        } else {
            uint32_t w[8];
#pragma unroll
            for (int j = 0; j < 8; j++) w[j] = __builtin_amdgcn_perm(t.w[e1][j], t.w[e0][j], sel);
            tq_codes(w);
#pragma unroll
            for (int c = 0; c < 16; c++) {
                v0[c] = tq_level(lvv, w[c & 7], c >> 3);
                v1[c] = tq_level(lvv, w[c & 7], 2 + (c >> 3));
            }
            const float s0 = tq_half(t.s[e0]), s1 = tq_half(t.s[e1]);
#pragma unroll
            for (int c = 0; c < 16; c++) {
                v0[c] *= s0;
                v1[c] *= s1;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 16; c++) {
            o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[e0], v0[c], o[c], 0, 0, 0);
            o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[e1], v1[c], o[c], 0, 0, 0);
        }
    }
}

// Mask byte of key (lane & 15) of round rho's group (0 past kv_len); the group's
// visibility bits are the ballot of the 16 bytes, taken when they are needed so that no
// earlier wait covers the load.
__device__ __forceinline__ uint32_t tq_mask_byte(__amdgpu_buffer_rsrc_t mr, int kv_len, int ngroups, int wv, int W,
                                                 int rho, int lane) {
    const int grp = wv + rho * W, pos = 16 * grp + (lane & 15);
    const bool ok = lane < 16 && grp < ngroups && pos < kv_len;
    return __builtin_amdgcn_raw_buffer_load_b8(mr, ok ? pos : TQ_OOB, 0, 0);
}
__device__ __forceinline__ uint32_t tq_ballot(uint32_t b) { return (uint32_t)__ballot(b != 0); }

struct TqLds {
    float lvk[256], lvv[256];                                  // codebooks of the K and V rows
    __attribute__((aligned(16))) float qsp[16][TT_QS];          // queries in score-step order
    float red[TT_WAVES][TQ_G][2];                               // each wave's max and sum a head
    __attribute__((aligned(16))) float osum[TT_WAVES][TQ_G][TQ_D];  // each wave's rescaled output
};

// The online softmax keeps a reference maximum per head and moves it only when a score
// exceeds it by more than TQ_TAU (natural-log units): the exponentials stay below e^8 and
// the accumulated output is rescaled rarely instead of every round.
constexpr float TQ_TAU = 8.0f;

template <int KB, int VB>
__global__ void __launch_bounds__(TT_WAVES * 64) attn_turbo_kernel(TurboArgs a) {
    constexpr bool ROT = KB != 0;
    constexpr int D = TQ_D, G = TQ_G;
    // one LDS object with the codebooks first: their addresses are constants that fold
    // into the lookups' offset field
    __shared__ TqLds sm;
    float* lvk = sm.lvk;
    float* lvv = sm.lvv;
    float(*qsp)[TT_QS] = sm.qsp;
    float(*red)[G][2] = sm.red;
    float(*osum)[G][D] = sm.osum;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 15, r = lane >> 4;
    const int kvh = blockIdx.y;
    const int kb = KB >= 0 ? KB : a.kb, vb = VB >= 0 ? VB : a.vb;
    const int krb = kv_row_bytes(D, kb), vrb = kv_row_bytes(D, vb);
    const int W = a.nblk * TT_WAVES, wv = blockIdx.x * TT_WAVES + wave;
    const int ngroups = (a.kv_len + 15) >> 4;
    const __amdgpu_buffer_rsrc_t mr = tq_rsrc(a.mask, a.kv_len);
    const __amdgpu_buffer_rsrc_t kr = tq_rsrc(a.k, a.kv_len * a.Hkv * krb);
    const __amdgpu_buffer_rsrc_t vr = tq_rsrc(a.v, a.kv_len * a.Hkv * vrb);

    // the small loads first (the first two rounds' mask bytes, this wave's query heads,
    // the codebooks), branch-free; the first round's rows go out as soon as its mask bytes
    // are in, and their latency hides behind the query rotation
    const __amdgpu_buffer_rsrc_t qr = tq_rsrc(a.q + (size_t)kvh * G * D, G * D * 4);
    const uint32_t b0 = tq_mask_byte(mr, a.kv_len, ngroups, wv, W, 0, lane);
    const uint32_t b1 = tq_mask_byte(mr, a.kv_len, ngroups, wv, W, 1, lane);
    // wave w rotates heads w and w + 8 (rows 12 .. 15 are zero); lane l holds coordinates
    // 4 l .. 4 l + 3
    uint4 qh[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int h = wave + TT_WAVES * j;
        qh[j] = ld16(qr, h < G ? (h * D + 4 * lane) * 4 : TQ_OOB);
    }
    float lk = 0.0f, lv = 0.0f;
    if constexpr (ROT) {
        const __amdgpu_buffer_rsrc_t lr = tq_rsrc(a.levels, TQ_LEVELS * 4);
        lk = ldf(lr, tid < (1 << kb) ? (codebook_offset(kb) + tid) * 4 : TQ_OOB);
        lv = ldf(lr, tid < (1 << vb) ? (codebook_offset(vb) + tid) * 4 : TQ_OOB);
    }
    uint32_t vis = tq_ballot(b0);
    TqK<KB> kbuf0, kbuf1;
    TqV<VB> vbuf;
    tq_load_k(kbuf0, a, kr, wv, vis, m, r, kvh, kb, krb);
    tq_load_v(vbuf, a, vr, wv, vis, m, r, kvh, vb, vrb);
    uint32_t vnext = tq_ballot(b1);

    if constexpr (ROT) {
        if (tid < 256) {
            lvk[tid] = lk;
            lvv[tid] = lv;
        }
    }
    // a rotated cache gets rotated queries: signs, then the Walsh-Hadamard butterflies in
    // the rotation's order (stages 1, 2 inside a lane, 4 .. 128 across lanes l ^ 1 ..
    // l ^ 32); the 1/16 normalisation is folded into the score scale (a power of two:
    // exact). The result goes to LDS in the order the score steps read it.
#pragma unroll
    for (int j = 0; j < 2; j++) {
        float x[4] = {__uint_as_float(qh[j].x), __uint_as_float(qh[j].y), __uint_as_float(qh[j].z),
                      __uint_as_float(qh[j].w)};
        if constexpr (ROT) {
#pragma unroll
            for (int i = 0; i < 4; i++) x[i] *= kv_sign(4 * lane + i);
            float y0 = x[0] + x[1], y1 = x[0] - x[1], y2 = x[2] + x[3], y3 = x[2] - x[3];
            x[0] = y0 + y2;
            x[2] = y0 - y2;
            x[1] = y1 + y3;
            x[3] = y1 - y3;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const bool upper = lane & o;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float y = __shfl_xor(x[i], o);
                    x[i] = upper ? y - x[i] : x[i] + y;
                }
            }
        }
        const int h = wave + TT_WAVES * j;
#pragma unroll
        for (int i = 0; i < 4; i++) qsp[h][tq_qperm(4 * lane + i)] = x[i];
    }
    __syncthreads();
    const float scale = ROT ? a.scale * (1.0f / 16.0f) : a.scale;

    tq_f4 o[16];
#pragma unroll
    for (int c = 0; c < 16; c++) o[c] = tq_f4{0.0f, 0.0f, 0.0f, 0.0f};
    float mrun = -INFINITY, lrun = 0.0f;  // reference maximum and sum of exponentials, head m
    // A round: the next group's K rows go out (into the other K buffer); this group's
    // scores; the online softmax; P V; the V buffer takes the next group's V rows. fp32
    // rows (four times the registers) keep one K buffer, refilled after the scores.
    constexpr bool KDB = KB != 0;
    auto round = [&](int rho, const TqK<KB>& kcur, TqK<KB>& knext) {
        const uint32_t bnn = tq_mask_byte(mr, a.kv_len, ngroups, wv, W, rho + 2, lane);
        if constexpr (KDB) tq_load_k(knext, a, kr, wv + (rho + 1) * W, vnext, m, r, kvh, kb, krb);
        tq_f4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
        if (vis) sc = tq_scores(kcur, qsp, lvk, m, r);
        if constexpr (!KDB) tq_load_k(knext, a, kr, wv + (rho + 1) * W, vnext, m, r, kvh, kb, krb);
        float s[4], mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            s[e] = (vis >> (4 * r + e)) & 1 ? sc[e] * scale : -INFINITY;
            mx = fmaxf(mx, s[e]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const bool grow = mx > mrun + TQ_TAU;  // (true for the first visible keys: mrun = -inf)
        if (__ballot(grow)) {
            const float mnew = grow ? mx : mrun;
            const float corr = grow ? __expf(mrun - mnew) : 1.0f;  // 0 from -inf
            lrun *= corr;
            if (__ballot(grow && mrun != -INFINITY)) {  // o is still zero while mrun is -inf
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float ce = __shfl(corr, 4 * r + e);
#pragma unroll
                    for (int c = 0; c < 16; c++) o[c][e] *= ce;
                }
            }
            mrun = mnew;
        }
        float p[4], ls = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            p[e] = s[e] == -INFINITY ? 0.0f : __expf(s[e] - mrun);
            ls += p[e];
        }
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        lrun += ls;
        if (vis) tq_pv(vbuf, p, o, lvv, m);
        tq_load_v(vbuf, a, vr, wv + (rho + 1) * W, vnext, m, r, kvh, vb, vrb);
        vis = vnext;
        vnext = tq_ballot(bnn);
    };
    if constexpr (KDB) {
        for (int rho = 0; wv + rho * W < ngroups; rho += 2) {
            round(rho, kbuf0, kbuf1);
            if (wv + (rho + 1) * W >= ngroups) break;
            round(rho + 1, kbuf1, kbuf0);
        }
    } else {
        for (int rho = 0; wv + rho * W < ngroups; rho++) round(rho, kbuf0, kbuf0);
    }

    // merge the block's waves: rescale each to the block max, sum in a fixed order
    if (r == 0 && m < G) {
        red[wave][m][0] = mrun;
        red[wave][m][1] = lrun;
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int h = 4 * r + e;
        if (h < G) {
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < TT_WAVES; w++) M = fmaxf(M, red[w][h][0]);
            const float mw = red[wave][h][0];
            const float f = mw == -INFINITY ? 0.0f : __expf(mw - M);
#pragma unroll
            for (int c4 = 0; c4 < 4; c4++) {
                const tq_f4 y = {o[4 * c4][e] * f, o[4 * c4 + 1][e] * f, o[4 * c4 + 2][e] * f, o[4 * c4 + 3][e] * f};
                *reinterpret_cast<tq_f4*>(&osum[wave][h][16 * m + 4 * c4]) = y;
            }
        }
    }
    __syncthreads();
    float* part = a.part + ((size_t)kvh * a.nblk + blockIdx.x) * G * D;
    for (int u = tid; u < G * D; u += blockDim.x) {
        const int h = u / D, c = u % D;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < TT_WAVES; w++) s += osum[w][h][c];
        part[u] = s;
    }
    if (tid < G) {
        float M = -INFINITY, L = 0.0f;
#pragma unroll
        for (int w = 0; w < TT_WAVES; w++) M = fmaxf(M, red[w][tid][0]);
#pragma unroll
        for (int w = 0; w < TT_WAVES; w++) {
            const float mw = red[w][tid][0];
            if (mw != -INFINITY) L += __expf(mw - M) * red[w][tid][1];
        }
        float* ml = a.ml + (((size_t)kvh * a.nblk + blockIdx.x) * G + tid) * 2;
        ml[0] = M;
        ml[1] = L;
    }
}

// out[h] = sum_b e^(m_b - M) O_b / sum_b e^(m_b - M) l_b over the blocks' partials of head
// h (a block with no visible key has m = -inf and weight 0), rotated back for a Turbo
// cache (x = s . (H y) / 16). One block of 1024 threads a head: four slices of the
// partials by 256 coordinates, each thread's loads in flight together.
template <bool ROT>
__global__ void __launch_bounds__(TC_THREADS) attn_turbo_combine_kernel(TurboArgs a) {
    constexpr int D = TQ_D, G = TQ_G, SL = TC_THREADS / D;
    __shared__ float wt[256];
    __shared__ float rm[TC_THREADS / 64], rl[TC_THREADS / 64];
    __shared__ float acc[SL][D];
    const int h = blockIdx.x, kvh = h / G, g = h % G, tid = threadIdx.x, n = a.nblk;
    const int lane = tid & 63, wave = tid >> 6;
    const int d = tid % D, sl = tid / D;
    const __amdgpu_buffer_rsrc_t pr = tq_rsrc(a.part + (size_t)kvh * n * G * D, n * G * D * 4);
    // the first TC_BATCH partials of this thread go out with the maxima and sums: one
    // memory round trip for both
    float x[TC_BATCH];
#pragma unroll
    for (int j = 0; j < TC_BATCH; j++) {
        const int p = sl + SL * j;
        x[j] = ldf(pr, p < n ? ((p * G + g) * D + d) * 4 : TQ_OOB);
    }
    const __amdgpu_buffer_rsrc_t mlr = tq_rsrc(a.ml + (size_t)kvh * n * G * 2, n * G * 2 * 4);
    const float mld = ldf(mlr, tid < n ? (tid * G + g) * 8 : TQ_OOB);
    const float lp = ldf(mlr, tid < n ? (tid * G + g) * 8 + 4 : TQ_OOB);
    const float mp = tid < n ? mld : -INFINITY;
    float M = wave_max(mp);
    if (lane == 0) rm[wave] = M;
    __syncthreads();
    M = -INFINITY;
#pragma unroll
    for (int w = 0; w < TC_THREADS / 64; w++) M = fmaxf(M, rm[w]);
    const float wp = mp == -INFINITY ? 0.0f : __expf(mp - M);
    if (tid < 256) wt[tid] = wp;  // zero for tid >= n
    float den = wave_sum(wp * lp);
    if (lane == 0) rl[wave] = den;
    __syncthreads();
    den = 0.0f;
#pragma unroll
    for (int w = 0; w < TC_THREADS / 64; w++) den += rl[w];
    float num = 0.0f;
#pragma unroll
    for (int j = 0; j < TC_BATCH; j++) num = fmaf(wt[sl + SL * j], x[j], num);
    for (int p0 = sl + SL * TC_BATCH; p0 < n; p0 += SL * TC_BATCH) {
#pragma unroll
        for (int j = 0; j < TC_BATCH; j++) {
            const int p = p0 + SL * j;
            x[j] = ldf(pr, p < n ? ((p * G + g) * D + d) * 4 : TQ_OOB);
        }
#pragma unroll
        for (int j = 0; j < TC_BATCH; j++) {
            const int p = p0 + SL * j;
            num = fmaf(wt[p < n ? p : 0], x[j], num);
        }
    }
    acc[sl][d] = num;
    __syncthreads();
    if (tid < D) {
        float y = 0.0f;
#pragma unroll
        for (int s = 0; s < SL; s++) y += acc[s][d];
        acc[0][d] = y / den;
    }
    __syncthreads();
    if constexpr (ROT) {
        // rotated back by the first wave: lane l takes coordinates 4 l .. 4 l + 3 through the
        // butterflies, then signs and the 1 / sqrt(D) = 1 / 16
        static_assert(D == 256, "one wave holds the head's 256 coordinates");
        if (wave == 0) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = acc[0][4 * lane + i];
            row_wht<D>(v, lane);
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = v[i] * kv_sign(4 * lane + i) * (1.0f / 16.0f);
#pragma unroll
            for (int i = 0; i < 4; i++) a.out[(size_t)h * D + 4 * lane + i] = v[i];
        }
    } else {
        if (tid < D) a.out[(size_t)h * D + tid] = acc[0][tid];
    }
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

// Rows of d coordinates stored at `bits` (0: fp32): d a multiple of 32 up to 256, and a
// power of two for the rotation (kv_row_shape, crates/oominf-cuda/src/attention.rs:351-356).
static bool kv_row_shape(int d, int bits) {
    return d >= 32 && d % 32 == 0 && d <= TQ_MAXD && (bits == 0 || ((d & (d - 1)) == 0 && bits >= 2 && bits <= 8));
}

// Blocks a KV head of the decode attention: enough that every wave has TT_GPW groups of
// 16 keys, at most 256 blocks over all KV heads (one a CU).
static int turbo_blocks(int kv_len, int kv_heads) {
    const int groups = (kv_len + 15) / 16;
    const int want = (groups + TT_WAVES * TT_GPW - 1) / (TT_WAVES * TT_GPW);
    return std::max(1, std::min(want, std::max(1, 256 / kv_heads)));
}

struct TurboWs {
    size_t part, ml, total;
    int nblk;
};

static size_t t_al256(size_t v) { return (v + 255) & ~size_t(255); }

static TurboWs turbo_ws(int kv_heads, int kv_len) {
    TurboWs w;
    w.nblk = turbo_blocks(kv_len, kv_heads);
    w.part = 0;
    w.ml = t_al256((size_t)kv_heads * w.nblk * TQ_G * TQ_D * 4);
    w.total = w.ml + t_al256((size_t)kv_heads * w.nblk * TQ_G * 2 * 4);
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

namespace oom {

// Blocks of the row kernels: TR_WAVES waves a block, 256 / d rows a wave.
static unsigned row_blocks(int64_t rows, int d) {
    const int64_t per = (int64_t)TR_WAVES * (256 / d);
    return (unsigned)((rows + per - 1) / per);
}

#define OOM_ROW_LAUNCH(KERNEL, d, ...)                                                                     \
    switch (d) {                                                                                           \
        case 32: hipLaunchKernelGGL(KERNEL<32>, dim3(grid), dim3(64 * TR_WAVES), 0, st, __VA_ARGS__); break;   \
        case 64: hipLaunchKernelGGL(KERNEL<64>, dim3(grid), dim3(64 * TR_WAVES), 0, st, __VA_ARGS__); break;   \
        case 128: hipLaunchKernelGGL(KERNEL<128>, dim3(grid), dim3(64 * TR_WAVES), 0, st, __VA_ARGS__); break; \
        default: hipLaunchKernelGGL(KERNEL<256>, dim3(grid), dim3(64 * TR_WAVES), 0, st, __VA_ARGS__); break;  \
    }

}  // namespace oom

extern "C" int oom_kv_rotate(float* x, int rows, int d, int inverse, void* stream) {
    using namespace oom;
    OOM_REQUIRE(kv_row_shape(d, 4) && rows >= 0, "oom_kv_rotate: d must be a power of two, 32..256");
    if (rows == 0) return OOM_OK;
    OOM_REQUIRE(x, "oom_kv_rotate: null buffer");
    const unsigned grid = row_blocks(rows, d);
    hipStream_t st = as_stream(stream);
    OOM_ROW_LAUNCH(kv_rotate_kernel, d, x, (int64_t)rows, inverse ? 1 : 0)
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
    hipStream_t st = as_stream(stream);
    if (!bits) {
        // fp32 rows are the values as they are: one contiguous copy
        if (hipMemcpyAsync(cache + start * kv_heads * (int64_t)d * 4, src, (size_t)rows * d * 4,
                           hipMemcpyDeviceToDevice, st) != hipSuccess)
            return launched("oom_kv_append");
        return OOM_OK;
    }
    const unsigned grid = row_blocks(rows, d);
    OOM_ROW_LAUNCH(kv_append_kernel, d, src, cache, start * kv_heads, rows, bits, levels)
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
    hipStream_t st = as_stream(stream);
    if (!bits) {
        if (hipMemcpyAsync(dst, cache, (size_t)rows * d * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
            return launched("oom_kv_read");
        return OOM_OK;
    }
    const unsigned grid = row_blocks(rows, d);
    OOM_ROW_LAUNCH(kv_read_kernel, d, cache, dst, rows, bits, levels)
    return launched("oom_kv_read");
}

#undef OOM_ROW_LAUNCH

extern "C" int oom_mask_compact(const uint8_t* mask, int32_t* sel, int n, void* stream) {
    using namespace oom;
    OOM_REQUIRE(n >= 0 && n < 0x7fff0000 && mask && sel, "oom_mask_compact: null buffer or length out of range");
    hipLaunchKernelGGL(mask_compact_kernel, dim3(1), dim3(TQ_MASK_THREADS), 0, as_stream(stream), mask, sel, n);
    return launched("oom_mask_compact");
}

extern "C" size_t oom_attn_decode_turbo_workspace_size(int heads, int kv_heads, int d, int kv_len) {
    if (heads < 1 || kv_heads < 1 || d < 1 || kv_len < 1 || heads % kv_heads) return 0;
    return oom::turbo_ws(kv_heads, kv_len).total;
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
    OOM_REQUIRE((int64_t)kv_len * kv_heads * kv_row_bytes(d, std::max(k_bits, v_bits)) < TQ_OOB,
                "oom_attn_decode_turbo: cache too large (rows of one cache under 1.75 GiB)");
    OOM_REQUIRE(q && k && v && mask && out && (k_bits == 0 || levels), "oom_attn_decode_turbo: null buffer");
    const TurboWs w = turbo_ws(kv_heads, kv_len);
    if (!ws || ws_bytes < w.total)
        return fail(OOM_ERR_WORKSPACE,
                    "oom_attn_decode_turbo: workspace smaller than oom_attn_decode_turbo_workspace_size()");
    OOM_REQUIRE(aligned(ws, 256), "oom_attn_decode_turbo: workspace must be 256-byte aligned");
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    hipStream_t st = as_stream(stream);
    TurboArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.mask = mask;
    a.levels = levels;
    a.part = reinterpret_cast<float*>(base + w.part);
    a.ml = reinterpret_cast<float*>(base + w.ml);
    a.out = out;
    a.Hkv = kv_heads;
    a.kv_len = kv_len;
    a.nblk = w.nblk;
    a.kb = k_bits;
    a.vb = v_bits;
    a.scale = scale;
    const dim3 grid((unsigned)w.nblk, (unsigned)kv_heads), block(TT_WAVES * 64);
    if (k_bits == 0) hipLaunchKernelGGL((attn_turbo_kernel<0, 0>), grid, block, 0, st, a);
    else if (k_bits == 8 && v_bits == 6) hipLaunchKernelGGL((attn_turbo_kernel<8, 6>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((attn_turbo_kernel<-1, -1>), grid, block, 0, st, a);
    if (int rc = launched("oom_attn_decode_turbo")) return rc;
    if (k_bits == 0) hipLaunchKernelGGL(attn_turbo_combine_kernel<false>, dim3((unsigned)heads), dim3(TC_THREADS), 0, st, a);
    else hipLaunchKernelGGL(attn_turbo_combine_kernel<true>, dim3((unsigned)heads), dim3(TC_THREADS), 0, st, a);
    return launched("oom_attn_decode_turbo");
}
