// Prefill over NVFP4 records on gfx950: the tiled grouped GEMM of one projection on the
// bf16 matrix cores, y[a, r] = x[row(a)] . W_e[r] * scale_2 (the semantics of moe_tiled,
// crates/oominf-cuda/kernels/moe.cu:166-335), and the elementwise SwiGLU over a range
// (moe_swiglu, moe.cu:338-341).
//
// Exactness (the reference's argument, restated): a weight e2m1(code) * e4m3(scale) has at
// most 6 significant bits, so it is a bf16 value with no rounding, and weight_scale_2
// multiplies the fp32 result instead of every weight. With OOM_EXPERT_EXACT each fp32
// activation is split into three bf16 terms (hi = bf16(x), mid = bf16(x - hi), lo =
// bf16(x - hi - mid); hi + mid + lo == x), every bf16 x bf16 product is exact in fp32,
// and the matrix cores accumulate in fp32: an fp32 GEMM in another summation order, three
// matrix-core passes. OOM_EXPERT_BF16 keeps the hi term only (x rounded to bf16), one pass.
//
// Layout of the work: a block of 4 waves takes 128 weight rows x 64 assignments of one
// expert; per K step of 32 the block decodes the 128 x 32 weights once into LDS as bf16
// (thread t: row t % 128, 16 columns, one 8-byte code load and one scale byte) and
// splits the 64 x 32 activations into their terms in LDS, while the next step's global
// loads are in flight. Wave w owns rows 32 w .. 32 w + 31 (two 16-row N subtiles) and all
// 64 assignments (four 16-row M subtiles; rows past the expert's assignments hold zeros):
// per step 8 v_mfma_f32_16x16x32_bf16 a term, with no branch in the step, so the
// compiler's waits for the load ring stay exact. LDS rows are 40 bf16 (80 bytes), so
// the 16 rows of an operand read fall in distinct bank groups. Grid (ceil(N / 128),
// ceil(max_per_expert / 64), n_experts), as the reference's.
#include "stream.hpp"

namespace oom {

constexpr int T4_BN = 128;       // weight rows a block
constexpr int T4_BM = 64;        // assignments a block
constexpr int T4_BK = 32;        // K step
constexpr int T4_THREADS = 256;  // 4 waves, 32 weight rows each
constexpr int T4_NX = T4_BM * T4_BK / 4 / T4_THREADS;  // activation float4s a thread loads a step
constexpr int T4_LS = 40;        // LDS row stride in bf16: 32 + 8

typedef __bf16 t4bf16x8 __attribute__((ext_vector_type(8)));
typedef float t4f4 __attribute__((ext_vector_type(4)));

struct TiledArgs {
    const uint64_t* recs;  // record of expert e
    const int32_t* off;    // assignments of expert e: [off[e], off[e + 1])
    const int32_t* rows;   // x row of assignment a (null: a)
    const float* x;        // [*, K]
    float* y;              // [A, N]
    int N, K;
    int64_t w_off, s_off;  // the projection's codes and e4m3 scales in a record
    int s2_idx;            // its weight_scale_2, in floats from the record start
};

typedef __bf16 t4bf16x2 __attribute__((ext_vector_type(2)));
typedef float t4f32x2 __attribute__((ext_vector_type(2)));

// Two f32 values as packed bf16 (v_cvt_pk_bf16_f32, round to nearest even; exact for the
// weights here, which are bf16 values).
__device__ __forceinline__ uint32_t t4_cvt(float lo, float hi) {
    const t4f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, t4bf16x2));
}

template <int TERMS>
__global__ void __launch_bounds__(T4_THREADS, 2) moe_tiled_nvfp4_kernel(TiledArgs g) {
    __shared__ __align__(16) uint16_t wsh[2][T4_BN][T4_LS];
    __shared__ __align__(16) uint16_t xsh[2][TERMS][T4_BM][T4_LS];
    const int e = blockIdx.z;
    const int a_begin = g.off[e] + (int)blockIdx.y * T4_BM, a_end = g.off[e + 1];
    if (a_begin >= a_end) return;
    const int nt = min(T4_BM, a_end - a_begin);
    const int r0 = (int)blockIdx.x * T4_BN;
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(g.recs[e]);
    const float s2 = reinterpret_cast<const float*>(rec)[g.s2_idx];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nkb = g.K / T4_BK;

    // ---- this thread's loads: weight row r0 + tid % 128, columns 16 (tid / 128) .. of a
    // step; activations idx = tid + 256 i (i < 2): assignment idx / 8, columns 4 (idx % 8) ..
    const int wr = tid & (T4_BN - 1), wh = tid / T4_BN;
    const bool wok = r0 + wr < g.N;
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(rec + g.w_off), (short)0, (int)((int64_t)g.N * g.K / 2), BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(rec + g.s_off), (short)0, (int)((int64_t)g.N * g.K / 16), BUF_FLAGS);
    const int cbase = wok ? (r0 + wr) * (g.K / 2) + 8 * wh : OOB;
    const int sbase = wok ? (r0 + wr) * (g.K / 16) + wh : OOB;
    // activation rows: past the expert's assignments a row reads assignment a_begin's row
    // (a valid address) and the value is dropped after the load, so no load is branched
    const float* xrow[T4_NX];
    bool xok[T4_NX];
#pragma unroll
    for (int i = 0; i < T4_NX; i++) {
        const int t = (tid + i * T4_THREADS) >> 3;
        xok[i] = t < nt;
        const int a = a_begin + (xok[i] ? t : 0);
        xrow[i] = g.x + (int64_t)(g.rows ? g.rows[a] : a) * g.K + ((tid + i * T4_THREADS) & 7) * 4;
    }
    struct Ld {
        uint2 codes;
        uint32_t sb;
        float4 xv[T4_NX];
    };
    // step kb's loads (kb clamped to the last step: the ring's loads past the end repeat it)
    auto load = [&](int kb, Ld& l) {
        const int k0 = min(kb, nkb - 1) * T4_BK;
        const auto c = __builtin_amdgcn_raw_buffer_load_b64(cr, cbase == OOB ? OOB : cbase + k0 / 2, 0, 0);
        l.codes = make_uint2(c[0], c[1]);
        l.sb = __builtin_amdgcn_raw_buffer_load_b8(sr, sbase == OOB ? OOB : sbase + k0 / 16, 0, 0);
#pragma unroll
        for (int i = 0; i < T4_NX; i++) l.xv[i] = *reinterpret_cast<const float4*>(xrow[i] + k0);
    };
    // decoded weights and split activations of a step into LDS buffer b
    auto stage = [&](int b, const Ld& l) {
        const float sc = __builtin_amdgcn_cvt_f32_fp8((int)l.sb, 0);
        uint32_t packed[8];
        const uint32_t cw[2] = {l.codes.x, l.codes.y};
#pragma unroll
        for (int i = 0; i < 2; i++) {
            // byte q of word i: columns 8 i + 2 q (low nibble) and 8 i + 2 q + 1
            const auto p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw[i], 1.0f, 0);
            const auto p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw[i], 1.0f, 1);
            const auto p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw[i], 1.0f, 2);
            const auto p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw[i], 1.0f, 3);
            packed[4 * i] = t4_cvt(p0[0] * sc, p0[1] * sc);
            packed[4 * i + 1] = t4_cvt(p1[0] * sc, p1[1] * sc);
            packed[4 * i + 2] = t4_cvt(p2[0] * sc, p2[1] * sc);
            packed[4 * i + 3] = t4_cvt(p3[0] * sc, p3[1] * sc);
        }
        uint4* dst = reinterpret_cast<uint4*>(&wsh[b][wr][16 * wh]);
        dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
        // activations as terms, two values a conversion: the remainder of a round to
        // nearest is exact in f32
#pragma unroll
        for (int i = 0; i < T4_NX; i++) {
            const int idx = tid + i * T4_THREADS, t = idx >> 3, kq = (idx & 7) * 4;
            const float4 x4 = xok[i] ? l.xv[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float v[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
            for (int p = 0; p < TERMS; p++) {
                const uint32_t w0 = t4_cvt(v[0], v[1]), w1 = t4_cvt(v[2], v[3]);
                *reinterpret_cast<uint2*>(&xsh[b][p][t][kq]) = make_uint2(w0, w1);
                if (p + 1 < TERMS) {
                    v[0] -= __uint_as_float(w0 << 16);
                    v[1] -= __uint_as_float(w0 & 0xffff0000u);
                    v[2] -= __uint_as_float(w1 << 16);
                    v[3] -= __uint_as_float(w1 & 0xffff0000u);
                }
            }
        }
    };

    t4f4 acc[4][2];
#pragma unroll
    for (int ms = 0; ms < 4; ms++)
#pragma unroll
        for (int ns = 0; ns < 2; ns++) acc[ms][ns] = t4f4{0.0f, 0.0f, 0.0f, 0.0f};
    const int kl = 8 * (lane >> 4);  // this lane's 8 columns of a step
    // a ring of four steps' loads in registers: step kb stages slot kb % 4 and refills it
    // with step kb + 4, so each step's loads have three steps of work to land in
    auto mfmas = [&](int b) {
        t4bf16x8 bop[2];
#pragma unroll
        for (int ns = 0; ns < 2; ns++)
            bop[ns] = *reinterpret_cast<const t4bf16x8*>(&wsh[b][32 * wave + 16 * ns + (lane & 15)][kl]);
#pragma unroll
        for (int ms = 0; ms < 4; ms++) {
#pragma unroll
            for (int p = 0; p < TERMS; p++) {
                const t4bf16x8 aop = *reinterpret_cast<const t4bf16x8*>(&xsh[b][p][16 * ms + (lane & 15)][kl]);
#pragma unroll
                for (int ns = 0; ns < 2; ns++)
                    acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop[ns], acc[ms][ns], 0, 0, 0);
            }
        }
    };
    Ld l0, l1, l2, l3;
    load(0, l0);
    load(1, l1);
    load(2, l2);
    load(3, l3);
#define T4_STEP(R)                  \
    {                               \
        stage(kb & 1, R);           \
        __syncthreads();            \
        load(kb + 4, R);            \
        mfmas(kb & 1);              \
        if (++kb == nkb) break;     \
    }
    int kb = 0;
    for (;;) {
        T4_STEP(l0)
        T4_STEP(l1)
        T4_STEP(l2)
        T4_STEP(l3)
    }
#undef T4_STEP
    // ---- y = acc * scale_2: lane l holds assignments 16 ms + 4 (l / 16) + i, row 16 ns + l % 16
#pragma unroll
    for (int ms = 0; ms < 4; ms++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * ms + 4 * (lane >> 4) + i;
            if (t >= nt) continue;
#pragma unroll
            for (int ns = 0; ns < 2; ns++) {
                const int r = r0 + 32 * wave + 16 * ns + (lane & 15);
                if (r < g.N) g.y[(int64_t)(a_begin + t) * g.N + r] = acc[ms][ns][i] * s2;
            }
        }
}

// ---- wide tiles: all 640 rows of a projection tile over 64 assignments ---------------
//
// The 128-row tiles above gather every activation row once per N tile, four times the
// bytes of the weights they meet. Here a block of 8 waves takes 640 weight rows (wave w:
// rows 80 w .. + 80, five 16-row N subtiles) x 64 assignments, so a gate or up projection
// (N 640) gathers each activation row once. The weights never pass through LDS: lane
// (r, q) of a wave (r = lane % 16, q = lane / 16) loads 16 contiguous code bytes of its row
// per K block of 128, codes k = 32 q .. 32 q + 31 of the block, and feeds them to four
// MFMAs, codes 8 s .. 8 s + 7 at step s. The activations sit in LDS in the same order
// (the lane's A operand at step s is x[m][32 q + 8 s .. + 8]), so every product pairs the
// same k on both sides and the sum is the plain dot product. Per K block the block loads
// 64 x 128 fp32 activations (four 16-byte loads a thread) while the previous block runs,
// splits them into their bf16 terms in LDS (row stride 272 bytes: the 16 rows of an
// operand read fall in distinct bank groups), and each wave decodes its own weights in
// registers: e2m1 -> f32 (v_cvt_scalef32_pk_f32_fp4 at scale 1), times the e4m3 group
// scale, -> bf16 (exact, as above). K must be a multiple of 128.
constexpr int TW_BN = 640;       // weight rows a block
constexpr int TW_NS = 5;         // N subtiles a wave
constexpr int TW_BK = 128;       // K block
constexpr int TW_THREADS = 512;  // 8 waves
constexpr int TW_LS = 136;       // LDS row stride in bf16 (272 bytes)
constexpr int TW_BM = 48;        // assignments a block (three M subtiles)
constexpr int TW_MS = TW_BM / 16;

template <int TERMS>
__global__ void __launch_bounds__(TW_THREADS) moe_tiled_nvfp4_wide_kernel(TiledArgs g) {
    __shared__ __align__(16) uint16_t xsh[2][TERMS][TW_BM][TW_LS];
    const int e = blockIdx.z;
    const int a_begin = g.off[e] + (int)blockIdx.y * TW_BM, a_end = g.off[e + 1];
    if (a_begin >= a_end) return;
    const int nt = min(TW_BM, a_end - a_begin);
    const int r0 = (int)blockIdx.x * TW_BN;
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(g.recs[e]);
    const float s2 = reinterpret_cast<const float*>(rec)[g.s2_idx];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nkb = g.K / TW_BK, q = lane >> 4;
    // ---- weights: lane (r, q)'s 16 code bytes and 2 scale bytes of N subtile ns, K block 0
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(rec + g.w_off), (short)0, (int)((int64_t)g.N * g.K / 2), BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(rec + g.s_off), (short)0, (int)((int64_t)g.N * g.K / 16), BUF_FLAGS);
    int coff[TW_NS], soff[TW_NS];
#pragma unroll
    for (int ns = 0; ns < TW_NS; ns++) {
        const int r = r0 + 80 * wave + 16 * ns + (lane & 15);
        coff[ns] = r < g.N ? r * (g.K / 2) + 16 * q : OOB;
        soff[ns] = r < g.N ? r * (g.K / 16) + 2 * q : OOB;
    }
    // ---- activations: thread t loads rows t / 32 + 16 i of the tile, columns 4 (t % 32) ..
    // of a K block (a row past the expert reads the tile's first row, dropped at staging)
    const float* xrow[TW_MS];
#pragma unroll
    for (int i = 0; i < TW_MS; i++) {
        const int m = (tid >> 5) + 16 * i;
        const int a = a_begin + (m < nt ? m : 0);
        xrow[i] = g.x + (int64_t)(g.rows ? g.rows[a] : a) * g.K + 4 * (tid & 31);
    }
    struct WLd {
        uint4 c[TW_NS];
        uint32_t s[TW_NS];
    };
    auto wload = [&](int kb, WLd& w) {
        const int k = min(kb, nkb - 1);
#pragma unroll
        for (int ns = 0; ns < TW_NS; ns++) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(cr, coff[ns] == OOB ? OOB : coff[ns] + 64 * k, 0, 0);
            w.c[ns] = make_uint4(v[0], v[1], v[2], v[3]);
            w.s[ns] = __builtin_amdgcn_raw_buffer_load_b16(sr, soff[ns] == OOB ? OOB : soff[ns] + 8 * k, 0, 0);
        }
    };
    float4 xv[TW_MS];
    auto xload = [&](int kb) {
        const int k = min(kb, nkb - 1) * TW_BK;
#pragma unroll
        for (int i = 0; i < TW_MS; i++) xv[i] = *reinterpret_cast<const float4*>(xrow[i] + k);
    };
    // the K block's activations as terms into LDS buffer b
    auto stage = [&](int b) {
#pragma unroll
        for (int i = 0; i < TW_MS; i++) {
            const int m = (tid >> 5) + 16 * i, kq = 4 * (tid & 31);
            const float4 x4 = m < nt ? xv[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float v[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
            for (int p = 0; p < TERMS; p++) {
                const uint32_t w0 = t4_cvt(v[0], v[1]), w1 = t4_cvt(v[2], v[3]);
                *reinterpret_cast<uint2*>(&xsh[b][p][m][kq]) = make_uint2(w0, w1);
                if (p + 1 < TERMS) {
                    v[0] -= __uint_as_float(w0 << 16);
                    v[1] -= __uint_as_float(w0 & 0xffff0000u);
                    v[2] -= __uint_as_float(w1 << 16);
                    v[3] -= __uint_as_float(w1 & 0xffff0000u);
                }
            }
        }
    };
    t4f4 acc[TW_MS][TW_NS];
#pragma unroll
    for (int ms = 0; ms < TW_MS; ms++)
#pragma unroll
        for (int ns = 0; ns < TW_NS; ns++) acc[ms][ns] = t4f4{0.0f, 0.0f, 0.0f, 0.0f};
    // one K block on the matrix cores: LDS buffer b, weights w
    auto mfmas = [&](int b, const WLd& w) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            t4bf16x8 bop[TW_NS];
#pragma unroll
            for (int ns = 0; ns < TW_NS; ns++) {
                const uint32_t cw = s == 0 ? w.c[ns].x : s == 1 ? w.c[ns].y : s == 2 ? w.c[ns].z : w.c[ns].w;
                const float sc = __builtin_amdgcn_cvt_f32_fp8((int)(w.s[ns] >> (s < 2 ? 0 : 8)), 0);
                const auto p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw, 1.0f, 0);
                const auto p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw, 1.0f, 1);
                const auto p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw, 1.0f, 2);
                const auto p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw, 1.0f, 3);
                bop[ns] = __builtin_bit_cast(
                    t4bf16x8, make_uint4(t4_cvt(p0[0] * sc, p0[1] * sc), t4_cvt(p1[0] * sc, p1[1] * sc),
                                         t4_cvt(p2[0] * sc, p2[1] * sc), t4_cvt(p3[0] * sc, p3[1] * sc)));
            }
#pragma unroll
            for (int ms = 0; ms < TW_MS; ms++) {
#pragma unroll
                for (int p = 0; p < TERMS; p++) {
                    const t4bf16x8 aop =
                        *reinterpret_cast<const t4bf16x8*>(&xsh[b][p][16 * ms + (lane & 15)][32 * q + 8 * s]);
#pragma unroll
                    for (int ns = 0; ns < TW_NS; ns++)
                        acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop[ns], acc[ms][ns], 0, 0, 0);
                }
            }
        }
    };
    // K block kb: its activations were loaded one block ahead (xv) and are staged into LDS
    // buffer kb % 2; its weights were loaded two blocks ahead (w0 / w1 alternate)
    WLd w0, w1;
    wload(0, w0);
    xload(0);
    wload(1, w1);
    // a scheduling barrier closes each step: no use of a weight block still loading (the
    // other register set) moves into the step before it, which would wait for that load
#define TW_STEP(KB, B, W)                       \
    {                                           \
        stage(B);                               \
        xload((KB) + 1);                        \
        __syncthreads();                        \
        mfmas(B, W);                            \
        wload((KB) + 2, W);                     \
        __builtin_amdgcn_sched_barrier(0);      \
    }
    // pairs of K blocks with no exit inside the body (an exit there merges states at the
    // loop head, where the compiler then waited for every load in flight), then the odd one
    for (int kb = 0; kb + 1 < nkb; kb += 2) {
        TW_STEP(kb, 0, w0)
        TW_STEP(kb + 1, 1, w1)
    }
    if (nkb & 1) TW_STEP(nkb - 1, 0, w0)
#undef TW_STEP
    // ---- y = acc * scale_2: lane l holds assignments 16 ms + 4 (l / 16) + i, row 16 ns + l % 16
#pragma unroll
    for (int ms = 0; ms < TW_MS; ms++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * ms + 4 * (lane >> 4) + i;
            if (t >= nt) continue;
#pragma unroll
            for (int ns = 0; ns < TW_NS; ns++) {
                const int r = r0 + 80 * wave + 16 * ns + (lane & 15);
                if (r < g.N) g.y[(int64_t)(a_begin + t) * g.N + r] = acc[ms][ns][i] * s2;
            }
        }
}

__global__ void __launch_bounds__(256) moe_swiglu_kernel(const float* __restrict__ gt, const float* __restrict__ up,
                                                         float* __restrict__ h, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = siluf(gt[i]) * up[i];
}

}  // namespace oom

extern "C" int oom_moe_tiled_nvfp4(const uint64_t* recs, const int32_t* off, const int32_t* rows, int n_experts,
                                   int max_per_expert, const float* x, float* y, int n, int k, int64_t w_off,
                                   int64_t s_off, int s2_idx, int precision, void* stream) {
    using namespace oom;
    OOM_REQUIRE(n_experts >= 0 && max_per_expert >= 0 && n >= 1 && k >= 32,
                "oom_moe_tiled_nvfp4: n_experts, max_per_expert >= 0; n >= 1; k >= 32");
    OOM_REQUIRE(k % 32 == 0, "oom_moe_tiled_nvfp4: k must be a multiple of 32");
    OOM_REQUIRE(precision == OOM_EXPERT_EXACT || precision == OOM_EXPERT_BF16,
                "oom_moe_tiled_nvfp4: precision must be OOM_EXPERT_EXACT or OOM_EXPERT_BF16");
    OOM_REQUIRE(n_experts <= 65535 && cdiv(max_per_expert, T4_BM) <= 65535, "oom_moe_tiled_nvfp4: grid too large");
    OOM_REQUIRE((int64_t)n * k / 2 < 0x7fff0000 && w_off >= 0 && s_off >= 0 && s2_idx >= 0,
                "oom_moe_tiled_nvfp4: projection offsets and size");
    if (n_experts == 0 || max_per_expert == 0) return OOM_OK;
    OOM_REQUIRE(recs && off && x && y, "oom_moe_tiled_nvfp4: null buffer");
    OOM_REQUIRE(aligned(x, 16), "oom_moe_tiled_nvfp4: x must be 16-byte aligned");
    TiledArgs a{recs, off, rows, x, y, n, k, w_off, s_off, s2_idx};
    if (k % TW_BK == 0 && w_off % 16 == 0 && s_off % 2 == 0) {
        // 640-row tiles, weights straight into registers (records' parts are 16-byte aligned
        // in the released layout)
        const dim3 grid((unsigned)cdiv(n, TW_BN), (unsigned)cdiv(max_per_expert, TW_BM), (unsigned)n_experts);
        if (precision == OOM_EXPERT_EXACT)
            hipLaunchKernelGGL(moe_tiled_nvfp4_wide_kernel<3>, grid, dim3(TW_THREADS), 0, as_stream(stream), a);
        else
            hipLaunchKernelGGL(moe_tiled_nvfp4_wide_kernel<1>, grid, dim3(TW_THREADS), 0, as_stream(stream), a);
        return launched("oom_moe_tiled_nvfp4");
    }
    const dim3 grid((unsigned)cdiv(n, T4_BN), (unsigned)cdiv(max_per_expert, T4_BM), (unsigned)n_experts);
    if (precision == OOM_EXPERT_EXACT)
        hipLaunchKernelGGL(moe_tiled_nvfp4_kernel<3>, grid, dim3(T4_THREADS), 0, as_stream(stream), a);
    else
        hipLaunchKernelGGL(moe_tiled_nvfp4_kernel<1>, grid, dim3(T4_THREADS), 0, as_stream(stream), a);
    return launched("oom_moe_tiled_nvfp4");
}

extern "C" int oom_moe_swiglu_range(const float* g, const float* u, float* h, int64_t start, int64_t end,
                                    void* stream) {
    using namespace oom;
    OOM_REQUIRE(start >= 0 && start <= end, "oom_moe_swiglu_range: need 0 <= start <= end");
    if (start == end) return OOM_OK;
    OOM_REQUIRE(g && u && h, "oom_moe_swiglu_range: null buffer");
    const int64_t n = end - start;
    hipLaunchKernelGGL(moe_swiglu_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, as_stream(stream), g + start,
                       u + start, h + start, n);
    return launched("oom_moe_swiglu_range");
}
