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
// 64 assignments (four 16-row M subtiles): per step 8 v_mfma_f32_16x16x32_bf16 a term,
// M subtiles past the expert's assignments skipped. LDS rows are 40 bf16 (80 bytes), so
// the 16 rows of an operand read fall in distinct bank groups. Grid (ceil(N / 128),
// ceil(max_per_expert / 64), n_experts), as the reference's.
#include "stream.hpp"

namespace oom {

constexpr int T4_BN = 128;       // weight rows a block
constexpr int T4_BM = 64;        // assignments a block
constexpr int T4_BK = 32;        // K step
constexpr int T4_THREADS = 256;  // 4 waves
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

// bf16 bits of an f32 value that is a bf16 value (the weights here): its top half.
__device__ __forceinline__ uint32_t t4_pack(float lo, float hi) {
    return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

// The term t of x: hi = bf16(x), then the same of each remainder (round to nearest even).
template <int TERMS>
__device__ __forceinline__ void t4_split(float x, uint16_t (&t)[TERMS]) {
    float r = x;
#pragma unroll
    for (int p = 0; p < TERMS; p++) {
        t[p] = f32_to_bf16(r);
        r -= bf16_to_f32(t[p]);
    }
}

template <int TERMS>
__global__ void __launch_bounds__(T4_THREADS) moe_tiled_nvfp4_kernel(TiledArgs g) {
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
    const int wr = tid & (T4_BN - 1), wh = tid >> 7;
    const bool wok = r0 + wr < g.N;
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(rec + g.w_off), (short)0, (int)((int64_t)g.N * g.K / 2), BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(rec + g.s_off), (short)0, (int)((int64_t)g.N * g.K / 16), BUF_FLAGS);
    const int cbase = wok ? (r0 + wr) * (g.K / 2) + 8 * wh : OOB;
    const int sbase = wok ? (r0 + wr) * (g.K / 16) + wh : OOB;
    const float* xrow[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = (tid + i * T4_THREADS) >> 3;
        xrow[i] = t < nt ? g.x + (int64_t)(g.rows ? g.rows[a_begin + t] : a_begin + t) * g.K : nullptr;
    }
    auto load = [&](int kb, uint2& codes, uint32_t& sb, float4 (&xv)[2]) {
        const int k0 = kb * T4_BK;
        const auto c = __builtin_amdgcn_raw_buffer_load_b64(cr, cbase == OOB ? OOB : cbase + k0 / 2, 0, 0);
        codes = make_uint2(c[0], c[1]);
        sb = __builtin_amdgcn_raw_buffer_load_b8(sr, sbase == OOB ? OOB : sbase + k0 / 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int kq = ((tid + i * T4_THREADS) & 7) * 4;
            xv[i] = xrow[i] ? *reinterpret_cast<const float4*>(xrow[i] + k0 + kq) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    // decoded weights and split activations of a step into LDS buffer b
    auto stage = [&](int b, const uint2& codes, uint32_t sb, const float4 (&xv)[2]) {
        const float sc = __builtin_amdgcn_cvt_f32_fp8((int)sb, 0);
        uint32_t packed[8];
        const uint32_t cw[2] = {codes.x, codes.y};
#pragma unroll
        for (int i = 0; i < 2; i++) {
            // byte q of word i: columns 8 i + 2 q (low nibble) and 8 i + 2 q + 1
            const auto p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw[i], 1.0f, 0);
            const auto p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw[i], 1.0f, 1);
            const auto p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw[i], 1.0f, 2);
            const auto p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(cw[i], 1.0f, 3);
            packed[4 * i] = t4_pack(p0[0] * sc, p0[1] * sc);
            packed[4 * i + 1] = t4_pack(p1[0] * sc, p1[1] * sc);
            packed[4 * i + 2] = t4_pack(p2[0] * sc, p2[1] * sc);
            packed[4 * i + 3] = t4_pack(p3[0] * sc, p3[1] * sc);
        }
        uint4* dst = reinterpret_cast<uint4*>(&wsh[b][wr][16 * wh]);
        dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int idx = tid + i * T4_THREADS, t = idx >> 3, kq = (idx & 7) * 4;
            const float v[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
            uint16_t parts[4][TERMS];
#pragma unroll
            for (int c = 0; c < 4; c++) t4_split<TERMS>(v[c], parts[c]);
#pragma unroll
            for (int p = 0; p < TERMS; p++)
                *reinterpret_cast<uint2*>(&xsh[b][p][t][kq]) =
                    make_uint2((uint32_t)parts[0][p] | ((uint32_t)parts[1][p] << 16),
                               (uint32_t)parts[2][p] | ((uint32_t)parts[3][p] << 16));
        }
    };

    t4f4 acc[4][2];
#pragma unroll
    for (int ms = 0; ms < 4; ms++)
#pragma unroll
        for (int ns = 0; ns < 2; ns++) acc[ms][ns] = t4f4{0.0f, 0.0f, 0.0f, 0.0f};
    const int msn = (nt + 15) >> 4;  // M subtiles holding assignments (block-uniform)
    const int kl = 8 * (lane >> 4);  // this lane's 8 columns of a step
    uint2 codes;
    uint32_t sb;
    float4 xv[2];
    load(0, codes, sb, xv);
    for (int kb = 0; kb < nkb; kb++) {
        const int b = kb & 1;
        stage(b, codes, sb, xv);
        __syncthreads();
        if (kb + 1 < nkb) load(kb + 1, codes, sb, xv);
        t4bf16x8 bop[2];
#pragma unroll
        for (int ns = 0; ns < 2; ns++)
            bop[ns] = *reinterpret_cast<const t4bf16x8*>(&wsh[b][32 * wave + 16 * ns + (lane & 15)][kl]);
#pragma unroll
        for (int ms = 0; ms < 4; ms++) {
            if (ms >= msn) break;
#pragma unroll
            for (int p = 0; p < TERMS; p++) {
                const t4bf16x8 aop = *reinterpret_cast<const t4bf16x8*>(&xsh[b][p][16 * ms + (lane & 15)][kl]);
#pragma unroll
                for (int ns = 0; ns < 2; ns++)
                    acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop[ns], acc[ms][ns], 0, 0, 0);
            }
        }
    }
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
