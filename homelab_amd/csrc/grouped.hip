// Prefill MoE on gfx950: per-token e4m3 activation quantiser, FP8 x FP8 grouped GEMM on
// the matrix cores (v_mfma_scale_f32_16x16x128_f8f6f4, unit block scales), the gate/up
// pass with SwiGLU in its epilogue, the down pass over h as one or two bf16 terms on
// v_mfma_f32_16x16x32_bf16, and the whole prefill step (router, plan, quantise, gate/up,
// down, combine) without a host round trip.
//
// Grouped GEMM: y[a, r] = xs(a) * sum_kb ws(r, kb) * sum_{c in kb} e4m3(xq[row(a), c]) *
// e4m3(W[r, c]) for the assignments a of each expert (the semantics of
// crates/oominf-cuda/kernels/moe.cu:166-335, moe_tiled, with e4m3 activations): each MFMA
// covers exactly one 128-column scale block, so its fp32 block sum is scaled by the
// weight's 128 x 128 block scale (and, for per-group activations, the row's group
// scale) before it joins the accumulator.
//
//  * oom_moe_grouped_gemm_fp8: a block takes a 128-assignment x 128-output tile of one
//    expert (8 waves, each 32 x 64); per K step of 128 the block stages the activation rows
//    (gathered by assignment) and the weight rows in LDS (16-byte chunks, swizzled), and the
//    next step's loads are in flight while the current step runs on the matrix cores.
//  * The prefill's gate/up pass (grouped_gate_up256_kernel): 256 assignments x 128 gate and
//    128 up rows, both weight tiles sharing the activation tile; the epilogue forms
//    h = silu(g) * u and writes hi = bf16(h) and, for the exact precision, lo =
//    bf16(h - hi) (16 significant bits, relative error <= 2^-17): h is not quantised
//    again. The two precisions are the reference's (ExpertPrecision,
//    crates/oominf-core/src/backend.rs:142-149): Bf16 rounds the activations to bf16 for
//    one matrix-core pass, Exact keeps them fp32 (crates/oominf-cuda/kernels/moe.cu:166-335
//    splits them into exact bf16 terms the same way).
//  * The prefill's down pass (grouped_down512_kernel): 128 assignments x 512 outputs, A =
//    the h term planes, B = e4m3 weight rows converted exactly to bf16 in registers; every
//    term runs on the bf16 matrix cores, fp32 accumulate, the weight's 128 x 128 block
//    scale applied to each block sum.
#include <algorithm>

#include "router.hpp"

namespace oom {

constexpr int GBM = 128;         // assignments per block tile
constexpr int GBN = 128;         // outputs per block tile (one 128-row weight scale block)
constexpr int GBK = 128;         // K step (one scale block)
constexpr int GTHREADS = 512;    // 8 waves: 4 x 2 of 32 x 64
constexpr int G_BUF_FLAGS = 0x00020000;

typedef int gi32x8 __attribute__((ext_vector_type(8)));
typedef float gf32x4 __attribute__((ext_vector_type(4)));

struct GArgs {
    const uint64_t* recs;   // record of expert i (plan order)
    const int32_t* off;     // assignments of expert i: [off[i], off[i + 1])
    const int32_t* rows;    // activation row of assignment a (null: a itself)
    const int32_t* tiles;   // device tile table: [2 mt] = expert, [2 mt + 1] = first assignment offset (or null)
    const int32_t* ntiles;  // number of tiles in the table
    const uint8_t* xq;      // e4m3 activations [rows, K]
    const float* xs;        // per row (x_group 0) or per row and 128-column group (x_group 128)
    int x_group;
    int64_t N, K;
    int64_t w_off, s_off;   // first (or only) weight part and its scales
    int64_t w2_off, s2_off; // up part (gate/up pass)
    float* y;               // [A, N] fp32 (plain and down passes)
    uint16_t* hh;           // [A, N] bf16 hi term of h (gate/up pass) / of the activations (down pass)
    uint16_t* hl;           // [A, N] bf16 lo term
#ifdef OOM_STAMPS
    uint64_t* stamps;       // per block: start, end, (expert, first assignment, N offset, assignments), where
#endif
};

// A profiling build (-DOOM_STAMPS) records each block's start and end on the 100 MHz clock,
// its tile and the XCC / HW_ID it ran on: 4 words per linear block id.
#ifdef OOM_STAMPS
uint64_t* stamps_buffer();
__device__ __forceinline__ void g_stamp(uint64_t* st, int L, int p, uint64_t v) {
    if (st && threadIdx.x == 0) st[4 * (size_t)L + p] = v;
}
#define G_STAMP_START(G, L, I, M0, N0, CNT)                                                                  \
    do {                                                                                                     \
        g_stamp((G).stamps, L, 0, wall_clock64());                                                           \
        g_stamp((G).stamps, L, 2, ((uint64_t)(I) << 48) | ((uint64_t)(M0) << 32) | ((uint64_t)(N0) << 16) |  \
                                      (uint64_t)(CNT));                                                      \
        g_stamp((G).stamps, L, 3, ((uint64_t)(uint32_t)__builtin_amdgcn_s_getreg(20 | (15 << 11)) << 32) |   \
                                      (uint32_t)__builtin_amdgcn_s_getreg(4 | (31 << 11)));                  \
    } while (0)
#define G_STAMP_END(G, L) g_stamp((G).stamps, L, 1, wall_clock64())
#else
#define G_STAMP_START(G, L, I, M0, N0, CNT) \
    do {                                    \
    } while (0)
#define G_STAMP_END(G, L) \
    do {                  \
    } while (0)
#endif

// e4m3fn code of v, round to nearest even, saturating at +-448 (the quantiser's rule,
// crates/oominf-core/src/fp8.rs:5-27), with the gfx950 OCP-FP8 conversion.
__device__ __forceinline__ uint32_t e4m3_pair(float v0, float v1) {
    v0 = fminf(fmaxf(v0, -448.0f), 448.0f);
    v1 = fminf(fmaxf(v1, -448.0f), 448.0f);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false) & 0xffffu;
}

// ---- per-row activation quantiser: scale = absmax / 448 (1 for a zero row), q = e4m3(x / scale)
// (crates/oominf-core/src/fp8.rs:52-88 applied per token). One block of 256 per row.
template <int XDT>
__global__ void __launch_bounds__(256) quant_rows_kernel(const void* __restrict__ x, int64_t cols,
                                                         uint8_t* __restrict__ q, float* __restrict__ scale) {
    __shared__ float wmax[4];
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float m = 0.0f;
    for (int64_t c = tid; c < cols; c += 256) m = fmaxf(m, fabsf(load_act<XDT>(x, r * cols + c)));
    m = wave_max(m);
    if (lane == 0) wmax[wave] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
    if (tid == 0) scale[r] = s;
    for (int64_t c = 2 * tid; c < cols; c += 512) {
        const float v0 = load_act<XDT>(x, r * cols + c) / s;
        const float v1 = c + 1 < cols ? load_act<XDT>(x, r * cols + c + 1) / s : 0.0f;
        const uint32_t p = e4m3_pair(v0, v1);
        q[r * cols + c] = (uint8_t)(p & 0xff);
        if (c + 1 < cols) q[r * cols + c + 1] = (uint8_t)(p >> 8);
    }
}

// The same quantiser for rows whose width is a multiple of 8 and at most QV_MAXC: one pass
// over memory. Thread t holds chunks of 8 consecutive elements (16-byte bf16 or 2 x 16-byte
// f32 loads) in registers, the row's absmax reduces over the block, and each chunk stores
// its 8 codes as one 8-byte word. Same arithmetic as quant_rows_kernel (bit-identical codes
// and scales).
constexpr int QV_CH = 4;                 // chunks a thread
constexpr int QV_MAXC = 256 * 8 * QV_CH; // widest row of the one-pass form
template <int XDT>
__global__ void __launch_bounds__(256) quant_rows_vec_kernel(const void* __restrict__ x, int64_t cols,
                                                             uint8_t* __restrict__ q, float* __restrict__ scale) {
    __shared__ float wmax[4];
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float v[QV_CH][8];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < QV_CH; j++) {
        const int64_t c = (int64_t)(j * 256 + tid) * 8;
        if (c < cols) {
            if constexpr (XDT == OOM_BF16) {
                const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + r * cols + c);
                const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[j][2 * i] = __uint_as_float(ww[i] << 16);
                    v[j][2 * i + 1] = __uint_as_float(ww[i] & 0xffff0000u);
                }
            } else {
                const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + r * cols + c);
                const float4 a = p[0], b = p[1];
                v[j][0] = a.x; v[j][1] = a.y; v[j][2] = a.z; v[j][3] = a.w;
                v[j][4] = b.x; v[j][5] = b.y; v[j][6] = b.z; v[j][7] = b.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[j][i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; i++) m = fmaxf(m, fabsf(v[j][i]));
    }
    m = wave_max(m);
    if (lane == 0) wmax[wave] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
    if (tid == 0) scale[r] = s;
#pragma unroll
    for (int j = 0; j < QV_CH; j++) {
        const int64_t c = (int64_t)(j * 256 + tid) * 8;
        if (c < cols) {
            uint32_t p[4];
#pragma unroll
            for (int i = 0; i < 4; i++) p[i] = e4m3_pair(v[j][2 * i] / s, v[j][2 * i + 1] / s);
            *reinterpret_cast<uint2*>(q + r * cols + c) = make_uint2(p[0] | (p[1] << 16), p[2] | (p[3] << 16));
        }
    }
}

// ---- the tile table of a device plan: tile mt = (expert i, assignments from off[i] + m0).
// One block of 1024 threads a table; experts in chunks of 1024 with a running carry. With
// light_rows > 0 the table lists the tiles of more than light_rows assignments first and
// then the others (each expert's last tile when it holds at most light_rows), so the
// blocks that take tiles in table order start the long ones first. Block 1, when
// launched, builds a second table (tile_rows2, light_rows2, tiles2, ntiles2).
struct TileTable {
    int tile_rows, light_rows;
    int32_t* tiles;
    int32_t* ntiles;
};
__global__ void __launch_bounds__(1024) grouped_tiles_kernel(const int32_t* __restrict__ n_e_p,
                                                             const int32_t* __restrict__ off, TileTable t0,
                                                             TileTable t1) {
    const TileTable tt = blockIdx.x == 0 ? t0 : t1;
    const int tile_rows = tt.tile_rows, light_rows = tt.light_rows;
    int32_t* __restrict__ tiles = tt.tiles;
    int32_t* __restrict__ ntiles = tt.ntiles;
    __shared__ int wsum[16];
    __shared__ int carry_s;
    const int n_e = *n_e_p, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) carry_s = 0;
    __syncthreads();
    for (int pass = 0; pass < (light_rows > 0 ? 2 : 1); pass++)
    for (int c0 = 0; c0 < n_e; c0 += (int)blockDim.x) {
        const int i = c0 + tid;
        const int n = i < n_e ? off[i + 1] - off[i] : 0, full = n / tile_rows, rem = n - full * tile_rows;
        // pass 0: every tile, or (light_rows > 0) all but a last tile of at most light_rows;
        // pass 1: that last tile
        const bool last_light = light_rows > 0 && rem > 0 && rem <= light_rows;
        const int cnt = pass == 0 ? full + (rem > 0 && !last_light ? 1 : 0) : (last_light ? 1 : 0);
        const int t0 = pass == 0 ? 0 : full;
        // inclusive scan within the wave, then over the waves
        int incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int before = carry_s;
        for (int w = 0; w < wave; w++) before += wsum[w];
        const int start = before + incl - cnt;
        for (int t = 0; t < cnt; t++) {
            tiles[2 * (start + t)] = i;
            tiles[2 * (start + t) + 1] = (t0 + t) * tile_rows;
        }
        __syncthreads();
        if (tid == (int)blockDim.x - 1) carry_s = start + cnt;
        __syncthreads();
    }
    if (tid == 0) *ntiles = carry_s;
}

constexpr int G_OOB = 0x7ffffff0;  // past every resource here (extents stay below 0x7fff0000): loads read 0

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// LDS image of a tile (rows x 128 bytes of one K step) as 16-byte chunks: chunk c of row
// r sits at position 8 r + (c ^ f(r)), f(r) = (r & 7) ^ ((r >> 3) & 1). An MFMA operand
// read takes one chunk column of 16 rows: any 8 consecutive of them (r = 8q .. 8q + 7)
// land in 8 different 16-byte bank groups of a 128-byte line, and all 16 in 16 different
// groups of a 256-byte line (f is a bijection on each 8 rows, and rows r, r + 8 differ in
// f's low bit, rows of one parity pair with a distinct f).
__device__ __forceinline__ int chunk_key(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int chunk_pos(int r, int c) { return 8 * r + (c ^ chunk_key(r)); }

// The inverse for the loads: position p of the tile holds row p / 8, chunk (p % 8) ^ f.
__device__ __forceinline__ void pos_chunk(int p, int& r, int& c) {
    r = p >> 3;
    c = (p & 7) ^ chunk_key(r);
}

// Activation rows of assignments a[i] (an assignment past a1 reads row `valid`'s entry), all
// loads in flight before the first use: under a per-row test the compiler moved each load
// into its branch, behind a wait for the load before (a round trip per row).
template <int N>
__device__ __forceinline__ void token_rows(const GArgs& g, const int (&a)[N], int a1, int valid, int (&r)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) {
        const int ac = a[i] < a1 ? a[i] : valid;
        r[i] = g.rows ? g.rows[ac] : ac;
    }
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(r[i]));
}

// The per-row activation scales xs of rows r[i], the same way.
template <int N>
__device__ __forceinline__ void row_scales(const GArgs& g, const int (&r)[N], float (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) x[i] = g.xs[r[i]];
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(x[i]));
}

// One 16-byte load per lane straight into LDS: lane l's bytes land at lds + 16 l.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, int off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, off, 0, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, void* lds, int off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 4, off, 0, 0, 0);
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding): this wave's loads but the newest n have
// completed, and its LDS accesses.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
}

// A workgroup barrier with no memory fence: the loop's only LDS writes are direct-to-LDS
// loads, and each wave waits for its own before arriving, so after the barrier every
// wave's loads of the stage have landed. (__syncthreads's release fence would wait for
// every load in flight, the next stages' too.) The signal fences keep the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void g_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The per-thread sources of a stage: A chunks (activation rows gathered by assignment),
// B chunks (weight rows), the activation group scale of tile row 16 wave + lane (lanes
// < 16, x_group 128) and the weight block scales (lanes < NB).
template <int NB>
struct GSrc {
    __amdgpu_buffer_rsrc_t xr, wr, xsr, sr;
    int xo[2], wo[NB][2];  // step-0 byte offsets (xo < 0: a row past the expert, loads zeros)
    int xso, so;           // step-0 byte offsets of this lane's scales (G_OOB: none)
};

// Stage of step kb into LDS: the operands into stage buffer `sb` (A tile, then NB B tiles),
// the scales into `scx` and `scw` (64 words per wave). kb >= nkb: every load reads zeros
// (offsets past their resources), which keeps each wave's load count fixed.
template <int NB>
__device__ __forceinline__ void g_issue(const GSrc<NB>& s, int kb, int nkb, uint8_t* sb, float* scx, float* scw,
                                        int wave) {
    const bool ok = kb < nkb;
    const int k0 = kb * GBK;
#pragma unroll
    for (int j = 0; j < 2; j++) dma16(s.xr, sb + (2 * wave + j) * 1024, ok && s.xo[j] >= 0 ? s.xo[j] + k0 : G_OOB);
#pragma unroll
    for (int m = 0; m < NB; m++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            dma16(s.wr, sb + GBM * GBK + m * GBN * GBK + (2 * wave + j) * 1024, ok ? s.wo[m][j] + k0 : G_OOB);
    // the scales, into the wave's 64-word slots (lane l writes word l): lanes 0..15 the
    // group scales of tile rows 16 wave + l, lanes 0 .. NB the weight block scales; the
    // other lanes read zeros past their resource. Every lane runs both loads, so each
    // wave's count of loads in flight is the same on every path.
    dma4(s.xsr, scx + 64 * wave, ok && s.xso != G_OOB ? s.xso + 4 * kb : G_OOB);
    dma4(s.sr, scw + 64 * wave, ok && s.so != G_OOB ? s.so + 4 * kb : G_OOB);
}

// 32 bytes of tile row `row` at K offset 32 (lane / 16): an MFMA operand (A: row = M
// index, B: row = N index; both layouts take k = 32 (lane / 16) + byte).
__device__ __forceinline__ gi32x8 gop(const uint8_t* base, int row, int lane) {
    const int c = 2 * (lane >> 4);
    const uint4 lo = *reinterpret_cast<const uint4*>(base + 16 * chunk_pos(row, c));
    const uint4 hi = *reinterpret_cast<const uint4*>(base + 16 * chunk_pos(row, c + 1));
    gi32x8 v;
    v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
    v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
    return v;
}

// One K step on the matrix cores from a stage buffer: acc += the block sums scaled by the
// weight's block scale (and the row's activation group scale). act: the wave's 16-row M
// subtiles that hold assignments (1 or 2; the others' products are never stored).
template <int NB>
__device__ __forceinline__ void g_step(const uint8_t* sb, const float* scx, const float* scw, bool xgrp, int wm,
                                       int wn, int wave, int lane, int act, float (&acc)[NB][2][4][4]) {
    // tile row r's group scale is word 64 (r / 16) + r % 16 of scx; the wave's weight
    // scales words 64 wave + m of scw
    float xsk[2][4];
    if (xgrp) {
#pragma unroll
        for (int ms = 0; ms < 2; ms++)
#pragma unroll
            for (int e = 0; e < 4; e++) xsk[ms][e] = scx[64 * (2 * wm + ms) + 4 * (lane >> 4) + e];
    }
    float wsk[NB];
#pragma unroll
    for (int m = 0; m < NB; m++) wsk[m] = scw[64 * wave + m];
    gi32x8 aop[2];
#pragma unroll
    for (int ms = 0; ms < 2; ms++) aop[ms] = gop(sb, 32 * wm + 16 * ms + (lane & 15), lane);
#pragma unroll
    for (int m = 0; m < NB; m++)
#pragma unroll
        for (int ns = 0; ns < 4; ns++) {
            const gi32x8 bop = gop(sb + GBM * GBK + m * GBN * GBK, 64 * wn + 16 * ns + (lane & 15), lane);
#pragma unroll
            for (int ms = 0; ms < 2; ms++) {
                if (ms >= act) continue;
                const gf32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                const gf32x4 blk =
                    __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aop[ms], bop, z, 0, 0, 0, 127, 0, 127);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float sc = xgrp ? wsk[m] * xsk[ms][e] : wsk[m];
                    acc[m][ms][ns][e] = fmaf(blk[e], sc, acc[m][ms][ns][e]);
                }
            }
        }
}

// y = scaled xq . W^T (oom_moe_grouped_gemm_fp8).
//
// K steps stream through two LDS stage buffers filled by direct-to-LDS buffer loads (two
// blocks per CU, which overlap each other's waits): at step kb a wave waits for its own
// loads of stage kb, the block synchronises (every wave's loads of kb have landed, and
// every wave is done reading the buffer stage kb + 1 takes), stage kb + 1 is issued, and
// step kb runs on the matrix cores while kb + 1 loads. Grid (N / 128, M-tiles, experts).
__global__ void __launch_bounds__(GTHREADS) grouped_gemm_kernel(GArgs g) {
    constexpr int NB = 1;
    constexpr int SBYTES = GBM * GBK + NB * GBN * GBK;  // one stage: the A tile and the B tile
    // each stage its own LDS object: the compiler's wait for direct-to-LDS loads then
    // covers only the loads into the buffer a read touches
    // a stage: the A tile, the B tile, then the activation and weight scales (64 words per
    // wave each)
    constexpr int STOT = SBYTES + 2 * GTHREADS * 4;
    __shared__ __align__(16) uint8_t sb0[STOT], sb1[STOT];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;  // rows 32 wm .. + 32, columns 64 wn .. + 64
    const int i = blockIdx.z, m0 = blockIdx.y * GBM, n0 = blockIdx.x * GBN;
    const int a0 = g.off[i], a1 = g.off[i + 1];
    if (a0 + m0 >= a1) return;
    const int Lb = (int)(blockIdx.x + blockIdx.y * gridDim.x);
    (void)Lb;
    G_STAMP_START(g, Lb, i, m0, n0, a1 - a0);
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(g.recs[i]);
    const int nkb = (int)(g.K / GBK);
    const bool xgrp = g.x_group != 0;
    // ---- this thread's sources: load j of the A (and each B) tile covers positions
    // (2 wave + j) 64 + lane, i.e. chunk c of tile row r (rows past the expert's range
    // load zeros from past the resource: no memory traffic, and their products are not
    // stored) ----
    GSrc<NB> src;
    src.xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(g.xq), (short)0, 0x7fff0000, G_BUF_FLAGS);
    const int wbytes = (int)(max(g.w_off, NB == 2 ? g.w2_off : g.w_off) + g.N * g.K);  // end of the weight parts
    src.wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(rec), (short)0, wbytes, G_BUF_FLAGS);
    int xa[2], xc[2], xrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int r;
        pos_chunk((2 * wave + j) * 64 + lane, r, xc[j]);
        xa[j] = a0 + m0 + r;
#pragma unroll
        for (int m = 0; m < NB; m++)
            src.wo[m][j] = (int)((m == 0 ? g.w_off : g.w2_off) + (int64_t)(n0 + r) * g.K) + 16 * xc[j];
    }
    token_rows(g, xa, a1, a0 + m0, xrow);
#pragma unroll
    for (int j = 0; j < 2; j++) src.xo[j] = xa[j] < a1 ? (int)(xrow[j] * g.K) + 16 * xc[j] : -1;
    // scales: lane l < 16 of wave w loads tile row 16 w + l's group scale (x_group 128),
    // lane m < NB the block scale of weight matrix m, once per K step
    src.sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(rec), (short)0, 0x7fff0000, G_BUF_FLAGS);
    src.xsr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.xs), (short)0, xgrp ? 0x7fff0000 : 0,
                                                G_BUF_FLAGS);
    src.xso = G_OOB;
    if (xgrp && lane < 16) {
        const int a = min(a0 + m0 + 16 * wave + lane, a1 - 1);
        src.xso = (int)((g.rows ? g.rows[a] : a) * nkb * 4);
    }
    src.so = lane < NB ? (int)((lane == 0 ? g.s_off : g.s2_off) + (int64_t)(n0 / 128) * nkb * 4) : G_OOB;
    const int left = a1 - (a0 + m0) - 32 * wm;  // assignments from this wave's first row on
    const int act = __builtin_amdgcn_readfirstlane(left <= 0 ? 0 : left <= 16 ? 1 : 2);
    // this lane's output rows (per 16-row M subtile ms, element e): assignment index
    int arow_out[2][4];
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
        for (int e = 0; e < 4; e++) arow_out[ms][e] = a0 + m0 + 32 * wm + 16 * ms + 4 * (lane >> 4) + e;
    float acc[NB][2][4][4];  // [matrix][M subtile][N subtile][element]
#pragma unroll
    for (int m = 0; m < NB; m++)
#pragma unroll
        for (int ms = 0; ms < 2; ms++)
#pragma unroll
            for (int ns = 0; ns < 4; ns++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[m][ms][ns][e] = 0.0f;
#define G_SX(B) reinterpret_cast<float*>((B) + SBYTES)
#define G_SW(B) reinterpret_cast<float*>((B) + SBYTES + GTHREADS * 4)
    // one step on stage buffer SB while stage kb + 1 goes into NSB
#define G_STEP(SB, NSB)                                                                             \
    {                                                                                               \
        wait_vm<0>();                                                                               \
        g_barrier();                                                                                \
        g_issue<NB>(src, kb + 1, nkb, NSB, G_SX(NSB), G_SW(NSB), wave);                             \
        if (act > 0) g_step<NB>(SB, G_SX(SB), G_SW(SB), xgrp, wm, wn, wave, lane, act, acc);        \
        if (++kb == nkb) break;                                                                     \
    }
    int kb = 0;
    g_issue<NB>(src, 0, nkb, sb0, G_SX(sb0), G_SW(sb0), wave);
    for (;;) {
        G_STEP(sb0, sb1)
        G_STEP(sb1, sb0)
    }
#undef G_SX
#undef G_SW
#undef G_STEP
    wait_vm<0>();  // the zero-filled stages past the end have landed before LDS is reused
    __syncthreads();
    // ---- epilogue ----
    float xsr[8];
    if (!g.x_group) {
        int orow[8];
        token_rows(g, reinterpret_cast<const int(&)[8]>(arow_out), a1, a0 + m0, orow);
        row_scales(g, orow, xsr);
    }
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int a = arow_out[ms][e];
            if (a >= a1) continue;
#pragma unroll
            for (int ns = 0; ns < 4; ns++) {
                const int64_t n = n0 + 64 * wn + 16 * ns + (lane & 15);
                if (n < g.N)
                    g.y[(int64_t)a * g.N + n] = g.x_group ? acc[0][ms][ns][e] : acc[0][ms][ns][e] * xsr[4 * ms + e];
            }
        }
    G_STAMP_END(g, Lb);
}

// ---- gate/up over 256-assignment tiles (the prefill step) -----------------------------
//
// A block takes 256 assignments x 128 gate rows and the same 128 up rows of one expert: a
// K step moves 64 KiB into LDS (the activation tile 32 KiB, each weight tile 16 KiB) for
// 256 x 256 x 128 multiply-adds, against 48 KiB for half of that in a 128-row tile, and an
// expert's weight slab is staged once per 256 assignments instead of once per 128. Wave
// (wm, wn) of the 8 takes rows 64 wm .. + 64 (4 M subtiles) and rows 64 wn .. + 64 of both
// weight tiles (4 N subtiles each): 128 accumulators a lane. Two LDS stages: at step kb a
// wave waits for its own loads of stage kb, the block synchronises (every wave's loads of
// kb have landed, every wave is done reading the other buffer), stage kb + 1 is issued, and
// step kb runs on the matrix cores while kb + 1 loads. Per-row activation scales only
// (x_group 0, the prefill's quantiser). Tiles come from a table of 256-row tiles.
//
// A tile of at most 32 assignments (a light expert, or a heavy expert's last rows) is a
// stream of its weight slab: its step time is the latency of a stage, whatever the stage
// holds. Its stages hold two K steps each (two 36 KiB halves: the 32-row activation tile
// and both weight tiles of a K step), so 64 KiB of weights are in flight instead of 32.
constexpr int GBM2 = 256;                                 // assignments per block tile
constexpr int GU2_SB = GBM2 * GBK + 2 * GBN * GBK;        // stage operands: A, gate, up tiles
constexpr int GU2_LROWS = 32;                             // assignments of a two-step (light) tile
constexpr int GU2_LA = GU2_LROWS * GBK;                   // its activation tile, one K step
constexpr int GU2_LHALF = GU2_LA + 2 * GBN * GBK;         // one K step of a light stage
constexpr int GU2_SCALES = GU2_SB > 2 * GU2_LHALF ? GU2_SB : 2 * GU2_LHALF;  // the scale words
constexpr int GU2_STOT = GU2_SCALES + GTHREADS * 4;       // + 64 words a wave

struct GU2Src {
    __amdgpu_buffer_rsrc_t xr, wr, sr;
    int xo[4], wo[2][2];  // step-0 byte offsets (xo < 0: a row past the expert, loads zeros)
    int so;               // step-0 byte offset of this lane's weight block scale (G_OOB: none)
    int lxo, lso;         // the light stages' activation chunk and scale (wave / 4: which K step)
};

__device__ __forceinline__ void gu2_issue(const GU2Src& s, int kb, int nkb, uint8_t* sb, int wave) {
    const bool ok = kb < nkb;
    const int k0 = kb * GBK;
#pragma unroll
    for (int j = 0; j < 4; j++) dma16(s.xr, sb + (4 * wave + j) * 1024, ok && s.xo[j] >= 0 ? s.xo[j] + k0 : G_OOB);
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            dma16(s.wr, sb + GBM2 * GBK + m * GBN * GBK + (2 * wave + j) * 1024, ok ? s.wo[m][j] + k0 : G_OOB);
    dma4(s.sr, reinterpret_cast<float*>(sb + GU2_SCALES) + 64 * wave, ok && s.so != G_OOB ? s.so + 4 * kb : G_OOB);
}

// A light stage: K steps kb and kb + 1 (kb even, K steps even in number). Waves 0-3 load
// the first step's 32-row activation tile, waves 4-7 the second's; every wave loads its
// chunks of both steps' weight tiles; lanes 0-3 the block scales (gate kb, up kb, gate
// kb + 1, up kb + 1).
__device__ __forceinline__ void gu2_issue_light(const GU2Src& s, int kb, int nkb, uint8_t* sb, int wave) {
    const bool ok = kb < nkb;
    const int k0 = kb * GBK;
    dma16(s.xr, sb + (wave >> 2) * GU2_LHALF + (wave & 3) * 1024, ok && s.lxo >= 0 ? s.lxo + k0 : G_OOB);
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int m = 0; m < 2; m++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                dma16(s.wr, sb + h * GU2_LHALF + GU2_LA + m * GBN * GBK + (2 * wave + j) * 1024,
                      ok ? s.wo[m][j] + k0 + h * GBK : G_OOB);
    dma4(s.sr, reinterpret_cast<float*>(sb + GU2_SCALES) + 64 * wave, ok && s.lso != G_OOB ? s.lso + 4 * kb : G_OOB);
}

// One K step: acc[m][ms][ns] += ws[m] * (block sum of M subtile ms and N subtile ns of
// weight matrix m), over the activation tile `at` and the weight tiles at `bt`. A wave with
// any assignment runs MS M subtiles (rows past the expert hold zeros and are not stored):
// per-subtile branches cost more registers than the matrix work they save.
template <int MS>
__device__ __forceinline__ void gu2_step(const uint8_t* at, const uint8_t* bt, const float* ws, int wm, int wn,
                                         int lane, float (&acc)[2][4][4][4]) {
    const float wsc[2] = {ws[0], ws[1]};
    gi32x8 aop[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++) aop[ms] = gop(at, 64 * wm + 16 * ms + (lane & 15), lane);
    // the 8 B operands (gate subtiles, then up) one read ahead of their products: holding
    // all of them beside the 128 accumulators spills
    const int brow = 64 * wn + (lane & 15);
    gi32x8 bcur = gop(bt, brow, lane);
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int m = q >> 2, ns = q & 3;
        gi32x8 bnext = bcur;
        if (q < 7) bnext = gop(bt + ((q + 1) >> 2) * GBN * GBK, brow + 16 * ((q + 1) & 3), lane);
#pragma unroll
        for (int ms = 0; ms < MS; ms++) {
            const gf32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            const gf32x4 blk = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aop[ms], bcur, z, 0, 0, 0, 127, 0, 127);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[m][ms][ns][e] = fmaf(blk[e], wsc[m], acc[m][ms][ns][e]);
        }
        __builtin_amdgcn_sched_barrier(0);
        bcur = bnext;
    }
}

__global__ void __launch_bounds__(GTHREADS) grouped_gate_up256_kernel(GArgs g) {
    // each stage its own LDS object, so the compiler's waits for direct-to-LDS loads cover
    // only the loads into the buffer a read touches
    __shared__ __align__(16) uint8_t sb0[GU2_STOT], sb1[GU2_STOT];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    // block L runs on XCD L % 8 as its item q = L / 8: tile 8 (q / NT) + L % 8, N-tile q % NT
    // (tiles dealt to the XCDs in turn, so each XCD gets its share of heavy and light tiles;
    // a tile's N-tiles run together and share its activation rows through that XCD's L2)
    const int NT = (int)gridDim.x, MT = *g.ntiles;
    const int L = (int)(blockIdx.x + blockIdx.y * gridDim.x), q = L >> 3;
    const int mt = 8 * (q / NT) + (L & 7), nt = q % NT;
    if (mt >= MT) return;
    const int i = g.tiles[2 * mt], m0 = g.tiles[2 * mt + 1], n0 = nt * GBN;
    const int a0 = g.off[i], a1 = g.off[i + 1];
    if (a0 + m0 >= a1) return;
    G_STAMP_START(g, L, i, m0, n0, a1 - a0);
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(g.recs[i]);
    const int nkb = (int)(g.K / GBK);
    GU2Src src;
    src.xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(g.xq), (short)0, 0x7fff0000, G_BUF_FLAGS);
    src.wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(rec), (short)0,
                                               (int)(max(g.w_off, g.w2_off) + g.N * g.K), G_BUF_FLAGS);
    src.sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(rec), (short)0, 0x7fff0000, G_BUF_FLAGS);
    // load j of the A tile covers positions (4 wave + j) 64 + lane, of each weight tile
    // (2 wave + j) 64 + lane: chunk c of tile row r
    // the A tile's rows (j < 4) and the light stages' row (j = 4), their row loads together
    int xa[5], xc[5], xrow[5];
#pragma unroll
    for (int j = 0; j < 5; j++) {
        int r;
        pos_chunk((j < 4 ? 4 * wave + j : wave & 3) * 64 + lane, r, xc[j]);
        xa[j] = a0 + m0 + r;
    }
    token_rows(g, xa, a1, a0 + m0, xrow);
#pragma unroll
    for (int j = 0; j < 4; j++) src.xo[j] = xa[j] < a1 ? (int)(xrow[j] * g.K) + 16 * xc[j] : -1;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int r, c;
        pos_chunk((2 * wave + j) * 64 + lane, r, c);
#pragma unroll
        for (int m = 0; m < 2; m++)
            src.wo[m][j] = (int)((m == 0 ? g.w_off : g.w2_off) + (int64_t)(n0 + r) * g.K) + 16 * c;
    }
    src.so = lane < 2 ? (int)((lane == 0 ? g.s_off : g.s2_off) + (int64_t)(n0 / 128) * nkb * 4) : G_OOB;
    const bool light = a1 - (a0 + m0) <= GU2_LROWS && (nkb & 1) == 0;
    {
        // light stages: activation chunk (wave % 4) 64 + lane of K step kb + wave / 4, and
        // lane 2 h + m's block scale of matrix m at K step kb + h
        src.lxo = xa[4] < a1 ? (int)(xrow[4] * g.K) + 16 * xc[4] + (wave >> 2) * GBK : -1;
        src.lso = lane < 4 ? (int)(((lane & 1) == 0 ? g.s_off : g.s2_off) + (int64_t)(n0 / 128) * nkb * 4) +
                                 4 * (lane >> 1)
                           : G_OOB;
    }
    const bool act = __builtin_amdgcn_readfirstlane(a1 - (a0 + m0) - 64 * wm > 0);  // the wave holds assignments
    float acc[2][4][4][4];
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int ms = 0; ms < 4; ms++)
#pragma unroll
            for (int ns = 0; ns < 4; ns++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[m][ms][ns][e] = 0.0f;
#define GU2_SW(B) (reinterpret_cast<const float*>((B) + GU2_SCALES) + 64 * wave)
#define GU2_STEP(SB, NSB)                                                                 \
    {                                                                                     \
        wait_vm<0>();                                                                     \
        g_barrier();                                                                      \
        gu2_issue(src, kb + 1, nkb, NSB, wave);                                           \
        if (act) gu2_step<4>(SB, SB + GBM2 * GBK, GU2_SW(SB), wm, wn, lane, acc);         \
        if (++kb == nkb) break;                                                           \
    }
#define GU2_LSTEP(SB, NSB)                                                                                     \
    {                                                                                                          \
        wait_vm<0>();                                                                                          \
        g_barrier();                                                                                           \
        gu2_issue_light(src, kb + 2, nkb, NSB, wave);                                                          \
        if (act) {                                                                                             \
            gu2_step<2>(SB, SB + GU2_LA, GU2_SW(SB), wm, wn, lane, acc);                                       \
            gu2_step<2>(SB + GU2_LHALF, SB + GU2_LHALF + GU2_LA, GU2_SW(SB) + 2, wm, wn, lane, acc);           \
        }                                                                                                      \
        kb += 2;                                                                                               \
        if (kb == nkb) break;                                                                                  \
    }
    int kb = 0;
    if (light) {
        gu2_issue_light(src, 0, nkb, sb0, wave);
        for (;;) {
            GU2_LSTEP(sb0, sb1)
            GU2_LSTEP(sb1, sb0)
        }
    } else {
        gu2_issue(src, 0, nkb, sb0, wave);
        for (;;) {
            GU2_STEP(sb0, sb1)
            GU2_STEP(sb1, sb0)
        }
    }
#undef GU2_STEP
#undef GU2_LSTEP
#undef GU2_SW
    wait_vm<0>();  // the zero-filled stage past the end has landed before the block ends
    // h = silu(xs g) * (xs u) as two bf16 terms: hi = bf16(h), lo = bf16(h - hi)
    float xsr[16];
    {
        int oa[16], orow[16];
#pragma unroll
        for (int i = 0; i < 16; i++) oa[i] = a0 + m0 + 64 * wm + 16 * (i >> 2) + 4 * (lane >> 4) + (i & 3);
        token_rows(g, oa, a1, a0 + m0, orow);
        row_scales(g, orow, xsr);
    }
#pragma unroll
    for (int ms = 0; ms < 4; ms++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int a = a0 + m0 + 64 * wm + 16 * ms + 4 * (lane >> 4) + e;
            if (a >= a1) continue;
            const float xs_a = xsr[4 * ms + e];
#pragma unroll
            for (int ns = 0; ns < 4; ns++) {
                const float h = siluf(acc[0][ms][ns][e] * xs_a) * (acc[1][ms][ns][e] * xs_a);
                const uint16_t hi = f32_to_bf16(h);
                const int64_t n = n0 + 64 * wn + 16 * ns + (lane & 15);
                g.hh[(int64_t)a * g.N + n] = hi;
                if (g.hl) g.hl[(int64_t)a * g.N + n] = f32_to_bf16(h - bf16_to_f32(hi));
            }
        }
    G_STAMP_END(g, L);
}

// ---- down pass over h as one or two bf16 terms ----------------------------------------
//
// y[a, r] = sum_kb ws(r, kb) * sum_{c in kb} (hi[a, c] (+ lo[a, c])) * e4m3(W[r, c]) for the
// assignments a of each expert (W = the down weights [N = hidden, K = inter]); e4m3 -> bf16
// is exact and bf16 products are exact in fp32, so each 64-column half of a 128-column
// scale block sums exact products in fp32, scaled by the weight's block scale as it joins
// the accumulator. One term (hi = bf16(h)) is the reference's ExpertPrecision::Bf16
// arithmetic; two (hi + lo, 16 significant bits of the fp32 h) stand for
// ExpertPrecision::Exact.
//
// K steps of 64 through LDS stages filled by direct-to-LDS loads, as the FP8 passes. An h
// term tile holds 64 bf16 (128 bytes) a row in 8 chunks with the FP8 tiles' chunk swizzle;
// the weight tile 64 bytes a row in 4 chunks, chunk c of row r at 4 r + (c ^ ((r >> 2) & 3)),
// so the 16 rows of an operand read, and any 8 of them, land in distinct 16-byte bank
// groups. Lane l of a wave takes K values 16 (l / 16) .. + 16 of the step for its row (A:
// assignment l % 16 of a 16-row subtile, B: weight row l % 16), as two 8-value halves, one
// per MFMA: the same K order on both sides, so the contraction is the plain sum.
constexpr int GBK2 = 64;                       // K step of the down pass
constexpr int D_HT = GBM * GBK2 * 2;           // bytes of one h term tile

typedef __bf16 gbf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ int wchunk_pos(int r, int c) { return 4 * r + (c ^ ((r >> 2) & 3)); }

constexpr int DL_ROWS = 32;                    // assignments of a light tile
constexpr int DL_HT = DL_ROWS * GBK2 * 2;      // bytes of one light h term tile

// ---- down over 512-output tiles (the prefill step) -------------------------------------
//
// A down tile waits on its loads more than on its work: a 256-output tile with the matrix
// cores, the conversions and the operand reads all switched off still took three quarters
// of its time. A tile of 128 assignments x 512 outputs moves 64 KiB a K step (the h term
// tiles 32 KiB, the weight tile 32 KiB) for twice the multiply-adds of a 256-output tile's
// 48 KiB. Wave (wm, wn) of the 8 takes h rows 32 wm .. + 32 (2 M subtiles) and weight rows
// 256 wn .. + 256 (16 N subtiles, two 128-row scale blocks): 128 accumulators a lane, so
// each K step's block sums are scaled into them at once (one K step is half a 128-column
// scale block; both halves take its scale) instead of held across the block. Two LDS
// stages (the two-stage protocol of grouped_gate_up256_kernel). A tile of at most 32
// assignments streams its weights instead: wave w takes weight rows 64 w .. + 64 over the
// tile's h rows, and a stage holds one K step's 32-row h term tiles and the weight tile.
constexpr int GBN5 = 512;                    // outputs per block tile
constexpr int D5_WT = GBN5 * GBK2;           // bytes of the weight tile, one K step
template <int TERMS>
constexpr int d5_scales() { return TERMS * D_HT + D5_WT > 2 * DL_HT + D5_WT ? TERMS * D_HT + D5_WT : 2 * DL_HT + D5_WT; }
template <int TERMS>
constexpr int d5_stot() { return d5_scales<TERMS>() + GTHREADS * 4; }

struct D5Src {
    __amdgpu_buffer_rsrc_t hr, wr, sr;
    int ho[2], wo[4];  // step-0 byte offsets (ho < 0: a row past the expert, loads zeros)
    int hl_off;        // bytes from the hi plane to the lo plane
    int so;            // this lane's block scale at K step 0 (G_OOB: none)
    int lho;           // light stages: this wave's h chunk (< 0: past the expert or no chunk)
};

// Heavy stage: h term t's chunks (2 wave + j) 64 + lane, the weight chunks (4 wave + j) 64
// + lane, lanes 0-1 the wave's two block scales.
template <int TERMS>
__device__ __forceinline__ void d5_issue(const D5Src& s, int kb, int nkb, uint8_t* sb, int wave) {
    const bool ok = kb < nkb;
    const int k0 = kb * GBK2 * 2;
#pragma unroll
    for (int t = 0; t < TERMS; t++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            dma16(s.hr, sb + t * D_HT + (2 * wave + j) * 1024, ok && s.ho[j] >= 0 ? s.ho[j] + t * s.hl_off + k0 : G_OOB);
#pragma unroll
    for (int j = 0; j < 4; j++)
        dma16(s.wr, sb + TERMS * D_HT + (4 * wave + j) * 1024, ok ? s.wo[j] + kb * GBK2 : G_OOB);
    dma4(s.sr, reinterpret_cast<float*>(sb + d5_scales<TERMS>()) + 64 * wave,
         ok && s.so != G_OOB ? s.so + 4 * (kb >> 1) : G_OOB);
}

// Light stage: one h chunk a wave (TERMS 2: term wave / 4; TERMS 1: waves 4-7 load zeros
// into the unused second term area), the weight chunks as above, lane 0 the block scale.
template <int TERMS>
__device__ __forceinline__ void d5_issue_light(const D5Src& s, int kb, int nkb, uint8_t* sb, int wave) {
    const bool ok = kb < nkb;
    const int k0 = kb * GBK2 * 2;
    dma16(s.hr, sb + (wave >> 2) * DL_HT + (wave & 3) * 1024, ok && s.lho >= 0 ? s.lho + k0 : G_OOB);
#pragma unroll
    for (int j = 0; j < 4; j++)
        dma16(s.wr, sb + 2 * DL_HT + (4 * wave + j) * 1024, ok ? s.wo[j] + kb * GBK2 : G_OOB);
    dma4(s.sr, reinterpret_cast<float*>(sb + d5_scales<TERMS>()) + 64 * wave,
         ok && s.so != G_OOB ? s.so + 4 * (kb >> 1) : G_OOB);
}

// One K step: NS N subtiles over the wave's 2 M subtiles (rows past the expert hold zeros
// and are not stored). at: the term-0 h tile (term t at + t * toff), bt: the weight tile,
// row0 / wrow0: the wave's first h row and weight row; scale words ws[ns / 8].
template <int TERMS, int NS>
__device__ __forceinline__ void d5_step(const uint8_t* at, int toff, const uint8_t* bt, const float* ws, int row0,
                                        int wrow0, int lane, float (&acc)[2][16][4]) {
    const int g = lane >> 4;
    uint4 ra[2][TERMS][2];
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
        for (int t = 0; t < TERMS; t++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++)
                ra[ms][t][hf] = *reinterpret_cast<const uint4*>(
                    at + t * toff + 16 * chunk_pos(row0 + 16 * ms + (lane & 15), 2 * g + hf));
    const float wsc[2] = {ws[0], NS > 8 ? ws[1] : ws[0]};
    // the weight subtiles one read ahead of their products (all of them at once beside the
    // 128 accumulators spill)
    auto bread = [&](int ns) {
        return *reinterpret_cast<const uint4*>(bt + 16 * wchunk_pos(wrow0 + 16 * ns + (lane & 15), g));
    };
    uint4 wcur = bread(0);
#pragma unroll
    for (int ns = 0; ns < NS; ns++) {
        uint4 wnext = wcur;
        if (ns + 1 < NS) wnext = bread(ns + 1);
        const uint32_t ww[4] = {wcur.x, wcur.y, wcur.z, wcur.w};
        gbf16x8 b[2];
#pragma unroll
        for (int hf = 0; hf < 2; hf++)
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(ww[2 * hf + q], 1.0f, false);
                const bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(ww[2 * hf + q], 1.0f, true);
                b[hf][4 * q] = p0[0];
                b[hf][4 * q + 1] = p0[1];
                b[hf][4 * q + 2] = p1[0];
                b[hf][4 * q + 3] = p1[1];
            }
        gf32x4 blk[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int hf = 0; hf < 2; hf++)
#pragma unroll
            for (int t = 0; t < TERMS; t++)
#pragma unroll
                for (int ms = 0; ms < 2; ms++)
                    blk[ms] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gbf16x8, ra[ms][t][hf]),
                                                                      b[hf], blk[ms], 0, 0, 0);
#pragma unroll
        for (int ms = 0; ms < 2; ms++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[ms][ns][e] = fmaf(blk[ms][e], wsc[ns >> 3], acc[ms][ns][e]);
        __builtin_amdgcn_sched_barrier(0);
        wcur = wnext;
    }
}

template <int TERMS>
__global__ void __launch_bounds__(GTHREADS) grouped_down512_kernel(GArgs g) {
    constexpr int STOT = d5_stot<TERMS>(), SCB = d5_scales<TERMS>();
    // each stage its own LDS object, so the compiler's waits for direct-to-LDS loads cover
    // only the loads into the buffer a read touches
    __shared__ __align__(16) uint8_t sb0[STOT], sb1[STOT];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    // block L runs on XCD L % 8 as its item q = L / 8: M-tile 8 (q / NT) + L % 8, N-tile q % NT
    const int NT = (int)gridDim.x, MT = *g.ntiles;
    const int L = (int)(blockIdx.x + blockIdx.y * gridDim.x), q = L >> 3;
    const int mt = 8 * (q / NT) + (L & 7), nt = q % NT;
    if (mt >= MT) return;
    const int i = g.tiles[2 * mt], m0 = g.tiles[2 * mt + 1], n0 = nt * GBN5;
    const int a0 = g.off[i], a1 = g.off[i + 1];
    if (a0 + m0 >= a1) return;
    G_STAMP_START(g, L, i, m0, n0, a1 - a0);
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(g.recs[i]);
    const int nkb = (int)(g.K / GBK2);
    const int rows = a1 - (a0 + m0);
    const bool light = rows <= DL_ROWS;
    D5Src src;
    src.hl_off = TERMS == 2 ? (int)((const uint8_t*)g.hl - (const uint8_t*)g.hh) : 0;
    src.hr = __builtin_amdgcn_make_buffer_rsrc(g.hh, (short)0, 0x7fff0000, G_BUF_FLAGS);
    src.wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(rec), (short)0, (int)(g.w_off + g.N * g.K),
                                               G_BUF_FLAGS);
    src.sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(rec), (short)0, 0x7fff0000, G_BUF_FLAGS);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int r, c;
        pos_chunk((2 * wave + j) * 64 + lane, r, c);
        const int a = a0 + m0 + r;
        src.ho[j] = a < a1 ? (int)(a * g.K * 2) + 16 * c : -1;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        // weight position (4 wave + j) 64 + lane = row p / 4, chunk (p % 4) ^ ((row >> 2) & 3);
        // rows past N read zeros (their outputs are not stored)
        const int p = (4 * wave + j) * 64 + lane, wr = p >> 2, wc = (p & 3) ^ ((wr >> 2) & 3);
        src.wo[j] = n0 + wr < g.N ? (int)(g.w_off + (int64_t)(n0 + wr) * g.K) + 16 * wc : G_OOB - GBK2 * 64;
    }
    {
        int r, c;
        pos_chunk((wave & 3) * 64 + lane, r, c);
        const int a = a0 + m0 + r;
        src.lho = a < a1 && (TERMS == 2 || wave < 4) ? (int)(a * g.K * 2) + 16 * c + (wave >> 2) * src.hl_off : -1;
    }
    // the wave's first h row and weight row, its first output, and its scale words
    const int row0 = light ? 0 : 32 * wm, wrow0 = light ? 64 * wave : 256 * wn;
    const int nw0 = n0 + wrow0;
    const int nsc = light ? 1 : 2;  // 128-row scale blocks the wave's rows span
    src.so = lane < nsc && nw0 + 128 * lane < g.N
                 ? (int)(g.s_off + (int64_t)(nw0 / 128 + lane) * (g.K / 128) * 4)
                 : G_OOB;
    const bool act = __builtin_amdgcn_readfirstlane(rows - row0 > 0);  // the wave holds assignments
    float acc[2][16][4];
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
        for (int ns = 0; ns < 16; ns++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[ms][ns][e] = 0.0f;
#define D5_SW(B) (reinterpret_cast<const float*>((B) + SCB) + 64 * wave)
#define D5_STEP(SB, NSB)                                                                          \
    {                                                                                             \
        wait_vm<0>();                                                                             \
        g_barrier();                                                                              \
        d5_issue<TERMS>(src, kb + 1, nkb, NSB, wave);                                             \
        if (act) d5_step<TERMS, 16>(SB, D_HT, SB + TERMS * D_HT, D5_SW(SB), row0, wrow0, lane, acc);        \
        if (++kb == nkb) break;                                                                   \
    }
#define D5_LSTEP(SB, NSB)                                                                         \
    {                                                                                             \
        wait_vm<0>();                                                                             \
        g_barrier();                                                                              \
        d5_issue_light<TERMS>(src, kb + 1, nkb, NSB, wave);                                       \
        if (act) d5_step<TERMS, 4>(SB, DL_HT, SB + 2 * DL_HT, D5_SW(SB), row0, wrow0, lane, acc);           \
        if (++kb == nkb) break;                                                                   \
    }
    int kb = 0;
    if (light) {
        d5_issue_light<TERMS>(src, 0, nkb, sb0, wave);
        for (;;) {
            D5_LSTEP(sb0, sb1)
            D5_LSTEP(sb1, sb0)
        }
    } else {
        d5_issue<TERMS>(src, 0, nkb, sb0, wave);
        for (;;) {
            D5_STEP(sb0, sb1)
            D5_STEP(sb1, sb0)
        }
    }
#undef D5_SW
#undef D5_STEP
#undef D5_LSTEP
    wait_vm<0>();  // the zero-filled stage past the end has landed before the block ends
    const int nsw = light ? 4 : 16;  // the wave's N subtiles
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int a = a0 + m0 + row0 + 16 * ms + 4 * (lane >> 4) + e;
            if (a >= a1) continue;
#pragma unroll
            for (int ns = 0; ns < 16; ns++) {
                const int64_t n = nw0 + 16 * ns + (lane & 15);
                if (ns < nsw && n < g.N) g.y[(int64_t)a * g.N + n] = acc[ms][ns][e];
            }
        }
    G_STAMP_END(g, L);
}

// ---- host side -----------------------------------------------------------------------

int launch_grouped(const GArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL(grouped_gemm_kernel, grid, dim3(GTHREADS), 0, st, a);
    return launched("grouped_gemm_fp8");
}

int launch_grouped_gate_up256(const GArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL(grouped_gate_up256_kernel, grid, dim3(GTHREADS), 0, st, a);
    return launched("grouped_gate_up_fp8");
}

int launch_grouped_down512(const GArgs& a, int terms, dim3 grid, hipStream_t st) {
    if (terms == 2) hipLaunchKernelGGL(grouped_down512_kernel<2>, grid, dim3(GTHREADS), 0, st, a);
    else hipLaunchKernelGGL(grouped_down512_kernel<1>, grid, dim3(GTHREADS), 0, st, a);
    return launched("grouped_down_bf16");
}

int launch_quant_rows(const void* x, int xdt, int64_t rows, int64_t cols, uint8_t* q, float* s, hipStream_t st) {
    if (rows == 0) return OOM_OK;
    if (cols % 8 == 0 && cols <= QV_MAXC && aligned(x, 16) && aligned(q, 8)) {
        if (xdt == OOM_BF16)
            hipLaunchKernelGGL(quant_rows_vec_kernel<OOM_BF16>, dim3((unsigned)rows), dim3(256), 0, st, x, cols, q, s);
        else
            hipLaunchKernelGGL(quant_rows_vec_kernel<OOM_F32>, dim3((unsigned)rows), dim3(256), 0, st, x, cols, q, s);
        return launched("quantize_rows_fp8");
    }
    if (xdt == OOM_BF16)
        hipLaunchKernelGGL(quant_rows_kernel<OOM_BF16>, dim3((unsigned)rows), dim3(256), 0, st, x, cols, q, s);
    else
        hipLaunchKernelGGL(quant_rows_kernel<OOM_F32>, dim3((unsigned)rows), dim3(256), 0, st, x, cols, q, s);
    return launched("quantize_rows_fp8");
}

int launch_grouped_tiles(const int32_t* n_e, const int32_t* off, TileTable t0, const TileTable* t1, hipStream_t st) {
    hipLaunchKernelGGL(grouped_tiles_kernel, dim3(t1 ? 2 : 1), dim3(1024), 0, st, n_e, off, t0, t1 ? *t1 : t0);
    return launched("grouped_tiles");
}

}  // namespace oom

// ---- C ABI -----------------------------------------------------------------------------

namespace oom {
int launch_combine(const float* y, const int32_t* slot, const float* w, void* out, int odt, int T, int H, int k,
                   hipStream_t st);
size_t plan_multi_counts(int A, int E);
int launch_plan_multi(const int32_t* ids, int T, int E, int k, const uint64_t* all_recs, int32_t* plan, uint64_t* recs,
                      int32_t* counts, hipStream_t st);
int check_geo(const OomFp8Record* g, const char* who);

// Workspace of oom_moe_prefill_fp8: plan | recs | xq | xs | tiles | tiles2 | hh | hl | y |
// counts (tiles: the 128-row tile table of the down pass, tiles2: the 256-row one of
// gate/up; hh and hl: the bf16 hi and lo terms of h [A, inter]; hl is written for the exact
// precision only; counts: the plan's per-block expert counts).
struct PrefillWs {
    size_t plan, recs, xq, xs, tiles, tiles2, hh, hl, y, counts, total;
    int max_tiles, max_tiles2;
};

static size_t p_al256(size_t v) { return (v + 255) & ~size_t(255); }

static PrefillWs prefill_ws(int T, int E, int k, const OomFp8Record& g) {
    PrefillWs w;
    const size_t A = (size_t)T * k, H = (size_t)g.hidden, I = (size_t)g.inter;
    w.max_tiles = (int)(cdiv((int64_t)A, GBM) + std::min<int64_t>(E, (int64_t)A));
    w.max_tiles2 = (int)(cdiv((int64_t)A, GBM2) + std::min<int64_t>(E, (int64_t)A));
    w.plan = 0;
    w.recs = p_al256(PlanView::size(E, (int)A) * sizeof(int32_t));
    w.xq = w.recs + p_al256((size_t)std::min<size_t>(E, A) * sizeof(uint64_t));
    w.xs = w.xq + p_al256((size_t)T * H);
    w.tiles = w.xs + p_al256((size_t)T * sizeof(float));
    w.tiles2 = w.tiles + p_al256((2 * (size_t)w.max_tiles + 1) * sizeof(int32_t));
    w.hh = w.tiles2 + p_al256((2 * (size_t)w.max_tiles2 + 1) * sizeof(int32_t));
    w.hl = w.hh + p_al256(A * I * sizeof(uint16_t));
    w.y = w.hl + p_al256(A * I * sizeof(uint16_t));
    w.counts = w.y + p_al256(A * H * sizeof(float));
    w.total = w.counts + p_al256(plan_multi_counts((int)A, E) * sizeof(int32_t));
    return w;
}
}  // namespace oom

extern "C" int oom_quantize_rows_fp8(const void* x, int x_dtype, int64_t rows, int64_t cols, uint8_t* q,
                                     float* scale, void* stream) {
    using namespace oom;
    OOM_REQUIRE(rows >= 0 && rows < (1ll << 31) && cols >= 1, "oom_quantize_rows_fp8: shape");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_quantize_rows_fp8: x_dtype");
    if (rows == 0) return OOM_OK;
    OOM_REQUIRE(x && q && scale, "oom_quantize_rows_fp8: null buffer");
    return launch_quant_rows(x, x_dtype, rows, cols, q, scale, as_stream(stream));
}

extern "C" int oom_moe_grouped_gemm_fp8(const uint64_t* recs, const int32_t* off, const int32_t* rows, int n_experts,
                                        int max_per_expert, const uint8_t* xq, const float* x_scale, int x_group,
                                        float* y, int64_t N, int64_t K, int64_t w_off, int64_t s_off, void* stream) {
    using namespace oom;
    OOM_REQUIRE(n_experts >= 0 && n_experts <= 65535 && max_per_expert >= 0, "oom_moe_grouped_gemm_fp8: experts");
    OOM_REQUIRE(N >= 128 && N % 128 == 0 && K >= 128 && K % 128 == 0 && N < (1 << 24) && K < (1 << 24),
                "oom_moe_grouped_gemm_fp8: N and K must be multiples of 128");
    OOM_REQUIRE(x_group == 0 || x_group == 128, "oom_moe_grouped_gemm_fp8: x_group must be 0 or 128");
    OOM_REQUIRE(w_off >= 0 && s_off >= 0 && w_off % 16 == 0 && s_off % 4 == 0, "oom_moe_grouped_gemm_fp8: part offsets");
    OOM_REQUIRE(w_off + N * K < 0x7fff0000ll, "oom_moe_grouped_gemm_fp8: weight part beyond 2 GiB of its record");
    if (n_experts == 0 || max_per_expert == 0) return OOM_OK;
    OOM_REQUIRE(recs && off && xq && x_scale && y, "oom_moe_grouped_gemm_fp8: null buffer");
    OOM_REQUIRE(aligned(xq, 16), "oom_moe_grouped_gemm_fp8: xq must be 16-byte aligned");
    GArgs a{};
    a.recs = recs;
    a.off = off;
    a.rows = rows;
    a.xq = xq;
    a.xs = x_scale;
    a.x_group = x_group;
    a.N = N;
    a.K = K;
    a.w_off = w_off;
    a.s_off = s_off;
    a.w2_off = w_off;
    a.s2_off = s_off;
    a.y = y;
    dim3 grid((unsigned)(N / GBN), (unsigned)cdiv(max_per_expert, GBM), (unsigned)n_experts);
    return launch_grouped(a, grid, as_stream(stream));
}

extern "C" size_t oom_moe_prefill_fp8_workspace_size(int T, int E, int k, const OomFp8Record* geo) {
    if (!geo || T < 1 || E < 1 || k < 1) return 0;
    return oom::prefill_ws(T, E, k, *geo).total;
}

extern "C" int oom_moe_prefill_fp8(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T,
                                   int E, int k, const OomFp8Record* geo, int precision, int32_t* ids, float* weights,
                                   void* out, int out_dtype, void* ws, size_t ws_bytes, void* stream) {
    using namespace oom;
    if (int rc = check_geo(geo, "oom_moe_prefill_fp8")) return rc;
    OOM_REQUIRE(geo->hidden % 128 == 0 && geo->inter % 128 == 0,
                "oom_moe_prefill_fp8: hidden and inter must be multiples of 128");
    OOM_REQUIRE(std::max({geo->gate_weight, geo->up_weight, geo->down_weight}) + geo->hidden * geo->inter < 0x7fff0000ll,
                "oom_moe_prefill_fp8: weight parts beyond 2 GiB of their record");
    OOM_REQUIRE(T >= 1 && (int64_t)T * k <= (1 << 24), "oom_moe_prefill_fp8: T must be >= 1 and T * k <= 2^24");
    // buffer-resource offsets are 32-bit: the e4m3 rows and both h planes stay below 2 GiB
    OOM_REQUIRE((int64_t)T * geo->hidden < 0x7fff0000ll && (int64_t)T * k * geo->inter * 4 < 0x7fff0000ll,
                "oom_moe_prefill_fp8: activations or h beyond 2 GiB (split the prefill into chunks of tokens)");
    OOM_REQUIRE(k >= 1 && k <= 32 && E >= k && E <= 8192, "oom_moe_prefill_fp8: router top-k > 32 or experts > 8192");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_moe_prefill_fp8: x_dtype");
    OOM_REQUIRE(out_dtype == OOM_F32 || out_dtype == OOM_BF16, "oom_moe_prefill_fp8: out_dtype");
    OOM_REQUIRE(precision == OOM_EXPERT_EXACT || precision == OOM_EXPERT_BF16, "oom_moe_prefill_fp8: precision");
    OOM_REQUIRE(logits && x && all_recs && ids && weights && out, "oom_moe_prefill_fp8: null buffer");
    const PrefillWs w = prefill_ws(T, E, k, *geo);
    if (!ws || ws_bytes < w.total)
        return fail(OOM_ERR_WORKSPACE, "oom_moe_prefill_fp8: workspace smaller than oom_moe_prefill_fp8_workspace_size()");
    OOM_REQUIRE(aligned(ws, 256), "oom_moe_prefill_fp8: workspace must be 256-byte aligned");
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    int32_t* plan = reinterpret_cast<int32_t*>(base + w.plan);
    uint64_t* recs = reinterpret_cast<uint64_t*>(base + w.recs);
    uint8_t* xq = base + w.xq;
    float* xs = reinterpret_cast<float*>(base + w.xs);
    int32_t* tiles = reinterpret_cast<int32_t*>(base + w.tiles);
    int32_t* ntiles = tiles + 2 * w.max_tiles;
    int32_t* tiles2 = reinterpret_cast<int32_t*>(base + w.tiles2);
    int32_t* ntiles2 = tiles2 + 2 * w.max_tiles2;
    uint16_t* hh = reinterpret_cast<uint16_t*>(base + w.hh);
    uint16_t* hl = reinterpret_cast<uint16_t*>(base + w.hl);
    float* y = reinterpret_cast<float*>(base + w.y);
    hipStream_t st = as_stream(stream);
    const int A = T * k;
    PlanView pv{plan, E, A};
    if (int rc = oom_router_topk(logits, ids, weights, T, E, k, stream)) return rc;
    if (int rc = launch_plan_multi(ids, T, E, k, all_recs, plan, recs, reinterpret_cast<int32_t*>(base + w.counts), st))
        return rc;
    if (int rc = launch_quant_rows(x, x_dtype, T, geo->hidden, xq, xs, st)) return rc;
    // both tile tables in one launch: 128-row tiles (down), 256-row tiles with the long ones first (gate/up)
    const TileTable tt2{GBM2, GU2_LROWS, tiles2, ntiles2};
    if (int rc = launch_grouped_tiles(pv.n_e(), pv.off(), TileTable{GBM, 0, tiles, ntiles}, &tt2, st)) return rc;
    GArgs a{};
    a.recs = recs;
    a.off = pv.off();
    a.rows = pv.assign_tok();
    a.tiles = tiles2;
    a.ntiles = ntiles2;
    a.xq = xq;
    a.xs = xs;
    a.x_group = 0;
    a.N = geo->inter;
    a.K = geo->hidden;
    a.w_off = geo->gate_weight;
    a.s_off = geo->gate_scale;
    a.w2_off = geo->up_weight;
    a.s2_off = geo->up_scale;
    a.hh = hh;
    a.hl = precision == OOM_EXPERT_EXACT ? hl : nullptr;
#ifdef OOM_STAMPS
    a.stamps = stamps_buffer();
#endif
    // 8 spare rows of blocks: the XCD-run order needs the grid to cover 8 ceil(W / 8) slots
    if (int rc = launch_grouped_gate_up256(a, dim3((unsigned)(geo->inter / GBN), (unsigned)w.max_tiles2 + 8, 1), st))
        return rc;
    GArgs d{};
    d.recs = recs;
    d.off = pv.off();
    d.tiles = tiles;
    d.ntiles = ntiles;
    d.N = geo->hidden;
    d.K = geo->inter;
    d.w_off = geo->down_weight;
    d.s_off = geo->down_scale;
    d.hh = hh;
    d.hl = hl;
    d.y = y;
#ifdef OOM_STAMPS
    // the down pass's blocks after the gate/up grid's
    d.stamps = a.stamps ? a.stamps + 4 * (size_t)(geo->inter / GBN) * (w.max_tiles2 + 8) : nullptr;
#endif
    const int terms = precision == OOM_EXPERT_EXACT ? 2 : 1;
    if (int rc = launch_grouped_down512(d, terms, dim3((unsigned)cdiv(geo->hidden, GBN5), (unsigned)w.max_tiles + 8, 1),
                                        st))
        return rc;
    return launch_combine(y, pv.slot_assign(), weights, out, out_dtype, T, (int)geo->hidden, k, st);
}
