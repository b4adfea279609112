// Decode GEMV over e4m3 weights: y[t, n] = sum_k x[t, k] * e4m3(q[n, k]) * scale(n, k).
//
// Layout of the work (gfx950, wave64):
//   - a block is 4 waves; each wave owns R consecutive rows; a split owns
//     KCH * 1024 columns (the last split may be shorter);
//   - lane l reads 16 e4m3 bytes (one 128-bit load) at columns c * 1024 + 16 l of
//     chunk c, so a wave-wide load is one contiguous 1 KiB run of a row and all R x
//     KCH loads of a wave are in flight before the first use;
//   - the split's activations sit in LDS as fp32 in lane order (float4 i of chunk c
//     of lane l at ((t * KCH + c) * 4 + i) * 64 + l), so a lane's ds_read_b128s are
//     conflict-free and each feeds all R rows;
//   - per (row, chunk) a lane's 16 products sum in fp32, are scaled by the weight
//     block's scale (one per lane: 16 columns never straddle a 128 block) and
//     accumulate; the R * T per-lane sums reduce over the wave in one multi-value
//     butterfly (R * T - 1 + log2(64 / (R * T)) exchanges);
//   - splits > 1 write fp32 partials [splits, T, N]; the last block of a row tile
//     (a ticket per tile, reset after use) adds them in split order, so the result
//     does not depend on block timing (crates/oominf-cuda/kernels/ops.cu:421-439);
//   - bf16 rows with few rows (N <= 512) and few tokens (T <= 4) take one row a wave and
//     up to 4 chunks a block, so a K of 4096 needs no split: the latency of the ticketed
//     sum is most of such a call;
//   - the workspace holds the tickets first, in an area sized for the most tiles any
//     T can have at this N (rows / 4), then the partials: a workspace left by a call
//     of another T or K still has zero tickets where this call looks (partials are
//     written before they are read), so calls with one N share a workspace.
#include "stream.hpp"

namespace oom {

constexpr int GEMV_WAVES = 4;

// WB: the weights are bf16 [N, K] (no scales): a lane's 16 columns of a chunk are two
// 16-byte loads, converted exactly to fp32.
template <int T, int R, int KCH, int SL, int XDT, int YDT, bool WB = false>
__global__ void __launch_bounds__(256) gemv_fp8_kernel(const void* __restrict__ x, const uint8_t* __restrict__ q,
                                                       const float* __restrict__ scale, void* __restrict__ y,
                                                       float* __restrict__ partial, uint32_t* __restrict__ tickets,
                                                       int tn, int N, int K) {
    extern __shared__ float4 xs4[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int split = blockIdx.y, splits = gridDim.y;
    const int klen = KCH * 1024;
    const int k0 = split * klen;
    const int kl = min(K, k0 + klen) - k0;
    const int row0 = (blockIdx.x * GEMV_WAVES + wave) * R;
    const int nkb = (K + 127) >> 7;
    // x's loads first (16 bytes: 8 bf16 or 4 f32 of one lane's 16 columns, when x is
    // 16-byte aligned; K % 16 == 0 keeps a load inside one row and on one side of kl), then
    // the weights': loads complete in issue order, so x can be staged in LDS while the
    // weights are still in flight
    // (buffer loads, no branch: an unaligned x or a lane past the data reads zeros through an
    // out-of-range offset, which keeps the compiler's count of loads in flight exact)
    const bool xal = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    constexpr int EPL = XDT == OOM_BF16 ? 8 : 4;
    constexpr int NV = T * KCH * 1024 / EPL;
    constexpr int NLD = (NV + 255) / 256;
    constexpr int XES = XDT == OOM_BF16 ? 2 : 4;
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(x), (short)0, tn * K * XES, BUF_FLAGS);
    uint4 v[NLD];
#pragma unroll
    for (int n = 0; n < NLD; n++) {
        const int i = threadIdx.x + 256 * n;
        const int t = i * EPL / klen, kk = i * EPL - t * klen;
        const bool ok = xal && i < NV && t < tn && kk < kl;
        v[n] = ld16(xr, ok ? (t * K + k0 + kk) * XES : OOB);
    }
    __builtin_amdgcn_sched_barrier(0);  // x's loads stay ahead of the weights
    // each row's split through a resource of its own (the row is uniform over the wave);
    // nontemporal: the weights are read once a call
    constexpr int NW = WB ? 2 : 1;  // 16-byte loads per lane per (row, chunk)
    uint4 w[R][KCH][NW];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(row0 + r, N - 1);
        const __amdgpu_buffer_rsrc_t wr =
            uniform_rsrc(reinterpret_cast<uint64_t>(q + ((size_t)row * K + k0) * NW), kl * NW);
#pragma unroll
        for (int c = 0; c < KCH; c++) {
            const int col = c * 1024 + lane * 16;
#pragma unroll
            for (int h = 0; h < NW; h++) w[r][c][h] = ld16nt(wr, col < kl ? col * NW + 16 * h : OOB);
        }
    }

    // stage x[t, k0 .. k0 + kl) in lane order (zeros past kl and for padded tokens): element
    // kk = c * 1024 + 16 l + j of token t sits at float index
    // (((t * KCH + c) * 4 + j / 4) * 64 + l) * 4 + j % 4
    // (written on every path, zeros for an unaligned x, so the loads stay ahead of the
    // weights' instead of moving into a branch)
    float* xs = reinterpret_cast<float*>(xs4);
    {
#pragma unroll
        for (int n = 0; n < NLD; n++) {
            const int i = threadIdx.x + 256 * n;
            if (NV % 256 != 0 && i >= NV) break;
            const int t = i * EPL / klen, kk = i * EPL - t * klen;
            const int c = kk >> 10, l = (kk & 1023) >> 4, j = kk & 15;
            float4* dst = &xs4[((t * KCH + c) * 4 + (j >> 2)) * 64 + l];
            if constexpr (XDT == OOM_BF16) {
                dst[0] = make_float4(__uint_as_float(v[n].x << 16), __uint_as_float(v[n].x & 0xffff0000u),
                                     __uint_as_float(v[n].y << 16), __uint_as_float(v[n].y & 0xffff0000u));
                dst[64] = make_float4(__uint_as_float(v[n].z << 16), __uint_as_float(v[n].z & 0xffff0000u),
                                      __uint_as_float(v[n].w << 16), __uint_as_float(v[n].w & 0xffff0000u));
            } else {
                dst[0] = make_float4(__uint_as_float(v[n].x), __uint_as_float(v[n].y), __uint_as_float(v[n].z),
                                     __uint_as_float(v[n].w));
            }
        }
    }
    if (!xal) {
        __syncthreads();
        for (int i = threadIdx.x; i < T * klen; i += blockDim.x) {
            int t = i / klen, kk = i - t * klen;
            int c = kk >> 10, l = (kk & 1023) >> 4, j = kk & 15;
            float v = (t < tn && kk < kl) ? load_act<XDT>(x, (size_t)t * K + k0 + kk) : 0.0f;
            xs[(((t * KCH + c) * 4 + (j >> 2)) * 64 + l) * 4 + (j & 3)] = v;
        }
    }
    __syncthreads();

    float acc[T * R];
#pragma unroll
    for (int i = 0; i < T * R; i++) acc[i] = 0.0f;
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        int col = k0 + c * 1024 + lane * 16;
        float sc[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int row = min(row0 + r, N - 1);
            if constexpr (WB || SL == OOM_SCALE_ROW) sc[r] = 1.0f;
            else if constexpr (SL == OOM_SCALE_1X128) sc[r] = col < K ? scale[(size_t)row * nkb + (col >> 7)] : 0.0f;
            else sc[r] = col < K ? scale[(size_t)(row >> 7) * nkb + (col >> 7)] : 0.0f;
        }
        float wf[R][16];
#pragma unroll
        for (int r = 0; r < R; r++) {
            if constexpr (WB) {
                const uint32_t u[8] = {w[r][c][0].x, w[r][c][0].y, w[r][c][0].z, w[r][c][0].w,
                                       w[r][c][NW - 1].x, w[r][c][NW - 1].y, w[r][c][NW - 1].z, w[r][c][NW - 1].w};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    wf[r][2 * i] = __uint_as_float(u[i] << 16);
                    wf[r][2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
                }
            } else {
                e4m3x16(w[r][c][0], wf[r]);
            }
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
            float xv[16];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float4 a = xs4[((t * KCH + c) * 4 + i) * 64 + lane];
                xv[4 * i] = a.x;
                xv[4 * i + 1] = a.y;
                xv[4 * i + 2] = a.z;
                xv[4 * i + 3] = a.w;
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) p = fmaf(wf[r][i], xv[i], p);
                acc[t * R + r] = fmaf(p, sc[r], acc[t * R + r]);
            }
        }
    }
    float tot = wave_sum_multi<T * R>(acc, lane);
    const int g = lane / (64 / (T * R));  // value g of the butterfly: t = g / R, r = g % R
    const bool writer = (lane % (64 / (T * R))) == 0;
    const int t = g / R, r = g % R, row = row0 + r;
    if (writer && row < N && t < tn) {
        if constexpr (!WB && SL == OOM_SCALE_ROW) tot *= scale[row];
        if (splits == 1) store_out<YDT>(y, (size_t)t * N + row, tot);
        else st_dev(&partial[((size_t)split * T + t) * N + row], tot);
    }
    if (splits == 1) return;
    // Partials move between blocks (of any XCD) as device-coherent stores and loads, and
    // the ticket is a relaxed device-scope add taken after this block's stores are
    // acknowledged: no agent-scope fence, whose L2 write-back and invalidate per block
    // cost ten times the whole GEMV.
    __shared__ bool last;
    wait_mem();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&tickets[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == (unsigned)splits - 1;
        if (last) __hip_atomic_store(&tickets[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    const int tile = GEMV_WAVES * R, first = blockIdx.x * tile;
    for (int i = threadIdx.x; i < tn * tile; i += blockDim.x) {
        int tt = i / tile, n = first + i % tile;
        if (n >= N) continue;
        float sum = 0.0f;
        for (int s = 0; s < splits; s++) sum += ld_dev(&partial[((size_t)s * T + tt) * N + n]);
        store_out<YDT>(y, (size_t)tt * N + n, sum);
    }
}

// Launch geometry of one call (shared by the workspace query and the launch).
struct GemvPlan {
    int tp, R, kch, splits, tiles;
    size_t lds;
};

static GemvPlan gemv_plan(int T, int64_t N, int64_t K, bool wb = false) {
    GemvPlan p;
    p.tp = T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : 16;
    p.R = p.tp >= 8 ? 2 : 4;
    int kchunks = (int)cdiv(K, 1024);
    if (wb && p.tp <= 4 && N <= 512) {
        // one row a wave, up to 4 chunks (x of a split: tp * 4 * 4 KiB <= 64 KiB)
        p.R = 1;
        p.tiles = (int)cdiv(N, (int64_t)GEMV_WAVES);
        p.kch = kchunks <= 1 ? 1 : kchunks <= 2 ? 2 : 4;
        p.splits = (int)cdiv(kchunks, p.kch);
        p.lds = (size_t)p.tp * p.kch * 1024 * sizeof(float);
        return p;
    }
    // x of one split in LDS: tp * kch * 4 KiB <= 64 KiB
    int kch_max = std::max(1, 16 / p.tp);
    kch_max = std::min(kch_max, wb ? 2 : 4);  // bf16 rows take twice the registers per chunk
    if (!wb && p.tp <= 4 && kchunks <= kch_max && cdiv(N, (int64_t)GEMV_WAVES * 2) >= 512) {
        // two rows a wave fill the chip (>= 512 blocks) with the whole of K in one block:
        // no split, so no second round trip through the partials
        p.R = 2;
        p.kch = kchunks <= 1 ? 1 : kchunks <= 2 ? 2 : 4;
        p.splits = 1;
        p.tiles = (int)cdiv(N, (int64_t)GEMV_WAVES * p.R);
        p.lds = (size_t)p.tp * p.kch * 1024 * sizeof(float);
        return p;
    }
    p.tiles = (int)cdiv(N, (int64_t)GEMV_WAVES * p.R);
    // enough blocks to cover the CUs (>= 512 blocks), but a split never shorter than 1 KiB
    int want = (int)std::max<int64_t>(1, cdiv(512, p.tiles));
    int splits = std::max<int>((int)cdiv(kchunks, kch_max), std::min(want, kchunks));
    p.kch = (int)cdiv(kchunks, splits);
    p.kch = p.kch <= 1 ? 1 : p.kch <= 2 ? 2 : 4;
    p.splits = (int)cdiv(kchunks, p.kch);
    p.lds = (size_t)p.tp * p.kch * 1024 * sizeof(float);
    return p;
}

template <int T, int R, int KCH, bool WB>
static void launch_gemv(const GemvPlan& p, int sl, int xdt, int ydt, const void* x, const uint8_t* q, const float* s,
                        void* y, float* part, uint32_t* tk, int tn, int N, int K, hipStream_t st) {
    dim3 grid(p.tiles, p.splits), block(256);
#define GEMV_CASE(SL, XD, YD)                                                                                     \
    if (sl == SL && xdt == XD && ydt == YD) {                                                                     \
        hipLaunchKernelGGL((gemv_fp8_kernel<T, R, KCH, SL, XD, YD, WB>), grid, block, p.lds, st, x, q, s, y, part, tk, \
                           tn, N, K);                                                                             \
        return;                                                                                                   \
    }
#define GEMV_DT(SL)                   \
    GEMV_CASE(SL, OOM_F32, OOM_F32)   \
    GEMV_CASE(SL, OOM_F32, OOM_BF16)  \
    GEMV_CASE(SL, OOM_BF16, OOM_F32)  \
    GEMV_CASE(SL, OOM_BF16, OOM_BF16)
    GEMV_DT(OOM_SCALE_ROW)
    if constexpr (!WB) {
        GEMV_DT(OOM_SCALE_1X128)
        GEMV_DT(OOM_SCALE_128X128)
    }
#undef GEMV_DT
#undef GEMV_CASE
}

template <int T, int R, bool WB = false>
static void launch_gemv_k(const GemvPlan& p, int sl, int xdt, int ydt, const void* x, const uint8_t* q,
                          const float* s, void* y, float* part, uint32_t* tk, int tn, int N, int K, hipStream_t st) {
    switch (p.kch) {
        case 1: launch_gemv<T, R, 1, WB>(p, sl, xdt, ydt, x, q, s, y, part, tk, tn, N, K, st); break;
        case 2: launch_gemv<T, R, 2, WB>(p, sl, xdt, ydt, x, q, s, y, part, tk, tn, N, K, st); break;
        default:
            if constexpr (T <= 4 && (!WB || R == 1))
                launch_gemv<T, R, 4, WB>(p, sl, xdt, ydt, x, q, s, y, part, tk, tn, N, K, st);
            break;
    }
}

static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Bytes of the ticket area at the start of a GEMV workspace: one ticket per row tile at the
// smallest tile (one row per wave, 4 rows), whatever T is.
static size_t gemv_ticket_bytes(int64_t N) { return align256((size_t)cdiv(N, (int64_t)GEMV_WAVES) * sizeof(uint32_t)); }

static size_t gemv_ws_bytes(const GemvPlan& p, int64_t N) {
    if (p.splits == 1) return 0;
    return gemv_ticket_bytes(N) + (size_t)p.splits * p.tp * N * sizeof(float);
}

}  // namespace oom

extern "C" size_t oom_gemv_fp8_workspace_size(int T, int64_t N, int64_t K) {
    if (T < 1 || N < 1 || K < 1) return 0;
    return oom::gemv_ws_bytes(oom::gemv_plan(T, N, K), N);
}

extern "C" int oom_gemv_fp8(const void* x, int x_dtype, const uint8_t* q, const float* scale, int scale_layout,
                            void* y, int y_dtype, int T, int64_t N, int64_t K, void* ws, size_t ws_bytes,
                            void* stream) {
    using namespace oom;
    OOM_REQUIRE(T >= 1 && T <= 16, "oom_gemv_fp8: T must be 1..16");
    OOM_REQUIRE(N >= 1 && K >= 16 && K % 16 == 0, "oom_gemv_fp8: K must be a positive multiple of 16");
    OOM_REQUIRE(N <= INT32_MAX && K <= INT32_MAX && N * K <= ((int64_t)1 << 40), "oom_gemv_fp8: shape too large");
    OOM_REQUIRE((int64_t)T * K * 4 < 0x7fff0000ll, "oom_gemv_fp8: x beyond 2 GiB");
    OOM_REQUIRE(x && q && scale && y, "oom_gemv_fp8: null buffer");
    OOM_REQUIRE(aligned(q, 16), "oom_gemv_fp8: weights must be 16-byte aligned");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_gemv_fp8: x_dtype");
    OOM_REQUIRE(y_dtype == OOM_F32 || y_dtype == OOM_BF16, "oom_gemv_fp8: y_dtype");
    OOM_REQUIRE(scale_layout >= OOM_SCALE_ROW && scale_layout <= OOM_SCALE_128X128, "oom_gemv_fp8: scale_layout");
    GemvPlan p = gemv_plan(T, N, K);
    float* part = nullptr;
    uint32_t* tk = nullptr;
    if (p.splits > 1) {
        size_t need = oom_gemv_fp8_workspace_size(T, N, K);
        if (ws_bytes < need || ws == nullptr)
            return fail(OOM_ERR_WORKSPACE, "oom_gemv_fp8: workspace smaller than oom_gemv_fp8_workspace_size()");
        OOM_REQUIRE(aligned(ws, 16), "oom_gemv_fp8: workspace must be 16-byte aligned");
        tk = reinterpret_cast<uint32_t*>(ws);
        part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) + gemv_ticket_bytes(N));
    }
    hipStream_t st = as_stream(stream);
    int n = (int)N, k = (int)K;
    switch (p.tp) {
#define GEMV_FP8_T(TP)                                                                                        \
    if (p.R == 2) launch_gemv_k<TP, 2>(p, scale_layout, x_dtype, y_dtype, x, q, scale, y, part, tk, T, n, k, st); \
    else launch_gemv_k<TP, 4>(p, scale_layout, x_dtype, y_dtype, x, q, scale, y, part, tk, T, n, k, st);         \
    break;
        case 1: GEMV_FP8_T(1)
        case 2: GEMV_FP8_T(2)
        case 4: GEMV_FP8_T(4)
#undef GEMV_FP8_T
        case 8: launch_gemv_k<8, 2>(p, scale_layout, x_dtype, y_dtype, x, q, scale, y, part, tk, T, n, k, st); break;
        default: launch_gemv_k<16, 2>(p, scale_layout, x_dtype, y_dtype, x, q, scale, y, part, tk, T, n, k, st); break;
    }
    return launched("oom_gemv_fp8");
}

extern "C" size_t oom_gemv_bf16_workspace_size(int T, int64_t N, int64_t K) {
    if (T < 1 || N < 1 || K < 1) return 0;
    return oom::gemv_ws_bytes(oom::gemv_plan(T, N, K, true), N);
}

extern "C" int oom_gemv_bf16(const void* x, int x_dtype, const uint16_t* w, void* y, int y_dtype, int T, int64_t N,
                             int64_t K, void* ws, size_t ws_bytes, void* stream) {
    using namespace oom;
    OOM_REQUIRE(T >= 1 && T <= 16, "oom_gemv_bf16: T must be 1..16");
    OOM_REQUIRE(N >= 1 && K >= 16 && K % 16 == 0, "oom_gemv_bf16: K must be a positive multiple of 16");
    OOM_REQUIRE(N <= INT32_MAX && K <= INT32_MAX && N * K <= ((int64_t)1 << 39), "oom_gemv_bf16: shape too large");
    OOM_REQUIRE((int64_t)T * K * 4 < 0x7fff0000ll, "oom_gemv_bf16: x beyond 2 GiB");
    OOM_REQUIRE(x && w && y, "oom_gemv_bf16: null buffer");
    OOM_REQUIRE(aligned(w, 16), "oom_gemv_bf16: weights must be 16-byte aligned");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_gemv_bf16: x_dtype");
    OOM_REQUIRE(y_dtype == OOM_F32 || y_dtype == OOM_BF16, "oom_gemv_bf16: y_dtype");
    GemvPlan p = gemv_plan(T, N, K, true);
    float* part = nullptr;
    uint32_t* tk = nullptr;
    if (p.splits > 1) {
        size_t need = oom_gemv_bf16_workspace_size(T, N, K);
        if (ws_bytes < need || ws == nullptr)
            return fail(OOM_ERR_WORKSPACE, "oom_gemv_bf16: workspace smaller than oom_gemv_bf16_workspace_size()");
        OOM_REQUIRE(aligned(ws, 16), "oom_gemv_bf16: workspace must be 16-byte aligned");
        tk = reinterpret_cast<uint32_t*>(ws);
        part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) + gemv_ticket_bytes(N));
    }
    hipStream_t st = as_stream(stream);
    const int n = (int)N, k = (int)K;
    const uint8_t* q = reinterpret_cast<const uint8_t*>(w);
    switch (p.tp) {
#define GEMV_BF16_T(TP)                                                                                          \
    if (p.R == 1)                                                                                                \
        launch_gemv_k<TP, 1, true>(p, OOM_SCALE_ROW, x_dtype, y_dtype, x, q, nullptr, y, part, tk, T, n, k, st);   \
    else                                                                                                         \
        launch_gemv_k<TP, 4, true>(p, OOM_SCALE_ROW, x_dtype, y_dtype, x, q, nullptr, y, part, tk, T, n, k, st);   \
    break;
        case 1: GEMV_BF16_T(1)
        case 2: GEMV_BF16_T(2)
        case 4: GEMV_BF16_T(4)
#undef GEMV_BF16_T
        case 8: launch_gemv_k<8, 2, true>(p, OOM_SCALE_ROW, x_dtype, y_dtype, x, q, nullptr, y, part, tk, T, n, k, st); break;
        default: launch_gemv_k<16, 2, true>(p, OOM_SCALE_ROW, x_dtype, y_dtype, x, q, nullptr, y, part, tk, T, n, k, st); break;
    }
    return launched("oom_gemv_bf16");
}
