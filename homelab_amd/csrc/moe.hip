// Routed experts over FP8 records read in place (fp8-e4m3-b128 layout, OomFp8Record).
//
// gate/up + SwiGLU: one block = 4 waves = 8 intermediate rows of one expert; each wave
// streams R = 2 gate rows and the same 2 up rows (16 x 128-bit loads in flight per
// lane for hidden 4096) against the expert's tokens staged in LDS (fp32, lane order),
// TB tokens per pass, and reduces its 4 * TB sums in one multi-value butterfly.
// down: one block = 4 waves = 16 output rows of one expert; h rows of the expert's
// assignments staged in LDS the same way.
// Both follow crates/oominf-cuda/kernels/moe.cu:52-151 (moe_gate_up / moe_down:
// expert e owns assignments [off[e], off[e+1]), records addressed through recs[]);
// the weight decode is e4m3 * 128x128 block scale, applied to each lane's 16-term
// partial (16 columns never straddle a 128-column block).
#include "router.hpp"
#include "stream.hpp"

namespace oom {

constexpr int MOE_WAVES = 4;
constexpr int GU_R = 2;   // gate/up rows per wave
constexpr int DN_R = 4;   // down rows per wave
constexpr int MOE_TB = 4; // assignments per pass

struct Rec {
    int64_t hidden, inter, gw, gs, uw, us, dw, ds;
};

__host__ __device__ inline Rec rec_of(const OomFp8Record& g) {
    return Rec{g.hidden, g.inter, g.gate_weight, g.gate_scale, g.up_weight, g.up_scale, g.down_weight, g.down_scale};
}

// Stages rows src[row(i)] (i < nb, width K, element type DT) of TB rows into LDS in
// lane order: float4 j of chunk c of lane l at ((i * CH + c) * 4 + j) * 64 + l, with
// CH = ceil(K / 1024); zeros past K and for i >= nb.
template <int TB, int DT, typename RowOf>
__device__ __forceinline__ void stage_rows(float* xs, const void* src, int K, int CH, int nb, RowOf row_of) {
    const int span = CH * 1024;
    for (int idx = threadIdx.x; idx < TB * span; idx += blockDim.x) {
        int i = idx / span, kk = idx - i * span;
        int c = kk >> 10, w = kk & 1023, l = w >> 4, j = w & 15;
        float v = 0.0f;
        if (i < nb && kk < K) v = load_act<DT>(src, (size_t)row_of(i) * K + kk);
        xs[(((i * CH + c) * 4 + (j >> 2)) * 64 + l) * 4 + (j & 3)] = v;
    }
}

// One pass of gate/up over TB staged tokens (nb real) for the wave's rows j0 .. j0 + GU_R.
template <int TB>
__device__ __forceinline__ void gate_up_pass(const float4* xs4, int CH, int nkb, int H, int I, int j0, int lane,
                                             const uint8_t* gw, const uint8_t* uw, const float* gs, const float* us,
                                             int nb, int a0, float* h) {
    float acc[2 * TB * GU_R];  // [gate|up][t][r]
#pragma unroll
    for (int i = 0; i < 2 * TB * GU_R; i++) acc[i] = 0.0f;
    for (int c0 = 0; c0 < CH; c0 += 4) {
        uint4 wg[GU_R][4], wu[GU_R][4];
#pragma unroll
        for (int r = 0; r < GU_R; r++) {
            const size_t row = (size_t)min(j0 + r, I - 1) * H;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                int col = (c0 + c) * 1024 + lane * 16;
                bool ok = c0 + c < CH && col < H;
                wg[r][c] = ok ? *reinterpret_cast<const uint4*>(gw + row + col) : make_uint4(0, 0, 0, 0);
                wu[r][c] = ok ? *reinterpret_cast<const uint4*>(uw + row + col) : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            if (c0 + c >= CH) break;
            int col = (c0 + c) * 1024 + lane * 16;
            float sg[GU_R], su[GU_R], fg[GU_R][16], fu[GU_R][16];
#pragma unroll
            for (int r = 0; r < GU_R; r++) {
                int jb = min(j0 + r, I - 1) >> 7;
                sg[r] = col < H ? gs[jb * nkb + (col >> 7)] : 0.0f;
                su[r] = col < H ? us[jb * nkb + (col >> 7)] : 0.0f;
                e4m3x16(wg[r][c], fg[r]);
                e4m3x16(wu[r][c], fu[r]);
            }
#pragma unroll
            for (int t = 0; t < TB; t++) {
                float xv[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float4 v = xs4[((t * CH + c0 + c) * 4 + i) * 64 + lane];
                    xv[4 * i] = v.x;
                    xv[4 * i + 1] = v.y;
                    xv[4 * i + 2] = v.z;
                    xv[4 * i + 3] = v.w;
                }
#pragma unroll
                for (int r = 0; r < GU_R; r++) {
                    float pg = 0.0f, pu = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        pg = fmaf(fg[r][i], xv[i], pg);
                        pu = fmaf(fu[r][i], xv[i], pu);
                    }
                    acc[(0 * TB + t) * GU_R + r] = fmaf(pg, sg[r], acc[(0 * TB + t) * GU_R + r]);
                    acc[(1 * TB + t) * GU_R + r] = fmaf(pu, su[r], acc[(1 * TB + t) * GU_R + r]);
                }
            }
        }
    }
    // value v = (gu * TB + t) * R + r ends in lane group v; its up sum TB * R groups later
    constexpr int NV = 2 * TB * GU_R, GROUP = 64 / NV;
    float tot = wave_sum_multi<NV>(acc, lane);
    float up = __shfl(tot, (lane + (NV / 2) * GROUP) & 63, 64);
    const int v = lane / GROUP;
    if (lane % GROUP == 0 && v < NV / 2) {
        const int t = v / GU_R, r = v % GU_R, j = j0 + r;
        if (t < nb && j < I) h[(size_t)(a0 + t) * I + j] = siluf(tot) * up;
    }
}

template <int XDT>
__global__ void __launch_bounds__(256) moe_gate_up_kernel(const uint64_t* __restrict__ recs,
                                                          const int32_t* __restrict__ off,
                                                          const int32_t* __restrict__ assign_tok,
                                                          const void* __restrict__ x, float* __restrict__ h, Rec g,
                                                          const int32_t* __restrict__ n_e_dev) {
    extern __shared__ float4 xs4[];
    const int e = blockIdx.y;
    if (n_e_dev && e >= *n_e_dev) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = (int)g.hidden, I = (int)g.inter;
    const int CH = (H + 1023) >> 10, nkb = (H + 127) >> 7;
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(recs[e]);
    const uint8_t* gw = rec + g.gw;
    const uint8_t* uw = rec + g.uw;
    const float* gs = reinterpret_cast<const float*>(rec + g.gs);
    const float* us = reinterpret_cast<const float*>(rec + g.us);
    const int j0 = (blockIdx.x * MOE_WAVES + wave) * GU_R;
    const int a_begin = off[e], a_end = off[e + 1];
    float* xs = reinterpret_cast<float*>(xs4);
    for (int a0 = a_begin; a0 < a_end; a0 += MOE_TB) {
        const int nb = min(MOE_TB, a_end - a0);
        __syncthreads();
        stage_rows<MOE_TB, XDT>(xs, x, H, CH, nb, [&](int i) { return assign_tok[a0 + i]; });
        __syncthreads();
        if (nb == 1) gate_up_pass<1>(xs4, CH, nkb, H, I, j0, lane, gw, uw, gs, us, nb, a0, h);
        else if (nb == 2) gate_up_pass<2>(xs4, CH, nkb, H, I, j0, lane, gw, uw, gs, us, nb, a0, h);
        else gate_up_pass<4>(xs4, CH, nkb, H, I, j0, lane, gw, uw, gs, us, nb, a0, h);
    }
}

// One pass of down over TB staged h rows (nb real) for the wave's rows r0 .. r0 + DN_R.
template <int TB>
__device__ __forceinline__ void down_pass(const float4* xs4, int CH, int nkb, int H, int I, int r0, int lane,
                                          const uint8_t* dw, const float* ds, int nb, int a0, float* y) {
    float acc[TB * DN_R];
#pragma unroll
    for (int i = 0; i < TB * DN_R; i++) acc[i] = 0.0f;
    for (int c0 = 0; c0 < CH; c0 += 2) {
        uint4 wd[DN_R][2];
#pragma unroll
        for (int r = 0; r < DN_R; r++) {
            const size_t row = (size_t)min(r0 + r, H - 1) * I;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                int col = (c0 + c) * 1024 + lane * 16;
                wd[r][c] = (c0 + c < CH && col < I) ? *reinterpret_cast<const uint4*>(dw + row + col)
                                                    : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int c = 0; c < 2; c++) {
            if (c0 + c >= CH) break;
            int col = (c0 + c) * 1024 + lane * 16;
            float sd[DN_R], fd[DN_R][16];
#pragma unroll
            for (int r = 0; r < DN_R; r++) {
                sd[r] = col < I ? ds[(min(r0 + r, H - 1) >> 7) * nkb + (col >> 7)] : 0.0f;
                e4m3x16(wd[r][c], fd[r]);
            }
#pragma unroll
            for (int t = 0; t < TB; t++) {
                float xv[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float4 v = xs4[((t * CH + c0 + c) * 4 + i) * 64 + lane];
                    xv[4 * i] = v.x;
                    xv[4 * i + 1] = v.y;
                    xv[4 * i + 2] = v.z;
                    xv[4 * i + 3] = v.w;
                }
#pragma unroll
                for (int r = 0; r < DN_R; r++) {
                    float p = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; i++) p = fmaf(fd[r][i], xv[i], p);
                    acc[t * DN_R + r] = fmaf(p, sd[r], acc[t * DN_R + r]);
                }
            }
        }
    }
    constexpr int NV = TB * DN_R, GROUP = 64 / NV;
    float tot = wave_sum_multi<NV>(acc, lane);
    const int v = lane / GROUP;
    if (lane % GROUP == 0) {
        const int t = v / DN_R, r = r0 + v % DN_R;
        if (t < nb && r < H) y[(size_t)(a0 + t) * H + r] = tot;
    }
}

__global__ void __launch_bounds__(256) moe_down_kernel(const uint64_t* __restrict__ recs, const int32_t* __restrict__ off,
                                                       const float* __restrict__ h, float* __restrict__ y, Rec g,
                                                       const int32_t* __restrict__ n_e_dev) {
    extern __shared__ float4 xs4[];
    const int e = blockIdx.y;
    if (n_e_dev && e >= *n_e_dev) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = (int)g.hidden, I = (int)g.inter;
    const int CH = (I + 1023) >> 10, nkb = (I + 127) >> 7;
    const uint8_t* rec = reinterpret_cast<const uint8_t*>(recs[e]);
    const uint8_t* dw = rec + g.dw;
    const float* ds = reinterpret_cast<const float*>(rec + g.ds);
    const int r0 = (blockIdx.x * MOE_WAVES + wave) * DN_R;
    const int a_begin = off[e], a_end = off[e + 1];
    float* xs = reinterpret_cast<float*>(xs4);
    for (int a0 = a_begin; a0 < a_end; a0 += MOE_TB) {
        const int nb = min(MOE_TB, a_end - a0);
        __syncthreads();
        stage_rows<MOE_TB, OOM_F32>(xs, h, I, CH, nb, [&](int i) { return a0 + i; });
        __syncthreads();
        if (nb == 1) down_pass<1>(xs4, CH, nkb, H, I, r0, lane, dw, ds, nb, a0, y);
        else if (nb == 2) down_pass<2>(xs4, CH, nkb, H, I, r0, lane, dw, ds, nb, a0, y);
        else down_pass<4>(xs4, CH, nkb, H, I, r0, lane, dw, ds, nb, a0, y);
    }
}

// out[t, c] = sum_s w[t, s] * y[slot_assign[t, s], c] in slot order
// (crates/oominf-cuda/kernels/moe.cu:153-164). Block (token t, column chunk of 1024): each
// thread 4 consecutive columns; the slots go 8 at a time, their indices and weights first,
// then the 8 rows' 16-byte loads together, then the multiply-adds in slot order.
template <int ODT>
__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ y, const int32_t* __restrict__ slot,
                                                          const float* __restrict__ w, void* __restrict__ out, int T,
                                                          int H, int k) {
    const int t = blockIdx.x, c0 = blockIdx.y * 1024 + 4 * threadIdx.x;
    if (c0 >= H) return;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool vec = c0 + 4 <= H && (H & 3) == 0;
    for (int s0 = 0; s0 < k; s0 += 8) {
        int sl[8];
        float ws[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const bool ok = s0 + i < k;
            sl[i] = ok ? slot[t * k + s0 + i] : 0;
            ws[i] = ok ? w[t * k + s0 + i] : 0.0f;
        }
        if (vec) {
            float4 v[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                v[i] = s0 + i < k ? *reinterpret_cast<const float4*>(y + (size_t)sl[i] * H + c0)
                                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (s0 + i >= k) break;
                acc[0] = fmaf(ws[i], v[i].x, acc[0]);
                acc[1] = fmaf(ws[i], v[i].y, acc[1]);
                acc[2] = fmaf(ws[i], v[i].z, acc[2]);
                acc[3] = fmaf(ws[i], v[i].w, acc[3]);
            }
        } else {
            for (int i = 0; i < 8 && s0 + i < k; i++)
                for (int j = 0; j < 4 && c0 + j < H; j++) acc[j] = fmaf(ws[i], y[(size_t)sl[i] * H + c0 + j], acc[j]);
        }
    }
    for (int j = 0; j < 4 && c0 + j < H; j++) store_out<ODT>(out, (size_t)t * H + c0 + j, acc[j]);
}

int check_geo(const OomFp8Record* geo, const char* who) {
    if (!geo) return fail(OOM_ERR_ARG, std::string(who) + ": null geometry");
    const OomFp8Record& g = *geo;
    bool ok = g.hidden >= 16 && g.inter >= 16 && g.hidden % 16 == 0 && g.inter % 16 == 0 && g.hidden <= (1 << 20) &&
              g.inter <= (1 << 20) && g.gate_weight % 16 == 0 && g.up_weight % 16 == 0 && g.down_weight % 16 == 0 &&
              g.gate_scale % 4 == 0 && g.up_scale % 4 == 0 && g.down_scale % 4 == 0 && g.gate_weight >= 0 &&
              g.up_weight >= 0 && g.down_weight >= 0 && g.gate_scale >= 0 && g.up_scale >= 0 && g.down_scale >= 0;
    if (!ok)
        return fail(OOM_ERR_ARG, std::string(who) +
                                     ": widths must be multiples of 16 and weight parts 16-byte aligned "
                                     "(buffer too small or shape unsupported)");
    return OOM_OK;
}

int launch_gate_up(const uint64_t* recs, const int32_t* off, const int32_t* tok, int grid_e, const void* x, int xdt,
                   float* h, const OomFp8Record& geo, const int32_t* n_e_dev, hipStream_t st) {
    Rec g = rec_of(geo);
    const int CH = (int)cdiv(geo.hidden, 1024);
    size_t lds = (size_t)MOE_TB * CH * 1024 * sizeof(float);
    dim3 grid((unsigned)cdiv(geo.inter, MOE_WAVES * GU_R), (unsigned)grid_e);
    if (xdt == OOM_BF16)
        hipLaunchKernelGGL((moe_gate_up_kernel<OOM_BF16>), grid, dim3(256), lds, st, recs, off, tok, x, h, g,
                           n_e_dev);
    else
        hipLaunchKernelGGL((moe_gate_up_kernel<OOM_F32>), grid, dim3(256), lds, st, recs, off, tok, x, h, g,
                           n_e_dev);
    return launched("moe_gate_up_fp8");
}

int launch_down(const uint64_t* recs, const int32_t* off, int grid_e, const float* h, float* y,
                const OomFp8Record& geo, const int32_t* n_e_dev, hipStream_t st) {
    Rec g = rec_of(geo);
    const int CH = (int)cdiv(geo.inter, 1024);
    size_t lds = (size_t)MOE_TB * CH * 1024 * sizeof(float);
    dim3 grid((unsigned)cdiv(geo.hidden, MOE_WAVES * DN_R), (unsigned)grid_e);
    hipLaunchKernelGGL(moe_down_kernel, grid, dim3(256), lds, st, recs, off, h, y, g, n_e_dev);
    return launched("moe_down_fp8");
}

int launch_combine(const float* y, const int32_t* slot, const float* w, void* out, int odt, int T, int H, int k,
                   hipStream_t st) {
    dim3 grid((unsigned)T, (unsigned)cdiv(H, 1024));
    if (odt == OOM_BF16)
        hipLaunchKernelGGL((moe_combine_kernel<OOM_BF16>), grid, dim3(256), 0, st, y, slot, w, out, T, H, k);
    else
        hipLaunchKernelGGL((moe_combine_kernel<OOM_F32>), grid, dim3(256), 0, st, y, slot, w, out, T, H, k);
    return launched("moe_combine_slots");
}

// LDS of one staged pass must fit 64 KiB.
static bool lds_fits(int64_t width) { return (size_t)MOE_TB * cdiv(width, 1024) * 1024 * sizeof(float) <= 65536; }

// The one-launch path (moe_fused.hip) and its workspace.
bool fused_supported(int T, int E, int k, const OomFp8Record& g);
size_t fused_workspace_size(int T, int E, int k, const OomFp8Record& g);
int launch_fused(const float* logits, const void* x, int xdt, const uint64_t* all_recs, int T, int E, int k,
                 const OomFp8Record& g, int32_t* ids, float* weights, void* out, int odt, void* ws, hipStream_t st);

// The one-launch bf16-MFMA path for 2..16 tokens (moe_batch.hip) and its workspace.
bool batch_supported(int T, int E, int k, const OomFp8Record& g, int xdt, const void* x);
size_t batch_workspace_size(int T, int k, const OomFp8Record& g);
int launch_batch(const float* logits, const void* x, const uint64_t* all_recs, int T, int E, int k,
                 const OomFp8Record& g, int32_t* ids, float* weights, void* out, int odt, void* ws, hipStream_t st);

// Workspace of the multi-launch path of oom_moe_decode_fp8: plan | recs | h | y.
struct DecodeWs {
    size_t plan, recs, h, y, total;
};

static size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

static DecodeWs decode_ws(int T, int E, int k, const OomFp8Record& g) {
    DecodeWs w;
    size_t A = (size_t)T * k;
    w.plan = WS_HEADER;  // the header holds the one-launch kernels' state between calls
    w.recs = w.plan + al256(PlanView::size(E, (int)A) * sizeof(int32_t));
    w.h = w.recs + al256((size_t)std::min<size_t>(E, A) * sizeof(uint64_t));
    w.y = w.h + al256(A * (size_t)g.inter * sizeof(float));
    w.total = w.y + al256(A * (size_t)g.hidden * sizeof(float));
    return w;
}

}  // namespace oom

extern "C" int oom_moe_gate_up_fp8(const uint64_t* recs, const int32_t* off, const int32_t* assign_tok,
                                   int n_experts, const void* x, int x_dtype, float* h, const OomFp8Record* geo,
                                   void* stream) {
    using namespace oom;
    if (int rc = check_geo(geo, "oom_moe_gate_up_fp8")) return rc;
    OOM_REQUIRE(n_experts >= 0 && n_experts <= 65535, "oom_moe_gate_up_fp8: n_experts");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_moe_gate_up_fp8: x_dtype");
    OOM_REQUIRE(lds_fits(geo->hidden), "oom_moe_gate_up_fp8: hidden > 4096 unsupported");
    if (n_experts == 0) return OOM_OK;
    OOM_REQUIRE(recs && off && assign_tok && x && h, "oom_moe_gate_up_fp8: null buffer");
    return launch_gate_up(recs, off, assign_tok, n_experts, x, x_dtype, h, *geo, nullptr, as_stream(stream));
}

extern "C" int oom_moe_down_fp8(const uint64_t* recs, const int32_t* off, int n_experts, const float* h, float* y,
                                const OomFp8Record* geo, void* stream) {
    using namespace oom;
    if (int rc = check_geo(geo, "oom_moe_down_fp8")) return rc;
    OOM_REQUIRE(n_experts >= 0 && n_experts <= 65535, "oom_moe_down_fp8: n_experts");
    OOM_REQUIRE(lds_fits(geo->inter), "oom_moe_down_fp8: inter > 4096 unsupported");
    if (n_experts == 0) return OOM_OK;
    OOM_REQUIRE(recs && off && h && y, "oom_moe_down_fp8: null buffer");
    return launch_down(recs, off, n_experts, h, y, *geo, nullptr, as_stream(stream));
}

extern "C" int oom_moe_combine_slots(const float* y, const int32_t* slot_assign, const float* w, void* out,
                                     int out_dtype, int T, int H, int k, void* stream) {
    using namespace oom;
    OOM_REQUIRE(T >= 0 && H >= 1 && k >= 1, "oom_moe_combine_slots: shape");
    OOM_REQUIRE(out_dtype == OOM_F32 || out_dtype == OOM_BF16, "oom_moe_combine_slots: out_dtype");
    if (T == 0) return OOM_OK;
    OOM_REQUIRE(y && slot_assign && w && out, "oom_moe_combine_slots: null buffer");
    return launch_combine(y, slot_assign, w, out, out_dtype, T, H, k, as_stream(stream));
}

extern "C" size_t oom_moe_decode_fp8_workspace_size(int T, int E, int k, const OomFp8Record* geo) {
    if (!geo || T < 1 || E < 1 || k < 1) return 0;
    return std::max({oom::decode_ws(T, E, k, *geo).total, oom::fused_workspace_size(T, E, k, *geo),
                     oom::batch_workspace_size(T, k, *geo)});
}

extern "C" int oom_moe_decode_fp8(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T,
                                  int E, int k, const OomFp8Record* geo, int32_t* ids, float* weights, void* out,
                                  int out_dtype, void* ws, size_t ws_bytes, void* stream) {
    using namespace oom;
    if (int rc = check_geo(geo, "oom_moe_decode_fp8")) return rc;
    OOM_REQUIRE(T >= 1 && (int64_t)T * k <= (1 << 24), "oom_moe_decode_fp8: T must be >= 1 and T * k <= 2^24");
    OOM_REQUIRE(k >= 1 && k <= 32 && E >= k && E <= 8192, "oom_moe_decode_fp8: router top-k > 32 or experts > 8192");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_moe_decode_fp8: x_dtype");
    OOM_REQUIRE(out_dtype == OOM_F32 || out_dtype == OOM_BF16, "oom_moe_decode_fp8: out_dtype");
    OOM_REQUIRE(lds_fits(geo->hidden) && lds_fits(geo->inter), "oom_moe_decode_fp8: widths > 4096 unsupported");
    OOM_REQUIRE(logits && x && all_recs && ids && weights && out, "oom_moe_decode_fp8: null buffer");
    DecodeWs w = decode_ws(T, E, k, *geo);
    if (!ws || ws_bytes < oom_moe_decode_fp8_workspace_size(T, E, k, geo))
        return fail(OOM_ERR_WORKSPACE, "oom_moe_decode_fp8: workspace smaller than oom_moe_decode_fp8_workspace_size()");
    OOM_REQUIRE(aligned(ws, 256), "oom_moe_decode_fp8: workspace must be 256-byte aligned");
    if (batch_supported(T, E, k, *geo, x_dtype, x))
        return launch_batch(logits, x, all_recs, T, E, k, *geo, ids, weights, out, out_dtype, ws, as_stream(stream));
    if (fused_supported(T, E, k, *geo))
        return launch_fused(logits, x, x_dtype, all_recs, T, E, k, *geo, ids, weights, out, out_dtype, ws,
                            as_stream(stream));
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    int32_t* plan = reinterpret_cast<int32_t*>(base + w.plan);
    uint64_t* recs = reinterpret_cast<uint64_t*>(base + w.recs);
    float* h = reinterpret_cast<float*>(base + w.h);
    float* y = reinterpret_cast<float*>(base + w.y);
    hipStream_t st = as_stream(stream);
    const int A = T * k;
    PlanView pv{plan, E, A};
    if (int rc = oom_router_topk(logits, ids, weights, T, E, k, stream)) return rc;
    if (int rc = oom_moe_plan(ids, T, E, k, all_recs, plan, recs, stream)) return rc;
    const int grid_e = std::min(E, A);
    if (int rc = launch_gate_up(recs, pv.off(), pv.assign_tok(), grid_e, x, x_dtype, h, *geo, pv.n_e(), st)) return rc;
    if (int rc = launch_down(recs, pv.off(), grid_e, h, y, *geo, pv.n_e(), st)) return rc;
    return launch_combine(y, pv.slot_assign(), weights, out, out_dtype, T, (int)geo->hidden, k, st);
}
