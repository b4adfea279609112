// Routed experts over NVFP4 records (layout nvfp4-modelopt-g16, OomNvfp4Record) read in
// place: gate/up + SwiGLU, down, and the one-call decode step over them.
//
// A weight is w = e2m1(code) * (e4m3(scale) * scale_2) (crates/oominf-cuda/kernels/moe.cu:17-45;
// crates/oominf-cpu/src/kernel.rs:76-98): two codes per byte, low nibble first, one e4m3
// scale byte per 16 inputs, one fp32 scale_2 per projection in the record's scalars part.
//
// Layout of the work (gfx950, wave64):
//   - a lane's 16-byte load holds 32 codes of one row: columns 1024 c + 32 l .. + 32 of
//     1024-column chunk c, l = lane % 32, two scale groups of 16;
//   - a wave streams two rows at a time, one per half (lanes 0..31 row 2p, 32..63 row
//     2p + 1), so a 640-column down row keeps 20 of each 32 lanes busy, not 20 of 64;
//   - the codes convert exactly to fp32 with v_cvt_scalef32_pk_f32_fp4 (scale 1), each
//     group's 16 products e2m1 * x sum in fp32, and the group sum is multiplied once by
//     e4m3(scale) * scale_2. The reference multiplies every weight first, (e2m1 * gs) * x,
//     so the rounding differs as well as the order (both within the f64 bars the tests
//     hold: 1e-5 of sum |x . w| per output);
//   - the inputs of a pass (x rows of up to TB assignments, or h rows) sit in LDS as fp32
//     in the same lane order (float4 i of lane l's 32 columns of chunk c of row t at
//     ((t * CH + c) * 8 + i) * 32 + l), staged with 16-byte loads all in flight before
//     the first store; both halves read the same words;
//   - gate/up: a block of 4 waves x 2 row pairs = 16 intermediate rows of one expert;
//     down: 4 waves x 4 row pairs = 32 output rows; grid (row blocks, experts), and a
//     block past the step's expert count (read from the device plan) returns at once;
//   - a scale group past the row's end reads as scale 0 (its codes would pair with the
//     next row's bytes and zero inputs), and loads past the record read zeros.
#include "router.hpp"
#include "stream.hpp"

extern "C" int oom_router_topk(const float* logits, int32_t* ids, float* weights, int T, int E, int k, void* stream);
extern "C" int oom_moe_plan(const int32_t* ids, int T, int E, int k, const uint64_t* all_recs, int32_t* plan,
                            uint64_t* recs, void* stream);

namespace oom {

int launch_combine(const float* y, const int32_t* slot, const float* w, void* out, int odt, int T, int H, int k,
                   hipStream_t st);

constexpr int N4_WAVES = 4;
constexpr int N4_GP = 2;  // gate/up row pairs per wave
constexpr int N4_DP = 4;  // down row pairs per wave
constexpr int N4_TB = 2;  // assignments per pass
constexpr int N4_KMAX = 4096;

struct Rec4 {
    int H, I;
    int gw, gs, uw, us, dw, ds;
    int s2g, s2u, s2d;  // byte offsets of the three weight_scale_2 floats
    int bytes;          // record span: end of its last part
};

static int64_t rec4_span(const OomNvfp4Record& g) {
    const int64_t H = g.hidden, I = g.inter;
    int64_t e = std::max({g.gate_weight + I * H / 2, g.gate_scale + I * H / 16, g.up_weight + I * H / 2,
                          g.up_scale + I * H / 16, g.down_weight + H * I / 2, g.down_scale + H * I / 16});
    for (int p = 0; p < 3; p++) e = std::max(e, (g.scale2[p] + 1) * 4);
    return e;
}

static Rec4 rec4_of(const OomNvfp4Record& g) {
    return Rec4{(int)g.hidden,         (int)g.inter,         (int)g.gate_weight,   (int)g.gate_scale,
                (int)g.up_weight,      (int)g.up_scale,      (int)g.down_weight,   (int)g.down_scale,
                (int)(g.scale2[0] * 4), (int)(g.scale2[1] * 4), (int)(g.scale2[2] * 4), (int)rec4_span(g)};
}

// The 32 E2M1 codes of a 16-byte piece to fp32, exactly: byte b holds columns 2b (low
// nibble) and 2b + 1.
__device__ __forceinline__ void e2m1x32(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const auto p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 0);
        const auto p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 1);
        const auto p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 2);
        const auto p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 3);
        f[8 * i + 0] = p0[0];
        f[8 * i + 1] = p0[1];
        f[8 * i + 2] = p1[0];
        f[8 * i + 3] = p1[1];
        f[8 * i + 4] = p2[0];
        f[8 * i + 5] = p2[1];
        f[8 * i + 6] = p3[0];
        f[8 * i + 7] = p3[1];
    }
}

__device__ __forceinline__ uint32_t ldb(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}

__device__ __forceinline__ float e4m3_byte(uint32_t b) { return __builtin_amdgcn_cvt_f32_fp8((int)b, 0); }

// Stages rows row_of(t) (t < nb) of src (width K, element type DT) into LDS in the lane
// order above; zeros past K and for t >= nb. 256 threads take part, thread ti of them.
template <int DT, typename RowOf>
__device__ __forceinline__ void stage4(float4* xs4, const void* src, int K, int CH, int nb, RowOf row_of,
                                       int ti = (int)threadIdx.x) {
    constexpr int EPL = DT == OOM_BF16 ? 8 : 4;  // elements per 16-byte load
    constexpr int ES = DT == OOM_BF16 ? 2 : 4;
    const int span = CH * 1024, nvec = N4_TB * span / EPL;
    for (int base = 0; base < nvec; base += 256 * 4) {
        uint4 v[4];
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const int i = base + ti + 256 * n;
            const int t = i * EPL / span, kk = i * EPL - t * span;
            const bool ok = i < nvec && t < nb && kk < K;
            v[n] = ok ? *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(src) +
                                                        ((size_t)row_of(t) * K + kk) * ES)
                      : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const int i = base + ti + 256 * n;
            if (i >= nvec) break;
            const int t = i * EPL / span, kk = i * EPL - t * span;
            const int c = kk >> 10, l = (kk & 1023) >> 5, j = kk & 31;
            float4* dst = &xs4[((t * CH + c) * 8 + (j >> 2)) * 32 + l];
            if constexpr (DT == OOM_BF16) {
                dst[0] = make_float4(__uint_as_float(v[n].x << 16), __uint_as_float(v[n].x & 0xffff0000u),
                                     __uint_as_float(v[n].y << 16), __uint_as_float(v[n].y & 0xffff0000u));
                dst[32] = make_float4(__uint_as_float(v[n].z << 16), __uint_as_float(v[n].z & 0xffff0000u),
                                      __uint_as_float(v[n].w << 16), __uint_as_float(v[n].w & 0xffff0000u));
            } else {
                dst[0] = make_float4(__uint_as_float(v[n].x), __uint_as_float(v[n].y), __uint_as_float(v[n].z),
                                     __uint_as_float(v[n].w));
            }
        }
    }
}

// The two group sums of one 32-column piece against staged row t: (cols 0..15, 16..31).
__device__ __forceinline__ void piece_dot(const float* f, const float4* xs4, int t, int CH, int c, int l, float& p0,
                                          float& p1) {
    float x[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = xs4[((t * CH + c) * 8 + i) * 32 + l];
        x[4 * i] = v.x;
        x[4 * i + 1] = v.y;
        x[4 * i + 2] = v.z;
        x[4 * i + 3] = v.w;
    }
    p0 = 0.0f;
    p1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        p0 = fmaf(f[i], x[i], p0);
        p1 = fmaf(f[16 + i], x[16 + i], p1);
    }
}

// One round of a gate/up pass's loads: chunks c0 .. c0 + CS - 1 (1024 columns each) of the
// wave's rows j0 + 2 p + half, codes and scale bytes (a chunk or group past the row reads 0).
template <int CS>
struct Gu4Ld {
    uint4 wg[N4_GP][CS], wu[N4_GP][CS];
    uint32_t bg[N4_GP][CS][2], bu[N4_GP][CS][2];
};
template <int CS>
__device__ __forceinline__ void gu4_load(const Rec4& g, __amdgpu_buffer_rsrc_t r, int j0, int lane, int c0,
                                         Gu4Ld<CS>& t) {
    const int H = g.H, I = g.I, CH = (H + 1023) >> 10, hg = H >> 4;
    const int half = lane >> 5, l = lane & 31;
#pragma unroll
    for (int p = 0; p < N4_GP; p++) {
        const int j = j0 + 2 * p + half;
#pragma unroll
        for (int c = 0; c < CS; c++) {
            const int col = (c0 + c) * 1024 + 32 * l;
            const bool ok = j < I && c0 + c < CH && col < H;
            t.wg[p][c] = ld16(r, ok ? g.gw + j * (H >> 1) + (col >> 1) : OOB);
            t.wu[p][c] = ld16(r, ok ? g.uw + j * (H >> 1) + (col >> 1) : OOB);
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const bool okq = ok && (col >> 4) + q < hg;
                t.bg[p][c][q] = ldb(r, okq ? g.gs + j * hg + (col >> 4) + q : OOB);
                t.bu[p][c][q] = ldb(r, okq ? g.us + j * hg + (col >> 4) + q : OOB);
            }
        }
    }
}

// That round's sums into acc[(gate|up, t, p)] over TB staged tokens.
template <int TB, int CS>
__device__ __forceinline__ void gu4_math(const float4* xs4, const Rec4& g, float s2g, float s2u, int lane, int c0,
                                         const Gu4Ld<CS>& t, float (&acc)[2 * TB * N4_GP]) {
    const int H = g.H, CH = (H + 1023) >> 10, hg = H >> 4;
    const int l = lane & 31;
#pragma unroll
    for (int c = 0; c < CS; c++) {
        if (c0 + c >= CH) break;
        const int col = (c0 + c) * 1024 + 32 * l;
#pragma unroll
        for (int p = 0; p < N4_GP; p++) {
            float sg[2], su[2];
#pragma unroll
            for (int q = 0; q < 2; q++) {
                // a group past the row's end scales to 0 (its byte read as 0); the select
                // is on scale_2, so the byte's load is used on every lane and stays where
                // it was issued (a select on the product let the compiler move the load
                // into a branch, whose wait then covered every load in flight)
                const bool okq = (col >> 4) + q < hg;
                sg[q] = e4m3_byte(t.bg[p][c][q]) * (okq ? s2g : 0.0f);
                su[q] = e4m3_byte(t.bu[p][c][q]) * (okq ? s2u : 0.0f);
            }
            // the gate piece, then the up piece: one set of 32 decoded weights at a time
            float f[32];
            e2m1x32(t.wg[p][c], f);
#pragma unroll
            for (int tt = 0; tt < TB; tt++) {
                float g0, g1;
                piece_dot(f, xs4, tt, CH, c0 + c, l, g0, g1);
                float& ag = acc[(0 * TB + tt) * N4_GP + p];
                ag = fmaf(g1, sg[1], fmaf(g0, sg[0], ag));
            }
            e2m1x32(t.wu[p][c], f);
#pragma unroll
            for (int tt = 0; tt < TB; tt++) {
                float u0, u1;
                piece_dot(f, xs4, tt, CH, c0 + c, l, u0, u1);
                float& au = acc[(1 * TB + tt) * N4_GP + p];
                au = fmaf(u1, su[1], fmaf(u0, su[0], au));
            }
        }
    }
}

// The pass's end: the wave sums, then put(t, j, silu(gate) * up) for each of the wave's rows.
template <int TB, typename Put>
__device__ __forceinline__ void gu4_put(float (&acc)[2 * TB * N4_GP], int I, int j0, int lane, int nb, Put put) {
    const int half = lane >> 5, l = lane & 31;
    // value v = (gu * TB + t) * GP + p ends in sub-group v of each half; its up sum sits
    // 16 lanes on, in the same half
    constexpr int NV = 2 * TB * N4_GP, GROUP = 32 / NV;
    const float tot = wave_sum_multi<NV, 16>(acc, lane);
    const float up = __shfl(tot, (lane & 32) | ((lane + 16) & 31), 64);
    const int v = l / GROUP;
    if (l % GROUP == 0 && v < NV / 2) {
        const int t = v / N4_GP, j = j0 + 2 * (v % N4_GP) + half;
        if (t < nb && j < I) put(t, j, siluf(tot) * up);
    }
}

// One gate/up pass over TB staged tokens (nb real): the wave's rows j0 + 2p + half;
// put(t, j, v) stores h of staged token t at intermediate row j.
// CS chunks of 1024 columns load per round (all of a row's with CS = 4).
template <int TB, int CS = 2, typename Put>
__device__ __forceinline__ void gu4_pass(const float4* xs4, const Rec4& g, __amdgpu_buffer_rsrc_t r, float s2g,
                                         float s2u, int j0, int lane, int nb, Put put) {
    const int CH = (g.H + 1023) >> 10;
    float acc[2 * TB * N4_GP];  // [gate|up][t][p]
#pragma unroll
    for (int i = 0; i < 2 * TB * N4_GP; i++) acc[i] = 0.0f;
    for (int c0 = 0; c0 < CH; c0 += CS) {
        Gu4Ld<CS> t;
        gu4_load<CS>(g, r, j0, lane, c0, t);
        gu4_math<TB, CS>(xs4, g, s2g, s2u, lane, c0, t, acc);
    }
    gu4_put<TB>(acc, g.I, j0, lane, nb, put);
}

template <int XDT>
__global__ void __launch_bounds__(256) moe_gate_up_nvfp4_kernel(const uint64_t* __restrict__ recs,
                                                                const int32_t* __restrict__ off,
                                                                const int32_t* __restrict__ assign_tok,
                                                                const void* __restrict__ x, float* __restrict__ h,
                                                                Rec4 g, const int32_t* __restrict__ n_e_dev) {
    extern __shared__ float4 xs4[];
    const int e = blockIdx.y;
    if (n_e_dev && e >= *n_e_dev) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const __amdgpu_buffer_rsrc_t r = uniform_rsrc(recs[e], g.bytes);
    const float s2g = ldf(r, g.s2g), s2u = ldf(r, g.s2u);
    const int j0 = (blockIdx.x * N4_WAVES + wave) * 2 * N4_GP;
    const int CH = (g.H + 1023) >> 10;
    const int a_begin = off[e], a_end = off[e + 1];
    for (int a0 = a_begin; a0 < a_end; a0 += N4_TB) {
        const int nb = min(N4_TB, a_end - a0);
        __syncthreads();
        stage4<XDT>(xs4, x, g.H, CH, nb, [&](int t) { return assign_tok[a0 + t]; });
        __syncthreads();
        const auto put = [&](int t, int j, float v) { h[(size_t)(a0 + t) * g.I + j] = v; };
        if (nb == 1) gu4_pass<1>(xs4, g, r, s2g, s2u, j0, lane, nb, put);
        else gu4_pass<2>(xs4, g, r, s2g, s2u, j0, lane, nb, put);
    }
}

// One down pass over TB staged h rows (nb real): the wave's output rows r0 + 2p + half;
// put(t, row, v) stores y of staged row t at output row `row`.
template <int TB, typename Put>
__device__ __forceinline__ void dn4_pass(const float4* xs4, const Rec4& g, __amdgpu_buffer_rsrc_t r, float s2,
                                         int r0, int lane, int nb, Put put) {
    const int H = g.H, I = g.I, CH = (I + 1023) >> 10, ig = I >> 4;
    const int half = lane >> 5, l = lane & 31;
    float acc[TB * N4_DP];
#pragma unroll
    for (int i = 0; i < TB * N4_DP; i++) acc[i] = 0.0f;
    for (int c0 = 0; c0 < CH; c0 += 2) {
        uint4 wd[N4_DP][2];
        uint32_t bd[N4_DP][2][2];
#pragma unroll
        for (int p = 0; p < N4_DP; p++) {
            const int row = r0 + 2 * p + half;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int col = (c0 + c) * 1024 + 32 * l;
                const bool ok = row < H && c0 + c < CH && col < I;
                wd[p][c] = ld16(r, ok ? g.dw + row * (I >> 1) + (col >> 1) : OOB);
#pragma unroll
                for (int q = 0; q < 2; q++)
                    bd[p][c][q] = ldb(r, ok && (col >> 4) + q < ig ? g.ds + row * ig + (col >> 4) + q : OOB);
            }
        }
#pragma unroll
        for (int c = 0; c < 2; c++) {
            if (c0 + c >= CH) break;
            const int col = (c0 + c) * 1024 + 32 * l;
#pragma unroll
            for (int p = 0; p < N4_DP; p++) {
                float sd[2];
#pragma unroll
                for (int q = 0; q < 2; q++) sd[q] = e4m3_byte(bd[p][c][q]) * ((col >> 4) + q < ig ? s2 : 0.0f);
                float f[32];
                e2m1x32(wd[p][c], f);
#pragma unroll
                for (int t = 0; t < TB; t++) {
                    float p0, p1;
                    piece_dot(f, xs4, t, CH, c0 + c, l, p0, p1);
                    float& a = acc[t * N4_DP + p];
                    a = fmaf(p1, sd[1], fmaf(p0, sd[0], a));
                }
            }
        }
    }
    constexpr int NV = TB * N4_DP, GROUP = 32 / NV;
    const float tot = wave_sum_multi<NV, 16>(acc, lane);
    const int v = l / GROUP;
    if (l % GROUP == 0) {
        const int t = v / N4_DP, row = r0 + 2 * (v % N4_DP) + half;
        if (t < nb && row < H) put(t, row, tot);
    }
}

__global__ void __launch_bounds__(256) moe_down_nvfp4_kernel(const uint64_t* __restrict__ recs,
                                                             const int32_t* __restrict__ off,
                                                             const float* __restrict__ h, float* __restrict__ y,
                                                             Rec4 g, const int32_t* __restrict__ n_e_dev) {
    extern __shared__ float4 xs4[];
    const int e = blockIdx.y;
    if (n_e_dev && e >= *n_e_dev) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const __amdgpu_buffer_rsrc_t r = uniform_rsrc(recs[e], g.bytes);
    const float s2 = ldf(r, g.s2d);
    const int r0 = (blockIdx.x * N4_WAVES + wave) * 2 * N4_DP;
    const int CH = (g.I + 1023) >> 10;
    const int a_begin = off[e], a_end = off[e + 1];
    for (int a0 = a_begin; a0 < a_end; a0 += N4_TB) {
        const int nb = min(N4_TB, a_end - a0);
        __syncthreads();
        stage4<OOM_F32>(xs4, h, g.I, CH, nb, [&](int t) { return a0 + t; });
        __syncthreads();
        const auto put = [&](int t, int row, float v) { y[(size_t)(a0 + t) * g.H + row] = v; };
        if (nb == 1) dn4_pass<1>(xs4, g, r, s2, r0, lane, nb, put);
        else dn4_pass<2>(xs4, g, r, s2, r0, lane, nb, put);
    }
}

static int check_geo4(const OomNvfp4Record* geo, const char* who) {
    if (!geo) return fail(OOM_ERR_ARG, std::string(who) + ": null geometry");
    const OomNvfp4Record& g = *geo;
    bool ok = g.hidden >= 16 && g.inter >= 16 && g.hidden % 16 == 0 && g.inter % 16 == 0 && g.hidden <= N4_KMAX &&
              g.inter <= N4_KMAX && g.gate_weight >= 0 && g.up_weight >= 0 && g.down_weight >= 0 &&
              g.gate_scale >= 0 && g.up_scale >= 0 && g.down_scale >= 0 && g.gate_weight % 16 == 0 &&
              g.up_weight % 16 == 0 && g.down_weight % 16 == 0;
    for (int p = 0; p < 3; p++) ok = ok && g.scale2[p] >= 0;
    ok = ok && rec4_span(g) < OOB;
    if (!ok)
        return fail(OOM_ERR_ARG, std::string(who) +
                                     ": widths must be multiples of 16 and at most 4096, weight parts 16-byte "
                                     "aligned (buffer too small or shape unsupported)");
    return OOM_OK;
}

static size_t stage_lds(int64_t width) { return (size_t)N4_TB * cdiv(width, 1024) * 1024 * sizeof(float); }

// ---- one token in one launch ---------------------------------------------------------------
// The step of oom_moe_decode_nvfp4 for T = 1 as one persistent kernel, the same arithmetic
// as the five-launch step (router, plan, gate/up, down, slot-order combine):
//   - every block routes the token on wave 0 (route_picks: the router kernel's picks and
//     weights, by a radix descent on ballots) while its other waves stage x into LDS; with one token each picked
//     expert has one assignment, so h row s belongs to slot s and no plan is built;
//   - phase 1: wave items (slot, 2 N4_GP intermediate rows) in global wave order, h stored
//     device-coherent (waves of other XCDs read it after the barrier);
//   - one grid barrier (every block resident: the grid never exceeds the occupancy limit);
//   - phase 1 loads all of an item's row chunks in one round (gu4_pass<1, 4>);
//   - phase 2: block b takes output tiles of 2 N4_DP rows b, b + G, ...; it stages the k
//     h rows once (device-coherent loads), its waves take the tile's rows of slots
//     wave, wave + 4, ... into LDS (inter <= 2048: one load round a slot, the next
//     slot's loads in flight), and the tile's outputs sum w[s] y_s in slot order
//     (moe_combine_kernel's fmaf order), so no y buffer or combine launch is needed.
constexpr int N4F_KMAX = 16;                 // expert slots of the one-launch step
constexpr size_t N4F_LDS_MAX = 64 * 1024;    // staged x or h rows

struct Fused4Args {
    const float* logits;
    const void* x;
    const uint64_t* all_recs;
    int E, k;
    Rec4 g;
    int32_t* ids;
    float* weights;
    void* out;
    float* h;  // [k, I]
    uint32_t* bar;
    uint32_t* status;  // the device's status word: 1 if the grid barrier's wait gave up
    uint32_t spin;     // polls before a wait gives up
#ifdef OOM_STAMPS
    uint64_t* stamps;  // phase timestamps (profiling build)
#endif
};

// Rows 0 .. rows - 1 of h (f32, width K) into LDS in stage4's lane order through
// device-coherent 16-byte loads, eight in flight per thread (one round for 10 rows of 640:
// each round costs a trip to the device's point of coherence); zeros past K. NT threads.
// Every load's value is stored, a load past the rows into one spare LDS slot: with a store
// under a branch the compiler moved each load into its branch, behind a wait for the one
// before (eight round trips instead of one).
template <int NT = 256>
__device__ __forceinline__ void stage_rows_dev(float4* xs4, const float* h, int K, int CH, int rows) {
    constexpr int R = 8;  // loads in flight per thread
    __shared__ float4 spare;
    const int span = CH * 1024, nvec = rows * span / 4;
    const __amdgpu_buffer_rsrc_t hr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(h), (short)0, rows * K * 4, BUF_FLAGS);
    for (int base = 0; base < nvec; base += NT * R) {
        uint4 v[R];
#pragma unroll
        for (int n = 0; n < R; n++) {
            const int i = base + (int)threadIdx.x + NT * n;
            const int t = i * 4 / span, kk = i * 4 - t * span;
            const auto q = __builtin_amdgcn_raw_buffer_load_b128(hr, i < nvec && kk < K ? (t * K + kk) * 4 : OOB, 0,
                                                                 BUF_SC1);
            v[n] = make_uint4(q[0], q[1], q[2], q[3]);
        }
#pragma unroll
        for (int n = 0; n < R; n++) {
            const int i = base + (int)threadIdx.x + NT * n;
            const int t = i * 4 / span, kk = i * 4 - t * span;
            const int c = kk >> 10, l = (kk & 1023) >> 5, j = kk & 31;
            float4* dst = i < nvec ? &xs4[((t * CH + c) * 8 + (j >> 2)) * 32 + l] : &spare;
            *dst = make_float4(__uint_as_float(v[n].x), __uint_as_float(v[n].y), __uint_as_float(v[n].z),
                               __uint_as_float(v[n].w));
        }
    }
}


// dn4_pass<1> in two halves for inter <= 2048 (one load round), so a wave's next slot
// loads while the current one is reduced: the loaded weights, scale bytes and scale_2 ...
struct Dn4W {
    uint4 wd[N4_DP][2];
    uint32_t bd[N4_DP][2][2];
    float s2;
};

__device__ __forceinline__ void dn4_load(Dn4W& w, const Rec4& g, __amdgpu_buffer_rsrc_t r, int r0, int lane) {
    const int H = g.H, I = g.I, CH = (I + 1023) >> 10, ig = I >> 4;
    const int half = lane >> 5, l = lane & 31;
#pragma unroll
    for (int p = 0; p < N4_DP; p++) {
        const int row = r0 + 2 * p + half;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int col = c * 1024 + 32 * l;
            const bool ok = row < H && c < CH && col < I;
            w.wd[p][c] = ld16(r, ok ? g.dw + row * (I >> 1) + (col >> 1) : OOB);
#pragma unroll
            for (int q = 0; q < 2; q++)
                w.bd[p][c][q] = ldb(r, ok && (col >> 4) + q < ig ? g.ds + row * ig + (col >> 4) + q : OOB);
        }
    }
    w.s2 = ldf(r, g.s2d);
}

// ... and dn4_pass<1>'s arithmetic on them against staged row 0 of xs4.
template <typename Put>
__device__ __forceinline__ void dn4_compute(const Dn4W& w, const float4* xs4, const Rec4& g, int r0, int lane,
                                            Put put) {
    const int H = g.H, I = g.I, CH = (I + 1023) >> 10, ig = I >> 4;
    const int half = lane >> 5, l = lane & 31;
    float acc[N4_DP];
#pragma unroll
    for (int p = 0; p < N4_DP; p++) acc[p] = 0.0f;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        if (c >= CH) break;
        const int col = c * 1024 + 32 * l;
#pragma unroll
        for (int p = 0; p < N4_DP; p++) {
            float sd[2];
#pragma unroll
            for (int q = 0; q < 2; q++) sd[q] = e4m3_byte(w.bd[p][c][q]) * ((col >> 4) + q < ig ? w.s2 : 0.0f);
            float f[32];
            e2m1x32(w.wd[p][c], f);
            float p0, p1;
            piece_dot(f, xs4, 0, CH, c, l, p0, p1);
            acc[p] = fmaf(p1, sd[1], fmaf(p0, sd[0], acc[p]));
        }
    }
    constexpr int GROUP = 32 / N4_DP;
    const float tot = wave_sum_multi<N4_DP, 16>(acc, lane);
    const int v = l / GROUP;
    if (l % GROUP == 0) {
        const int row = r0 + 2 * v + half;
        if (row < H) put(row, tot);
    }
}

template <int XDT, int EQ, int ODT>
__global__ void __launch_bounds__(256) moe_decode_nvfp4_1_kernel(Fused4Args a) {
    const uint32_t bbase = grid_barrier_base(a.bar);
    extern __shared__ float4 xs4[];
    __shared__ uint64_t recs_l[N4F_KMAX];
    __shared__ float w_l[N4F_KMAX];
    __shared__ uint64_t pk_keys[64];  // routing scratch (route_picks: 64 entries with 8 logits a lane)
    __shared__ int pk_ids[N4F_KMAX];
    __shared__ float pk_p[N4F_KMAX];
    __shared__ float ylds[N4F_KMAX][2 * N4_DP];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const Rec4& g = a.g;
    const int k = a.k, H = g.H, I = g.I;
    OOM_STAMP(a.stamps, N4_WAVES, 0);
    if (wave == 0) {
        // every expert's record address (lane l holds experts l + 64 q) loads beside the
        // logits, so no load waits on the picks
        uint64_t rr[EQ];
#pragma unroll
        for (int q = 0; q < EQ; q++) rr[q] = lane + 64 * q < a.E ? a.all_recs[lane + 64 * q] : 0ull;
        int id = 0;
        float w = 0.0f;
        route_picks<EQ>(a.logits, a.E, k, lane, pk_keys, pk_ids, pk_p, id, w);
        // pick `lane`'s record: register id / 64 of lane id % 64
        uint64_t rec = 0;
#pragma unroll
        for (int q = 0; q < EQ; q++) {
            const uint64_t v = (uint64_t)__shfl((long long)rr[q], id & 63, 64);
            if ((id >> 6) == q) rec = v;
        }
        OOM_STAMP_AFTER(a.stamps, N4_WAVES, 1, rec);  // routed (wave 0)
        if (lane < k) {
            recs_l[lane] = rec;
            w_l[lane] = w;
            if (blockIdx.x == 0) {
                a.ids[lane] = id;
                a.weights[lane] = w;
            }
        }
    }
    const int CHH = (H + 1023) >> 10, CHI = (I + 1023) >> 10;
    stage4<XDT>(xs4, a.x, H, CHH, 1, [](int) { return 0; });
    __syncthreads();
    OOM_STAMP(a.stamps, N4_WAVES, 2);  // x staged, the picks shared
    // ---- phase 1: h[s, j0 .. j0 + 2 N4_GP) per wave item ----
    const int ipe = (I + 2 * N4_GP - 1) / (2 * N4_GP), NG = k * ipe;
    const int NW = gridDim.x * N4_WAVES;
    for (int it = blockIdx.x * N4_WAVES + wave; it < NG; it += NW) {
        const int s = it / ipe, j0 = (it - s * ipe) * 2 * N4_GP;
        const __amdgpu_buffer_rsrc_t r = uniform_rsrc(recs_l[s], g.bytes);
        const float s2g = ldf(r, g.s2g), s2u = ldf(r, g.s2u);
        float* hs = a.h + (size_t)s * I;
        gu4_pass<1, 4>(xs4, g, r, s2g, s2u, j0, lane, 1, [&](int, int j, float v) { st_dev(hs + j, v); });
    }
    OOM_STAMP(a.stamps, N4_WAVES, 3);  // gate/up items done
    wait_mem();  // this wave's h stores are complete before its block arrives
    grid_barrier_words(a.bar, bbase, a.status, a.spin);
    OOM_STAMP(a.stamps, N4_WAVES, 4);  // the grid barrier released
    // ---- phase 2: the k h rows once, then per output tile the slot rows and the combine ----
    // slots wave, wave + 4, ...: the next slot's loads are in flight while the current one
    // is reduced (a slot past k loads through an empty resource: zeros, no access); the
    // first tile's first slot loads before h is staged, so the two loads' latencies overlap
    const int tiles = (H + 2 * N4_DP - 1) / (2 * N4_DP);
    const auto rsrc_of = [&](int s) { return uniform_rsrc(recs_l[s < k ? s : 0], s < k ? g.bytes : 0); };
    Dn4W wa, wb;
    if ((int)blockIdx.x < tiles) dn4_load(wa, g, rsrc_of(wave), (int)blockIdx.x * 2 * N4_DP, lane);
    stage_rows_dev(xs4, a.h, I, CHI, k);
    __syncthreads();
    OOM_STAMP(a.stamps, N4_WAVES, 5);  // h staged
    for (int tb = blockIdx.x; tb < tiles; tb += gridDim.x) {
        const int r0 = tb * 2 * N4_DP;
        if (tb != (int)blockIdx.x) dn4_load(wa, g, rsrc_of(wave), r0, lane);
        for (int s = wave; s < k;) {
            dn4_load(wb, g, rsrc_of(s + N4_WAVES), r0, lane);
            dn4_compute(wa, xs4 + (size_t)s * CHI * 256, g, r0, lane, [&](int row, float v) { ylds[s][row - r0] = v; });
            s += N4_WAVES;
            if (s >= k) break;
            dn4_load(wa, g, rsrc_of(s + N4_WAVES), r0, lane);
            dn4_compute(wb, xs4 + (size_t)s * CHI * 256, g, r0, lane, [&](int row, float v) { ylds[s][row - r0] = v; });
            s += N4_WAVES;
        }
        __syncthreads();
        const int row = r0 + (int)threadIdx.x;
        if (threadIdx.x < 2 * N4_DP && row < H) {
            float acc = 0.0f;
            for (int s = 0; s < k; s++) acc = fmaf(w_l[s], ylds[s][threadIdx.x], acc);
            store_out<ODT>(a.out, row, acc);
        }
        __syncthreads();
        if (tb == (int)blockIdx.x) OOM_STAMP(a.stamps, N4_WAVES, 6);  // first tile combined
    }
    OOM_STAMP(a.stamps, N4_WAVES, 7);
    grid_barrier_exit(a.bar);
}

// ---- one token in one launch, one block per CU -----------------------------------------------
// The step above for hidden <= 3072 and inter <= 1024 (the released geometry: 2560 / 640),
// with the same arithmetic and another schedule:
//   - blocks of 8 waves, one a CU; wave w of block b takes the items (slot, 2 N4_GP rows)
//     b + G (w + 8 n), so every block holds 6 or 7 of the step's 1600 items;
//   - block b's output tile is rows 10 b .. + 10 (2560 outputs over 256 blocks); its (slot,
//     row pair) units are u = w + 8 m of wave w, and the first N4P_UP of them load into
//     registers right behind the loads of the wave's first gate/up item (so the rows h
//     needs arrive first), so the down weights stream in phase 1 and after the barrier a
//     block only stages h;
//   - a unit's lane partial and the 32-lane butterfly are dn4_compute's, so the outputs equal
//     the staged launches' bit for bit. Units past N4P_UP (k > 11) and tiles past the grid
//     load after the barrier.
constexpr int N4P_WAVES = 8;  // waves per block
constexpr int N4P_DP = 5;     // row pairs of a block's output tile
constexpr int N4P_UP = 7;     // units a wave prefetches in phase 1 (k * N4P_DP <= 8 * 7 with k <= 11)

// A unit of a down tile (inter <= 1024: one 1024-column chunk): lane l of half `half` holds
// row r0 + 2 p + half's columns 32 (l % 32) .. + 32, their two scale bytes and the record's
// weight_scale_2.
struct Dn4U {
    uint4 wd;
    uint32_t bd[2];
    float s2;
};

// row2: the pair's first row (the same on every lane); the row's offsets are a scalar product
// plus the lane's part, so no vector multiply-add reads a register a load in flight will write.
__device__ __forceinline__ void dnu_load(Dn4U& w, const Rec4& g, __amdgpu_buffer_rsrc_t r, int row2, int lane) {
    const int I = g.I, ig = I >> 4, half = lane >> 5, col = 32 * (lane & 31);
    const bool ok = row2 + half < g.H && col < I;
    const int wrow = __builtin_amdgcn_readfirstlane(g.dw + row2 * (I >> 1)), srow = __builtin_amdgcn_readfirstlane(g.ds + row2 * ig);
    w.wd = ld16(r, ok ? wrow + half * (I >> 1) + (col >> 1) : OOB);
#pragma unroll
    for (int q = 0; q < 2; q++) w.bd[q] = ldb(r, ok && (col >> 4) + q < ig ? srow + half * ig + (col >> 4) + q : OOB);
    w.s2 = ldf(r, g.s2d);
}

// The unit's lane partial against the slot's staged h row (dn4_compute's per-lane sum for one chunk).
__device__ __forceinline__ float dnu_part(const Dn4U& w, const float4* hs4, int I, int lane) {
    const int ig = I >> 4, l = lane & 31, col = 32 * l;
    float sd[2];
#pragma unroll
    for (int q = 0; q < 2; q++) sd[q] = e4m3_byte(w.bd[q]) * ((col >> 4) + q < ig ? w.s2 : 0.0f);
    float f[32];
    e2m1x32(w.wd, f);
    float p0, p1;
    piece_dot(f, hs4, 0, 1, 0, l, p0, p1);
    return fmaf(p1, sd[1], fmaf(p0, sd[0], 0.0f));
}

template <int XDT, int EQ, int ODT>
__global__ void __launch_bounds__(64 * N4P_WAVES) moe_decode_nvfp4_1p_kernel(Fused4Args a) {
    const uint32_t bbase = grid_barrier_base(a.bar);
    extern __shared__ float4 xs4[];
    __shared__ uint64_t recs_l[N4F_KMAX];
    __shared__ float w_l[N4F_KMAX];
    __shared__ uint64_t pk_keys[64];  // routing scratch (route_picks: 64 entries with 8 logits a lane)
    __shared__ int pk_ids[N4F_KMAX];
    __shared__ float pk_p[N4F_KMAX];
    __shared__ float ylds[N4F_KMAX][2 * N4P_DP];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5, l = lane & 31;
    const Rec4& g = a.g;
    const int k = a.k, H = g.H, I = g.I;
    OOM_STAMP(a.stamps, N4P_WAVES, 0);
    OOM_STAMP_WHERE(a.stamps, N4P_WAVES);
    if (wave == 0) {
        // the record addresses (lane l holds experts l + 64 q) load beside the logits
        uint64_t rr[EQ];
#pragma unroll
        for (int q = 0; q < EQ; q++) rr[q] = lane + 64 * q < a.E ? a.all_recs[lane + 64 * q] : 0ull;
        int id = 0;
        float w = 0.0f;
        route_picks<EQ>(a.logits, a.E, k, lane, pk_keys, pk_ids, pk_p, id, w);
        uint64_t rec = 0;
#pragma unroll
        for (int q = 0; q < EQ; q++) {
            const uint64_t v = (uint64_t)__shfl((long long)rr[q], id & 63, 64);
            if ((id >> 6) == q) rec = v;
        }
        OOM_STAMP_AFTER(a.stamps, N4P_WAVES, 1, rec);  // routed (wave 0)
        if (lane < k) {
            recs_l[lane] = rec;
            w_l[lane] = w;
            if (blockIdx.x == 0) {
                a.ids[lane] = id;
                a.weights[lane] = w;
            }
        }
    }
    if (wave >= 4) stage4<XDT>(xs4, a.x, H, (H + 1023) >> 10, 1, [](int) { return 0; }, tid - 256);
    __syncthreads();
    OOM_STAMP(a.stamps, N4P_WAVES, 2);  // x staged, the picks shared
    const int G = gridDim.x, b = blockIdx.x;
    const int ipe = (I + 2 * N4_GP - 1) / (2 * N4_GP), NG = k * ipe;
    const int tiles = (H + 2 * N4P_DP - 1) / (2 * N4P_DP), NU = k * N4P_DP;
    // a slot past k loads through an empty resource: zeros, no memory access
    const auto rsrc_of = [&](int s) { return uniform_rsrc(recs_l[s < k ? s : 0], s < k ? g.bytes : 0); };
    Dn4U du[N4P_UP];
    const auto prefetch = [&]() {  // (one call)
#pragma unroll
        for (int m = 0; m < N4P_UP; m++) {
            const int u = wave + N4P_WAVES * m, s = u / N4P_DP, p = u - s * N4P_DP;
            const bool ok = b < tiles && u < NU;
            dnu_load(du[m], g, rsrc_of(ok ? s : k), b * 2 * N4P_DP + 2 * p, lane);
        }
    };
    // ---- phase 1: items b + G (wave + 8 n); the down prefetch goes out behind the first
    // item's loads, so the rows h needs arrive first. The first item is straight-line code
    // (its one round of loads, the prefetch, its math: CH <= 3 here), so the item's waits
    // leave the prefetch in flight ----
    int it = b + G * wave;
    if (it < NG) {
        const int s = it / ipe, j0 = (it - s * ipe) * 2 * N4_GP;
        const __amdgpu_buffer_rsrc_t r = uniform_rsrc(recs_l[s], g.bytes);
        const float s2g = ldf(r, g.s2g), s2u = ldf(r, g.s2u);
        float* hs = a.h + (size_t)s * I;
        float acc[2 * N4_GP];
#pragma unroll
        for (int i = 0; i < 2 * N4_GP; i++) acc[i] = 0.0f;
        {
            Gu4Ld<3> t;
            gu4_load<3>(g, r, j0, lane, 0, t);
            __builtin_amdgcn_sched_barrier(0);
            prefetch();
            __builtin_amdgcn_sched_barrier(0);
            gu4_math<1, 3>(xs4, g, s2g, s2u, lane, 0, t, acc);
        }
        for (int c0 = 3; c0 < (H + 1023) >> 10; c0 += 3) {  // hidden > 3072: not launched here
            Gu4Ld<3> t;
            gu4_load<3>(g, r, j0, lane, c0, t);
            gu4_math<1, 3>(xs4, g, s2g, s2u, lane, c0, t, acc);
        }
        gu4_put<1>(acc, I, j0, lane, 1, [&](int, int j, float v) { st_dev(hs + j, v); });
        for (it += G * N4P_WAVES; it < NG; it += G * N4P_WAVES) {
            const int s = it / ipe, j0 = (it - s * ipe) * 2 * N4_GP;
            const __amdgpu_buffer_rsrc_t r = uniform_rsrc(recs_l[s], g.bytes);
            const float s2g = ldf(r, g.s2g), s2u = ldf(r, g.s2u);
            float* hs = a.h + (size_t)s * I;
            gu4_pass<1, 3>(xs4, g, r, s2g, s2u, j0, lane, 1, [&](int, int j, float v) { st_dev(hs + j, v); });
        }
    } else {
        prefetch();
    }
    OOM_STAMP(a.stamps, N4P_WAVES, 3);  // gate/up items done, the down units loaded
    wait_mem();  // this wave's h stores are complete before its block arrives
    grid_barrier_words(a.bar, bbase, a.status, a.spin);
    OOM_STAMP(a.stamps, N4P_WAVES, 4);  // the grid barrier released
    // ---- phase 2: the k h rows once, the units' rows into LDS, the slot-order combine ----
    stage_rows_dev<64 * N4P_WAVES>(xs4, a.h, I, 1, k);
    __syncthreads();
    OOM_STAMP(a.stamps, N4P_WAVES, 5);  // h staged
    const auto put_unit = [&](int u, int r0, float tot) {
        const int s = u / N4P_DP, p = u - s * N4P_DP;
        if (r0 + 2 * p + half < H) ylds[s][2 * p + half] = tot;
    };
    const auto combine = [&](int r0) {
        const int row = r0 + tid;
        if (tid < 2 * N4P_DP && row < H) {
            float acc = 0.0f;
            for (int s = 0; s < k; s++) acc = fmaf(w_l[s], ylds[s][tid], acc);
            store_out<ODT>(a.out, row, acc);
        }
    };
    // units loaded after the barrier, one at a time
    const auto late_units = [&](int u0, int r0) {
        for (int u = u0; u < NU; u += N4P_WAVES) {
            const int s = u / N4P_DP, p = u - s * N4P_DP;
            Dn4U d;
            dnu_load(d, g, rsrc_of(s), r0 + 2 * p, lane);
            float v[1] = {dnu_part(d, xs4 + (size_t)s * 256, I, lane)};
            const float tot = wave_sum_multi<1, 16>(v, lane);
            if (l == 0) put_unit(u, r0, tot);
        }
    };
    if (b < tiles) {
        const int r0 = b * 2 * N4P_DP;
        constexpr int NV = 8;  // N4P_UP values (and one zero) in the butterfly
        static_assert(N4P_UP < NV, "one butterfly for the prefetched units");
        float v[NV];
#pragma unroll
        for (int m = 0; m < NV; m++) {
            const int u = wave + N4P_WAVES * m;
            v[m] = m < N4P_UP && u < NU ? dnu_part(du[m < N4P_UP ? m : 0], xs4 + (size_t)(u / N4P_DP) * 256, I, lane)
                                        : 0.0f;
        }
        const float tot = wave_sum_multi<NV, 16>(v, lane);
        const int m = l / (32 / NV), u = wave + N4P_WAVES * m;
        if (l % (32 / NV) == 0 && m < N4P_UP && u < NU) put_unit(u, r0, tot);
        late_units(wave + N4P_WAVES * N4P_UP, r0);
        __syncthreads();
        combine(r0);
        OOM_STAMP(a.stamps, N4P_WAVES, 6);  // the tile combined
    }
    // tiles past the grid: their units load after the barrier
    for (int tb = b + G; tb < tiles; tb += G) {
        __syncthreads();  // the last tile's combine has read ylds
        late_units(wave, tb * 2 * N4P_DP);
        __syncthreads();
        combine(tb * 2 * N4P_DP);
    }
    grid_barrier_exit(a.bar);
}

// LDS of the one-launch kernel: x staged for one token, then the k h rows.
static size_t fused4_lds(const OomNvfp4Record& g, int k) {
    return std::max(stage_lds(g.hidden), (size_t)k * cdiv(g.inter, 1024) * 1024 * sizeof(float));
}

static bool fused4_ok(int T, int E, int k, const OomNvfp4Record& g) {
    return T == 1 && E <= 512 && k <= N4F_KMAX && g.inter <= 2048 && fused4_lds(g, k) <= N4F_LDS_MAX &&
           (int64_t)k * g.inter * 4 < OOB;
}

// The one-block-per-CU kernel's limits (beyond fused4_ok's): three chunks of hidden, one of inter.
static bool fused4p_ok(int H, int I) { return H <= 3072 && I <= 1024; }

// P: the one-block-per-CU kernel (8 waves), else the 4-wave kernel.
template <bool P, int XDT, int EQ, int ODT>
static int launch_fused4_t(const Fused4Args& a, size_t lds, hipStream_t st) {
    static thread_local int cached_dev = -1, cached_blocks = 0;
    static thread_local size_t cached_lds = 0;
    const auto kernel = P ? moe_decode_nvfp4_1p_kernel<XDT, EQ, ODT> : moe_decode_nvfp4_1_kernel<XDT, EQ, ODT>;
    const int threads = P ? 64 * N4P_WAVES : 64 * N4_WAVES;
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != cached_dev || lds != cached_lds) {
        int cus = 0, per = 0;
        cached_blocks = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, lds) == hipSuccess)
            cached_blocks = cus * per;
        cached_dev = dev;
        cached_lds = lds;
    }
    if (cached_blocks <= 0) return fail(OOM_ERR_LAUNCH, "oom_moe_decode_nvfp4: occupancy query failed");
    // enough blocks for one item a wave or one output tile each, never more than fit
    const int64_t items = cdiv((int64_t)a.k * cdiv(a.g.I, 2 * N4_GP), P ? N4P_WAVES : N4_WAVES);
    const int64_t tiles = cdiv(a.g.H, P ? 2 * N4P_DP : 2 * N4_DP);
    const int blocks = (int)std::max<int64_t>(1, std::min<int64_t>(cached_blocks, std::max(items, tiles)));
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(threads), lds, st, a);
    return launched("oom_moe_decode_nvfp4");
}

template <bool P, int XDT, int EQ>
static int launch_fused4_o(const Fused4Args& a, int odt, size_t lds, hipStream_t st) {
    return odt == OOM_BF16 ? launch_fused4_t<P, XDT, EQ, OOM_BF16>(a, lds, st)
                           : launch_fused4_t<P, XDT, EQ, OOM_F32>(a, lds, st);
}

template <int XDT>
static int launch_fused4_e(const Fused4Args& a, int odt, size_t lds, hipStream_t st) {
    if (fused4p_ok(a.g.H, a.g.I))
        return a.E <= 256 ? launch_fused4_o<true, XDT, 4>(a, odt, lds, st) : launch_fused4_o<true, XDT, 8>(a, odt, lds, st);
    return a.E <= 256 ? launch_fused4_o<false, XDT, 4>(a, odt, lds, st) : launch_fused4_o<false, XDT, 8>(a, odt, lds, st);
}

static int launch_gate_up4(const uint64_t* recs, const int32_t* off, const int32_t* tok, int grid_e, const void* x,
                           int xdt, float* h, const OomNvfp4Record& geo, const int32_t* n_e_dev, hipStream_t st) {
    const Rec4 g = rec4_of(geo);
    const dim3 grid((unsigned)cdiv(geo.inter, N4_WAVES * 2 * N4_GP), (unsigned)grid_e);
    const size_t lds = stage_lds(geo.hidden);
    if (xdt == OOM_BF16)
        hipLaunchKernelGGL((moe_gate_up_nvfp4_kernel<OOM_BF16>), grid, dim3(256), lds, st, recs, off, tok, x, h, g,
                           n_e_dev);
    else
        hipLaunchKernelGGL((moe_gate_up_nvfp4_kernel<OOM_F32>), grid, dim3(256), lds, st, recs, off, tok, x, h, g,
                           n_e_dev);
    return launched("oom_moe_gate_up_nvfp4");
}

static int launch_down4(const uint64_t* recs, const int32_t* off, int grid_e, const float* h, float* y,
                        const OomNvfp4Record& geo, const int32_t* n_e_dev, hipStream_t st) {
    const Rec4 g = rec4_of(geo);
    const dim3 grid((unsigned)cdiv(geo.hidden, N4_WAVES * 2 * N4_DP), (unsigned)grid_e);
    hipLaunchKernelGGL(moe_down_nvfp4_kernel, grid, dim3(256), stage_lds(geo.inter), st, recs, off, h, y, g, n_e_dev);
    return launched("oom_moe_down_nvfp4");
}

// Workspace of oom_moe_decode_nvfp4: the decode workspace header (barrier words and
// status of the one-launch kernel) | plan | recs | h | y.
struct Decode4Ws {
    size_t plan, recs, h, y, total;
};

static size_t a256(size_t v) { return (v + 255) & ~size_t(255); }

static Decode4Ws decode4_ws(int T, int E, int k, const OomNvfp4Record& g) {
    Decode4Ws w;
    const size_t A = (size_t)T * k;
    w.plan = WS_HEADER;
    w.recs = w.plan + a256(PlanView::size(E, (int)A) * sizeof(int32_t));
    w.h = w.recs + a256(std::min<size_t>(E, A) * sizeof(uint64_t));
    w.y = w.h + a256(A * (size_t)g.inter * sizeof(float));
    w.total = w.y + a256(A * (size_t)g.hidden * sizeof(float));
    return w;
}

}  // namespace oom

extern "C" int oom_moe_gate_up_nvfp4(const uint64_t* recs, const int32_t* off, const int32_t* assign_tok,
                                     int n_experts, const void* x, int x_dtype, float* h, const OomNvfp4Record* geo,
                                     void* stream) {
    using namespace oom;
    if (int rc = check_geo4(geo, "oom_moe_gate_up_nvfp4")) return rc;
    OOM_REQUIRE(n_experts >= 0 && n_experts <= 65535, "oom_moe_gate_up_nvfp4: n_experts");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_moe_gate_up_nvfp4: x_dtype");
    if (n_experts == 0) return OOM_OK;
    OOM_REQUIRE(recs && off && assign_tok && x && h, "oom_moe_gate_up_nvfp4: null buffer");
    OOM_REQUIRE(aligned(x, 16), "oom_moe_gate_up_nvfp4: x must be 16-byte aligned");
    return launch_gate_up4(recs, off, assign_tok, n_experts, x, x_dtype, h, *geo, nullptr, as_stream(stream));
}

extern "C" int oom_moe_down_nvfp4(const uint64_t* recs, const int32_t* off, int n_experts, const float* h, float* y,
                                  const OomNvfp4Record* geo, void* stream) {
    using namespace oom;
    if (int rc = check_geo4(geo, "oom_moe_down_nvfp4")) return rc;
    OOM_REQUIRE(n_experts >= 0 && n_experts <= 65535, "oom_moe_down_nvfp4: n_experts");
    if (n_experts == 0) return OOM_OK;
    OOM_REQUIRE(recs && off && h && y, "oom_moe_down_nvfp4: null buffer");
    OOM_REQUIRE(aligned(h, 16), "oom_moe_down_nvfp4: h must be 16-byte aligned");
    return launch_down4(recs, off, n_experts, h, y, *geo, nullptr, as_stream(stream));
}

extern "C" size_t oom_moe_decode_nvfp4_workspace_size(int T, int E, int k, const OomNvfp4Record* geo) {
    if (!geo || T < 1 || E < 1 || k < 1) return 0;
    return oom::decode4_ws(T, E, k, *geo).total;
}

extern "C" int oom_moe_decode_nvfp4(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T,
                                    int E, int k, const OomNvfp4Record* geo, int32_t* ids, float* weights, void* out,
                                    int out_dtype, void* ws, size_t ws_bytes, void* stream) {
    using namespace oom;
    if (int rc = check_geo4(geo, "oom_moe_decode_nvfp4")) return rc;
    OOM_REQUIRE(T >= 1 && (int64_t)T * k <= (1 << 24), "oom_moe_decode_nvfp4: T must be >= 1 and T * k <= 2^24");
    OOM_REQUIRE(k >= 1 && k <= 32 && E >= k && E <= 8192, "oom_moe_decode_nvfp4: router top-k > 32 or experts > 8192");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_moe_decode_nvfp4: x_dtype");
    OOM_REQUIRE(out_dtype == OOM_F32 || out_dtype == OOM_BF16, "oom_moe_decode_nvfp4: out_dtype");
    OOM_REQUIRE(logits && x && all_recs && ids && weights && out, "oom_moe_decode_nvfp4: null buffer");
    OOM_REQUIRE(aligned(x, 16), "oom_moe_decode_nvfp4: x must be 16-byte aligned");
    const Decode4Ws w = decode4_ws(T, E, k, *geo);
    if (!ws || ws_bytes < w.total)
        return fail(OOM_ERR_WORKSPACE,
                    "oom_moe_decode_nvfp4: workspace smaller than oom_moe_decode_nvfp4_workspace_size()");
    OOM_REQUIRE(aligned(ws, 256), "oom_moe_decode_nvfp4: workspace must be 256-byte aligned");
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    int32_t* plan = reinterpret_cast<int32_t*>(base + w.plan);
    uint64_t* recs = reinterpret_cast<uint64_t*>(base + w.recs);
    float* h = reinterpret_cast<float*>(base + w.h);
    float* y = reinterpret_cast<float*>(base + w.y);
    hipStream_t st = as_stream(stream);
    if (fused4_ok(T, E, k, *geo)) {
        uint32_t* status = status_word();
        if (!status) return fail(OOM_ERR_LAUNCH, "oom_moe_decode_nvfp4: the device status word has no address");
        Fused4Args a{logits, x, all_recs, E, k, rec4_of(*geo), ids, weights, out, h,
                     reinterpret_cast<uint32_t*>(base + WS_BAR), status, wait_limit()};
#ifdef OOM_STAMPS
        a.stamps = stamps_buffer();
#endif
        const size_t lds = fused4_lds(*geo, k);
        return x_dtype == OOM_BF16 ? launch_fused4_e<OOM_BF16>(a, out_dtype, lds, st)
                                   : launch_fused4_e<OOM_F32>(a, out_dtype, lds, st);
    }
    const int A = T * k;
    const PlanView pv{plan, E, A};
    if (int rc = oom_router_topk(logits, ids, weights, T, E, k, stream)) return rc;
    if (int rc = oom_moe_plan(ids, T, E, k, all_recs, plan, recs, stream)) return rc;
    const int grid_e = std::min(E, A);
    if (int rc = launch_gate_up4(recs, pv.off(), pv.assign_tok(), grid_e, x, x_dtype, h, *geo, pv.n_e(), st)) return rc;
    if (int rc = launch_down4(recs, pv.off(), grid_e, h, y, *geo, pv.n_e(), st)) return rc;
    return launch_combine(y, pv.slot_assign(), weights, out, out_dtype, T, (int)geo->hidden, k, st);
}
