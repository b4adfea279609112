// Routed experts over bf16 records read in place (the `bf16` layout tag, weights as
// released: gate.weight and up.weight bf16 [inter, hidden], down.weight bf16 [hidden, inter],
// row-major; OomBf16Record holds the parts' byte offsets).
//
// gate/up + SwiGLU: a block is 4 waves of one expert, a wave one intermediate row j: its
// gate row and its up row stream with every 128-bit load in flight at once (lane l holds
// columns 512 c + 8 l .. + 8 of chunk c: 8 weights a load), and each of the expert's
// tokens meets them in registers: the token's activations load in the same lane layout
// (from L2 after the first wave), each bf16 weight widens to fp32 exactly (a 16-bit shift)
// and the lane's partial sums reduce in one butterfly. down: the same over the expert's
// h rows, a wave MB_DR output rows. No LDS: a token costs a wave one 8 or 16 KiB read of
// L2 and its multiply-adds. fp32 products and accumulation throughout.
// Semantics of crates/oominf-cuda/kernels/moe.cu:343-443 (moe_gate_up_bf16 and
// moe_down_bf16: expert e owns assignments [off[e], off[e+1]), its record at recs[e]);
// only the summation order differs.
#include <algorithm>

#include "stream.hpp"

namespace oom {

constexpr int MB_WAVES = 4;    // waves a block
constexpr int MB_DR = 4;       // down rows a wave
constexpr int MB_MAXW = 4096;  // widths (hidden, inter): at most 8 chunks of 512 a lane row

// Eight activations of a row (columns col .. col + 8): their loads (one 16-byte load of
// bf16, two of f32; zeros when !ok) ...
template <int DT>
__device__ __forceinline__ void mb_act8_load(__amdgpu_buffer_rsrc_t r, int col, bool ok, uint4 (&w)[DT == OOM_BF16 ? 1 : 2]) {
    if constexpr (DT == OOM_BF16) {
        w[0] = ld16(r, ok ? col * 2 : OOB);
    } else {
        w[0] = ld16(r, ok ? col * 4 : OOB);
        w[1] = ld16(r, ok ? col * 4 + 16 : OOB);
    }
}

// ... and their eight values as fp32.
template <int DT>
__device__ __forceinline__ void mb_act8_cvt(const uint4 (&w)[DT == OOM_BF16 ? 1 : 2], float (&v)[8]) {
    if constexpr (DT == OOM_BF16) {
        const uint32_t ww[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v[2 * q] = __uint_as_float(ww[q] << 16);
            v[2 * q + 1] = __uint_as_float(ww[q] & 0xffff0000u);
        }
    } else {
        const uint32_t ww[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] = __uint_as_float(ww[q]);
    }
}

// An assignment's activations (or h) for every chunk of a lane row, all loads in flight
// before the first use (loaded chunk by chunk, the compiler put a wait for each chunk's
// loads before the next chunk's went out).
template <int DT, int CH>
__device__ __forceinline__ void mb_act_row(__amdgpu_buffer_rsrc_t r, int width, int lane,
                                           uint4 (&w)[CH][DT == OOM_BF16 ? 1 : 2]) {
#pragma unroll
    for (int c = 0; c < CH; c++) mb_act8_load<DT>(r, c * 512 + lane * 8, c * 512 + lane * 8 < width, w[c]);
#pragma unroll
    for (int c = 0; c < CH; c++)
#pragma unroll
        for (int q = 0; q < (DT == OOM_BF16 ? 1 : 2); q++)
            asm volatile("" : "+v"(w[c][q].x), "+v"(w[c][q].y), "+v"(w[c][q].z), "+v"(w[c][q].w));
}

// Eight bf16 weights (one 16-byte load) times eight activations, into acc.
__device__ __forceinline__ float mb_dot8(const uint4& w, const float (&x)[8], float acc) {
    acc = fmaf(__uint_as_float(w.x << 16), x[0], acc);
    acc = fmaf(__uint_as_float(w.x & 0xffff0000u), x[1], acc);
    acc = fmaf(__uint_as_float(w.y << 16), x[2], acc);
    acc = fmaf(__uint_as_float(w.y & 0xffff0000u), x[3], acc);
    acc = fmaf(__uint_as_float(w.z << 16), x[4], acc);
    acc = fmaf(__uint_as_float(w.z & 0xffff0000u), x[5], acc);
    acc = fmaf(__uint_as_float(w.w << 16), x[6], acc);
    acc = fmaf(__uint_as_float(w.w & 0xffff0000u), x[7], acc);
    return acc;
}

// h[a, j] = silu(x . gate row j) * (x . up row j) for the expert's assignments; CH chunks of
// 512 columns a row.
template <int XDT, int CH>
__global__ void __launch_bounds__(64 * MB_WAVES) moe_gate_up_bf16_kernel(const uint64_t* __restrict__ recs,
                                                                         const int32_t* __restrict__ off,
                                                                         const int32_t* __restrict__ assign_tok,
                                                                         const void* __restrict__ x,
                                                                         float* __restrict__ h, OomBf16Record g,
                                                                         int rec_bytes) {
    constexpr int ES = XDT == OOM_BF16 ? 2 : 4;
    const int e = blockIdx.y, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = (int)g.hidden, I = (int)g.inter;
    const int j = blockIdx.x * MB_WAVES + wave;
    const int a_begin = off[e], a_end = off[e + 1];
    const __amdgpu_buffer_rsrc_t r = uniform_rsrc(recs[e], j < I && a_begin < a_end ? rec_bytes : 0);
    uint4 wg[CH], wu[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int col = c * 512 + lane * 8;
        const bool ok = col < H;
        wg[c] = ld16nt(r, ok ? (int)(g.gate_weight + ((int64_t)j * H + col) * 2) : OOB);
        wu[c] = ld16nt(r, ok ? (int)(g.up_weight + ((int64_t)j * H + col) * 2) : OOB);
    }
    for (int a = a_begin; a < a_end; a++) {
        const int t = assign_tok[a];
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(reinterpret_cast<const uint8_t*>(x) + (size_t)t * H * ES), (short)0, H * ES, BUF_FLAGS);
        float acc[2] = {0.0f, 0.0f};
        uint4 xw[CH][XDT == OOM_BF16 ? 1 : 2];
        mb_act_row<XDT, CH>(xr, H, lane, xw);
#pragma unroll
        for (int c = 0; c < CH; c++) {
            float xv[8];
            mb_act8_cvt<XDT>(xw[c], xv);
            acc[0] = mb_dot8(wg[c], xv, acc[0]);
            acc[1] = mb_dot8(wu[c], xv, acc[1]);
        }
        // gate total in lanes 0..31, up total in lanes 32..63
        const float tot = wave_sum_multi<2>(acc, lane);
        const float up = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot), 32));
        if (lane == 0 && j < I) h[(size_t)a * I + j] = siluf(tot) * up;
    }
}

// y[a, r] = h[a] . down row r for the expert's assignments; CH chunks of 512 columns a row.
template <int CH>
__global__ void __launch_bounds__(64 * MB_WAVES) moe_down_bf16_kernel(const uint64_t* __restrict__ recs,
                                                                      const int32_t* __restrict__ off,
                                                                      const float* __restrict__ h,
                                                                      float* __restrict__ y, OomBf16Record g,
                                                                      int rec_bytes) {
    const int e = blockIdx.y, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int H = (int)g.hidden, I = (int)g.inter;
    const int r0 = (blockIdx.x * MB_WAVES + wave) * MB_DR;
    const int a_begin = off[e], a_end = off[e + 1];
    const __amdgpu_buffer_rsrc_t r = uniform_rsrc(recs[e], a_begin < a_end ? rec_bytes : 0);
    uint4 wd[MB_DR][CH];
#pragma unroll
    for (int q = 0; q < MB_DR; q++)
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int col = c * 512 + lane * 8, row = r0 + q;
            wd[q][c] = ld16nt(r, row < H && col < I ? (int)(g.down_weight + ((int64_t)row * I + col) * 2) : OOB);
        }
    for (int a = a_begin; a < a_end; a++) {
        const __amdgpu_buffer_rsrc_t hr =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(h + (size_t)a * I), (short)0, I * 4, BUF_FLAGS);
        float acc[MB_DR];
#pragma unroll
        for (int q = 0; q < MB_DR; q++) acc[q] = 0.0f;
        uint4 hw[CH][2];
        mb_act_row<OOM_F32, CH>(hr, I, lane, hw);
#pragma unroll
        for (int c = 0; c < CH; c++) {
            float hv[8];
            mb_act8_cvt<OOM_F32>(hw[c], hv);
#pragma unroll
            for (int q = 0; q < MB_DR; q++) acc[q] = mb_dot8(wd[q][c], hv, acc[q]);
        }
        // row q's total in lane group q of 16 lanes
        const float tot = wave_sum_multi<MB_DR>(acc, lane);
        const int row = r0 + (lane >> 4);
        if ((lane & 15) == 0 && row < H) y[(size_t)a * H + row] = tot;
    }
}

// Bytes of a bf16 record up to the end of its last part.
static int64_t bf16_span(const OomBf16Record& g) {
    const int64_t m = g.hidden * g.inter * 2;
    return std::max({g.gate_weight + m, g.up_weight + m, g.down_weight + m});
}

static int check_bf16_geo(const OomBf16Record* geo, const char* who) {
    if (!geo) return fail(OOM_ERR_ARG, std::string(who) + ": null geometry");
    const OomBf16Record& g = *geo;
    const bool ok = g.hidden >= 8 && g.inter >= 8 && g.hidden % 8 == 0 && g.inter % 8 == 0 && g.hidden <= MB_MAXW &&
                    g.inter <= MB_MAXW && g.gate_weight >= 0 && g.up_weight >= 0 && g.down_weight >= 0 &&
                    g.gate_weight % 16 == 0 && g.up_weight % 16 == 0 && g.down_weight % 16 == 0 &&
                    bf16_span(g) < OOB;
    if (!ok)
        return fail(OOM_ERR_ARG, std::string(who) +
                                     ": widths must be multiples of 8 up to 4096 and weight parts 16-byte aligned "
                                     "(buffer too small or shape unsupported)");
    return OOM_OK;
}

template <int XDT>
static void launch_gu_bf16(int ch, dim3 grid, hipStream_t st, const uint64_t* recs, const int32_t* off,
                           const int32_t* tok, const void* x, float* h, const OomBf16Record& g, int rb) {
#define MB_GU(C)                                                                                                  \
    case C:                                                                                                       \
        hipLaunchKernelGGL((moe_gate_up_bf16_kernel<XDT, C>), grid, dim3(64 * MB_WAVES), 0, st, recs, off, tok, x, h, \
                           g, rb);                                                                                \
        break;
    switch (ch) { MB_GU(1) MB_GU(2) MB_GU(3) MB_GU(4) MB_GU(5) MB_GU(6) MB_GU(7) default: MB_GU(8) }
#undef MB_GU
}

}  // namespace oom

extern "C" int oom_moe_gate_up_bf16(const uint64_t* recs, const int32_t* off, const int32_t* assign_tok,
                                    int n_experts, const void* x, int x_dtype, float* h, const OomBf16Record* geo,
                                    void* stream) {
    using namespace oom;
    if (int rc = check_bf16_geo(geo, "oom_moe_gate_up_bf16")) return rc;
    OOM_REQUIRE(n_experts >= 0 && n_experts <= 65535, "oom_moe_gate_up_bf16: n_experts");
    OOM_REQUIRE(x_dtype == OOM_F32 || x_dtype == OOM_BF16, "oom_moe_gate_up_bf16: x_dtype");
    if (n_experts == 0) return OOM_OK;
    OOM_REQUIRE(recs && off && assign_tok && x && h, "oom_moe_gate_up_bf16: null buffer");
    const int ch = (int)cdiv(geo->hidden, 512);
    const dim3 grid((unsigned)cdiv(geo->inter, MB_WAVES), (unsigned)n_experts);
    const int rb = (int)bf16_span(*geo);
    hipStream_t st = as_stream(stream);
    if (x_dtype == OOM_BF16) launch_gu_bf16<OOM_BF16>(ch, grid, st, recs, off, assign_tok, x, h, *geo, rb);
    else launch_gu_bf16<OOM_F32>(ch, grid, st, recs, off, assign_tok, x, h, *geo, rb);
    return launched("oom_moe_gate_up_bf16");
}

extern "C" int oom_moe_down_bf16(const uint64_t* recs, const int32_t* off, int n_experts, const float* h, float* y,
                                 const OomBf16Record* geo, void* stream) {
    using namespace oom;
    if (int rc = check_bf16_geo(geo, "oom_moe_down_bf16")) return rc;
    OOM_REQUIRE(n_experts >= 0 && n_experts <= 65535, "oom_moe_down_bf16: n_experts");
    if (n_experts == 0) return OOM_OK;
    OOM_REQUIRE(recs && off && h && y, "oom_moe_down_bf16: null buffer");
    const int ch = (int)cdiv(geo->inter, 512);
    const dim3 grid((unsigned)cdiv(geo->hidden, MB_WAVES * MB_DR), (unsigned)n_experts);
    const int rb = (int)bf16_span(*geo);
    hipStream_t st = as_stream(stream);
#define MB_DN(C)                                                                                                 \
    case C:                                                                                                      \
        hipLaunchKernelGGL((moe_down_bf16_kernel<C>), grid, dim3(64 * MB_WAVES), 0, st, recs, off, h, y, *geo, rb); \
        break;
    switch (ch) { MB_DN(1) MB_DN(2) MB_DN(3) MB_DN(4) MB_DN(5) MB_DN(6) MB_DN(7) default: MB_DN(8) }
#undef MB_DN
    return launched("oom_moe_down_bf16");
}
