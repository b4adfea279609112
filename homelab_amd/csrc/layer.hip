// A whole decode MoE layer as one call, with no host synchronisation: the router GEMV over
// bf16 weights, the routed experts (the one-launch decode step), the shared expert and its
// sigmoid gate, and the combine out = routed + sigmoid(gate_logit) * shared: the device
// half of Moe::forward (crates/oominf-models-qwen/src/moe.rs:254-366) with every routed
// expert resident, and Moe::shared (moe.rs:498-527).
//
// One token with bf16 activations and a shared expert of the routed geometry takes two
// launches: the router GEMV, then the one-token decode kernel with the shared expert as one
// more plan slot (its gate/up rows beside the routed ones, one row pair of each down tile
// per wave) and the gate logit and gated add inside it. A batch of 2..16 such tokens takes
// two as well: the router GEMV, then the batch kernel with the shared expert as one more
// plan entry holding every token, the gate logits and the gated add inside it.
//
// Otherwise the shared expert is an FP8 record of the routed experts' format (gate, up, down
// with 128 x 128 block scales, hidden x shared_inter). It runs through the same one-launch decode
// step as a single expert with top-1 routing: softmax over one logit is exactly 1, so the
// step computes down(silu(x Wg^T) * (x Wu^T)) with weight 1, which is the reference's
// gemm_w(gate_up) -> silu_mul_rows -> gemm_w(down) (moe.rs:507-513) in the same fp32
// arithmetic, summed in another order.
#include <algorithm>

#include "common.hpp"

extern "C" int oom_moe_decode_fp8(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T,
                                  int E, int k, const OomFp8Record* geo, int32_t* ids, float* weights, void* out,
                                  int out_dtype, void* ws, size_t ws_bytes, void* stream);
extern "C" size_t oom_moe_decode_fp8_workspace_size(int T, int E, int k, const OomFp8Record* geo);
extern "C" int oom_gemv_bf16(const void* x, int x_dtype, const uint16_t* w, void* y, int y_dtype, int T, int64_t N,
                             int64_t K, void* ws, size_t ws_bytes, void* stream);
extern "C" size_t oom_gemv_bf16_workspace_size(int T, int64_t N, int64_t K);

namespace oom {
int check_geo(const OomFp8Record* g, const char* who);
bool fused_shared_supported(int T, int E, int k, const OomFp8Record& g, const OomFp8Record& sg, int xdt);
int launch_fused_shared(const float* logits, const void* x, const uint64_t* all_recs, int E, int k,
                        const OomFp8Record& g, const uint64_t* shared_rec, const uint16_t* gate_w, float* gate,
                        int32_t* ids, float* weights, void* out, int odt, void* ws, hipStream_t st);
bool batch_shared_supported(int T, int E, int k, const OomFp8Record& g, const OomFp8Record& sg, int xdt,
                            const void* x);
size_t batch_shared_workspace_size(int T, int k, const OomFp8Record& g);
int launch_batch_shared(const float* logits, const void* x, const uint64_t* all_recs, int T, int E, int k,
                        const OomFp8Record& g, const uint64_t* shared_rec, const uint16_t* gate_w, int32_t* ids,
                        float* weights, void* out, int odt, void* ws, hipStream_t st);

// out[t, c] = routed[t, c] + sigmoid(gate[t]) * shared[t, c], sigmoid(v) = 1 / (1 + e^-v)
// (crates/oominf-cuda/kernels/ops.cu:10,310-316). Four columns per thread.
template <int ODT>
__global__ void __launch_bounds__(256) moe_combine_shared_kernel(const float* __restrict__ routed,
                                                                 const float* __restrict__ shared,
                                                                 const float* __restrict__ gate, void* out, int T,
                                                                 int H) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= (int64_t)T * H) return;
    const int t = (int)(i / H);
    const float sg = 1.0f / (1.0f + expf(-gate[t]));
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (i + e < (int64_t)T * H) store_out<ODT>(out, i + e, routed[i + e] + sg * shared[i + e]);
}

static int launch_combine_shared(const float* routed, const float* shared, const float* gate, void* out, int odt,
                                 int T, int H, hipStream_t st) {
    const int64_t n4 = cdiv((int64_t)T * H, 4);
    const dim3 grid((unsigned)cdiv(n4, 256));
    if (odt == OOM_BF16)
        hipLaunchKernelGGL(moe_combine_shared_kernel<OOM_BF16>, grid, dim3(256), 0, st, routed, shared, gate, out, T, H);
    else
        hipLaunchKernelGGL(moe_combine_shared_kernel<OOM_F32>, grid, dim3(256), 0, st, routed, shared, gate, out, T, H);
    return launched("oom_moe_combine_shared");
}

// Workspace of oom_moe_layer_decode_fp8: the router GEMV's region | the gate GEMV's region |
// the decode steps' region (their state header at its start) | logits | gate | routed |
// shared | shared ids and weights. The first three sit at offsets that depend on E, k and
// the geometries but not on T, so calls of any T up to the workspace's share one: each
// GEMV keeps its tickets and each decode step its header where every call looks, and the
// rest is written before it is read.
struct LayerWs {
    size_t rgemv, ggemv, decode, logits, gate, routed, shared, sids, sw, total;
};

static size_t l_al256(size_t v) { return (v + 255) & ~size_t(255); }

// The GEMV workspace of N rows over the hidden width at the largest T bucket it can take.
static size_t gemv_region(int64_t N, int64_t H) {
    size_t b = 0;
    for (int t = 1; t <= 16; t *= 2) b = std::max(b, oom_gemv_bf16_workspace_size(t, N, H));
    return l_al256(b);
}

static LayerWs layer_ws(int T, int E, int k, const OomFp8Record* geo, const OomFp8Record* sgeo) {
    LayerWs w;
    const size_t H = (size_t)geo->hidden;
    w.rgemv = 0;
    w.ggemv = gemv_region(E, (int64_t)H);
    w.decode = w.ggemv + gemv_region(1, (int64_t)H);
    const size_t dec = std::max({oom_moe_decode_fp8_workspace_size(T, E, k, geo),
                                 oom_moe_decode_fp8_workspace_size(T, 1, 1, sgeo),
                                 batch_shared_workspace_size(T, k, *geo)});
    w.logits = w.decode + l_al256(dec);
    w.gate = w.logits + l_al256((size_t)T * E * sizeof(float));
    w.routed = w.gate + l_al256((size_t)T * sizeof(float));
    w.shared = w.routed + l_al256((size_t)T * H * sizeof(float));
    w.sids = w.shared + l_al256((size_t)T * H * sizeof(float));
    w.sw = w.sids + l_al256((size_t)T * sizeof(int32_t));
    w.total = w.sw + l_al256((size_t)T * sizeof(float));
    return w;
}

}  // namespace oom

extern "C" int oom_moe_combine_shared(const float* routed, const float* shared, const float* gate_logit, void* out,
                                      int out_dtype, int T, int H, void* stream) {
    using namespace oom;
    OOM_REQUIRE(T >= 0 && H >= 1, "oom_moe_combine_shared: shape");
    OOM_REQUIRE(out_dtype == OOM_F32 || out_dtype == OOM_BF16, "oom_moe_combine_shared: out_dtype");
    if (T == 0) return OOM_OK;
    OOM_REQUIRE(routed && shared && gate_logit && out, "oom_moe_combine_shared: null buffer");
    return launch_combine_shared(routed, shared, gate_logit, out, out_dtype, T, H, as_stream(stream));
}

extern "C" size_t oom_moe_layer_decode_fp8_workspace_size(int T, int E, int k, const OomFp8Record* geo,
                                                          const OomFp8Record* shared_geo) {
    if (!geo || !shared_geo || T < 1 || E < 1 || k < 1) return 0;
    return oom::layer_ws(T, E, k, geo, shared_geo).total;
}

extern "C" int oom_moe_layer_decode_fp8(const void* x, int x_dtype, const uint16_t* router_w, const uint64_t* all_recs,
                                        int T, int E, int k, const OomFp8Record* geo, const uint64_t* shared_rec,
                                        const OomFp8Record* shared_geo, const uint16_t* shared_gate_w, int32_t* ids,
                                        float* weights, void* out, int out_dtype, void* ws, size_t ws_bytes,
                                        void* stream) {
    using namespace oom;
    if (int rc = check_geo(geo, "oom_moe_layer_decode_fp8")) return rc;
    if (int rc = check_geo(shared_geo, "oom_moe_layer_decode_fp8")) return rc;
    OOM_REQUIRE(shared_geo->hidden == geo->hidden, "oom_moe_layer_decode_fp8: the shared expert's hidden differs");
    OOM_REQUIRE(T >= 1 && T <= 16, "oom_moe_layer_decode_fp8: T must be 1..16 (a decode step)");
    OOM_REQUIRE(geo->hidden % 16 == 0, "oom_moe_layer_decode_fp8: hidden must be a multiple of 16");
    OOM_REQUIRE(x && router_w && all_recs && shared_rec && shared_gate_w && ids && weights && out,
                "oom_moe_layer_decode_fp8: null buffer");
    OOM_REQUIRE(aligned(router_w, 16) && aligned(shared_gate_w, 16),
                "oom_moe_layer_decode_fp8: router and gate weights must be 16-byte aligned");
    OOM_REQUIRE(out_dtype == OOM_F32 || out_dtype == OOM_BF16, "oom_moe_layer_decode_fp8: out_dtype");
    const LayerWs w = layer_ws(T, E, k, geo, shared_geo);
    if (!ws || ws_bytes < w.total)
        return fail(OOM_ERR_WORKSPACE,
                    "oom_moe_layer_decode_fp8: workspace smaller than oom_moe_layer_decode_fp8_workspace_size()");
    OOM_REQUIRE(aligned(ws, 256), "oom_moe_layer_decode_fp8: workspace must be 256-byte aligned");
    uint8_t* base = reinterpret_cast<uint8_t*>(ws);
    float* logits = reinterpret_cast<float*>(base + w.logits);
    float* gate = reinterpret_cast<float*>(base + w.gate);
    float* routed = reinterpret_cast<float*>(base + w.routed);
    float* shared = reinterpret_cast<float*>(base + w.shared);
    int32_t* sids = reinterpret_cast<int32_t*>(base + w.sids);
    float* sw = reinterpret_cast<float*>(base + w.sw);
    void* dws = base + w.decode;
    const size_t dws_bytes = w.logits - w.decode;
    const int64_t H = geo->hidden;
    // router logits [T, E] and the shared expert's gate logit [T] (Moe::forward's gemm_w of
    // the router, moe.rs:290-298; Moe::shared's gate, moe.rs:515-524)
    OOM_REQUIRE(k >= 1 && k <= 32 && E >= k && E <= 8192, "oom_moe_layer_decode_fp8: router top-k > 32 or experts > 8192");
    if (int rc = oom_gemv_bf16(x, x_dtype, router_w, logits, OOM_F32, T, E, H, base + w.rgemv, w.ggemv - w.rgemv,
                               stream))
        return rc;
    if (fused_shared_supported(T, E, k, *geo, *shared_geo, x_dtype))
        return launch_fused_shared(logits, x, all_recs, E, k, *geo, shared_rec, shared_gate_w, gate, ids, weights, out,
                                   out_dtype, dws, as_stream(stream));
    if (batch_shared_supported(T, E, k, *geo, *shared_geo, x_dtype, x))
        return launch_batch_shared(logits, x, all_recs, T, E, k, *geo, shared_rec, shared_gate_w, ids, weights, out,
                                   out_dtype, dws, as_stream(stream));
    if (int rc = oom_gemv_bf16(x, x_dtype, shared_gate_w, gate, OOM_F32, T, 1, H, base + w.ggemv, w.decode - w.ggemv,
                               stream))
        return rc;
    // the routed experts, then the shared expert as one expert with top-1 routing (any
    // finite logit routes to it with weight 1: the gate logits serve)
    if (int rc = oom_moe_decode_fp8(logits, x, x_dtype, all_recs, T, E, k, geo, ids, weights, routed, OOM_F32, dws,
                                    dws_bytes, stream))
        return rc;
    if (int rc = oom_moe_decode_fp8(gate, x, x_dtype, shared_rec, T, 1, 1, shared_geo, sids, sw, shared, OOM_F32, dws,
                                    dws_bytes, stream))
        return rc;
    return launch_combine_shared(routed, shared, gate, out, out_dtype, T, (int)H, as_stream(stream));
}
