/*
 * oom_hip.h -- C ABI of the MI355X (gfx950) decode hot path of oom-inference.
 *
 * These entry points are what an `oominf-rocm` backend crate binds to implement
 * the reference's operation traits (crates/oominf-core/src/backend.rs:1020-1049)
 * on ROCm. Every call:
 *   - takes device pointers, sizes and a HIP stream (`stream`, a hipStream_t;
 *     NULL is the null stream) and enqueues work on that stream in order;
 *   - returns OOM_OK (0) or a negative OOM_ERR_*; the message of the last failure
 *     on the calling thread is oom_last_error() (as the reference's
 *     "...: buffer too small or shape unsupported", crates/oominf-cuda/src/lib.rs:157-160);
 *   - allocates nothing: scratch comes from a caller workspace whose size the
 *     matching *_workspace_size() returns. A workspace must be zero-filled once
 *     before its first use (oom_workspace_init); calls leave it ready for the next
 *     call of the same entry point (any T up to the size it was made for; for the
 *     GEMVs, the same N: their split tickets sit in an area sized by N). Calls
 *     sharing one workspace must be ordered (one stream).
 *   - is deterministic: the same inputs give the same bits.
 * Activations are fp32 or bf16 (OOM_F32 / OOM_BF16); accumulation is fp32.
 */
#ifndef OOM_HIP_H
#define OOM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OOM_OK 0
#define OOM_ERR_ARG (-1)       /* shape unsupported, null pointer, misaligned buffer */
#define OOM_ERR_WORKSPACE (-2) /* workspace smaller than *_workspace_size() */
#define OOM_ERR_LAUNCH (-3)    /* the HIP runtime refused a launch */
#define OOM_ERR_KERNEL (-4)    /* a bounded wait inside an earlier kernel gave up (oom_status) */

/* Element types of activations and outputs. */
#define OOM_F32 0
#define OOM_BF16 1

/* Scale layouts of e4m3 weights [n, k] (w = e4m3(q) * scale):
 *   OOM_SCALE_ROW      scale[r]                              one per output row
 *   OOM_SCALE_1X128    scale[r * ceil(k/128) + c/128]        the reference's Weight::Fp8
 *                                                            (crates/oominf-core/src/backend.rs:163-167)
 *   OOM_SCALE_128X128  scale[(r/128) * ceil(k/128) + c/128]  128 x 128 blocks */
#define OOM_SCALE_ROW 0
#define OOM_SCALE_1X128 1
#define OOM_SCALE_128X128 2

/* Byte layout of an FP8 expert record (layout tag "fp8-e4m3-b128"): byte offsets of
 * each part from the record start, every part 256-byte aligned (the reference's
 * PART_ALIGN, docs/dev/format.md:37-39). gate and up weights are e4m3 [inter,
 * hidden], down e4m3 [hidden, inter], all row-major; each scale part is fp32 in
 * the OOM_SCALE_128X128 layout of its weight. The FP8 counterpart of
 * Nvfp4Record (crates/oominf-core/src/backend.rs:780-796). */
typedef struct OomFp8Record {
    int64_t hidden;
    int64_t inter;
    int64_t gate_weight;
    int64_t gate_scale;
    int64_t up_weight;
    int64_t up_scale;
    int64_t down_weight;
    int64_t down_scale;
} OomFp8Record;

/* Byte layout of a bf16 expert record (layout tag "bf16", docs/dev/format.md:72-73:
 * unquantised weights as released): byte offsets of gate.weight and up.weight (bf16
 * [inter, hidden]) and down.weight (bf16 [hidden, inter]), row-major, each 16-byte
 * aligned. The reference's Bf16Record (crates/oominf-core/src/backend.rs:800-807). */
typedef struct OomBf16Record {
    int64_t hidden;
    int64_t inter;
    int64_t gate_weight;
    int64_t up_weight;
    int64_t down_weight;
} OomBf16Record;

/* Message of the last failed call on this thread ("" if none). */
const char* oom_last_error(void);

/* Kernel-side failures. The persistent decode kernels meet across the grid through
 * bounded waits; a wait that gives up (the grid was not resident at once, or a limit
 * set by oom_set_wait_limit) lets the kernel end normally with invalid outputs and
 * sets the current device's status word. Like the reference's asynchronous CUDA
 * errors, which surface at its next synchronising call as an Err (its error contract:
 * crates/oominf-cuda/src/lib.rs:157-160), that failure is reported at a sync point:
 * oom_status waits for `stream`, then returns OOM_ERR_KERNEL if any kernel of this
 * library on the current device gave up a wait since the last oom_status, else OOM_OK;
 * it reads and clears the word in one atomic exchange. oom_stream_sync reports it the
 * same way. The word is per device, not per stream: a give-up in a kernel on any stream
 * of the device is reported by the next oom_status (or oom_stream_sync) on that device,
 * whichever stream it names, and only once; a backend that drives several streams of one
 * device checks it once per step. */
int oom_status(void* stream);

/* Polls of each bounded wait before it gives up, for later launches of this process
 * (0 restores the default, 2^22 polls of about 0.1 us). A tiny limit makes waits give
 * up at once: kernels still end normally, and oom_status then reports OOM_ERR_KERNEL;
 * tests use it to exercise the failure path without a GPU fault. */
int oom_set_wait_limit(uint32_t spins);

/* Zero-fills `bytes` of workspace at `ws` on `stream` with a fill kernel (no
 * hipMemset node, so it is safe inside graph capture). */
int oom_workspace_init(void* ws, size_t bytes, void* stream);

/* Byte offsets of the parts of an NVFP4 expert record (layout nvfp4-modelopt-g16,
 * docs/dev/format.md:63-68,111-118): weights two E2M1 codes per byte, row-major, low
 * nibble first (gate/up [inter, hidden], down [hidden, inter]); weight_scale one e4m3
 * byte per 16 inputs, row-major; scale2[p] the index, in floats from the record start, of
 * projection p's weight_scale_2 (gate, up, down). Weight w = e2m1(code) *
 * (e4m3(scale) * scale_2). Mirrors Nvfp4Record (crates/oominf-core/src/backend.rs:783-796). */
typedef struct OomNvfp4Record {
    int64_t hidden;
    int64_t inter;
    int64_t gate_weight;
    int64_t gate_scale;
    int64_t up_weight;
    int64_t up_scale;
    int64_t down_weight;
    int64_t down_scale;
    int64_t scale2[3];
} OomNvfp4Record;

/* Router: softmax over E logits per token, top k (ties to the lower id), weights
 * renormalised over the k picks, in pick order. logits f32 [T, E]; ids i32 [T, k];
 * weights f32 [T, k]. k <= 32, E <= 8192.
 * Replaces Experts::router_topk (crates/oominf-core/src/backend.rs:814-824;
 * crates/oominf-cuda/src/experts.rs:10-38). */
int oom_router_topk(const float* logits, int32_t* ids, float* weights, int T, int E, int k, void* stream);

/* Decode GEMV over e4m3 weights: y[t, n] = sum_k x[t, k] * e4m3(q[n, k]) * scale(n, k)
 * for t < T <= 16. x [T, K] in x_dtype; q [N, K] (16-byte aligned, K % 16 == 0);
 * scale in scale_layout; y [T, N] in y_dtype.
 * Replaces Linear::gemm_fp8 at decode sizes (crates/oominf-core/src/backend.rs:194-209;
 * crates/oominf-cuda/src/linear.rs:35-56,220-350). */
size_t oom_gemv_fp8_workspace_size(int T, int64_t N, int64_t K);
int oom_gemv_fp8(const void* x, int x_dtype, const uint8_t* q, const float* scale, int scale_layout, void* y,
                 int y_dtype, int T, int64_t N, int64_t K, void* ws, size_t ws_bytes, void* stream);

/* Decode GEMV over bf16 weights: y[t, n] = sum_k x[t, k] * w[n, k] (fp32 accumulate) for
 * t < T <= 16. x [T, K] in x_dtype; w bf16 [N, K] (16-byte aligned, K % 16 == 0); y [T, N]
 * in y_dtype. Replaces Linear::gemm_bf16 at decode sizes (crates/oominf-core/src/backend.rs:
 * 222-234; crates/oominf-cuda/kernels/ops.cu:329-440,568-576): the router GEMV. */
size_t oom_gemv_bf16_workspace_size(int T, int64_t N, int64_t K);
int oom_gemv_bf16(const void* x, int x_dtype, const uint16_t* w, void* y, int y_dtype, int T, int64_t N, int64_t K,
                  void* ws, size_t ws_bytes, void* stream);

/* Routed-expert gate/up + SwiGLU over FP8 records read in place:
 * h[a, j] = silu(x[assign_tok[a]] . Wg_e[j]) * (x[assign_tok[a]] . Wu_e[j]) for the
 * assignments a in [off[i], off[i+1]) of expert i < n_experts, whose record starts
 * at device address recs[i]. x [T, hidden] in x_dtype; h f32 [A, inter].
 * Replaces Experts::moe_gate_up (crates/oominf-core/src/backend.rs:825-836;
 * crates/oominf-cuda/src/experts.rs:43-93). */
int oom_moe_gate_up_fp8(const uint64_t* recs, const int32_t* off, const int32_t* assign_tok, int n_experts,
                        const void* x, int x_dtype, float* h, const OomFp8Record* geo, void* stream);

/* Down projection: y[a, r] = h[a] . Wd_e[r]; h f32 [A, inter]; y f32 [A, hidden].
 * Replaces Experts::moe_down (crates/oominf-core/src/backend.rs:859-868;
 * crates/oominf-cuda/src/experts.rs:174-209). */
int oom_moe_down_fp8(const uint64_t* recs, const int32_t* off, int n_experts, const float* h, float* y,
                     const OomFp8Record* geo, void* stream);

/* The routed experts' gate/up + SwiGLU and down projection over bf16 records read in
 * place, for decode-sized steps: the arguments and results of oom_moe_gate_up_fp8 and
 * oom_moe_down_fp8 with the weights bf16 (widened exactly to fp32), fp32 products and
 * accumulation, x in x_dtype (f32 or bf16). hidden and inter multiples of 8 up to 4096.
 * Replace Experts::moe_gate_up_bf16 and Experts::moe_down_bf16
 * (crates/oominf-core/src/backend.rs:837-858; crates/oominf-cuda/kernels/moe.cu:343-443),
 * called by run_group for Geometry::Bf16 (crates/oominf-models-qwen/src/moe.rs:741-744). */
int oom_moe_gate_up_bf16(const uint64_t* recs, const int32_t* off, const int32_t* assign_tok, int n_experts,
                         const void* x, int x_dtype, float* h, const OomBf16Record* geo, void* stream);
int oom_moe_down_bf16(const uint64_t* recs, const int32_t* off, int n_experts, const float* h, float* y,
                      const OomBf16Record* geo, void* stream);

/* out[t, c] = sum_s w[t, s] * y[slot_assign[t, s], c], summed in slot order.
 * y f32 [A, H]; w f32 [T, k]; out [T, H] in out_dtype.
 * Replaces Experts::moe_combine_slots (crates/oominf-core/src/backend.rs:896-907;
 * crates/oominf-cuda/src/experts.rs:303-329). */
int oom_moe_combine_slots(const float* y, const int32_t* slot_assign, const float* w, void* out, int out_dtype,
                          int T, int H, int k, void* stream);

/* Routing plan on the device: groups the T*k slots of `ids` by expert in id
 * order, as the host does in crates/oominf-models-qwen/src/moe.rs:539-582,638-649.
 * Writes plan[0] = n_e, then experts[E] (distinct ids, ascending; unused entries
 * -1), off[E + 1], assign_tok[T*k], slot_assign[T*k], all i32 in that order
 * (oom_moe_plan_size() elements), and recs[i] = all_recs[experts[i]] for i < n_e.
 * No host synchronisation: later kernels read n_e from the device. */
size_t oom_moe_plan_size(int T, int E, int k);
int oom_moe_plan(const int32_t* ids, int T, int E, int k, const uint64_t* all_recs, int32_t* plan, uint64_t* recs,
                 void* stream);

/* One decode MoE FFN step on the device, with no host synchronisation: router
 * top-k over logits f32 [T, E], routing plan, gate/up + SwiGLU, down projection
 * and slot-order weighted combine, reading the records of the routed experts
 * (all_recs[e] = device address of expert e's record, for all E experts) once per
 * step for all their tokens. x [T, hidden] in x_dtype; out [T, hidden] in
 * out_dtype; ids i32 [T, k] and weights f32 [T, k] are written as by
 * oom_router_topk. Steps with T * k <= 512, E <= 256, hidden <= 4096 and inter <= 2048 run
 * as one persistent kernel (2..16 tokens with bf16 x, k <= 8 and 16-byte aligned x: the
 * products on bf16 matrix cores; otherwise on the vector ALUs); larger steps as router,
 * plan, gate/up, down and combine launches. The fused equivalent of Moe::forward's routed part
 * (crates/oominf-models-qwen/src/moe.rs:290-366: router_topk, begin_routed,
 * finish_routed, run_group, moe_combine_slots). */
size_t oom_moe_decode_fp8_workspace_size(int T, int E, int k, const OomFp8Record* geo);
int oom_moe_decode_fp8(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T, int E,
                       int k, const OomFp8Record* geo, int32_t* ids, float* weights, void* out, int out_dtype,
                       void* ws, size_t ws_bytes, void* stream);

/* oom_moe_decode_fp8 without a caller workspace: the same step, same kernels, same bits,
 * with its scratch in a device array of the library (oom_moe_decode_fp8_noalloc_max_bytes()
 * bytes, 4 MiB: every step with T <= 16, k <= 8, hidden <= 4096 and inter <= 2048 fits;
 * a larger step returns OOM_ERR_WORKSPACE). It allocates nothing, not even on its first
 * call, so callers that cannot allocate can use it: code under graph capture, tight
 * serving loops, harnesses that forbid allocation. Every call on one device shares that
 * device's array and leaves it ready for the next call; calls that overlap in time on
 * one device (two streams, two threads) race, so order them on one stream. No counterpart
 * in the reference, whose backend keeps its scratch in a per-device workspace. */
size_t oom_moe_decode_fp8_noalloc_max_bytes(void);
int oom_moe_decode_fp8_noalloc(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T,
                               int E, int k, const OomFp8Record* geo, int32_t* ids, float* weights, void* out,
                               int out_dtype, void* stream);

/* The shared expert's gated add: out[t, c] = routed[t, c] + sigmoid(gate_logit[t]) *
 * shared[t, c], sigmoid(v) = 1 / (1 + e^-v); routed and shared f32 [T, H], gate_logit f32
 * [T]; out [T, H] in out_dtype. Replaces Elementwise::moe_combine
 * (crates/oominf-core/src/backend.rs:909-917; crates/oominf-cuda/kernels/ops.cu:310-316). */
int oom_moe_combine_shared(const float* routed, const float* shared, const float* gate_logit, void* out,
                           int out_dtype, int T, int H, void* stream);

/* One decode MoE layer with no host synchronisation: logits = x Wr^T over bf16 router
 * weights router_w [E, hidden]; the routed step of oom_moe_decode_fp8 (ids, weights written
 * as there); the shared expert, an FP8 record (device address at shared_rec[0], geometry
 * shared_geo with the same hidden) run as one expert with weight 1; its gate logit
 * x . shared_gate_w (bf16 [hidden]); out = routed + sigmoid(gate logit) * shared, in
 * out_dtype. T <= 16; one workspace made for T serves every step of 1..T tokens. The
 * device half of Moe::forward with every routed expert resident
 * (crates/oominf-models-qwen/src/moe.rs:254-366) and Moe::shared (moe.rs:498-527). */
size_t oom_moe_layer_decode_fp8_workspace_size(int T, int E, int k, const OomFp8Record* geo,
                                               const OomFp8Record* shared_geo);
int oom_moe_layer_decode_fp8(const void* x, int x_dtype, const uint16_t* router_w, const uint64_t* all_recs, int T,
                             int E, int k, const OomFp8Record* geo, const uint64_t* shared_rec,
                             const OomFp8Record* shared_geo, const uint16_t* shared_gate_w, int32_t* ids,
                             float* weights, void* out, int out_dtype, void* ws, size_t ws_bytes, void* stream);

/* Routed-expert gate/up + SwiGLU over NVFP4 records read in place: as
 * oom_moe_gate_up_fp8, weights decoded as e2m1(code) * (e4m3(scale) * scale_2), fp32
 * accumulate. hidden and inter multiples of 16, hidden <= 4096; x 16-byte aligned.
 * Replaces Experts::moe_gate_up (crates/oominf-core/src/backend.rs:825-836;
 * crates/oominf-cuda/src/experts.rs:43-93; crates/oominf-cuda/kernels/moe.cu:52-106). */
int oom_moe_gate_up_nvfp4(const uint64_t* recs, const int32_t* off, const int32_t* assign_tok, int n_experts,
                          const void* x, int x_dtype, float* h, const OomNvfp4Record* geo, void* stream);

/* Down projection over NVFP4 records: y[a, r] = h[a] . Wd_e[r]; h f32 [A, inter]
 * (inter <= 4096); y f32 [A, hidden]. Replaces Experts::moe_down (backend.rs:859-868;
 * experts.rs:174-209; moe.cu:108-151). */
int oom_moe_down_nvfp4(const uint64_t* recs, const int32_t* off, int n_experts, const float* h, float* y,
                       const OomNvfp4Record* geo, void* stream);

/* One decode MoE FFN step over NVFP4 records with no host synchronisation: router
 * top-k, device routing plan, gate/up + SwiGLU, down and slot-order weighted combine, as
 * oom_moe_decode_fp8 (same arguments, NVFP4 geometry). The routed part of Moe::forward
 * (crates/oominf-models-qwen/src/moe.rs:290-366) on the released record format. One
 * token (T = 1, E <= 512, k <= 16, inter <= 2048) runs as one launch with one grid
 * barrier over the workspace header, with the staged launches' arithmetic; the workspace
 * must be zero-filled once before its first use (oom_workspace_init). */
size_t oom_moe_decode_nvfp4_workspace_size(int T, int E, int k, const OomNvfp4Record* geo);
int oom_moe_decode_nvfp4(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T, int E,
                         int k, const OomNvfp4Record* geo, int32_t* ids, float* weights, void* out, int out_dtype,
                         void* ws, size_t ws_bytes, void* stream);

/* Per-row e4m3 quantisation of activations: scale[r] = max_c |x[r, c]| / 448 (1 for an
 * all-zero row), q[r, c] = e4m3(x[r, c] / scale[r]) rounded to nearest even and
 * saturating at +-448 (crates/oominf-core/src/fp8.rs:5-88, block = one row). x [rows,
 * cols] in x_dtype; q u8 [rows, cols]; scale f32 [rows]. The prefill's per-token
 * activation quantiser. */
int oom_quantize_rows_fp8(const void* x, int x_dtype, int64_t rows, int64_t cols, uint8_t* q, float* scale,
                          void* stream);

/* FP8 x FP8 grouped GEMM of one projection of each expert, on the matrix cores:
 *   y[a, r] = xs(a) * sum_kb ws_e(r, kb) * sum_{c in kb} e4m3(xq[row(a), c]) * e4m3(W_e[r, c])
 * for the assignments a in [off[i], off[i+1]) of expert i < n_experts (record at
 * recs[i]; W_e [N, K] e4m3 at byte w_off, its 128 x 128 fp32 scales at s_off),
 * row(a) = rows ? rows[a] : a. x_group 0: xs(a) = x_scale[row(a)] multiplies the result;
 * x_group 128: x_scale[row(a) * K / 128 + kb] joins ws inside the kb sum. y f32 [A, N].
 * N, K multiples of 128; max_per_expert bounds off[i+1] - off[i] (the host plan's).
 * Replaces Experts::moe_tiled (crates/oominf-core/src/backend.rs:869-883;
 * crates/oominf-cuda/src/experts.rs:214-260; crates/oominf-cuda/kernels/moe.cu:166-335)
 * for e4m3 records and e4m3 activations. */
int oom_moe_grouped_gemm_fp8(const uint64_t* recs, const int32_t* off, const int32_t* rows, int n_experts,
                             int max_per_expert, const uint8_t* xq, const float* x_scale, int x_group, float* y,
                             int64_t N, int64_t K, int64_t w_off, int64_t s_off, void* stream);

/* Activation precision of the prefill's down projection: the reference's ExpertPrecision
 * (crates/oominf-core/src/backend.rs:142-149). OOM_EXPERT_BF16 rounds h to bf16 (one
 * matrix-core pass); OOM_EXPERT_EXACT keeps 16 significant bits of the fp32 h as two
 * bf16 terms (two passes). */
#define OOM_EXPERT_EXACT 0
#define OOM_EXPERT_BF16 1

/* One prefill MoE FFN step on the device, with no host synchronisation: router top-k,
 * routing plan, x quantised per token to e4m3, gate and up grouped GEMMs with
 * h = silu(g) * u formed in the same pass (in `precision`), down grouped GEMM on the bf16
 * matrix cores, slot-order weighted combine. logits f32 [T, E]; x [T, hidden] in x_dtype;
 * out [T, hidden] in out_dtype; ids / weights as oom_router_topk. hidden and inter
 * multiples of 128. The tiled prefill of Moe::forward (crates/oominf-models-qwen/src/moe.rs:700,
 * 746-758: run_group over moe_tiled and moe_swiglu_range) with FP8 activations. */
size_t oom_moe_prefill_fp8_workspace_size(int T, int E, int k, const OomFp8Record* geo);
int oom_moe_prefill_fp8(const float* logits, const void* x, int x_dtype, const uint64_t* all_recs, int T, int E,
                        int k, const OomFp8Record* geo, int precision, int32_t* ids, float* weights, void* out,
                        int out_dtype, void* ws, size_t ws_bytes, void* stream);

/* Tiled grouped GEMM of one NVFP4 projection (prefill): y[a, r] = x[row(a)] . W_e[r] for
 * the assignments a in [off[e], off[e + 1]) of each of n_experts experts, row(a) = rows[a]
 * (rows null: a), W_e the projection (codes at byte w_off, e4m3 scales at byte s_off,
 * weight_scale_2 at float s2_idx of expert e's record recs[e]; layout
 * nvfp4-modelopt-g16, n rows of k inputs), decoded exactly to bf16 with scale_2 applied
 * to the fp32 result. x f32 [*, k] (16-byte aligned); y f32 [A, n]. precision
 * OOM_EXPERT_EXACT splits x into three exact bf16 terms (an fp32 GEMM in another
 * summation order); OOM_EXPERT_BF16 rounds x to bf16 (one matrix-core pass). k a
 * multiple of 32; max_per_expert bounds any expert's assignment count (the grid).
 * Replaces Experts::moe_tiled (crates/oominf-core/src/backend.rs:869-886;
 * crates/oominf-cuda/src/experts.rs:214-267; crates/oominf-cuda/kernels/moe.cu:166-335). */
int oom_moe_tiled_nvfp4(const uint64_t* recs, const int32_t* off, const int32_t* rows, int n_experts,
                        int max_per_expert, const float* x, float* y, int n, int k, int64_t w_off, int64_t s_off,
                        int s2_idx, int precision, void* stream);

/* h[i] = silu(g[i]) * u[i] for i in [start, end), silu(v) = v / (1 + e^-v), fp32.
 * Replaces Experts::moe_swiglu_range (crates/oominf-core/src/backend.rs:887-895;
 * crates/oominf-cuda/src/experts.rs:269-299; crates/oominf-cuda/kernels/moe.cu:338-341). */
int oom_moe_swiglu_range(const float* g, const float* u, float* h, int64_t start, int64_t end, void* stream);

/* Paged GQA decode attention for one query token: out[h, :] = sum_j softmax_j(q_h . k_j
 * * scale) v_j over the kv_len keys, query head h reading KV head h / (heads / kv_heads).
 * q [heads, d] in q_dtype; k_pages and v_pages bf16 [n_pages, kv_heads, page_size, d]
 * (16-byte aligned); key j lives in physical page page_table[j / page_size] (i32, one
 * entry per page of the sequence; an entry outside [0, n_pages) reads zeros) at slot
 * j % page_size. d = 128, heads / kv_heads <= 8, page_size a multiple of 16. fp32 dot
 * products, exp and accumulation (fp32 q enters the bf16 matrix cores as an exact
 * three-term split); out [heads, d] in out_dtype. Every key up to kv_len is visible
 * (the decode position is the last one).
 * Replaces Attention::attention at decode (crates/oominf-core/src/backend.rs:545-568;
 * crates/oominf-cuda/src/attention.rs:265-346, which routes D=128, G=8 to attn_prefill,
 * crates/oominf-cuda/kernels/attention.cu:419-553), over a paged bf16 cache. */
size_t oom_attn_decode_workspace_size(int kv_len, int heads, int kv_heads, int d);
int oom_attn_decode_paged(const void* q, int q_dtype, const uint16_t* k_pages, const uint16_t* v_pages,
                          const int32_t* page_table, int n_pages, int page_size, int kv_len, int heads, int kv_heads,
                          int d, float scale, void* out, int out_dtype, void* ws, size_t ws_bytes, void* stream);

/* ---- Turbo KV cache and the D = 256, G = 12 decode attention ----
 * KvFormat (crates/oominf-core/src/backend.rs:571-635): a cache row is one head vector of
 * d coordinates; bits 0: d fp32 values; bits 2..8 (Turbo): the vector rotated by a fixed
 * randomized Walsh-Hadamard transform, then per 32 coordinates an fp16 scale (their RMS;
 * the scales padded to 16 bytes) and `bits` 32-bit words, word j holding bit j of the 32
 * codebook indices. A cache holds rows [len, kv_heads]. `levels` is the device copy of
 * oom_kv_codebooks' table (null for fp32 rows). */

/* KvFormat::codebooks (backend.rs:637-700): the Lloyd-Max levels of a unit Gaussian for
 * 2..8 bits, ascending, concatenated (the 2^b levels for b bits start at 2^b - 4); 508
 * floats into `levels` (n >= oom_kv_codebook_size()). Computed on the host once. */
size_t oom_kv_codebook_size(void);
int oom_kv_codebooks(float* levels, size_t n);
/* KvFormat::row_bytes (backend.rs:605-611); 0 for a shape the kernels do not take (d a
 * multiple of 32 up to 256, a power of two for bits 2..8). */
size_t oom_kv_row_bytes(int d, int bits);
/* Gpu::kv_rotate (crates/oominf-cuda/src/attention.rs:476-496; attention.cu:63-73): rows
 * [rows, d] f32 in place into (inverse 0) or out of (inverse 1) the rotated space. */
int oom_kv_rotate(float* x, int rows, int d, int inverse, void* stream);
/* Attention::kv_append (attention.rs:172-214; attention.cu:75-112): src f32 [t, kv_heads,
 * d] appended at sequence position `start` (cache row start * kv_heads), rotated and
 * quantised for bits 2..8. */
int oom_kv_append(const float* src, uint8_t* cache, int64_t start, int t, int kv_heads, int d, int bits,
                  const float* levels, void* stream);
/* Attention::kv_read (attention.rs:216-254; attention.cu:114-131): len * kv_heads rows back
 * as f32 [len, kv_heads, d], decoded and un-rotated. */
int oom_kv_read(const uint8_t* cache, float* dst, int len, int kv_heads, int d, int bits, const float* levels,
                void* stream);
/* mask_compact (attention.cu:363-374): the positions j < n with mask[j] != 0, in order:
 * sel[0] = count, sel[1 ..] = positions (sel: n + 1 int32). */
int oom_mask_compact(const uint8_t* mask, int32_t* sel, int n, void* stream);
/* One query token of Attention::attention with d = 256 and 12 query heads a KV head, the
 * flash-decode path (attention.rs:265-346,365-447; attention.cu:584-686): q f32 [heads,
 * 256] (rotated on the device for a Turbo cache), the keys j < kv_len with mask[j] != 0
 * (u8 [kv_len]), out f32 [heads, 256] = sum_j softmax_j(q_h . k_j * scale) v_j (rotated
 * back), query head h reading KV head h / 12. k_bits and v_bits both 0 or both 2..8.
 * fp32 dot products, exp and accumulation. */
size_t oom_attn_decode_turbo_workspace_size(int heads, int kv_heads, int d, int kv_len);
int oom_attn_decode_turbo(const float* q, const uint8_t* k, const uint8_t* v, int k_bits, int v_bits,
                          const float* levels, const uint8_t* mask, int heads, int kv_heads, int d, int kv_len,
                          float scale, float* out, void* ws, size_t ws_bytes, void* stream);


/* ---- copies beside compute (expert offload) ----
 * The Transfer trait (crates/oominf-core/src/backend.rs:945-1018; CUDA form
 * crates/oominf-cuda/src/memory.rs:300-380): a copy queue runs beside the compute stream,
 * events order the two, so TieredExperts can stage host-tier expert records into device
 * slots while the previous layer computes. Queues and events are opaque handles. */

/* Transfer::copy_queue: a stream of its own at default priority, non-blocking. */
int oom_copy_queue_create(void** queue);
int oom_copy_queue_destroy(void* queue);
/* Pinned host memory, the source of asynchronous copies. Replaces Transfer::pin_host /
 * unpin_host (backend.rs:956-963): registering existing memory is not offered, so a host
 * expert tier is allocated here instead. */
int oom_host_alloc(void** ptr, size_t bytes);
int oom_host_free(void* ptr);
/* Transfer::copy_to_device (backend.rs:964-976): len bytes from pinned host src to device
 * address dst, queued on `queue`. */
int oom_copy_to_device(void* queue, uint64_t dst, const void* src, size_t len);
/* Transfer::copy_on_device (backend.rs:998-1006). */
int oom_copy_on_device(void* queue, uint64_t dst, uint64_t src, size_t len);
/* n records of `bytes` each, src[i] (pinned host) -> dst[i] (device), in order on `queue`:
 * the per-layer staging loop of TieredExperts over copy_to_device (crates/oominf-core/src/experts.rs). */
int oom_copy_records_to_device(void* queue, const uint64_t* dst, const void* const* src, size_t bytes, int n);
/* Transfer::download_async (backend.rs:977-985): after the work queued on `stream` so far,
 * len bytes from device src to pinned host dst. */
int oom_download_async(void* stream, void* dst, const void* src, size_t len);
/* Transfer events (backend.rs:1007-1017): record_compute / record_copies are
 * oom_event_record on the compute stream or the queue; compute_wait / copies_wait are
 * oom_stream_wait_event; event_done returns 1 (done), 0 (pending) or an error;
 * event_wait and copies_sync block the host. */
int oom_event_create(void** event);
int oom_event_destroy(void* event);
int oom_event_record(void* event, void* stream);
int oom_stream_wait_event(void* stream, void* event);
int oom_event_done(void* event);
int oom_event_wait(void* event);
int oom_stream_sync(void* stream);

#ifdef __cplusplus
}
#endif
#endif
