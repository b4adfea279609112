/*
 * oom_oracle.h -- CPU restatement of oom-inference's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests/, the smoke entry
 * point and the bench's CPU-baseline leg may load it; the product library
 * (homelab_amd/liboom_hip.so) never does, and no product path falls back to it.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * projects/oom-inference/). Arithmetic is fp32 with the reference's operation
 * order where the reference fixes one, and serial order elsewhere.
 *
 * Parity pins (what checks this oracle, independently of itself) are listed in
 * tests/test_oracle_*.py next to each function. Functions with no such check say
 * "parity unpinned" here: none at present.
 */
#ifndef OOM_ORACLE_H
#define OOM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/oom_hip.h" /* OomFp8Record, scale-layout and dtype enums */

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats ---------------------------------------------------- */

/* e4m3fn code nearest x, ties to even, saturating at +-448 (0x7e / 0xfe); NaN
 * saturates too. crates/oominf-core/src/fp8.rs:5-27. */
uint8_t oracle_e4m3_from_f32(float x);

/* Value of an e4m3fn code, exactly; 0x7f / 0xff are NaN as in
 * crates/oominf-cpu/src/kernel.rs:14-27 (fp8.rs:29-42 reads them as 448; the
 * quantiser never emits them). */
float oracle_e4m3_to_f32(uint8_t b);

/* bf16 bits of v, round to nearest even (crates/oominf-cuda/tests/gemv.rs:23-27). */
uint16_t oracle_bf16_from_f32(float v);
float oracle_bf16_to_f32(uint16_t b);
void oracle_bf16_from_f32_n(const float* v, uint16_t* out, size_t n);
void oracle_bf16_to_f32_n(const uint16_t* b, float* out, size_t n);

/* Blocked FP8 quantisation of bf16 weights w [n, k] (crates/oominf-core/src/
 * fp8.rs:44-88): a block's scale is its absolute maximum over 448 (1.0 for an
 * all-zero block) and q = e4m3(w / scale). `layout` picks the block shape:
 *   OOM_SCALE_ROW      one block per row            scale [n]
 *   OOM_SCALE_1X128    1 x 128 (the reference's)    scale [n, ceil(k/128)]
 *   OOM_SCALE_128X128  128 x 128                    scale [ceil(n/128), ceil(k/128)]
 * Returns 0, or -1 for an unknown layout. */
int oracle_quantize(const uint16_t* w, int64_t n, int64_t k, int layout, uint8_t* q, float* scale);

/* Number of fp32 scales `layout` holds for an [n, k] matrix. */
int64_t oracle_scale_count(int64_t n, int64_t k, int layout);

/* scale applied to weight (r, c) under `layout`. */
float oracle_scale_at(const float* scale, int64_t n, int64_t k, int layout, int64_t r, int64_t c);

/* Per-row e4m3 quantisation of activations x [rows, cols] (fp32): scale = row
 * absmax / 448 (1.0 for a zero row), q = e4m3(x / scale). `group` = 0 gives one
 * scale per row, else one per `group` columns ([rows, ceil(cols/group)]). */
void oracle_quantize_act(const float* x, int64_t rows, int64_t cols, int64_t group, uint8_t* q, float* scale);

/* ---- deterministic generators ------------------------------------------ */

/* xorshift64* step (crates/oominf-cuda/tests/moe_tiled.rs:15-20). */
uint64_t oracle_xorshift64s(uint64_t* state);

/* splitmix64 of a value: derives independent non-zero stream seeds. */
uint64_t oracle_seed(uint64_t base, uint64_t stream);

/* n standard normals * std from one xorshift64* + Box-Muller stream (cos branch
 * only, two uniforms per sample): crates/oominf-cuda/tests/kv_cache.rs:10-24. */
void oracle_gaussian(float* out, size_t n, uint64_t seed, float std);

/* As oracle_gaussian, rounded to bf16 (RNE). The tensor is split into chunks of
 * `chunk` values, chunk c drawn from stream oracle_seed(seed, c), so large tensors
 * generate in parallel over `threads` threads with the same result. */
void oracle_gaussian_bf16(uint16_t* out, size_t n, uint64_t seed, float std, size_t chunk, int threads);

/* Zipf(s) popularity bias over E experts: a seeded Fisher-Yates permutation gives
 * each expert a rank, p_e = rank_e^-s / sum_r r^-s, bias_e = ln p_e. */
void oracle_zipf_bias(float* bias, int E, double s, uint64_t seed);

/* Seeded Fisher-Yates permutation of 0..n-1 (page order of a KV cache). */
void oracle_permutation(int32_t* out, int n, uint64_t seed);

/* ---- router ------------------------------------------------------------ */

/* Softmax over E logits per row, top k (ties to the lower id), weights
 * renormalised over the picks, in pick order (descending probability).
 * crates/oominf-cuda/kernels/ops.cu:230-294, with the kernel's 256-thread
 * block_sum order for the softmax denominator (ops.cu:16-31). */
void oracle_router_topk(const float* logits, int T, int E, int k, int32_t* ids, float* weights);

/* The softmax probabilities the router ranks (same arithmetic): p [T, E]. */
void oracle_router_probs(const float* logits, int T, int E, float* p);

/* ---- dense FP8 GEMV ----------------------------------------------------- */

/* y[t, n] = sum_k x[t, k] * (e4m3(q[n, k]) * scale(n, k)), fp32, k ascending.
 * crates/oominf-cuda/kernels/ops.cu:339-440 (gemv_impl<T, true>). */
void oracle_gemv_fp8(const float* x, int T, const uint8_t* q, const float* scale, int layout, int64_t N,
                     int64_t K, float* y);

/* y[t, n] = sum_k x[t, k] * bf16(w[n, k]), fp32, k ascending (the router GEMV).
 * crates/oominf-cuda/kernels/ops.cu:329-440 (gemv_impl<T, false>). */
void oracle_gemv_bf16(const float* x, int T, const uint16_t* w, int64_t N, int64_t K, float* y);

/* ---- routed experts ---------------------------------------------------- */

/* Routing plan of one step with every expert resident: slots t*k+s grouped by
 * expert in id order; off[n_e + 1], assign_tok[A], slot_assign[A], experts[n_e]
 * (the distinct ids). crates/oominf-models-qwen/src/moe.rs:539-582 (grouping)
 * and :638-649 (meta). Returns n_e, or -1 for an out-of-range id. */
int oracle_moe_plan(const int32_t* ids, int T, int k, int E, int32_t* experts, int32_t* off,
                    int32_t* assign_tok, int32_t* slot_assign);

/* h[a, j] = silu(x[tok(a)] . Wg[j]) * (x[tok(a)] . Wu[j]) for every assignment of
 * the n_e experts whose records start at recs[i] (host pointers).
 * crates/oominf-cuda/kernels/moe.cu:52-106 (silu = v / (1 + expf(-v)), :50). */
void oracle_moe_gate_up_fp8(const uint8_t* const* recs, const int32_t* off, const int32_t* assign_tok, int n_e,
                            const float* x, float* h, const OomFp8Record* geo);

/* y[a, r] = h[a] . Wd[r]. crates/oominf-cuda/kernels/moe.cu:108-151. */
void oracle_moe_down_fp8(const uint8_t* const* recs, const int32_t* off, int n_e, const float* h, float* y,
                         const OomFp8Record* geo);

/* out[t, c] = sum_s w[t, s] * y[slot_assign[t, s], c], slots in order.
 * crates/oominf-cuda/kernels/moe.cu:153-164. */
void oracle_moe_combine_slots(const float* y, const int32_t* slot_assign, const float* w, float* out, int T,
                              int H, int k);

/* One whole decode MoE FFN step (router -> plan -> gate/up -> down -> combine)
 * over records all_recs[e] for all E experts; x fp32 [T, H]; out fp32 [T, H];
 * ids / weights [T, k]. crates/oominf-models-qwen/src/moe.rs:254-366 minus the
 * shared expert and router GEMV. Returns 0 or -1. */
int oracle_moe_decode_fp8(const float* logits, const float* x, const uint8_t* const* all_recs, int T, int E, int k,
                          const OomFp8Record* geo, int32_t* ids, float* weights, float* out);

/* NVFP4 (nvfp4-modelopt-g16) routed experts. E2M1 value of a 4-bit code
 * (crates/oominf-cpu/src/kernel.rs:8-11). */
float oracle_e2m1_to_f32(uint8_t code);
/* y[t, r] = sum_c e2m1(code(r, c)) * (e4m3(scale(r, c / 16)) * s2) * x[t, c], column order
 * (kernel.rs:76-98); packed [rows, cols / 2], scales [rows, cols / 16]; y [T, rows]. */
void oracle_nvfp4_rows(const uint8_t* packed, const uint8_t* scales, float s2, int64_t rows, int64_t cols,
                       const float* x, int T, float* y);
/* gate/up + SwiGLU and down over NVFP4 records (moe.cu:52-151 semantics). */
/* bf16 records (layout tag bf16; bf16rec.c): the reference's moe_gate_up_bf16 and
 * moe_down_bf16 (crates/oominf-cuda/kernels/moe.cu:343-443). */
void oracle_moe_gate_up_bf16(const uint8_t* const* recs, const int32_t* off, const int32_t* assign_tok, int n_e,
                             const float* x, float* h, const OomBf16Record* geo);
void oracle_moe_down_bf16(const uint8_t* const* recs, const int32_t* off, int n_e, const float* h, float* y,
                          const OomBf16Record* geo);

void oracle_moe_gate_up_nvfp4(const uint8_t* const* recs, const int32_t* off, const int32_t* assign_tok, int n_e,
                              const float* x, float* h, const OomNvfp4Record* geo);
void oracle_moe_down_nvfp4(const uint8_t* const* recs, const int32_t* off, int n_e, const float* h, float* y,
                           const OomNvfp4Record* geo);
/* The tiled NVFP4 grouped GEMM of one projection (moe.cu:166-335): y[a, r] = x[row(a)] .
 * W_e[r] * s2 with x as `terms` bf16 terms (3: exact, 1: x rounded to bf16), fp32 sums;
 * rows null: row(a) = a. x [*, K]; y [A, N]. */
void oracle_moe_tiled_nvfp4(const uint8_t* const* recs, const int32_t* off, const int32_t* rows, int n_e,
                            const float* x, float* y, int64_t N, int64_t K, int64_t w_off, int64_t s_off, int s2_idx,
                            int terms);
/* The whole routed decode step over NVFP4 records (router, plan, gate/up, down, combine). */
int oracle_moe_decode_nvfp4(const float* logits, const float* x, const uint8_t* const* all_recs, int T, int E, int k,
                            const OomNvfp4Record* geo, int32_t* ids, float* weights, float* out);

/* ---- prefill grouped GEMM (FP8 x FP8) ---------------------------------- */

/* y[a, r] = xs(a) * sum_kb ws(r, kb) * sum_{c in kb} e4m3(xq[row(a), c]) * e4m3(W[r, c])
 * for one projection of each expert (W at rec + w_off, 128x128 scales at rec +
 * s_off), row(a) = rows ? rows[a] : a, xs(a) = x_scale[row(a)] (per-row) or
 * x_scale[row(a) * ceil(K/128) + kb] (per-row 128-column groups, then inside the
 * kb sum). Semantics of crates/oominf-cuda/kernels/moe.cu:166-335 (moe_tiled:
 * grouped y = x[row(a)] . W_e^T, weight scale applied to the fp32 block sums)
 * with e4m3 activations instead of fp32. */
void oracle_grouped_gemm_fp8(const uint8_t* const* recs, const int32_t* off, const int32_t* rows, int n_e,
                             const uint8_t* xq, const float* x_scale, int x_group, float* y, int64_t N, int64_t K,
                             int64_t w_off, int64_t s_off);

/* Whole prefill MoE FFN over the routed assignments of T tokens: x fp32 [T, H]
 * quantised per token, gate and up grouped GEMMs, h = silu(g) * u kept in fp32 (the
 * reference's exact tiled path, ExpertPrecision::Exact) or, with h_bf16, rounded to bf16
 * to nearest even (ExpertPrecision::Bf16), the down projection as oracle_moe_down_fp8,
 * slot-order combine.
 * crates/oominf-models-qwen/src/moe.rs:746-758 (tiled run_group) + :700.
 * Returns n_e or -1. */
int oracle_moe_prefill_fp8(const float* logits, const float* x, const uint8_t* const* all_recs, int T, int E, int k,
                           const OomFp8Record* geo, int h_bf16, int32_t* ids, float* weights, float* out);

/* ---- paged GQA decode attention ---------------------------------------- */

/* One query token: out[h, :] = softmax_j(q_h . k_j * scale) v_j over kv_len keys,
 * GQA (head h reads KV head h / (H / Hkv)), keys in 16-token... `page_size`-token
 * pages: token j lives in physical page page_table[j / page_size], slot
 * j % page_size; a page is [page_size, Hkv, D] bf16. fp32 dots, expf and
 * accumulation with an online softmax over key tiles of 16, as
 * crates/oominf-cuda/kernels/attention.cu:419-553 (attn_prefill, which the
 * reference dispatches for D=128, G=8: crates/oominf-cuda/src/attention.rs:300-303). */
void oracle_attn_decode_paged(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                              const int32_t* page_table, int page_size, int kv_len, int H, int Hkv, int D,
                              float scale, float* out);

/* ---- reference CPU path (timed as the CPU baseline) --------------------- */

/* Routed experts on host cores, restating crates/oominf-cpu/src/lib.rs:175-323
 * (HostExperts::run) for e4m3 records: gate/up work items of 32 rows and down
 * items of 128 rows over a pool of `threads` threads; jobs of <= 4 tokens use the
 * per-row vector kernel (kernel.rs:374-412 shape, AVX-512 when the CPU has it),
 * larger jobs decode rows once and run the register-tiled GEMM over token
 * columns padded to 16 (lib.rs:386-438, kernel.rs:164-185). Output: per job in
 * order, one H-wide unweighted row per token. Returns 0. */
int oracle_host_experts(const OomFp8Record* geo, const uint8_t* const* records, const int32_t* job_tokens,
                        const int32_t* job_off, int n_jobs, const float* x, float* y, int threads);

/* Whether the AVX-512 kernels are in use on this CPU. */
int oracle_host_has_avx512(void);

/* ---- Turbo KV cache and the d = 256, G = 12 decode attention (turbo.c) ---- */

/* fp16 bits of f, round to nearest even (IEEE binary16); and back, exactly. */
uint16_t oracle_f16_from_f32(float f);
float oracle_f16_to_f32(uint16_t h);
/* KvFormat::codebooks (crates/oominf-core/src/backend.rs:637-700): 508 levels, the 2^b
 * Lloyd-Max levels of a unit Gaussian for b = 2..8, ascending, concatenated. */
void oracle_kv_codebooks(float* levels);
/* KvFormat::row_bytes (backend.rs:605-611). */
size_t oracle_kv_row_bytes(int D, int bits);
/* kv_rotate (crates/oominf-cuda/kernels/attention.cu:63-73): rows [rows, D] in place. */
void oracle_kv_rotate(float* x, int rows, int D, int inverse);
/* kv_append (attention.cu:75-112): rows [rows, D] into cache rows row0 .. + rows. */
void oracle_kv_append(const float* src, uint8_t* cache, int64_t row0, int rows, int D, int bits,
                      const float* levels);
/* kv_read (attention.cu:114-131). */
void oracle_kv_read(const uint8_t* cache, float* dst, int rows, int D, int bits, const float* levels);
/* mask_compact (attention.cu:363-374); returns the count. */
int oracle_mask_compact(const uint8_t* mask, int32_t* sel, int n);
/* Attention::attention for one token with d = 256, 12 query heads a KV head: q [H, 256]
 * rotated for a Turbo cache, mask_compact, the partials of attn_decode_partial_g12 (P =
 * ceil(min(kv_len, 4096) / 16) rounded up to 8, even chunks of the list, lane l of a
 * partial owning d = l + 32 e), attn_decode_combine, the output rotated back
 * (crates/oominf-cuda/src/attention.rs:265-447; attention.cu:584-686). */
void oracle_attn_decode_turbo(const float* q, const uint8_t* k, const uint8_t* v, int kb, int vb,
                              const float* levels, const uint8_t* mask, int H, int Hkv, int kv_len, float scale,
                              float* out);

#ifdef __cplusplus
}
#endif

/* out[t, c] = routed[t, c] + sigmoid(gate[t]) * shared[t, c], sigmoid(v) = 1 / (1 + expf(-v)).
 * crates/oominf-cuda/kernels/ops.cu:10,310-316 (moe_combine). */
void oracle_moe_combine_shared(const float* routed, const float* shared, const float* gate, float* out, int T, int H);

/* One decode MoE layer: logits = x Wr^T (bf16 router_w [E, H]), the routed step as
 * oracle_moe_decode_fp8, the shared expert (record shared_rec, geometry sgeo) as one
 * expert of weight 1, gate = x . gate_w (bf16 [H]), out = routed + sigmoid(gate) * shared.
 * crates/oominf-models-qwen/src/moe.rs:254-366 (all routed experts resident) and :498-527.
 * Returns 0 or -1. */
int oracle_moe_layer_decode_fp8(const float* x, int T, const uint16_t* router_w, const uint8_t* const* all_recs,
                                int E, int k, const OomFp8Record* geo, const uint8_t* shared_rec,
                                const OomFp8Record* sgeo, const uint16_t* gate_w, float* logits, float* gate,
                                int32_t* ids, float* weights, float* out);

#endif
