/*
 * paths.c -- router, FP8 GEMV, routed experts, prefill grouped GEMM and paged
 * decode attention, restated on the CPU in fp32.
 * TEST INFRASTRUCTURE (the oracle): never linked into the product library.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oom_oracle.h"

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

/* ---- router ---------------------------------------------------------------- */

/* v[i] += v[i ^ o] for o = 16, 8, 4, 2, 1 over one 32-lane warp; lane 0's value.
 * The __shfl_xor_sync reduction of crates/oominf-cuda/kernels/ops.cu:17,24. */
static float warp_xor_sum(float* v) {
    for (int o = 16; o > 0; o >>= 1) {
        float n[32];
        for (int i = 0; i < 32; i++) n[i] = v[i] + v[i ^ o];
        memcpy(v, n, sizeof(n));
    }
    return v[0];
}

/* block_sum for a 256-thread block (ops.cu:15-31): per-warp xor sums, then warp 0
 * xor-sums the 8 warp totals (lanes past 8 hold 0). */
static float block_sum_256(const float* per_thread) {
    float warp_sums[8];
    for (int w = 0; w < 8; w++) {
        float v[32];
        memcpy(v, per_thread + 32 * w, sizeof(v));
        warp_sums[w] = warp_xor_sum(v);
    }
    float v[32] = {0};
    for (int i = 0; i < 8; i++) v[i] = warp_sums[i];
    return warp_xor_sum(v);
}

/* ops.cu:234-258: max, then per-thread serial sums of exp(l - max) over e = tid,
 * tid + 256, ..., block_sum, p = exp(l - max) / sum. */
static void router_row_probs(const float* l, int E, float* p) {
    float mx = -INFINITY;
    for (int e = 0; e < E; e++) mx = fmaxf(mx, l[e]);
    float part[256];
    for (int t = 0; t < 256; t++) {
        float s = 0.0f;
        for (int e = t; e < E; e += 256) s += expf(l[e] - mx);
        part[t] = s;
    }
    float sum = block_sum_256(part);
    for (int e = 0; e < E; e++) p[e] = expf(l[e] - mx) / sum;
}

void oracle_router_probs(const float* logits, int T, int E, float* p) {
    for (int t = 0; t < T; t++) router_row_probs(logits + (size_t)t * E, E, p + (size_t)t * E);
}

/* ops.cu:259-293: k rounds of argmax (ties to the lower id), picks marked -2;
 * weights = p / (sum of picked p in pick order). */
void oracle_router_topk(const float* logits, int T, int E, int k, int32_t* ids, float* weights) {
    float* p = (float*)malloc(sizeof(float) * (size_t)E);
    for (int t = 0; t < T; t++) {
        router_row_probs(logits + (size_t)t * E, E, p);
        float chosen_p[32];
        int chosen[32];
        for (int r = 0; r < k; r++) {
            float bv = -3.0f;
            int bi = 0x7fffffff;
            for (int e = 0; e < E; e++)
                if (p[e] > bv || (p[e] == bv && e < bi)) {
                    bv = p[e];
                    bi = e;
                }
            chosen[r] = bi;
            chosen_p[r] = bv;
            p[bi] = -2.0f;
        }
        float picked = 0.0f;
        for (int r = 0; r < k; r++) picked += chosen_p[r];
        for (int r = 0; r < k; r++) {
            ids[t * k + r] = chosen[r];
            weights[t * k + r] = chosen_p[r] / picked;
        }
    }
    free(p);
}

/* ---- dense FP8 GEMV ---------------------------------------------------------- */

/* ops.cu:374-399: w = e4m3(q) * scale, acc += x * w, fp32. */
void oracle_gemv_fp8(const float* x, int T, const uint8_t* q, const float* scale, int layout, int64_t N,
                     int64_t K, float* y) {
    for (int t = 0; t < T; t++)
        for (int64_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int64_t c = 0; c < K; c++)
                acc += x[(size_t)t * K + c] * (oracle_e4m3_to_f32(q[n * K + c]) * oracle_scale_at(scale, N, K, layout, n, c));
            y[(size_t)t * N + n] = acc;
        }
}

/* ---- dense bf16 GEMV (the router) ---------------------------------------------- */

/* ops.cu:329-440 (gemv_impl<T, false>): acc += x * bf16(w), fp32, k ascending. */
void oracle_gemv_bf16(const float* x, int T, const uint16_t* w, int64_t N, int64_t K, float* y) {
    for (int t = 0; t < T; t++)
        for (int64_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int64_t c = 0; c < K; c++) {
                uint32_t bits = (uint32_t)w[n * K + c] << 16;
                float wf;
                memcpy(&wf, &bits, sizeof(wf));
                acc += x[(size_t)t * K + c] * wf;
            }
            y[(size_t)t * N + n] = acc;
        }
}

/* ---- routed experts ---------------------------------------------------------- */

int oracle_moe_plan(const int32_t* ids, int T, int k, int E, int32_t* experts, int32_t* off, int32_t* assign_tok,
                    int32_t* slot_assign) {
    int A = T * k;
    int32_t* count = (int32_t*)calloc((size_t)E, sizeof(int32_t));
    for (int s = 0; s < A; s++) {
        if (ids[s] < 0 || ids[s] >= E) {
            free(count);
            return -1;
        }
        count[ids[s]]++;
    }
    /* moe.rs:549-551: the distinct experts in id order (all resident: no reorder). */
    int n_e = 0;
    int32_t* start = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    int a = 0;
    for (int e = 0; e < E; e++) {
        start[e] = a;
        if (count[e]) {
            experts[n_e] = e;
            off[n_e] = a;
            n_e++;
            a += count[e];
        }
    }
    off[n_e] = a;
    /* moe.rs:641-647: within an expert, its slots in slot order. */
    for (int s = 0; s < A; s++) {
        int pos = start[ids[s]]++;
        assign_tok[pos] = s / k;
        slot_assign[s] = pos;
    }
    free(start);
    free(count);
    return n_e;
}

static inline float siluf(float v) { return v / (1.0f + expf(-v)); }

/* row `r` of an e4m3 [rows, cols] matrix with 128x128 scales, dotted with x. */
static float dot_row(const uint8_t* w, const float* s, int64_t rows, int64_t cols, int64_t r, const float* x) {
    float acc = 0.0f;
    for (int64_t c = 0; c < cols; c++)
        acc += x[c] * (oracle_e4m3_to_f32(w[r * cols + c]) * oracle_scale_at(s, rows, cols, OOM_SCALE_128X128, r, c));
    return acc;
}

void oracle_moe_gate_up_fp8(const uint8_t* const* recs, const int32_t* off, const int32_t* assign_tok, int n_e,
                            const float* x, float* h, const OomFp8Record* geo) {
    int64_t H = geo->hidden, I = geo->inter;
    for (int i = 0; i < n_e; i++) {
        const uint8_t* rec = recs[i];
        const uint8_t* gw = rec + geo->gate_weight;
        const uint8_t* uw = rec + geo->up_weight;
        const float* gs = (const float*)(rec + geo->gate_scale);
        const float* us = (const float*)(rec + geo->up_scale);
        for (int a = off[i]; a < off[i + 1]; a++) {
            const float* xt = x + (size_t)assign_tok[a] * H;
            for (int64_t j = 0; j < I; j++) {
                float g = dot_row(gw, gs, I, H, j, xt);
                float u = dot_row(uw, us, I, H, j, xt);
                h[(size_t)a * I + j] = siluf(g) * u;
            }
        }
    }
}

void oracle_moe_down_fp8(const uint8_t* const* recs, const int32_t* off, int n_e, const float* h, float* y,
                         const OomFp8Record* geo) {
    int64_t H = geo->hidden, I = geo->inter;
    for (int i = 0; i < n_e; i++) {
        const uint8_t* rec = recs[i];
        const uint8_t* dw = rec + geo->down_weight;
        const float* ds = (const float*)(rec + geo->down_scale);
        for (int a = off[i]; a < off[i + 1]; a++)
            for (int64_t r = 0; r < H; r++) y[(size_t)a * H + r] = dot_row(dw, ds, H, I, r, h + (size_t)a * I);
    }
}

void oracle_moe_combine_slots(const float* y, const int32_t* slot_assign, const float* w, float* out, int T,
                              int H, int k) {
    for (int t = 0; t < T; t++)
        for (int c = 0; c < H; c++) {
            float acc = 0.0f;
            for (int s = 0; s < k; s++) acc += w[t * k + s] * y[(size_t)slot_assign[t * k + s] * H + c];
            out[(size_t)t * H + c] = acc;
        }
}

int oracle_moe_decode_fp8(const float* logits, const float* x, const uint8_t* const* all_recs, int T, int E, int k,
                          const OomFp8Record* geo, int32_t* ids, float* weights, float* out) {
    int A = T * k;
    int64_t H = geo->hidden, I = geo->inter;
    oracle_router_topk(logits, T, E, k, ids, weights);
    int32_t* experts = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A + 1));
    int32_t* off = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A + 2));
    int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    int32_t* slot = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    int n_e = oracle_moe_plan(ids, T, k, E, experts, off, tok, slot);
    if (n_e < 0) {
        free(experts); free(off); free(tok); free(slot);
        return -1;
    }
    const uint8_t** recs = (const uint8_t**)malloc(sizeof(void*) * (size_t)(n_e ? n_e : 1));
    for (int i = 0; i < n_e; i++) recs[i] = all_recs[experts[i]];
    float* h = (float*)malloc(sizeof(float) * (size_t)A * (size_t)I);
    float* y = (float*)malloc(sizeof(float) * (size_t)A * (size_t)H);
    oracle_moe_gate_up_fp8(recs, off, tok, n_e, x, h, geo);
    oracle_moe_down_fp8(recs, off, n_e, h, y, geo);
    oracle_moe_combine_slots(y, slot, weights, out, T, (int)H, k);
    free(h); free(y); free(recs); free(experts); free(off); free(tok); free(slot);
    return 0;
}

/* ---- NVFP4 routed experts (nvfp4-modelopt-g16) ------------------------------------- */

/* E2M1 values by 4-bit code: low three bits the magnitude, bit 3 the sign
 * (crates/oominf-cpu/src/kernel.rs:8-11). */
static const float E2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                               -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

float oracle_e2m1_to_f32(uint8_t code) { return E2M1[code & 15]; }

/* One row of an NVFP4 matrix against x (crates/oominf-cpu/src/kernel.rs:76-98,
 * nvfp4_rows_scalar): w = e2m1(code) * (e4m3(scale) * scale_2), code c the low nibble of
 * byte c / 2 for even c and the high nibble for odd c; acc += w * x in column order. */
static float nvfp4_dot(const uint8_t* packed, const uint8_t* scales, float s2, int64_t cols, const float* x) {
    float acc = 0.0f;
    for (int64_t c = 0; c < cols; c++) {
        uint8_t byte = packed[c / 2];
        uint8_t code = (c % 2 == 0) ? (uint8_t)(byte & 0x0f) : (uint8_t)(byte >> 4);
        float w = E2M1[code] * (oracle_e4m3_to_f32(scales[c / 16]) * s2);
        acc += w * x[c];
    }
    return acc;
}

void oracle_nvfp4_rows(const uint8_t* packed, const uint8_t* scales, float s2, int64_t rows, int64_t cols,
                       const float* x, int T, float* y) {
    for (int64_t r = 0; r < rows; r++)
        for (int t = 0; t < T; t++)
            y[(size_t)t * rows + r] = nvfp4_dot(packed + r * cols / 2, scales + r * cols / 16, s2, cols,
                                                x + (size_t)t * cols);
}

static float rec_f32(const uint8_t* rec, int64_t index) {
    float v;
    memcpy(&v, rec + index * 4, 4);
    return v;
}

/* h[a, j] = silu(x_t . gate_j) * (x_t . up_j) over NVFP4 records (the HostExperts
 * gate/up of crates/oominf-cpu/src/lib.rs:355-369 on kernel.rs:52-98; the device's
 * moe_gate_up, crates/oominf-cuda/kernels/moe.cu:52-106). */
void oracle_moe_gate_up_nvfp4(const uint8_t* const* recs, const int32_t* off, const int32_t* assign_tok, int n_e,
                              const float* x, float* h, const OomNvfp4Record* geo) {
    int64_t H = geo->hidden, I = geo->inter;
    for (int i = 0; i < n_e; i++) {
        const uint8_t* rec = recs[i];
        float s2g = rec_f32(rec, geo->scale2[0]), s2u = rec_f32(rec, geo->scale2[1]);
        for (int a = off[i]; a < off[i + 1]; a++) {
            const float* xt = x + (size_t)assign_tok[a] * H;
            for (int64_t j = 0; j < I; j++) {
                float g = nvfp4_dot(rec + geo->gate_weight + j * H / 2, rec + geo->gate_scale + j * H / 16, s2g, H, xt);
                float u = nvfp4_dot(rec + geo->up_weight + j * H / 2, rec + geo->up_scale + j * H / 16, s2u, H, xt);
                h[(size_t)a * I + j] = siluf(g) * u;
            }
        }
    }
}

/* y[a, r] = h[a] . down_r over NVFP4 records (moe.cu:108-151; kernel.rs:76-98). */
void oracle_moe_down_nvfp4(const uint8_t* const* recs, const int32_t* off, int n_e, const float* h, float* y,
                           const OomNvfp4Record* geo) {
    int64_t H = geo->hidden, I = geo->inter;
    for (int i = 0; i < n_e; i++) {
        const uint8_t* rec = recs[i];
        float s2 = rec_f32(rec, geo->scale2[2]);
        for (int a = off[i]; a < off[i + 1]; a++)
            for (int64_t r = 0; r < H; r++)
                y[(size_t)a * H + r] = nvfp4_dot(rec + geo->down_weight + r * I / 2, rec + geo->down_scale + r * I / 16,
                                                 s2, I, h + (size_t)a * I);
    }
}

/* The tiled NVFP4 grouped GEMM of one projection (moe_tiled, crates/oominf-cuda/kernels/
 * moe.cu:166-335): y[a, r] = (sum_c sum_p term_p(x[row(a), c]) * w(r, c)) * s2, with
 * w(r, c) = e2m1(code) * e4m3(scale) exact (at most 6 significant bits: a bf16 value) and
 * x split into `terms` bf16 terms, hi = bf16(x), each next term bf16 of the remainder
 * (moe.cu:263-273; with three terms they sum to x exactly). The products are exact in
 * fp32 and summed in fp32, term-major within each 16-column group and the groups in
 * column order (the reference's tensor-core passes sum in their own order). The
 * weight_scale_2 scalar sits at float s2_idx of the record. */
void oracle_moe_tiled_nvfp4(const uint8_t* const* recs, const int32_t* off, const int32_t* rows, int n_e,
                            const float* x, float* y, int64_t N, int64_t K, int64_t w_off, int64_t s_off, int s2_idx,
                            int terms) {
    float* wrow = (float*)malloc(sizeof(float) * (size_t)K);
    float* xt = (float*)malloc(sizeof(float) * (size_t)K * 3);
    for (int e = 0; e < n_e; e++) {
        const uint8_t* rec = recs[e];
        float s2 = rec_f32(rec, s2_idx);
        for (int a = off[e]; a < off[e + 1]; a++) {
            const float* xr = x + (size_t)(rows ? rows[a] : a) * K;
            for (int64_t c = 0; c < K; c++) {
                float rem = xr[c];
                for (int p = 0; p < terms; p++) {
                    float tp = oracle_bf16_to_f32(oracle_bf16_from_f32(rem));
                    xt[(size_t)p * K + c] = tp;
                    rem -= tp;
                }
            }
            for (int64_t r = 0; r < N; r++) {
                const uint8_t* cw = rec + w_off + r * K / 2;
                const uint8_t* sc = rec + s_off + r * K / 16;
                for (int64_t c = 0; c < K; c++) {
                    uint8_t code = (c & 1) ? (uint8_t)(cw[c / 2] >> 4) : (uint8_t)(cw[c / 2] & 15);
                    wrow[c] = oracle_e2m1_to_f32(code) * oracle_e4m3_to_f32(sc[c / 16]);
                }
                float acc = 0.0f;
                for (int64_t g = 0; g < K; g += 16)
                    for (int p = 0; p < terms; p++)
                        for (int64_t c = g; c < g + 16; c++) acc += xt[(size_t)p * K + c] * wrow[c];
                y[(size_t)a * N + r] = acc * s2;
            }
        }
    }
    free(wrow);
    free(xt);
}

int oracle_moe_decode_nvfp4(const float* logits, const float* x, const uint8_t* const* all_recs, int T, int E, int k,
                            const OomNvfp4Record* geo, int32_t* ids, float* weights, float* out) {
    int A = T * k;
    int64_t H = geo->hidden, I = geo->inter;
    oracle_router_topk(logits, T, E, k, ids, weights);
    int32_t* experts = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A + 1));
    int32_t* off = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A + 2));
    int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    int32_t* slot = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    int n_e = oracle_moe_plan(ids, T, k, E, experts, off, tok, slot);
    if (n_e < 0) {
        free(experts); free(off); free(tok); free(slot);
        return -1;
    }
    const uint8_t** recs = (const uint8_t**)malloc(sizeof(void*) * (size_t)(n_e ? n_e : 1));
    for (int i = 0; i < n_e; i++) recs[i] = all_recs[experts[i]];
    float* h = (float*)malloc(sizeof(float) * (size_t)A * (size_t)I);
    float* y = (float*)malloc(sizeof(float) * (size_t)A * (size_t)H);
    oracle_moe_gate_up_nvfp4(recs, off, tok, n_e, x, h, geo);
    oracle_moe_down_nvfp4(recs, off, n_e, h, y, geo);
    oracle_moe_combine_slots(y, slot, weights, out, T, (int)H, k);
    free(h); free(y); free(recs); free(experts); free(off); free(tok); free(slot);
    return 0;
}

/* ---- prefill grouped GEMM (FP8 x FP8) ---------------------------------------- */

void oracle_grouped_gemm_fp8(const uint8_t* const* recs, const int32_t* off, const int32_t* rows, int n_e,
                             const uint8_t* xq, const float* x_scale, int x_group, float* y, int64_t N, int64_t K,
                             int64_t w_off, int64_t s_off) {
    int64_t nkb = cdiv(K, 128);
    float* xd = (float*)malloc(sizeof(float) * (size_t)K);
    for (int i = 0; i < n_e; i++) {
        const uint8_t* W = recs[i] + w_off;
        const float* S = (const float*)(recs[i] + s_off);
        for (int a = off[i]; a < off[i + 1]; a++) {
            int64_t row = rows ? rows[a] : a;
            for (int64_t c = 0; c < K; c++) xd[c] = oracle_e4m3_to_f32(xq[row * K + c]);
            for (int64_t r = 0; r < N; r++) {
                float acc = 0.0f;
                for (int64_t kb = 0; kb < nkb; kb++) {
                    float blk = 0.0f;
                    for (int64_t c = kb * 128; c < K && c < (kb + 1) * 128; c++)
                        blk += xd[c] * oracle_e4m3_to_f32(W[r * K + c]);
                    float ws = S[(r / 128) * nkb + kb];
                    if (x_group) acc += blk * (ws * x_scale[row * nkb + kb]);
                    else acc += blk * ws;
                }
                y[(size_t)a * N + r] = x_group ? acc : acc * x_scale[row];
            }
        }
    }
    free(xd);
}

int oracle_moe_prefill_fp8(const float* logits, const float* x, const uint8_t* const* all_recs, int T, int E, int k,
                           const OomFp8Record* geo, int h_bf16, int32_t* ids, float* weights, float* out) {
    int A = T * k;
    int64_t H = geo->hidden, I = geo->inter;
    oracle_router_topk(logits, T, E, k, ids, weights);
    int32_t* experts = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A + 1));
    int32_t* off = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A + 2));
    int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    int32_t* slot = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    int n_e = oracle_moe_plan(ids, T, k, E, experts, off, tok, slot);
    if (n_e < 0) {
        free(experts); free(off); free(tok); free(slot);
        return -1;
    }
    const uint8_t** recs = (const uint8_t**)malloc(sizeof(void*) * (size_t)(n_e ? n_e : 1));
    for (int i = 0; i < n_e; i++) recs[i] = all_recs[experts[i]];
    uint8_t* xq = (uint8_t*)malloc((size_t)T * (size_t)H);
    float* xs = (float*)malloc(sizeof(float) * (size_t)T);
    oracle_quantize_act(x, T, H, 0, xq, xs);
    float* g = (float*)malloc(sizeof(float) * (size_t)A * (size_t)I);
    float* u = (float*)malloc(sizeof(float) * (size_t)A * (size_t)I);
    oracle_grouped_gemm_fp8(recs, off, tok, n_e, xq, xs, 0, g, I, H, geo->gate_weight, geo->gate_scale);
    oracle_grouped_gemm_fp8(recs, off, tok, n_e, xq, xs, 0, u, I, H, geo->up_weight, geo->up_scale);
    for (size_t i = 0; i < (size_t)A * (size_t)I; i++) g[i] = siluf(g[i]) * u[i];
    /* h into the down projection: fp32, as the reference's exact tiled path keeps its
     * activations (ExpertPrecision::Exact, crates/oominf-core/src/backend.rs:144-149;
     * crates/oominf-cuda/kernels/moe.cu:166-335 with three bf16 terms), or rounded to bf16
     * (ExpertPrecision::Bf16, one tensor-core pass; h_bf16 set); then the decode path's
     * down, per-128-column block sums times the block scale. */
    if (h_bf16)
        for (size_t i = 0; i < (size_t)A * (size_t)I; i++) g[i] = oracle_bf16_to_f32(oracle_bf16_from_f32(g[i]));
    float* y = (float*)malloc(sizeof(float) * (size_t)A * (size_t)H);
    oracle_moe_down_fp8(recs, off, n_e, g, y, geo);
    oracle_moe_combine_slots(y, slot, weights, out, T, (int)H, k);
    free(y); free(g); free(u); free(xq); free(xs);
    free(recs); free(experts); free(off); free(tok); free(slot);
    return n_e;
}

/* ---- paged GQA decode attention ---------------------------------------------- */

/* attention.cu:449-548 for one query token: key tiles of 16; per row the tile's
 * scores s = (q . k) * scale (dot in d order), tile max by a 16-lane xor tree,
 * e = exp(s - m_new), tile sum by the same tree, l = l * exp(m_old - m_new) + sum,
 * acc = acc * corr + sum_j e_j v_j in key order; out = acc / l. */
static float tree16_sum(const float* v) {
    float a[16];
    memcpy(a, v, sizeof(a));
    for (int o = 8; o > 0; o >>= 1) {
        float n[16];
        for (int i = 0; i < 16; i++) n[i] = a[i] + a[i ^ o];
        memcpy(a, n, sizeof(a));
    }
    return a[0];
}

void oracle_attn_decode_paged(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                              const int32_t* page_table, int page_size, int kv_len, int H, int Hkv, int D,
                              float scale, float* out) {
    int G = H / Hkv;
    float* qf = (float*)malloc(sizeof(float) * (size_t)D);
    float* acc = (float*)malloc(sizeof(float) * (size_t)D);
    float* vrow = (float*)malloc(sizeof(float) * 16 * (size_t)D);
    for (int h = 0; h < H; h++) {
        int kvh = h / G;
        for (int d = 0; d < D; d++) qf[d] = oracle_bf16_to_f32(q[(size_t)h * D + d]);
        for (int d = 0; d < D; d++) acc[d] = 0.0f;
        float m = -INFINITY, l = 0.0f;
        for (int j0 = 0; j0 < kv_len; j0 += 16) {
            float s[16], e[16];
            for (int jj = 0; jj < 16; jj++) {
                int j = j0 + jj;
                if (j >= kv_len) {
                    s[jj] = -INFINITY;
                    continue;
                }
                /* pages [n_pages, Hkv, page_size, D]: KV head kvh's slot j % page_size */
                size_t row = ((size_t)page_table[j / page_size] * Hkv + kvh) * page_size + (size_t)(j % page_size);
                const uint16_t* kr = k_pages + row * D;
                const uint16_t* vr = v_pages + row * D;
                float dot = 0.0f;
                for (int d = 0; d < D; d++) dot += qf[d] * oracle_bf16_to_f32(kr[d]);
                s[jj] = dot * scale;
                for (int d = 0; d < D; d++) vrow[jj * D + d] = oracle_bf16_to_f32(vr[d]);
            }
            float mt = -INFINITY;
            for (int jj = 0; jj < 16; jj++) mt = fmaxf(mt, s[jj]);
            float mn = fmaxf(m, mt);
            for (int jj = 0; jj < 16; jj++) e[jj] = (mn == -INFINITY || s[jj] == -INFINITY) ? 0.0f : expf(s[jj] - mn);
            float sum = tree16_sum(e);
            float corr = mn == -INFINITY ? 1.0f : expf(m - mn);
            l = l * corr + sum;
            m = mn;
            for (int d = 0; d < D; d++) {
                float a = acc[d] * corr;
                for (int jj = 0; jj < 16; jj++)
                    if (j0 + jj < kv_len) a += e[jj] * vrow[jj * D + d];
                acc[d] = a;
            }
        }
        for (int d = 0; d < D; d++) out[(size_t)h * D + d] = acc[d] / l;
    }
    free(qf);
    free(acc);
    free(vrow);
}

/* ---- the shared expert and the whole decode layer --------------------------------- */

/* ops.cu:10,310-316: out = routed + sigmoid(gate[t]) * shared, sigmoid(v) = 1 / (1 + expf(-v)). */
void oracle_moe_combine_shared(const float* routed, const float* shared, const float* gate, float* out, int T, int H) {
    for (int t = 0; t < T; t++) {
        const float sg = 1.0f / (1.0f + expf(-gate[t]));
        for (int c = 0; c < H; c++) out[(size_t)t * H + c] = routed[(size_t)t * H + c] + sg * shared[(size_t)t * H + c];
    }
}

/* moe.rs:254-366 with every routed expert resident and moe.rs:498-527 (the shared
 * expert: gemm_w of the stacked gate/up, silu_mul_rows, gemm_w of down; its gate logit by
 * gemm_w; moe_combine). logits [T, E] and gate [T] are written too. */
int oracle_moe_layer_decode_fp8(const float* x, int T, const uint16_t* router_w, const uint8_t* const* all_recs,
                                int E, int k, const OomFp8Record* geo, const uint8_t* shared_rec,
                                const OomFp8Record* sgeo, const uint16_t* gate_w, float* logits, float* gate,
                                int32_t* ids, float* weights, float* out) {
    const int64_t H = geo->hidden;
    oracle_gemv_bf16(x, T, router_w, E, H, logits);
    oracle_gemv_bf16(x, T, gate_w, 1, H, gate);
    float* routed = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* shared = (float*)malloc(sizeof(float) * (size_t)T * H);
    int32_t* sids = (int32_t*)malloc(sizeof(int32_t) * (size_t)T);
    float* sw = (float*)malloc(sizeof(float) * (size_t)T);
    int rc = oracle_moe_decode_fp8(logits, x, all_recs, T, E, k, geo, ids, weights, routed);
    if (rc == 0) {
        /* the shared expert: one expert, weight 1 */
        const uint8_t* srecs[1] = {shared_rec};
        rc = oracle_moe_decode_fp8(gate, x, srecs, T, 1, 1, sgeo, sids, sw, shared);
    }
    if (rc == 0) oracle_moe_combine_shared(routed, shared, gate, out, T, (int)H);
    free(routed);
    free(shared);
    free(sids);
    free(sw);
    return rc;
}
