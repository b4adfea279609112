/*
 * bf16rec.c -- the routed experts over bf16 records (layout tag "bf16"), restated on the
 * CPU. TEST INFRASTRUCTURE ONLY (see oom_oracle.h).
 *
 * Paths relative to projects/oom-inference/:
 *   moe_gate_up_bf16 / moe_down_bf16   crates/oominf-cuda/kernels/moe.cu:343-443
 *   trait methods                      crates/oominf-core/src/backend.rs:837-858
 *   Bf16Record                         crates/oominf-core/src/backend.rs:800-807
 * A row dot product follows the reference kernel's order: 32 lanes, lane t adding the
 * 8-weight groups t, t + 32, ... in order, each group as two halves of four products
 * summed left to right ((w0 x0 + w1 x1) + w2 x2) + w3 x3 onto the lane's sum; then the
 * lanes' sums by a 32-way xor butterfly (partner offsets 16, 8, 4, 2, 1). Weights widen
 * exactly from bf16; fp32 products and sums, no fused multiply-adds.
 */
#include <math.h>
#include <string.h>

#include "oom_oracle.h"

static float bf(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float lanes_xor32(float* v) {
    float n[32];
    for (int o = 16; o > 0; o >>= 1) {
        for (int l = 0; l < 32; l++) n[l] = v[l] + v[l ^ o];
        memcpy(v, n, sizeof(n));
    }
    return v[0];
}

/* sum_c w[c] * x[c] over a row of n (a multiple of 8) bf16 weights. */
static float bf16_row_dot(const uint16_t* w, const float* x, int64_t n) {
    float lanes[32];
    for (int t = 0; t < 32; t++) {
        float acc = 0.0f;
        for (int64_t g = t; g < n / 8; g += 32)
            for (int q = 0; q < 2; q++) {
                const uint16_t* wq = w + g * 8 + 4 * q;
                const float* xq = x + g * 8 + 4 * q;
                acc += bf(wq[0]) * xq[0] + bf(wq[1]) * xq[1] + bf(wq[2]) * xq[2] + bf(wq[3]) * xq[3];
            }
        lanes[t] = acc;
    }
    return lanes_xor32(lanes);
}

static float silu(float v) { return v / (1.0f + expf(-v)); }

void oracle_moe_gate_up_bf16(const uint8_t* const* recs, const int32_t* off, const int32_t* assign_tok, int n_e,
                             const float* x, float* h, const OomBf16Record* geo) {
    const int64_t H = geo->hidden, I = geo->inter;
    for (int i = 0; i < n_e; i++) {
        const uint16_t* gw = (const uint16_t*)(recs[i] + geo->gate_weight);
        const uint16_t* uw = (const uint16_t*)(recs[i] + geo->up_weight);
        for (int a = off[i]; a < off[i + 1]; a++) {
            const float* xt = x + (size_t)assign_tok[a] * H;
            for (int64_t j = 0; j < I; j++) {
                const float g = bf16_row_dot(gw + j * H, xt, H);
                const float u = bf16_row_dot(uw + j * H, xt, H);
                h[(size_t)a * I + j] = silu(g) * u;
            }
        }
    }
}

void oracle_moe_down_bf16(const uint8_t* const* recs, const int32_t* off, int n_e, const float* h, float* y,
                          const OomBf16Record* geo) {
    const int64_t H = geo->hidden, I = geo->inter;
    for (int i = 0; i < n_e; i++) {
        const uint16_t* dw = (const uint16_t*)(recs[i] + geo->down_weight);
        for (int a = off[i]; a < off[i + 1]; a++)
            for (int64_t r = 0; r < H; r++) y[(size_t)a * H + r] = bf16_row_dot(dw + r * I, h + (size_t)a * I, I);
    }
}
