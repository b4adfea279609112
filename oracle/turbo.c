/*
 * turbo.c -- Turbo KV cache rows, mask_compact and the D = 256, G = 12 flash-decode
 * attention of oom-inference, restated on the CPU. TEST INFRASTRUCTURE ONLY (see
 * oom_oracle.h).
 *
 * Paths relative to projects/oom-inference/:
 *   KvFormat rows and codebooks   crates/oominf-core/src/backend.rs:571-700
 *   kv_rotate / kv_append / kv_read  crates/oominf-cuda/kernels/attention.cu:9-131
 *   mask_compact                  crates/oominf-cuda/kernels/attention.cu:363-374
 *   flash decode (partial, combine)  crates/oominf-cuda/kernels/attention.cu:584-686,
 *                                 dispatch crates/oominf-cuda/src/attention.rs:265-447
 * fp32 with the reference's operation order (butterflies, per-lane dot then a 32-lane xor
 * tree, online softmax per key); the multiply-adds of the partials and the combine are
 * written as fused multiply-adds, the form the device kernels use.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oom_oracle.h"

/* ---- fp16 ---------------------------------------------------------------------- */

/* m >> s rounded to nearest, ties to even (s >= 1). */
static uint32_t rne_shift(uint32_t m, int s) {
    if (s >= 32) return 0;
    uint32_t q = m >> s, rem = m & ((1u << s) - 1u), half = 1u << (s - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return q;
}

uint16_t oracle_f16_from_f32(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, mant = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    if (exp == 0u) return (uint16_t)sign; /* f32 subnormals are far below f16's range */
    const uint32_t M = mant | 0x800000u;  /* value = M * 2^(exp - 150) */
    const int e = (int)exp - 112;         /* f16 biased exponent */
    if (e >= 1) {
        uint32_t q = rne_shift(M, 13); /* 11 significant bits */
        int ee = e;
        if (q == 0x800u) {
            q = 0x400u;
            ee++;
        }
        if (ee >= 31) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | ((uint32_t)ee << 10) | (q & 0x3ffu));
    }
    /* subnormal f16: units of 2^-24 */
    return (uint16_t)(sign | rne_shift(M, 126 - (int)exp));
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    float v;
    if (exp == 0) v = ldexpf((float)mant, -24);
    else if (exp == 31) v = mant ? NAN : INFINITY;
    else v = ldexpf((float)(mant | 0x400u), (int)exp - 25);
    return sign ? -v : v;
}

/* ---- codebooks (backend.rs:637-700) ------------------------------------------- */

static void lloyd_max(int bits, float* out) {
    const int n = 1 << bits;
    const double SQRT_2 = 1.4142135623730951, TWO_PI = 6.283185307179586;
    double* c = (double*)malloc(sizeof(double) * (size_t)n);
    double* nx = (double*)malloc(sizeof(double) * (size_t)n);
    const double span = 4.0 + bits * 0.25;
    for (int i = 0; i < n; i++) c[i] = -span + 2.0 * span * (i + 0.5) / n;
    for (int round = 0; round < 200000; round++) {
        double moved = 0.0;
        for (int i = 0; i < n; i++) {
            const double a = i == 0 ? -INFINITY : 0.5 * (c[i - 1] + c[i]);
            const double b = i + 1 == n ? INFINITY : 0.5 * (c[i] + c[i + 1]);
            const double pa = isfinite(a) ? exp(-0.5 * a * a) / sqrt(TWO_PI) : 0.0;
            const double pb = isfinite(b) ? exp(-0.5 * b * b) / sqrt(TWO_PI) : 0.0;
            double qv[2];
            const double xs[2] = {a, b};
            for (int s = 0; s < 2; s++) { /* upper tail Q(x) from the Numerical Recipes erfcc */
                const double x = xs[s], z = fabs(x) / SQRT_2, t = 1.0 / (1.0 + 0.5 * z);
                const double erfc =
                    t * exp(-z * z - 1.26551223 +
                            t * (1.00002368 +
                                 t * (0.37409196 +
                                      t * (0.09678418 +
                                           t * (-0.18628806 +
                                                t * (0.27886807 +
                                                     t * (-1.13520398 +
                                                          t * (1.48851587 + t * (-0.82215223 + t * 0.17087277)))))))));
                qv[s] = x >= 0.0 ? 0.5 * erfc : 1.0 - 0.5 * erfc;
            }
            const double mass = qv[0] - qv[1];
            const double m = mass > 0.0 ? (pa - pb) / mass : c[i];
            if (fabs(m - c[i]) > moved) moved = fabs(m - c[i]);
            nx[i] = m;
        }
        double* tmp = c;
        c = nx;
        nx = tmp;
        if (moved < 1e-12) break;
    }
    for (int i = 0; i < n; i++) out[i] = (float)c[i];
    free(c);
    free(nx);
}

void oracle_kv_codebooks(float* levels) {
    int at = 0;
    for (int b = 2; b <= 8; b++) {
        lloyd_max(b, levels + at);
        at += 1 << b;
    }
}

/* ---- rows (attention.cu:9-131) -------------------------------------------------- */

static int scale_bytes(int D) { return ((D / 32) * 2 + 15) & ~15; }
size_t oracle_kv_row_bytes(int D, int bits) {
    return bits ? (size_t)scale_bytes(D) + (size_t)(D / 32) * bits * 4 : (size_t)D * 4;
}
static float sign_of(int i) { return (((unsigned)i * 2654435761u) >> 31) ? -1.0f : 1.0f; }

/* unnormalised Walsh-Hadamard transform, stages h = 1, 2, 4, ... */
static void wht(float* s, int D) {
    for (int h = 1; h < D; h <<= 1)
        for (int i = 0; i < D; i++)
            if ((i & h) == 0) {
                const float a = s[i], b = s[i + h];
                s[i] = a + b;
                s[i + h] = a - b;
            }
}

void oracle_kv_rotate(float* x, int rows, int D, int inverse) {
    float s[256];
    const float norm = 1.0f / sqrtf((float)D);
    for (int r = 0; r < rows; r++) {
        float* v = x + (size_t)r * D;
        for (int i = 0; i < D; i++) s[i] = inverse ? v[i] : v[i] * sign_of(i);
        wht(s, D);
        for (int i = 0; i < D; i++) v[i] = inverse ? s[i] * sign_of(i) * norm : s[i] * norm;
    }
}

/* The sum of v[0..32) by the xor butterfly 16, 8, 4, 2, 1 (the value every lane holds). */
static float xor_tree32(const float* v0) {
    float v[32], n[32];
    memcpy(v, v0, sizeof(v));
    for (int o = 16; o > 0; o >>= 1) {
        for (int l = 0; l < 32; l++) n[l] = v[l] + v[l ^ o];
        memcpy(v, n, sizeof(v));
    }
    return v[0];
}

void oracle_kv_append(const float* src, uint8_t* cache, int64_t row0, int rows, int D, int bits,
                      const float* levels) {
    const size_t rb = oracle_kv_row_bytes(D, bits);
    float s[256], y2[32];
    for (int r = 0; r < rows; r++) {
        const float* x = src + (size_t)r * D;
        uint8_t* row = cache + ((size_t)row0 + r) * rb;
        if (!bits) {
            memcpy(row, x, (size_t)D * 4);
            continue;
        }
        const float* lv = levels + ((1 << bits) - 4);
        for (int i = 0; i < D; i++) s[i] = x[i] * sign_of(i);
        wht(s, D);
        for (int b = 0; b < D / 32; b++) {
            float y[32];
            int idx[32];
            for (int l = 0; l < 32; l++) {
                y[l] = s[32 * b + l] / sqrtf((float)D);
                y2[l] = y[l] * y[l];
            }
            const float ss = xor_tree32(y2);
            const uint16_t hs = oracle_f16_from_f32(sqrtf(ss / 32.0f));
            const float sc = oracle_f16_to_f32(hs);
            for (int l = 0; l < 32; l++) {
                const float u = sc > 0.0f ? y[l] / sc : 0.0f;
                int lo = 0, hi = (1 << bits) - 1;
                while (hi - lo > 1) {
                    const int mid = (lo + hi) >> 1;
                    if (lv[mid] <= u) lo = mid;
                    else hi = mid;
                }
                idx[l] = fabsf(u - lv[lo]) <= fabsf(u - lv[hi]) ? lo : hi;
            }
            memcpy(row + 2 * b, &hs, 2);
            for (int j = 0; j < bits; j++) {
                uint32_t w = 0;
                for (int l = 0; l < 32; l++) w |= (uint32_t)((idx[l] >> j) & 1) << l;
                memcpy(row + scale_bytes(D) + ((size_t)b * bits + j) * 4, &w, 4);
            }
        }
    }
}

static float row_value(const uint8_t* row, int d, int D, int bits, const float* lv) {
    if (!bits) {
        float v;
        memcpy(&v, row + 4 * (size_t)d, 4);
        return v;
    }
    const int b = d >> 5, lane = d & 31;
    uint16_t hs;
    memcpy(&hs, row + 2 * b, 2);
    int idx = 0;
    for (int j = 0; j < bits; j++) {
        uint32_t w;
        memcpy(&w, row + scale_bytes(D) + ((size_t)b * bits + j) * 4, 4);
        idx |= (int)((w >> lane) & 1u) << j;
    }
    return lv[idx] * oracle_f16_to_f32(hs);
}

void oracle_kv_read(const uint8_t* cache, float* dst, int rows, int D, int bits, const float* levels) {
    const size_t rb = oracle_kv_row_bytes(D, bits);
    const float* lv = bits ? levels + ((1 << bits) - 4) : NULL;
    float s[256];
    for (int r = 0; r < rows; r++) {
        const uint8_t* row = cache + (size_t)r * rb;
        float* out = dst + (size_t)r * D;
        for (int i = 0; i < D; i++) s[i] = row_value(row, i, D, bits, lv);
        if (!bits) {
            memcpy(out, s, (size_t)D * 4);
            continue;
        }
        wht(s, D);
        for (int i = 0; i < D; i++) out[i] = s[i] * sign_of(i) / sqrtf((float)D);
    }
}

/* ---- mask_compact (attention.cu:363-374) ----------------------------------------- */

int oracle_mask_compact(const uint8_t* mask, int32_t* sel, int n) {
    int c = 0;
    for (int j = 0; j < n; j++)
        if (mask[j]) sel[1 + c++] = j;
    sel[0] = c;
    return c;
}

/* ---- flash decode, d = 256, G = 12 (attention.cu:584-686; attention.rs:365-447) --- */

void oracle_attn_decode_turbo(const float* q, const uint8_t* k, const uint8_t* v, int kb, int vb,
                              const float* levels, const uint8_t* mask, int H, int Hkv, int kv_len, float scale,
                              float* out) {
    enum { D = 256, G = 12, E = 8 };
    const size_t krow = oracle_kv_row_bytes(D, kb), vrow = oracle_kv_row_bytes(D, vb);
    const float* lvk = kb ? levels + ((1 << kb) - 4) : NULL;
    const float* lvv = vb ? levels + ((1 << vb) - 4) : NULL;
    float* qr = (float*)malloc(sizeof(float) * (size_t)H * D);
    memcpy(qr, q, sizeof(float) * (size_t)H * D);
    if (kb) oracle_kv_rotate(qr, H, D, 0);
    int32_t* sel = (int32_t*)malloc(sizeof(int32_t) * (size_t)(kv_len + 1));
    const int count = oracle_mask_compact(mask, sel, kv_len);
    int P = ((kv_len < 4096 ? kv_len : 4096) + 15) / 16;
    P = (P + 7) / 8 * 8;
    const int chunk = (count + P - 1) / P;
    /* part[kvh][p][g]: acc[D], m, l */
    float* part = (float*)malloc(sizeof(float) * (size_t)Hkv * P * G * (D + 2));
    float kk[D], vv[D], dl[32];
    for (int kvh = 0; kvh < Hkv; kvh++)
        for (int p = 0; p < P; p++) {
            float acc[G][D], m[G], l[G];
            for (int g = 0; g < G; g++) {
                m[g] = -INFINITY;
                l[g] = 0.0f;
                for (int d = 0; d < D; d++) acc[g][d] = 0.0f;
            }
            int i0 = p * chunk < count ? p * chunk : count;
            int i1 = i0 + chunk < count ? i0 + chunk : count;
            for (int i = i0; i < i1; i++) {
                const int j = sel[1 + i];
                const uint8_t* kr = k + ((size_t)j * Hkv + kvh) * krow;
                const uint8_t* vr = v + ((size_t)j * Hkv + kvh) * vrow;
                for (int d = 0; d < D; d++) {
                    kk[d] = row_value(kr, d, D, kb, lvk);
                    vv[d] = row_value(vr, d, D, vb, lvv);
                }
                for (int g = 0; g < G; g++) {
                    const float* qg = qr + ((size_t)kvh * G + g) * D;
                    for (int lane = 0; lane < 32; lane++) { /* lane owns d = lane + 32 e */
                        float dot = 0.0f;
                        for (int e = 0; e < E; e++) dot = fmaf(qg[32 * e + lane], kk[32 * e + lane], dot);
                        dl[lane] = dot;
                    }
                    const float s = xor_tree32(dl) * scale;
                    const float mn = fmaxf(m[g], s);
                    const float corr = expf(m[g] - mn);
                    const float w = expf(s - mn);
                    l[g] = l[g] * corr + w;
                    for (int d = 0; d < D; d++) acc[g][d] = fmaf(acc[g][d], corr, w * vv[d]);
                    m[g] = mn;
                }
            }
            for (int g = 0; g < G; g++) {
                float* o = part + (((size_t)kvh * P + p) * G + g) * (D + 2);
                memcpy(o, acc[g], sizeof(float) * D);
                o[D] = m[g];
                o[D + 1] = l[g];
            }
        }
    for (int h = 0; h < H; h++) {
        const int kvh = h / G, g = h % G;
        float M = -INFINITY;
        for (int p = 0; p < P; p++) M = fmaxf(M, part[(((size_t)kvh * P + p) * G + g) * (D + 2) + D]);
        for (int d = 0; d < D; d++) {
            float num = 0.0f, den = 0.0f;
            for (int p = 0; p < P; p++) {
                const float* pr = part + (((size_t)kvh * P + p) * G + g) * (D + 2);
                if (pr[D] == -INFINITY) continue;
                const float w = expf(pr[D] - M);
                num = fmaf(w, pr[d], num);
                den = fmaf(w, pr[D + 1], den);
            }
            out[(size_t)h * D + d] = num / den;
        }
    }
    if (kb) oracle_kv_rotate(out, H, D, 1);
    free(part);
    free(sel);
    free(qr);
}
