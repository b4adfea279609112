/*
 * formats.c -- e4m3fn / bf16 encodings, block quantisers and seeded generators.
 * TEST INFRASTRUCTURE (the oracle): never linked into the product library.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "oom_oracle.h"

static inline uint32_t f32_bits(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return b;
}

static inline float bits_f32(uint32_t b) {
    float v;
    memcpy(&v, &b, 4);
    return v;
}

/* crates/oominf-core/src/fp8.rs:5-27: sign, saturation at 448, subnormals in steps
 * of 2^-9 (rounding up to 8 steps gives the smallest normal, code 0x08), normals by
 * exponent and a 3-bit mantissa rounded to nearest even, carry into the exponent. */
uint8_t oracle_e4m3_from_f32(float x) {
    uint8_t sign = signbit(x) ? 0x80 : 0;
    float a = fabsf(x);
    if (isnan(a) || a >= 448.0f) return sign | 0x7e;
    if (a < 0x1p-6f) return sign | (uint8_t)rintf(a * 512.0f);
    int e = (int)((f32_bits(a) >> 23) & 0xff) - 127;
    int m = (int)rintf((a / ldexpf(1.0f, e) - 1.0f) * 8.0f);
    if (m == 8) {
        m = 0;
        e += 1;
    }
    int biased = e + 7;
    if (biased > 15 || (biased == 15 && m == 7)) return sign | 0x7e;
    return sign | (uint8_t)(biased << 3) | (uint8_t)m;
}

/* crates/oominf-cpu/src/kernel.rs:14-27: exact value; S.1111.111 is NaN. */
float oracle_e4m3_to_f32(uint8_t b) {
    float s = (b & 0x80) ? -1.0f : 1.0f;
    int e = (b >> 3) & 0x0f;
    int m = b & 0x07;
    if (e == 0x0f && m == 0x07) return NAN;
    float mag = e == 0 ? (float)m / 8.0f * 0x1p-6f : (1.0f + (float)m / 8.0f) * ldexpf(1.0f, e - 7);
    return s * mag;
}

/* crates/oominf-cuda/tests/gemv.rs:23-27 (round to nearest even). */
uint16_t oracle_bf16_from_f32(float v) {
    uint32_t b = f32_bits(v);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

void oracle_bf16_from_f32_n(const float* v, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_bf16_from_f32(v[i]);
}

void oracle_bf16_to_f32_n(const uint16_t* b, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_bf16_to_f32(b[i]);
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int64_t oracle_scale_count(int64_t n, int64_t k, int layout) {
    switch (layout) {
        case OOM_SCALE_ROW: return n;
        case OOM_SCALE_1X128: return n * cdiv(k, 128);
        case OOM_SCALE_128X128: return cdiv(n, 128) * cdiv(k, 128);
        default: return -1;
    }
}

float oracle_scale_at(const float* scale, int64_t n, int64_t k, int layout, int64_t r, int64_t c) {
    (void)n;
    switch (layout) {
        case OOM_SCALE_ROW: return scale[r];
        case OOM_SCALE_1X128: return scale[r * cdiv(k, 128) + c / 128];
        default: return scale[(r / 128) * cdiv(k, 128) + c / 128];
    }
}

/* fp8.rs:48-88 generalised over the block shape: each block's scale is its
 * absolute maximum over 448 (1 for an all-zero block) and q = e4m3(w / scale). */
int oracle_quantize(const uint16_t* w, int64_t n, int64_t k, int layout, uint8_t* q, float* scale) {
    int64_t br, bc;
    switch (layout) {
        case OOM_SCALE_ROW: br = 1; bc = k; break;
        case OOM_SCALE_1X128: br = 1; bc = 128; break;
        case OOM_SCALE_128X128: br = 128; bc = 128; break;
        default: return -1;
    }
    int64_t nbc = cdiv(k, bc);
    for (int64_t r0 = 0; r0 < n; r0 += br) {
        for (int64_t b = 0; b < nbc; b++) {
            int64_t c0 = b * bc, c1 = c0 + bc < k ? c0 + bc : k;
            int64_t r1 = r0 + br < n ? r0 + br : n;
            float amax = 0.0f;
            for (int64_t r = r0; r < r1; r++)
                for (int64_t c = c0; c < c1; c++) amax = fmaxf(amax, fabsf(oracle_bf16_to_f32(w[r * k + c])));
            float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            scale[(r0 / br) * nbc + b] = s;
            for (int64_t r = r0; r < r1; r++)
                for (int64_t c = c0; c < c1; c++) q[r * k + c] = oracle_e4m3_from_f32(oracle_bf16_to_f32(w[r * k + c]) / s);
        }
    }
    return 0;
}

void oracle_quantize_act(const float* x, int64_t rows, int64_t cols, int64_t group, uint8_t* q, float* scale) {
    int64_t g = group > 0 ? group : cols;
    int64_t ng = cdiv(cols, g);
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t b = 0; b < ng; b++) {
            int64_t c0 = b * g, c1 = c0 + g < cols ? c0 + g : cols;
            float amax = 0.0f;
            for (int64_t c = c0; c < c1; c++) amax = fmaxf(amax, fabsf(x[r * cols + c]));
            float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            scale[r * ng + b] = s;
            for (int64_t c = c0; c < c1; c++) q[r * cols + c] = oracle_e4m3_from_f32(x[r * cols + c] / s);
        }
    }
}

/* ---- generators ---------------------------------------------------------- */

uint64_t oracle_xorshift64s(uint64_t* s) {
    uint64_t x = *s;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return x * 0x2545F4914F6CDD1DULL;
}

uint64_t oracle_seed(uint64_t base, uint64_t stream) {
    uint64_t z = base + (stream + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return z ? z : 1;
}

/* crates/oominf-cuda/tests/kv_cache.rs:10-24: uniforms ((s * M) >> 11 + 0.5) / 2^53
 * from xorshift64*, one normal sqrt(-2 ln u) cos(2 pi v) per pair, in f64, cast to f32. */
void oracle_gaussian(float* out, size_t n, uint64_t seed, float std) {
    uint64_t s = seed ? seed : 1;
    const double tau = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i++) {
        double u = ((double)(oracle_xorshift64s(&s) >> 11) + 0.5) / 9007199254740992.0;
        double v = ((double)(oracle_xorshift64s(&s) >> 11) + 0.5) / 9007199254740992.0;
        float g = (float)(sqrt(-2.0 * log(u)) * cos(tau * v));
        out[i] = g * std;
    }
}

typedef struct {
    uint16_t* out;
    size_t n, chunk, c0, c1;
    uint64_t seed;
    float std;
} GaussJob;

static void* gauss_worker(void* p) {
    GaussJob* j = (GaussJob*)p;
    float* tmp = (float*)malloc(j->chunk * sizeof(float));
    for (size_t c = j->c0; c < j->c1; c++) {
        size_t a = c * j->chunk, len = a + j->chunk <= j->n ? j->chunk : j->n - a;
        oracle_gaussian(tmp, len, oracle_seed(j->seed, c), j->std);
        oracle_bf16_from_f32_n(tmp, j->out + a, len);
    }
    free(tmp);
    return NULL;
}

void oracle_gaussian_bf16(uint16_t* out, size_t n, uint64_t seed, float std, size_t chunk, int threads) {
    if (chunk == 0) chunk = n ? n : 1;
    size_t chunks = (n + chunk - 1) / chunk;
    if (threads < 1) threads = 1;
    if ((size_t)threads > chunks) threads = (int)(chunks ? chunks : 1);
    pthread_t tid[256];
    GaussJob jobs[256];
    if (threads > 256) threads = 256;
    size_t per = (chunks + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; t++) {
        jobs[t] = (GaussJob){out, n, chunk, t * per, (t + 1) * per < chunks ? (t + 1) * per : chunks, seed, std};
        if (jobs[t].c0 >= jobs[t].c1) break;
        if (t == threads - 1 || pthread_create(&tid[t], NULL, gauss_worker, &jobs[t]) != 0) {
            gauss_worker(&jobs[t]);
            tid[t] = 0;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; t++)
        if (tid[t]) pthread_join(tid[t], NULL);
}

void oracle_permutation(int32_t* out, int n, uint64_t seed) {
    uint64_t s = seed ? seed : 1;
    for (int i = 0; i < n; i++) out[i] = i;
    for (int i = n - 1; i > 0; i--) {
        int j = (int)(oracle_xorshift64s(&s) % (uint64_t)(i + 1));
        int32_t t = out[i];
        out[i] = out[j];
        out[j] = t;
    }
}

void oracle_zipf_bias(float* bias, int E, double s, uint64_t seed) {
    int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    oracle_permutation(perm, E, seed);
    double h = 0.0;
    for (int r = 1; r <= E; r++) h += pow((double)r, -s);
    /* perm[i] is the expert of rank i + 1 */
    for (int i = 0; i < E; i++) bias[perm[i]] = (float)log(pow((double)(i + 1), -s) / h);
    free(perm);
}
