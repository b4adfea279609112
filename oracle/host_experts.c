/*
 * host_experts.c -- the reference's CPU path for routed experts (crates/oominf-cpu),
 * restated for e4m3 records with 128x128 block scales. Timed as the CPU baseline.
 * TEST INFRASTRUCTURE (the oracle): never linked into the product library.
 *
 * Structure (crates/oominf-cpu/src/lib.rs:175-323, HostExperts::run):
 *   1. jobs with more than MAX_TOKENS (4) tokens get their inputs by column,
 *      [hidden, s] with s = tokens rounded up to LANES (16) (lib.rs:190-211);
 *   2. gate/up rows in work items of GATE_ROWS (32) rows, SwiGLU in place
 *      (lib.rs:227-257);
 *   3. down rows in items of DOWN_ROWS (128) (lib.rs:276-302);
 *   4. output rows by job, then token (lib.rs:305-316).
 * Small jobs run the per-row vector kernel (kernel.rs:374-412 shape), large jobs
 * decode each item's rows once and run the register-tiled GEMM over token
 * columns (lib.rs:386-438, kernel.rs:164-185, 329-372). e4m3 decodes by exact bit
 * construction (crates/oominf-metal/src/kernels.metal:5-11).
 */
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#include "oom_oracle.h"

#define MAX_TOKENS 4
#define LANES 16
#define GATE_ROWS 32
#define DOWN_ROWS 128

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
static inline float siluf(float v) { return v / (1.0f + expf(-v)); }

/* ---- a persistent worker pool (the rayon pool of HostExperts::new) -------------- */

typedef void (*ItemFn)(void* ctx, int64_t item);

typedef struct {
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    int threads;          /* workers, the caller included */
    pthread_t* tid;
    uint64_t generation;  /* bumped per dispatch */
    int running;          /* workers still on the current dispatch */
    ItemFn fn;
    void* ctx;
    int64_t items;
    atomic_llong next;
} Pool;

static Pool g_pool;
static pthread_mutex_t g_pool_mu = PTHREAD_MUTEX_INITIALIZER;

static void pool_drain(Pool* p) {
    for (;;) {
        int64_t i = atomic_fetch_add(&p->next, 1);
        if (i >= p->items) break;
        p->fn(p->ctx, i);
    }
}

static void* pool_worker(void* arg) {
    Pool* p = (Pool*)arg;
    uint64_t seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (p->generation == seen) pthread_cond_wait(&p->go, &p->mu);
        seen = p->generation;
        pthread_mutex_unlock(&p->mu);
        pool_drain(p);
        pthread_mutex_lock(&p->mu);
        if (--p->running == 0) pthread_cond_signal(&p->done);
        pthread_mutex_unlock(&p->mu);
    }
    return NULL;
}

static void pool_ensure(int threads) {
    if (threads < 1) threads = 1;
    if (g_pool.threads == threads) return;
    if (g_pool.threads != 0) return; /* one pool per process, sized by its first use */
    pthread_mutex_init(&g_pool.mu, NULL);
    pthread_cond_init(&g_pool.go, NULL);
    pthread_cond_init(&g_pool.done, NULL);
    g_pool.threads = threads;
    g_pool.tid = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    for (int t = 1; t < threads; t++) pthread_create(&g_pool.tid[t], NULL, pool_worker, &g_pool);
}

/* Runs fn(ctx, i) for i < items over the pool; the caller works too. */
static void pool_run(ItemFn fn, void* ctx, int64_t items) {
    Pool* p = &g_pool;
    pthread_mutex_lock(&p->mu);
    p->fn = fn;
    p->ctx = ctx;
    p->items = items;
    atomic_store(&p->next, 0);
    p->running = p->threads - 1;
    p->generation++;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    pool_drain(p);
    pthread_mutex_lock(&p->mu);
    while (p->running > 0) pthread_cond_wait(&p->done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

/* ---- e4m3 rows ------------------------------------------------------------------ */

typedef struct {
    const uint8_t* w; /* e4m3 [rows, cols] */
    const float* s;   /* 128x128 scales */
    int64_t rows, cols;
} Mat;

static inline float scale_of(Mat m, int64_t r, int64_t c) { return m.s[(r / 128) * cdiv(m.cols, 128) + c / 128]; }

int oracle_host_has_avx512(void) {
#if defined(__x86_64__)
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
#else
    return 0;
#endif
}

#if defined(__x86_64__)
/* 16 e4m3 codes to fp32 exactly: |code| << 20 is the fp32 pattern of the value
 * times 2^-120 (subnormal codes land on fp32 subnormals), then * 2^120 and the sign;
 * S.1111.111 is NaN. */
__attribute__((target("avx512f,avx512bw"))) static inline __m512 e4m3x16(const uint8_t* p) {
    __m512i b = _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i*)p));
    __m512i mag = _mm512_slli_epi32(_mm512_and_si512(b, _mm512_set1_epi32(0x7f)), 20);
    __m512 v = _mm512_mul_ps(_mm512_castsi512_ps(mag), _mm512_set1_ps(0x1p120f));
    __m512i sign = _mm512_slli_epi32(_mm512_and_si512(b, _mm512_set1_epi32(0x80)), 24);
    v = _mm512_castsi512_ps(_mm512_or_si512(_mm512_castps_si512(v), sign));
    __mmask16 nan = _mm512_cmpeq_epi32_mask(_mm512_and_si512(b, _mm512_set1_epi32(0x7f)), _mm512_set1_epi32(0x7f));
    return _mm512_mask_mov_ps(v, nan, _mm512_set1_ps(NAN));
}

/* out[r * nt + t] = W[row0 + r] . xs[t] (kernel.rs:374-412 with e4m3 weights). */
__attribute__((target("avx512f,avx512bw"))) static void rows_avx512(Mat m, int64_t row0, int64_t n_rows,
                                                                     const float* const* xs, int nt, float* out) {
    for (int64_t r = 0; r < n_rows; r++) {
        int64_t row = row0 + r;
        __m512 acc[MAX_TOKENS];
        for (int t = 0; t < MAX_TOKENS; t++) acc[t] = _mm512_setzero_ps();
        for (int64_t g = 0; g < m.cols / 16; g++) {
            __m512 w = _mm512_mul_ps(e4m3x16(m.w + row * m.cols + g * 16), _mm512_set1_ps(scale_of(m, row, g * 16)));
            for (int t = 0; t < nt; t++) acc[t] = _mm512_fmadd_ps(w, _mm512_loadu_ps(xs[t] + g * 16), acc[t]);
        }
        for (int t = 0; t < nt; t++) out[r * nt + t] = _mm512_reduce_add_ps(acc[t]);
    }
}

/* rows decoded to fp32 [n_rows, cols] (w = e4m3 * scale). */
__attribute__((target("avx512f,avx512bw"))) static void decode_avx512(Mat m, int64_t row0, int64_t n_rows, float* w) {
    for (int64_t r = 0; r < n_rows; r++)
        for (int64_t g = 0; g < m.cols / 16; g++)
            _mm512_storeu_ps(w + r * m.cols + g * 16, _mm512_mul_ps(e4m3x16(m.w + (row0 + r) * m.cols + g * 16),
                                                                     _mm512_set1_ps(scale_of(m, row0 + r, g * 16))));
}

/* Register tile of R rows x TV vectors of 16 token columns over columns [k0, k0+kc)
 * (kernel.rs:248-279). */
#define KC 512
#define TILE_FN(R, TV)                                                                                         \
    __attribute__((target("avx512f"))) static void tile_##R##_##TV(const float* w, int64_t stride, int64_t kc, \
                                                                   const float* xt, int64_t ntp, int64_t t0,    \
                                                                   int first, float* out) {                    \
        __m512 acc[R][TV];                                                                                     \
        for (int r = 0; r < R; r++)                                                                            \
            for (int v = 0; v < TV; v++)                                                                       \
                acc[r][v] = first ? _mm512_setzero_ps() : _mm512_loadu_ps(out + r * ntp + t0 + v * 16);        \
        for (int64_t c = 0; c < kc; c++) {                                                                     \
            __m512 xv[TV];                                                                                     \
            for (int v = 0; v < TV; v++) xv[v] = _mm512_loadu_ps(xt + c * ntp + t0 + v * 16);                  \
            for (int r = 0; r < R; r++) {                                                                      \
                __m512 wv = _mm512_set1_ps(w[r * stride + c]);                                                 \
                for (int v = 0; v < TV; v++) acc[r][v] = _mm512_fmadd_ps(wv, xv[v], acc[r][v]);                \
            }                                                                                                  \
        }                                                                                                      \
        for (int r = 0; r < R; r++)                                                                            \
            for (int v = 0; v < TV; v++) _mm512_storeu_ps(out + r * ntp + t0 + v * 16, acc[r][v]);              \
    }
TILE_FN(16, 1)
TILE_FN(12, 2)
TILE_FN(8, 3)
TILE_FN(6, 4)
TILE_FN(8, 1) TILE_FN(4, 1) TILE_FN(2, 1) TILE_FN(1, 1)
TILE_FN(8, 2) TILE_FN(4, 2) TILE_FN(2, 2) TILE_FN(1, 2)
TILE_FN(4, 3) TILE_FN(2, 3) TILE_FN(1, 3)
TILE_FN(4, 4) TILE_FN(2, 4) TILE_FN(1, 4)

typedef void (*TileFn)(const float*, int64_t, int64_t, const float*, int64_t, int64_t, int, float*);

/* out[r * ntp + t] = sum_c w[r, c] * xt[c, t] (kernel.rs:335-372): passes of KC
 * columns, row tiles of R then smaller remainders, 1..4 token vectors at a time. */
__attribute__((target("avx512f"))) static void gemm_avx512(const float* w, int64_t n_rows, int64_t cols,
                                                            const float* xt, int64_t ntp, float* out) {
    int64_t vectors = ntp / 16;
    for (int64_t v = 0; v < vectors;) {
        int64_t left = vectors - v;
        int tv = left >= 4 ? 4 : (int)left;
        TileFn big, rem[4];
        int R;
        switch (tv) {
            case 1: big = tile_16_1; R = 16; rem[0] = tile_8_1; rem[1] = tile_4_1; rem[2] = tile_2_1; rem[3] = tile_1_1; break;
            case 2: big = tile_12_2; R = 12; rem[0] = tile_8_2; rem[1] = tile_4_2; rem[2] = tile_2_2; rem[3] = tile_1_2; break;
            case 3: big = tile_8_3; R = 8; rem[0] = tile_4_3; rem[1] = tile_4_3; rem[2] = tile_2_3; rem[3] = tile_1_3; break;
            default: big = tile_6_4; R = 6; rem[0] = tile_4_4; rem[1] = tile_4_4; rem[2] = tile_2_4; rem[3] = tile_1_4; break;
        }
        static const int sizes[4] = {8, 4, 2, 1};
        for (int64_t k0 = 0; k0 < cols; k0 += KC) {
            int64_t kc = cols - k0 < KC ? cols - k0 : KC;
            int first = k0 == 0;
            int64_t r = 0;
            for (; r + R <= n_rows; r += R) big(w + r * cols + k0, cols, kc, xt + k0 * ntp, ntp, v * 16, first, out + r * ntp);
            for (int s = 0; s < 4; s++) {
                int size = sizes[s];
                if (tv >= 3 && size == 8) continue;
                while (size < R && r + size <= n_rows) {
                    rem[s](w + r * cols + k0, cols, kc, xt + k0 * ntp, ntp, v * 16, first, out + r * ntp);
                    r += size;
                }
            }
        }
        v += tv;
    }
}
#endif

static void rows_scalar(Mat m, int64_t row0, int64_t n_rows, const float* const* xs, int nt, float* out) {
    for (int64_t r = 0; r < n_rows; r++) {
        int64_t row = row0 + r;
        for (int t = 0; t < nt; t++) {
            float acc = 0.0f;
            for (int64_t c = 0; c < m.cols; c++)
                acc += (oracle_e4m3_to_f32(m.w[row * m.cols + c]) * scale_of(m, row, c)) * xs[t][c];
            out[r * nt + t] = acc;
        }
    }
}

static void gemm_scalar(const float* w, int64_t n_rows, int64_t cols, const float* xt, int64_t ntp, float* out) {
    for (int64_t r = 0; r < n_rows; r++)
        for (int64_t t = 0; t < ntp; t++) {
            float acc = 0.0f;
            for (int64_t c = 0; c < cols; c++) acc = fmaf(w[r * cols + c], xt[c * ntp + t], acc);
            out[r * ntp + t] = acc;
        }
}

static void project_rows(Mat m, int64_t row0, int64_t n_rows, const float* const* xs, int nt, float* out) {
#if defined(__x86_64__)
    if (oracle_host_has_avx512() && m.cols % 16 == 0) {
        rows_avx512(m, row0, n_rows, xs, nt, out);
        return;
    }
#endif
    rows_scalar(m, row0, n_rows, xs, nt, out);
}

static void project_gemm(Mat m, int64_t row0, int64_t n_rows, const float* xt, int64_t s, float* out) {
    float* w = (float*)malloc(sizeof(float) * (size_t)(n_rows * m.cols));
#if defined(__x86_64__)
    if (oracle_host_has_avx512() && m.cols % 16 == 0) {
        decode_avx512(m, row0, n_rows, w);
        gemm_avx512(w, n_rows, m.cols, xt, s, out);
        free(w);
        return;
    }
#endif
    for (int64_t r = 0; r < n_rows; r++)
        for (int64_t c = 0; c < m.cols; c++)
            w[r * m.cols + c] = oracle_e4m3_to_f32(m.w[(row0 + r) * m.cols + c]) * scale_of(m, row0 + r, c);
    gemm_scalar(w, n_rows, m.cols, xt, s, out);
    free(w);
}

/* ---- HostExperts::run ------------------------------------------------------------ */

typedef struct {
    const OomFp8Record* geo;
    const uint8_t* const* recs;
    const int32_t* tok;
    const int32_t* joff;
    int n_jobs;
    const float* x;
    float** cols;   /* [H, s] per GEMM job */
    float** acts;   /* [I, s] per job */
    float** arows;  /* [nt, I] per vector job */
    float** downs;  /* [H, s] per job */
    int64_t* gate_items; /* prefix sums of items per job */
    int64_t* down_items;
} Ctx;

static int64_t stride_of(int nt) { return nt <= MAX_TOKENS ? nt : cdiv(nt, LANES) * LANES; }

static int job_of(const int64_t* prefix, int n_jobs, int64_t item) {
    int j = 0;
    while (j + 1 < n_jobs + 1 && prefix[j + 1] <= item) j++;
    return j;
}

static void gate_up_item(void* p, int64_t item) {
    Ctx* c = (Ctx*)p;
    int j = job_of(c->gate_items, c->n_jobs, item);
    int64_t row0 = (item - c->gate_items[j]) * GATE_ROWS;
    int64_t H = c->geo->hidden, I = c->geo->inter;
    int64_t rows = I - row0 < GATE_ROWS ? I - row0 : GATE_ROWS;
    int nt = c->joff[j + 1] - c->joff[j];
    int64_t s = stride_of(nt);
    const uint8_t* rec = c->recs[j];
    Mat g = {rec + c->geo->gate_weight, (const float*)(rec + c->geo->gate_scale), I, H};
    Mat u = {rec + c->geo->up_weight, (const float*)(rec + c->geo->up_scale), I, H};
    float* out = c->acts[j] + row0 * s;
    float* up = (float*)malloc(sizeof(float) * (size_t)(rows * s));
    if (nt <= MAX_TOKENS) {
        const float* xs[MAX_TOKENS];
        for (int t = 0; t < nt; t++) xs[t] = c->x + (size_t)c->tok[c->joff[j] + t] * H;
        project_rows(g, row0, rows, xs, nt, out);
        project_rows(u, row0, rows, xs, nt, up);
    } else {
        project_gemm(g, row0, rows, c->cols[j], s, out);
        project_gemm(u, row0, rows, c->cols[j], s, up);
    }
    for (int64_t i = 0; i < rows * s; i++) out[i] = siluf(out[i]) * up[i];
    free(up);
}

static void down_item(void* p, int64_t item) {
    Ctx* c = (Ctx*)p;
    int j = job_of(c->down_items, c->n_jobs, item);
    int64_t row0 = (item - c->down_items[j]) * DOWN_ROWS;
    int64_t H = c->geo->hidden, I = c->geo->inter;
    int64_t rows = H - row0 < DOWN_ROWS ? H - row0 : DOWN_ROWS;
    int nt = c->joff[j + 1] - c->joff[j];
    int64_t s = stride_of(nt);
    const uint8_t* rec = c->recs[j];
    Mat d = {rec + c->geo->down_weight, (const float*)(rec + c->geo->down_scale), H, I};
    float* out = c->downs[j] + row0 * s;
    if (nt <= MAX_TOKENS) {
        const float* xs[MAX_TOKENS];
        for (int t = 0; t < nt; t++) xs[t] = c->arows[j] + (size_t)t * I;
        project_rows(d, row0, rows, xs, nt, out);
    } else {
        project_gemm(d, row0, rows, c->acts[j], s, out);
    }
}

int oracle_host_experts(const OomFp8Record* geo, const uint8_t* const* records, const int32_t* job_tokens,
                        const int32_t* job_off, int n_jobs, const float* x, float* y, int threads) {
    pthread_mutex_lock(&g_pool_mu);
    pool_ensure(threads);
    int64_t H = geo->hidden, I = geo->inter;
    Ctx c = {geo, records, job_tokens, job_off, n_jobs, x, NULL, NULL, NULL, NULL, NULL, NULL};
    c.cols = (float**)calloc((size_t)n_jobs + 1, sizeof(float*));
    c.acts = (float**)calloc((size_t)n_jobs + 1, sizeof(float*));
    c.arows = (float**)calloc((size_t)n_jobs + 1, sizeof(float*));
    c.downs = (float**)calloc((size_t)n_jobs + 1, sizeof(float*));
    c.gate_items = (int64_t*)calloc((size_t)n_jobs + 1, sizeof(int64_t));
    c.down_items = (int64_t*)calloc((size_t)n_jobs + 1, sizeof(int64_t));
    for (int j = 0; j < n_jobs; j++) {
        int nt = job_off[j + 1] - job_off[j];
        int64_t s = stride_of(nt);
        if (nt > MAX_TOKENS) {
            c.cols[j] = (float*)calloc((size_t)(H * s), sizeof(float));
            for (int t = 0; t < nt; t++)
                for (int64_t col = 0; col < H; col++) c.cols[j][col * s + t] = x[(size_t)job_tokens[job_off[j] + t] * H + col];
        }
        c.acts[j] = (float*)calloc((size_t)(I * s), sizeof(float));
        c.downs[j] = (float*)calloc((size_t)(H * s), sizeof(float));
        c.gate_items[j + 1] = c.gate_items[j] + cdiv(I, GATE_ROWS);
        c.down_items[j + 1] = c.down_items[j] + cdiv(H, DOWN_ROWS);
    }
    pool_run(gate_up_item, &c, c.gate_items[n_jobs]);
    for (int j = 0; j < n_jobs; j++) {
        int nt = job_off[j + 1] - job_off[j];
        if (nt > MAX_TOKENS) continue;
        c.arows[j] = (float*)malloc(sizeof(float) * (size_t)(nt * I));
        for (int t = 0; t < nt; t++)
            for (int64_t r = 0; r < I; r++) c.arows[j][t * I + r] = c.acts[j][r * nt + t];
    }
    pool_run(down_item, &c, c.down_items[n_jobs]);
    int64_t row = 0;
    for (int j = 0; j < n_jobs; j++) {
        int nt = job_off[j + 1] - job_off[j];
        int64_t s = stride_of(nt);
        for (int t = 0; t < nt; t++, row++)
            for (int64_t i = 0; i < H; i++) y[row * H + i] = c.downs[j][i * s + t];
    }
    for (int j = 0; j < n_jobs; j++) {
        free(c.cols[j]);
        free(c.acts[j]);
        free(c.arows[j]);
        free(c.downs[j]);
    }
    free(c.cols); free(c.acts); free(c.arows); free(c.downs); free(c.gate_items); free(c.down_items);
    pthread_mutex_unlock(&g_pool_mu);
    return 0;
}
