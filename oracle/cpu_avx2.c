/*
 * cpu_avx2.c — restatement of Yule's x86 CPU decode path: the AVX2+FMA
 * vec_dot bodies of yule-core/src/simd/avx2.rs and the threaded qmv row
 * loop of yule-infer/src/model_runner.rs:152-244.
 *
 * TEST INFRASTRUCTURE ONLY: the CPU oracle for the end-to-end runner and
 * the timed CPU baseline in bench.py.  Never linked into the product.
 *
 * Compiled with -O3 -mavx2 -mfma -mf16c -ffp-contract=off: the explicit
 * intrinsics carry the reference's FMAs, and the scalar glue (scale * dot -
 * min * sum) stays unfused as in Rust.
 *
 * Q4_K: Yule links its hand-written assembly (yule-core/src/kernels/
 * q4k_gemv_avx2.S) when clang is found at build time, else the Rust
 * intrinsics fallback (avx2.rs:100-152).  This file restates the fallback;
 * tests/test_oracle.py checks it against the assembly built from the
 * reference sources into oracle/_ref/ (tolerance 1e-1, as avx2.rs:437).
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include "yule_oracle.h"

int yo_have_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

static int g_level = 0; /* simd/mod.rs:20-34: 0 unknown, 1 scalar, 2 avx2 */

static inline float f16le(const uint8_t *p) { return yo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* avx2.rs:9-19 — (lo128+hi128), movehl, then lane0+lane1 */
__attribute__((target("avx2,fma"))) static inline float hsum(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
    return _mm_cvtss_f32(s);
}

/* avx2.rs:38-56 */
__attribute__((target("avx2,fma"))) static float dot_q8_0(const uint8_t *blk, const float *act) {
    float d = f16le(blk);
    const uint8_t *qs = blk + 2;
    __m256 acc = _mm256_setzero_ps();
    for (int g = 0; g < 4; g++) {
        __m128i qi = _mm_loadl_epi64((const __m128i *)(qs + g * 8));
        __m256 f = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(qi));
        acc = _mm256_fmadd_ps(f, _mm256_loadu_ps(act + g * 8), acc);
    }
    return hsum(acc) * d;
}

/* avx2.rs:58-83 — interleaved nibbles, (w - 8) then FMA */
__attribute__((target("avx2,fma"))) static float dot_q4_0(const uint8_t *blk, const float *act) {
    float d = f16le(blk);
    const uint8_t *qs = blk + 2;
    __m256 bias = _mm256_set1_ps(8.0f), acc = _mm256_setzero_ps();
    for (int g = 0; g < 4; g++) {
        float w[8];
        for (int i = 0; i < 4; i++) {
            uint8_t b = qs[g * 4 + i];
            w[2 * i] = (float)(b & 0x0F);
            w[2 * i + 1] = (float)(b >> 4);
        }
        __m256 wv = _mm256_sub_ps(_mm256_loadu_ps(w), bias);
        acc = _mm256_fmadd_ps(wv, _mm256_loadu_ps(act + g * 8), acc);
    }
    return hsum(acc) * d;
}

/* avx2.rs:100-152 (Rust intrinsics fallback of the Q4_K kernel) */
__attribute__((target("avx2,fma"))) static float dot_q4_k(const uint8_t *blk, const float *act) {
    float d = f16le(blk), dmin = f16le(blk + 2);
    uint8_t sc[8], mn[8];
    yo_extract_q4k_scales_mins(blk + 4, sc, mn);
    float sum = 0.0f;
    for (int j = 0; j < 4; j++) {
        const uint8_t *ql = blk + 16 + 32 * j;
        for (int h = 0; h < 2; h++) {
            __m256 dacc = _mm256_setzero_ps(), sacc = _mm256_setzero_ps();
            for (int g = 0; g < 4; g++) {
                float w[8];
                for (int l = 0; l < 8; l++)
                    w[l] = (float)(h == 0 ? (ql[g * 8 + l] & 0xF) : (ql[g * 8 + l] >> 4));
                __m256 a = _mm256_loadu_ps(act + 64 * j + 32 * h + g * 8);
                dacc = _mm256_fmadd_ps(_mm256_loadu_ps(w), a, dacc);
                sacc = _mm256_add_ps(sacc, a);
            }
            int k = 2 * j + h;
            float t1 = d * (float)sc[k] * hsum(dacc);
            float t2 = dmin * (float)mn[k] * hsum(sacc);
            sum += t1 - t2;
        }
    }
    return sum;
}

/* avx2.rs:238-303 — per sub-block, 4 groups of 8 weights (5-bit levels built
 * in scalar), FMA into one accumulator and add into another, hsum each */
__attribute__((target("avx2,fma"))) static float dot_q5_k(const uint8_t *blk, const float *act) {
    float d = f16le(blk), dmin = f16le(blk + 2);
    uint8_t sc[8], mn[8];
    yo_extract_q4k_scales_mins(blk + 4, sc, mn);
    const uint8_t *qh = blk + 16;
    float sum = 0.0f;
    for (int j = 0; j < 4; j++) {
        const uint8_t *ql = blk + 48 + 32 * j;
        const uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
        for (int half = 0; half < 2; half++) {
            const int k = 2 * j + half;
            float scale = d * (float)sc[k], mins = dmin * (float)mn[k];
            __m256 dacc = _mm256_setzero_ps(), sacc = _mm256_setzero_ps();
            for (int g = 0; g < 4; g++) {
                float w[8];
                for (int l = 0; l < 8; l++) {
                    const int idx = 8 * g + l;
                    const int q = half ? (ql[idx] >> 4) + ((qh[idx] & u2) ? 16 : 0)
                                       : (ql[idx] & 0x0F) + ((qh[idx] & u1) ? 16 : 0);
                    w[l] = (float)q;
                }
                const __m256 a = _mm256_loadu_ps(act + 64 * j + 32 * half + 8 * g);
                dacc = _mm256_fmadd_ps(_mm256_loadu_ps(w), a, dacc);
                sacc = _mm256_add_ps(sacc, a);
            }
            sum += scale * hsum(dacc) - mins * hsum(sacc);
        }
    }
    return sum;
}

/* avx2.rs:305-337 — the AVX2 Q6_K body is the scalar loop */
static float dot_q6_k(const uint8_t *blk, const float *act) { return yo_vec_dot_q6_k(blk, act); }

/* The reference's AVX2 build runs Q4_K through its hand-written assembly
 * kernel when that is compiled in (simd/avx2.rs:84-96,
 * kernels/q4k_gemv_avx2.S); yo_set_q4k_dot installs that function (loaded
 * from oracle/_ref by the caller) in place of the Rust-fallback restatement
 * above, NULL restores the restatement. */
static yo_q4k_dot_fn g_q4k_dot = NULL;
void yo_set_q4k_dot(yo_q4k_dot_fn fn) { g_q4k_dot = fn; }

/* simd::vec_dot, simd/mod.rs:38-47 */
int yo_vec_dot_block(int dtype, const uint8_t *blk, const float *act, float *res) {
    if (g_level == 0) g_level = yo_have_avx2() ? 2 : 1;
    if (g_level == 2) {
        switch (dtype) {
        case YO_Q8_0: *res = dot_q8_0(blk, act); return 0;
        case YO_Q4_0: *res = dot_q4_0(blk, act); return 0;
        case YO_Q4_K: *res = g_q4k_dot ? g_q4k_dot(blk, act) : dot_q4_k(blk, act); return 0;
        case YO_Q6_K: *res = dot_q6_k(blk, act); return 0;
        case YO_Q5_K: *res = dot_q5_k(blk, act); return 0;
        default: break;
        }
    }
    return yo_vec_dot_block_scalar(dtype, blk, act, res);
}

typedef struct {
    int dtype, bs, bb;
    const uint8_t *w;
    const float *x;
    float *y;
    uint32_t row0, nrows, n_rows_total;
    size_t bpr;
} qmv_job;

/* one row chunk of model_runner.rs:176-204, with the _mm_prefetch of the
 * next block (:101-130) */
static void *qmv_rows(void *p) {
    qmv_job *j = (qmv_job *)p;
    for (uint32_t i = 0; i < j->nrows; i++) {
        uint32_t row = j->row0 + i;
        size_t row_off = (size_t)row * j->bpr * j->bb;
        float sum = 0.0f;
        for (size_t b = 0; b < j->bpr; b++) {
            size_t start = row_off + b * j->bb;
            size_t next = 0;
            int have_next = 1;
            if (b + 1 < j->bpr) next = row_off + (b + 1) * j->bb;
            else if (row + 1 < j->n_rows_total) next = (size_t)(row + 1) * j->bpr * j->bb;
            else have_next = 0;
            if (have_next) {
                _mm_prefetch((const char *)(j->w + next), _MM_HINT_T0);
                if (j->bb > 64) _mm_prefetch((const char *)(j->w + next + 64), _MM_HINT_T0);
            }
            float v;
            yo_vec_dot_block(j->dtype, j->w + start, j->x + b * j->bs, &v);
            sum += v;
        }
        j->y[row] = sum;
    }
    return NULL;
}

int yo_qmv(int dtype, const uint8_t *w, const float *x, float *y,
           uint32_t n_rows, uint32_t n_cols, int n_threads) {
    int bs = yo_block_size(dtype), bb = yo_block_bytes(dtype);
    if (!bs || bs == 1) return -1;
    if (n_threads <= 0) n_threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (n_threads < 1) n_threads = 1;
    qmv_job base = {dtype, bs, bb, w, x, y, 0, n_rows, n_rows, n_cols / (uint32_t)bs};
    if (n_rows < 128 || n_threads == 1) {   /* QMV_PARALLEL_THRESHOLD, :149 */
        qmv_rows(&base);
        return 0;
    }
    /* std::thread::scope with rows chunked by ceil(n_rows / n_threads), one
     * thread spawned per chunk on every call (:164-211) */
    uint32_t chunk = (n_rows + (uint32_t)n_threads - 1) / (uint32_t)n_threads;
    int n_chunks = (int)((n_rows + chunk - 1) / chunk);
    pthread_t tid[512];
    qmv_job jobs[512];
    if (n_chunks > 512) n_chunks = 512;
    for (int c = 0; c < n_chunks; c++) {
        jobs[c] = base;
        jobs[c].row0 = (uint32_t)c * chunk;
        jobs[c].nrows = (c == n_chunks - 1) ? n_rows - jobs[c].row0 : chunk;
        pthread_create(&tid[c], NULL, qmv_rows, &jobs[c]);
    }
    for (int c = 0; c < n_chunks; c++) pthread_join(tid[c], NULL);
    return 0;
}
