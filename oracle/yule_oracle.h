/*
 * yule_oracle.h — CPU restatement of Yule's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libyule_hip.so, the
 * yule_amd package's compute path) links, loads or calls this code; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do, and
 * only as the checker / the timed CPU baseline.
 *
 * Every function cites the reference file:line it restates
 * (paths relative to the visualstudioblyat/yule source tree).
 *
 * Parity pinning (what checks each function against something other than a
 * retyped formula) is listed per function in tests/test_oracle.py; see the
 * header comment of each definition for the pin.
 */
#ifndef YULE_ORACLE_H
#define YULE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids, yule-core/src/dtype.rs:21-33 */
enum {
    YO_F32 = 0,
    YO_F16 = 1,
    YO_Q4_0 = 2,
    YO_Q8_0 = 8,
    YO_Q4_K = 12,
    YO_Q5_K = 13,
    YO_Q6_K = 14,
    YO_Q8_K = 15,
};

/* block geometry, yule-core/src/dtype.rs:62-118 (0 = unsupported here) */
int yo_block_size(int dtype);
int yo_block_bytes(int dtype);

/* ---- scalar restatement of yule-core/src/dequant.rs ---- */
float yo_f16_to_f32(uint16_t bits);                                  /* :20-49 */
void yo_extract_q4k_scales_mins(const uint8_t q[12], uint8_t sc[8], uint8_t mn[8]); /* :176-190 */
void yo_dequant_q4_0(const uint8_t *blk, float *out);                /* :77-86 */
void yo_dequant_q8_0(const uint8_t *blk, float *out);                /* :142-150 */
void yo_dequant_q4_k(const uint8_t *blk, float *out);                /* :260-290 */
void yo_dequant_q6_k(const uint8_t *blk, float *out);                /* :346-372 */
void yo_dequant_q5_k(const uint8_t *blk, float *out);                /* :297-338 */
void yo_dequant_q8_k(const uint8_t *blk, float *out);                /* :376-384 */
float yo_vec_dot_q4_0(const uint8_t *blk, const float *act);         /* :902-913 */
float yo_vec_dot_q8_0(const uint8_t *blk, const float *act);         /* :916-926 */
float yo_vec_dot_q4_k(const uint8_t *blk, const float *act);         /* :929-972 */
float yo_vec_dot_q6_k(const uint8_t *blk, const float *act);         /* :976-1009 */
float yo_vec_dot_q5_k(const uint8_t *blk, const float *act);         /* :1088-1140 */
/* dequant_block / vec_dot_block dispatch, dequant.rs:1232-1282. Returns 0 ok, -1 unsupported. */
int yo_dequant_block(int dtype, const uint8_t *blk, float *out);
int yo_dequant_rows(int dtype, const uint8_t *w, size_t n_blocks, float *out);
int yo_vec_dot_block_scalar(int dtype, const uint8_t *blk, const float *act, float *res);

/* CpuBackend::quantized_matmul, yule-gpu/src/cpu.rs:544-590 (scalar vec_dot,
 * blocks_per_row = n_cols / block_size, single thread). */
int yo_qmv_scalar(int dtype, const uint8_t *w, const float *x, float *y,
                  uint32_t n_rows, uint32_t n_cols);
/* Accuracy reference: bit-exact f32 dequantized weights, f64 accumulation. */
int yo_qmv_f64(int dtype, const uint8_t *w, const float *x, double *y,
               uint32_t n_rows, uint32_t n_cols);

/* ---- AVX2 CPU baseline, yule-core/src/simd/avx2.rs + model_runner.rs:152-244 ---- */
int yo_have_avx2(void);
/* vec_dot with the reference's runtime dispatch (simd/mod.rs:38-47): AVX2
 * bodies when AVX2+FMA are present, scalar otherwise. */
int yo_vec_dot_block(int dtype, const uint8_t *blk, const float *act, float *res);
/* qmv of model_runner.rs:152-244: rows split over n_threads std::threads
 * spawned per call when n_rows >= 128 (n_threads <= 0: all online CPUs). */
/* Q4_K block dot of the AVX2 path: the reference's assembly kernel when
 * installed (simd/avx2.rs:84-96), else the Rust-fallback restatement. */
typedef float (*yo_q4k_dot_fn)(const uint8_t *blk, const float *act);
void yo_set_q4k_dot(yo_q4k_dot_fn fn);

int yo_qmv(int dtype, const uint8_t *w, const float *x, float *y,
           uint32_t n_rows, uint32_t n_cols, int n_threads);

/* ---- TransformerRunner restatement, yule-infer/src/model_runner.rs ---- */
typedef struct {
    const float *attn_norm;     /* f32[dim] */
    const uint8_t *wq, *wk, *wv, *wo;
    int wq_t, wk_t, wv_t, wo_t;
    const float *ffn_norm;      /* f32[dim] */
    const uint8_t *w_gate, *w_up, *w_down;
    int w_gate_t, w_up_t, w_down_t;
} yo_layer;

typedef struct {
    uint32_t n_layers, dim, n_heads, n_kv_heads, ff_dim, vocab, max_seq;
    float norm_eps, rope_base;
    const uint8_t *token_embd; int token_embd_t;   /* [vocab][dim] quantized rows */
    const float *output_norm;                      /* f32[dim] */
    const uint8_t *output; int output_t;           /* [vocab][dim] */
    const yo_layer *layers;
} yo_model;

typedef struct yo_runner yo_runner;
yo_runner *yo_runner_new(const yo_model *m, int n_threads);
void yo_runner_free(yo_runner *r);
void yo_runner_reset(yo_runner *r);
/* forward one token (model_runner.rs:533-1036); logits written to out[vocab]. */
int yo_runner_forward(yo_runner *r, uint32_t token, float *logits);
uint32_t yo_runner_pos(const yo_runner *r);

/* argmax_ct, yule-infer/src/sampler.rs:150-163: last maximal index wins. */
uint32_t yo_argmax(const float *v, uint32_t n);

/* RopeTable::new, model_runner.rs:77-100 (fills cos/sin [max_seq][rot/2]). */
void yo_rope_table(uint32_t max_seq, uint32_t rot_dim, float base, float *cos_t, float *sin_t);

#ifdef __cplusplus
}
#endif
#endif
