/*
 * runner.c — restatement of Yule's CPU TransformerRunner forward pass
 * (yule-infer/src/model_runner.rs:384-531 construction, :533-1036 forward,
 * :1075-1092 prefill/decode/reset) for the dense Llama branch the
 * TinyLlama-shaped config takes: no MoE, no Mixture-of-Depths (n_layers <
 * 32), no streaming KV (context < 8192), no QKV bias, no post norms, no
 * softcap, SwiGLU, norm weight offset 0.
 *
 * TEST INFRASTRUCTURE ONLY: the greedy-token oracle for the HIP runner and
 * the CPU decode baseline.  Never linked into the product.
 *
 * Every linear layer goes through yo_qmv (the AVX2 vec_dot + per-call thread
 * split of model_runner.rs:152-244), exactly as the reference's CPU runner
 * does on an AVX2 host.  Compiled with -ffp-contract=off.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include "yule_oracle.h"

struct yo_runner {
    yo_model m;
    int n_threads;
    uint32_t pos, head_dim, half;
    float *k_cache, *v_cache;       /* [n_layers][max_seq][n_kv*hd] */
    float *cos_t, *sin_t;
    float *hidden, *residual, *normed, *q, *k, *v, *attn_out, *attn_proj, *scores;
    float *gate, *up, *ffn_out;
};

yo_runner *yo_runner_new(const yo_model *m, int n_threads) {
    yo_runner *r = (yo_runner *)calloc(1, sizeof(*r));
    if (!r) return NULL;
    r->m = *m;
    r->n_threads = n_threads;
    r->head_dim = m->dim / m->n_heads;
    r->half = r->head_dim / 2;
    size_t kv = (size_t)m->n_layers * m->max_seq * m->n_kv_heads * r->head_dim;
    r->k_cache = (float *)calloc(kv, 4);
    r->v_cache = (float *)calloc(kv, 4);
    r->cos_t = (float *)malloc((size_t)m->max_seq * r->half * 4);
    r->sin_t = (float *)malloc((size_t)m->max_seq * r->half * 4);
    yo_rope_table(m->max_seq, r->head_dim, m->rope_base, r->cos_t, r->sin_t);
    size_t qd = (size_t)m->n_heads * r->head_dim, kd = (size_t)m->n_kv_heads * r->head_dim;
    r->hidden = (float *)calloc(m->dim, 4);
    r->residual = (float *)calloc(m->dim, 4);
    r->normed = (float *)calloc(m->dim, 4);
    r->q = (float *)calloc(qd, 4);
    r->k = (float *)calloc(kd, 4);
    r->v = (float *)calloc(kd, 4);
    r->attn_out = (float *)calloc(qd, 4);
    r->attn_proj = (float *)calloc(m->dim, 4);
    r->scores = (float *)calloc(m->max_seq, 4);
    r->gate = (float *)calloc(m->ff_dim, 4);
    r->up = (float *)calloc(m->ff_dim, 4);
    r->ffn_out = (float *)calloc(m->dim, 4);
    if (!r->k_cache || !r->v_cache || !r->ffn_out) { yo_runner_free(r); return NULL; }
    return r;
}

void yo_runner_free(yo_runner *r) {
    if (!r) return;
    free(r->k_cache); free(r->v_cache); free(r->cos_t); free(r->sin_t);
    free(r->hidden); free(r->residual); free(r->normed); free(r->q); free(r->k); free(r->v);
    free(r->attn_out); free(r->attn_proj); free(r->scores); free(r->gate); free(r->up);
    free(r->ffn_out);
    free(r);
}

/* model_runner.rs:1087-1092: only the position is reset; stale cache rows
 * are overwritten before they are read again. */
void yo_runner_reset(yo_runner *r) { r->pos = 0; }
uint32_t yo_runner_pos(const yo_runner *r) { return r->pos; }

/* model_runner.rs:246-275 with f32 weights and offset 0 */
static void rms_norm(const float *x, const float *w, float eps, uint32_t n, float *out) {
    float ss = 0.0f;
    for (uint32_t i = 0; i < n; i++) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (uint32_t i = 0; i < n; i++) out[i] = x[i] * inv * (w[i] + 0.0f);
}

/* model_runner.rs:277-293 (interleaved pairs) */
static void apply_rope(float *v, uint32_t len, uint32_t pos, uint32_t hd, uint32_t half,
                       const float *cos_t, const float *sin_t) {
    uint32_t nh = len / hd;
    size_t base = (size_t)pos * half;
    for (uint32_t h = 0; h < nh; h++)
        for (uint32_t i = 0; i < half; i++) {
            float c = cos_t[base + i], s = sin_t[base + i];
            float x0 = v[h * hd + 2 * i], x1 = v[h * hd + 2 * i + 1];
            v[h * hd + 2 * i] = x0 * c - x1 * s;
            v[h * hd + 2 * i + 1] = x0 * s + x1 * c;
        }
}

int yo_runner_forward(yo_runner *r, uint32_t token, float *logits) {
    const yo_model *m = &r->m;
    uint32_t dim = m->dim, pos = r->pos, hd = r->head_dim;
    if (pos >= m->max_seq || token >= m->vocab) return -1;

    /* 1. embedding: dequantize the token's row (:543-566) */
    int ebs = yo_block_size(m->token_embd_t), ebb = yo_block_bytes(m->token_embd_t);
    size_t row_bytes = (size_t)(dim / ebs) * ebb;
    if (yo_dequant_rows(m->token_embd_t, m->token_embd + (size_t)token * row_bytes, dim / ebs, r->hidden))
        return -1;

    uint32_t nh = m->n_heads, nkv = m->n_kv_heads, group = nh / nkv;
    uint32_t kv_stride = nkv * hd, seq_len = pos + 1;
    float scale = 1.0f / sqrtf((float)hd);

    for (uint32_t L = 0; L < m->n_layers; L++) {
        const yo_layer *ly = &m->layers[L];
        memcpy(r->residual, r->hidden, dim * 4);
        rms_norm(r->hidden, ly->attn_norm, m->norm_eps, dim, r->normed);          /* :621-629 */
        yo_qmv(ly->wq_t, ly->wq, r->normed, r->q, nh * hd, dim, r->n_threads);     /* :636-638 */
        yo_qmv(ly->wk_t, ly->wk, r->normed, r->k, kv_stride, dim, r->n_threads);
        yo_qmv(ly->wv_t, ly->wv, r->normed, r->v, kv_stride, dim, r->n_threads);
        apply_rope(r->q, nh * hd, pos, hd, r->half, r->cos_t, r->sin_t);           /* :654-655 */
        apply_rope(r->k, kv_stride, pos, hd, r->half, r->cos_t, r->sin_t);
        float *kc = r->k_cache + (size_t)L * m->max_seq * kv_stride;
        float *vc = r->v_cache + (size_t)L * m->max_seq * kv_stride;
        memcpy(kc + (size_t)pos * kv_stride, r->k, kv_stride * 4);                  /* :665-669 */
        memcpy(vc + (size_t)pos * kv_stride, r->v, kv_stride * 4);

        memset(r->attn_out, 0, (size_t)nh * hd * 4);                                /* :679-758 */
        for (uint32_t h = 0; h < nh; h++) {
            uint32_t kvh = h / group;
            const float *qh = r->q + h * hd;
            for (uint32_t t = 0; t < seq_len; t++) {
                const float *kh = kc + (size_t)t * kv_stride + kvh * hd;
                float dot = 0.0f;
                for (uint32_t d = 0; d < hd; d++) dot += qh[d] * kh[d];
                r->scores[t] = dot * scale;
            }
            float mx = -INFINITY;
            for (uint32_t t = 0; t < seq_len; t++) mx = fmaxf(mx, r->scores[t]);
            float sum = 0.0f;
            for (uint32_t t = 0; t < seq_len; t++) { r->scores[t] = expf(r->scores[t] - mx); sum += r->scores[t]; }
            float inv = 1.0f / sum;
            for (uint32_t t = 0; t < seq_len; t++) r->scores[t] *= inv;
            float *oh = r->attn_out + h * hd;
            for (uint32_t t = 0; t < seq_len; t++) {
                float w = r->scores[t];
                const float *vh = vc + (size_t)t * kv_stride + kvh * hd;
                for (uint32_t d = 0; d < hd; d++) oh[d] += w * vh[d];
            }
        }
        yo_qmv(ly->wo_t, ly->wo, r->attn_out, r->attn_proj, dim, nh * hd, r->n_threads); /* :762 */
        for (uint32_t i = 0; i < dim; i++) r->hidden[i] = r->residual[i] + r->attn_proj[i];

        memcpy(r->residual, r->hidden, dim * 4);                                       /* :792 */
        rms_norm(r->hidden, ly->ffn_norm, m->norm_eps, dim, r->normed);
        uint32_t ff = m->ff_dim;
        yo_qmv(ly->w_gate_t, ly->w_gate, r->normed, r->gate, ff, dim, r->n_threads);  /* :963-964 */
        yo_qmv(ly->w_up_t, ly->w_up, r->normed, r->up, ff, dim, r->n_threads);
        for (uint32_t i = 0; i < ff; i++) {                                            /* :967-972 */
            float sg = 1.0f / (1.0f + expf(-r->gate[i]));
            r->gate[i] = r->gate[i] * sg * r->up[i];
        }
        yo_qmv(ly->w_down_t, ly->w_down, r->gate, r->ffn_out, dim, ff, r->n_threads);  /* :982 */
        for (uint32_t i = 0; i < dim; i++) r->hidden[i] = r->residual[i] + r->ffn_out[i];
    }
    rms_norm(r->hidden, m->output_norm, m->norm_eps, dim, r->normed);                  /* :1008-1016 */
    yo_qmv(m->output_t, m->output, r->normed, logits, m->vocab, dim, r->n_threads);   /* :1019-1025 */
    r->pos++;
    return 0;
}
