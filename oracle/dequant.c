/*
 * dequant.c — scalar restatement of yule-core/src/dequant.rs for the four
 * GGUF block formats on the hot path (Q4_0, Q8_0, Q4_K, Q6_K) plus f16.
 *
 * TEST INFRASTRUCTURE ONLY (the CPU oracle); never linked into the product.
 *
 * Built with -ffp-contract=off: the reference evaluates every product and
 * sum as a separately rounded f32 operation (Rust never contracts a*b+c),
 * and the bit-exact dequant parity depends on keeping that.
 *
 * Pins (tests/test_oracle.py):
 *  - yo_f16_to_f32: all 65536 bit patterns vs numpy float16->float32
 *    (NaN payload compared bitwise), plus the dequant.rs:1288-1298 KATs.
 *  - yo_extract_q4k_scales_mins: every 6-bit scale/min vector packed by an
 *    independent bit-level packer round-trips; ggml get_scale_min_k4 KATs.
 *  - dequant_q4_0/q8_0: dequant.rs:1308-1359 KATs (0x88, 0xF0 interleave,
 *    127/-128), exhaustive byte x scale brute force.
 *  - dequant_q4_k/q6_k: special cases (sc=1,mn=0,d=1 -> raw nibble; mins
 *    only -> constant), bit-plane probes that flip one quant and check one
 *    output moves, and a numpy restatement written from the GLSL/CUDA
 *    kernels' indexing (yule-gpu/shaders/qmv_q4_k.comp, qmv_q6_k.comp).
 *  - vec_dot_*: dequant.rs:1361-1375 KAT, f64 dot of dequantized weights,
 *    and the reference's own hand-written AVX2 assembly for Q4_K
 *    (yule-core/src/kernels/q4k_gemv_avx2.S, built into oracle/_ref/).
 */
#include <math.h>
#include <string.h>
#include "yule_oracle.h"

int yo_block_size(int dtype) {
    switch (dtype) {                      /* dtype.rs:99-118 */
    case YO_Q4_0: case YO_Q8_0: return 32;
    case YO_Q4_K: case YO_Q5_K: case YO_Q6_K: case YO_Q8_K: return 256;
    case YO_F32: case YO_F16: return 1;
    default: return 0;
    }
}

int yo_block_bytes(int dtype) {
    switch (dtype) {                      /* dtype.rs:62-96 */
    case YO_Q4_0: return 18;
    case YO_Q8_0: return 34;
    case YO_Q4_K: return 144;
    case YO_Q5_K: return 176;
    case YO_Q6_K: return 210;
    case YO_Q8_K: return 292;
    case YO_F32: return 4;
    case YO_F16: return 2;
    default: return 0;
    }
}

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* dequant.rs:20-49 — exact bit manipulation; denormals renormalised,
 * inf/NaN keep their payload shifted into the f32 mantissa. */
float yo_f16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u;
    uint32_t exp = (bits >> 10) & 0x1Fu;
    uint32_t mant = bits & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return bits_to_f32(sign << 31);
        uint32_t m = mant;
        int e = -14;
        while ((m & 0x400u) == 0) { m <<= 1; e -= 1; }
        m &= 0x3FFu;
        uint32_t fe = (uint32_t)(e + 127) & 0xFFu;
        return bits_to_f32((sign << 31) | (fe << 23) | (m << 13));
    }
    if (exp == 31) return bits_to_f32((sign << 31) | (0xFFu << 23) | (mant << 13));
    return bits_to_f32((sign << 31) | ((exp - 15 + 127) << 23) | (mant << 13));
}

/* dequant.rs:59-62, little-endian u16 */
static inline float read_f16(const uint8_t *p) { return yo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* dequant.rs:176-190 (ggml get_scale_min_k4) */
void yo_extract_q4k_scales_mins(const uint8_t q[12], uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 4; j++) {
        sc[j] = q[j] & 63;
        mn[j] = q[j + 4] & 63;
    }
    for (int j = 4; j < 8; j++) {
        sc[j] = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        mn[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* dequant.rs:77-86 — Yule's interleaved order: byte 2+i/2, low nibble for even i */
void yo_dequant_q4_0(const uint8_t *blk, float *out) {
    float d = read_f16(blk);
    for (int i = 0; i < 32; i++) {
        uint8_t byte = blk[2 + i / 2];
        uint8_t nib = (i % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
        out[i] = ((float)nib - 8.0f) * d;
    }
}

/* dequant.rs:142-150 */
void yo_dequant_q8_0(const uint8_t *blk, float *out) {
    float d = read_f16(blk);
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)blk[2 + i] * d;
}

/* dequant.rs:260-290 — q*(d*sc) - dmin*mn, two separately rounded ops */
void yo_dequant_q4_k(const uint8_t *blk, float *out) {
    float d = read_f16(blk), dmin = read_f16(blk + 2);
    uint8_t sc[8], mn[8];
    yo_extract_q4k_scales_mins(blk + 4, sc, mn);
    for (int j = 0; j < 4; j++) {
        const uint8_t *qs = blk + 16 + 32 * j;
        float scale0 = d * (float)sc[2 * j], min0 = dmin * (float)mn[2 * j];
        for (int l = 0; l < 32; l++) out[64 * j + l] = (float)(qs[l] & 0x0F) * scale0 - min0;
        float scale1 = d * (float)sc[2 * j + 1], min1 = dmin * (float)mn[2 * j + 1];
        for (int l = 0; l < 32; l++) out[64 * j + 32 + l] = (float)(qs[l] >> 4) * scale1 - min1;
    }
}

/* dequant.rs:297-338 — Q4_K's layout plus a 5th bit per weight from qh[32]
 * (bit 2j for the low-nibble sub-block of group j, bit 2j+1 for the high);
 * q*(d*sc) - dmin*mn as two separately rounded ops */
void yo_dequant_q5_k(const uint8_t *blk, float *out) {
    float d = read_f16(blk), dmin = read_f16(blk + 2);
    uint8_t sc[8], mn[8];
    yo_extract_q4k_scales_mins(blk + 4, sc, mn);
    const uint8_t *qh = blk + 16;
    for (int j = 0; j < 4; j++) {
        const uint8_t *ql = blk + 48 + 32 * j;
        const uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
        float d1 = d * (float)sc[2 * j], m1 = dmin * (float)mn[2 * j];
        for (int l = 0; l < 32; l++)
            out[64 * j + l] = (float)((ql[l] & 0x0F) + ((qh[l] & u1) ? 16 : 0)) * d1 - m1;
        float d2 = d * (float)sc[2 * j + 1], m2 = dmin * (float)mn[2 * j + 1];
        for (int l = 0; l < 32; l++)
            out[64 * j + 32 + l] = (float)((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) * d2 - m2;
    }
}

/* dequant.rs:376-384 — f32 d (little-endian) at 0, 256 int8 at 4; the
 * 32-byte bsums tail is not read */
void yo_dequant_q8_k(const uint8_t *blk, float *out) {
    float d;
    memcpy(&d, blk, 4);
    for (int i = 0; i < 256; i++) out[i] = (float)(int8_t)blk[4 + i] * d;
}

/* the four 6-bit quants of position l in a Q6_K half, dequant.rs:358-361 */
static inline void q6k_quads(const uint8_t *ql, const uint8_t *qh, int l, int q[4]) {
    q[0] = (int)(int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
    q[1] = (int)(int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
    q[2] = (int)(int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
    q[3] = (int)(int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
}

/* dequant.rs:346-372 — value = (d * sc) * q, evaluated left to right */
void yo_dequant_q6_k(const uint8_t *blk, float *out) {
    float d = read_f16(blk + 208);
    const int8_t *sc = (const int8_t *)(blk + 192);
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = blk + half * 64, *qh = blk + 128 + half * 32;
        int ob = half * 128, sb = half * 8;
        for (int l = 0; l < 32; l++) {
            int is = l / 16, q[4];
            q6k_quads(ql, qh, l, q);
            for (int g = 0; g < 4; g++)
                out[ob + l + 32 * g] = d * (float)sc[sb + is + 2 * g] * (float)q[g];
        }
    }
}

/* dequant.rs:902-913 — sum first, scale last */
float yo_vec_dot_q4_0(const uint8_t *blk, const float *act) {
    float d = read_f16(blk), sum = 0.0f;
    for (int i = 0; i < 32; i++) {
        uint8_t byte = blk[2 + i / 2];
        uint8_t nib = (i % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
        sum += ((float)nib - 8.0f) * act[i];
    }
    return sum * d;
}

/* dequant.rs:916-926 */
float yo_vec_dot_q8_0(const uint8_t *blk, const float *act) {
    float d = read_f16(blk), sum = 0.0f;
    for (int i = 0; i < 32; i++) sum += (float)(int8_t)blk[2 + i] * act[i];
    return sum * d;
}

/* dequant.rs:929-972 — per sub-block: scale*dot - min*sum(act) */
float yo_vec_dot_q4_k(const uint8_t *blk, const float *act) {
    float d = read_f16(blk), dmin = read_f16(blk + 2);
    uint8_t sc[8], mn[8];
    yo_extract_q4k_scales_mins(blk + 4, sc, mn);
    float sum = 0.0f;
    for (int j = 0; j < 4; j++) {
        const uint8_t *qs = blk + 16 + 32 * j;
        float scale0 = d * (float)sc[2 * j], min0 = dmin * (float)mn[2 * j];
        float sb = 0.0f, ms = 0.0f;
        for (int l = 0; l < 32; l++) {
            sb += (float)(qs[l] & 0x0F) * act[64 * j + l];
            ms += act[64 * j + l];
        }
        sum += scale0 * sb - min0 * ms;
        float scale1 = d * (float)sc[2 * j + 1], min1 = dmin * (float)mn[2 * j + 1];
        sb = 0.0f; ms = 0.0f;
        for (int l = 0; l < 32; l++) {
            sb += (float)(qs[l] >> 4) * act[64 * j + 32 + l];
            ms += act[64 * j + 32 + l];
        }
        sum += scale1 * sb - min1 * ms;
    }
    return sum;
}

/* dequant.rs:976-1009 — term order q1..q4 per l; each term ((d*sc)*q)*act */
float yo_vec_dot_q6_k(const uint8_t *blk, const float *act) {
    float d = read_f16(blk + 208), sum = 0.0f;
    const int8_t *sc = (const int8_t *)(blk + 192);
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = blk + half * 64, *qh = blk + 128 + half * 32;
        int ab = half * 128, sb = half * 8;
        for (int l = 0; l < 32; l++) {
            int is = l / 16, q[4];
            q6k_quads(ql, qh, l, q);
            for (int g = 0; g < 4; g++)
                sum += d * (float)sc[sb + is + 2 * g] * (float)q[g] * act[ab + l + 32 * g];
        }
    }
    return sum;
}

/* dequant.rs:1088-1140 — per sub-block: scale*dot - min*sum(act) */
float yo_vec_dot_q5_k(const uint8_t *blk, const float *act) {
    float d = read_f16(blk), dmin = read_f16(blk + 2);
    uint8_t sc[8], mn[8];
    yo_extract_q4k_scales_mins(blk + 4, sc, mn);
    const uint8_t *qh = blk + 16;
    float sum = 0.0f;
    for (int j = 0; j < 4; j++) {
        const uint8_t *ql = blk + 48 + 32 * j;
        const uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
        float scale0 = d * (float)sc[2 * j], min0 = dmin * (float)mn[2 * j];
        float dot0 = 0.0f, asum0 = 0.0f;
        for (int l = 0; l < 32; l++) {
            dot0 += (float)((ql[l] & 0x0F) + ((qh[l] & u1) ? 16 : 0)) * act[64 * j + l];
            asum0 += act[64 * j + l];
        }
        sum += scale0 * dot0 - min0 * asum0;
        float scale1 = d * (float)sc[2 * j + 1], min1 = dmin * (float)mn[2 * j + 1];
        float dot1 = 0.0f, asum1 = 0.0f;
        for (int l = 0; l < 32; l++) {
            dot1 += (float)((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) * act[64 * j + 32 + l];
            asum1 += act[64 * j + 32 + l];
        }
        sum += scale1 * dot1 - min1 * asum1;
    }
    return sum;
}

/* dequant.rs:1232-1275 (the hot-path formats and Q5_K/Q8_K plus F32/F16 scalars) */
int yo_dequant_block(int dtype, const uint8_t *blk, float *out) {
    switch (dtype) {
    case YO_Q4_0: yo_dequant_q4_0(blk, out); return 0;
    case YO_Q8_0: yo_dequant_q8_0(blk, out); return 0;
    case YO_Q4_K: yo_dequant_q4_k(blk, out); return 0;
    case YO_Q6_K: yo_dequant_q6_k(blk, out); return 0;
    case YO_Q5_K: yo_dequant_q5_k(blk, out); return 0;
    case YO_Q8_K: yo_dequant_q8_k(blk, out); return 0;
    case YO_F16: out[0] = read_f16(blk); return 0;
    case YO_F32: memcpy(out, blk, 4); return 0;
    default: return -1;
    }
}

int yo_dequant_rows(int dtype, const uint8_t *w, size_t n_blocks, float *out) {
    int bs = yo_block_size(dtype), bb = yo_block_bytes(dtype);
    if (!bs) return -1;
    for (size_t b = 0; b < n_blocks; b++)
        if (yo_dequant_block(dtype, w + b * (size_t)bb, out + b * (size_t)bs)) return -1;
    return 0;
}

/* scalar::vec_dot_dispatch, yule-core/src/simd/scalar.rs:4-22 */
int yo_vec_dot_block_scalar(int dtype, const uint8_t *blk, const float *act, float *res) {
    switch (dtype) {
    case YO_Q4_0: *res = yo_vec_dot_q4_0(blk, act); return 0;
    case YO_Q8_0: *res = yo_vec_dot_q8_0(blk, act); return 0;
    case YO_Q4_K: *res = yo_vec_dot_q4_k(blk, act); return 0;
    case YO_Q6_K: *res = yo_vec_dot_q6_k(blk, act); return 0;
    case YO_Q5_K: *res = yo_vec_dot_q5_k(blk, act); return 0;
    default: return -1;   /* Q8_K: no vec_dot in the reference (scalar.rs:4-22) */
    }
}

/* yule-gpu/src/cpu.rs:544-590 */
int yo_qmv_scalar(int dtype, const uint8_t *w, const float *x, float *y,
                  uint32_t n_rows, uint32_t n_cols) {
    int bs = yo_block_size(dtype), bb = yo_block_bytes(dtype);
    if (!bs || bs == 1) return -1;
    size_t bpr = n_cols / (uint32_t)bs;
    for (uint32_t r = 0; r < n_rows; r++) {
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            float v;
            yo_vec_dot_block_scalar(dtype, w + ((size_t)r * bpr + b) * bb, x + b * bs, &v);
            sum += v;
        }
        y[r] = sum;
    }
    return 0;
}

int yo_qmv_f64(int dtype, const uint8_t *w, const float *x, double *y,
               uint32_t n_rows, uint32_t n_cols) {
    int bs = yo_block_size(dtype), bb = yo_block_bytes(dtype);
    if (!bs || bs == 1) return -1;
    size_t bpr = n_cols / (uint32_t)bs;
    float tmp[256];
    for (uint32_t r = 0; r < n_rows; r++) {
        double sum = 0.0;
        for (size_t b = 0; b < bpr; b++) {
            yo_dequant_block(dtype, w + ((size_t)r * bpr + b) * bb, tmp);
            for (int i = 0; i < bs; i++) sum += (double)tmp[i] * (double)x[b * bs + i];
        }
        y[r] = sum;
    }
    return 0;
}

/* argmax_ct, sampler.rs:142-163: starts at values[0]; an element replaces the
 * best when the sign bit of (v - best) is clear, so the last maximal index
 * wins (for finite values that test equals v >= best). */
uint32_t yo_argmax(const float *v, uint32_t n) {
    if (n == 0) return 0;
    uint32_t best_i = 0;
    float best = v[0];
    for (uint32_t i = 1; i < n; i++) {
        float diff = v[i] - best;
        uint32_t bits;
        memcpy(&bits, &diff, 4);
        if ((bits >> 31) == 0) { best = v[i]; best_i = i; }
    }
    return best_i;
}

/* RopeTable::new, model_runner.rs:77-100: freq = 1/base^(2i/rot), theta = pos*freq */
void yo_rope_table(uint32_t max_seq, uint32_t rot_dim, float base, float *cos_t, float *sin_t) {
    uint32_t half = rot_dim / 2;
    for (uint32_t pos = 0; pos < max_seq; pos++)
        for (uint32_t i = 0; i < half; i++) {
            float freq = 1.0f / powf(base, 2.0f * (float)i / (float)rot_dim);
            float theta = (float)pos * freq;
            cos_t[pos * half + i] = cosf(theta);
            sin_t[pos * half + i] = sinf(theta);
        }
}
