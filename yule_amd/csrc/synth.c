/*
 * synth.c — seeded synthetic weights and activations, and f32 -> GGUF block
 * quantizers (Q4_0 in Yule's interleaved nibble order, Q8_0, Q4_K, Q6_K).
 *
 * Yule has no quantizer and no seeded Gaussian generator; these produce the
 * bytes every parity check and benchmark consumes.  Quantization quality is
 * not parity-critical (GPU and CPU read the same bytes), but generation is
 * deterministic: same seed -> same bytes on any x86-64 host with this glibc.
 *
 * Generator: row r of a tensor draws from a SplitMix64 stream seeded with
 * mix(seed ^ (r * golden)); pairs of 53-bit uniforms feed Box-Muller
 * (u1 in (0,1], radius sqrt(-2 ln u1), angle 2*pi*u2), computed in double
 * and rounded to f32.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GOLDEN 0x9E3779B97F4A7C15ull

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t splitmix_next(uint64_t *s) {
    *s += GOLDEN;
    return mix64(*s);
}

uint64_t ys_splitmix64_next(uint64_t *state) { return splitmix_next(state); }

static void gauss_row(uint64_t seed, uint64_t row, float sigma, float *out, size_t n) {
    uint64_t s = mix64(seed ^ (row * GOLDEN));
    for (size_t i = 0; i < n; i += 2) {
        double u1 = ((double)(splitmix_next(&s) >> 11) + 1.0) * 0x1.0p-53;
        double u2 = (double)(splitmix_next(&s) >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
        out[i] = (float)(sigma * r * cos(t));
        if (i + 1 < n) out[i + 1] = (float)(sigma * r * sin(t));
    }
}

/* out[n_rows][n_cols] ~ N(0, sigma^2) */
void ys_gauss(uint64_t seed, float sigma, size_t n_rows, size_t n_cols, float *out) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)n_rows; r++) gauss_row(seed, (uint64_t)r, sigma, out + (size_t)r * n_cols, n_cols);
}

/* uniform integers in [0, bound) from one SplitMix64 stream (token ids) */
void ys_uniform_u32(uint64_t seed, uint32_t bound, size_t n, uint32_t *out) {
    uint64_t s = mix64(seed);
    for (size_t i = 0; i < n; i++) out[i] = (uint32_t)(splitmix_next(&s) % bound);
}

/* f32 -> IEEE half, round to nearest even */
uint16_t ys_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);           /* overflow -> inf */
    if (ax < 0x38800000u) {                                              /* subnormal / zero */
        if (ax < 0x33000000u) return (uint16_t)sign;
        uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126 - e;                                        /* 14 - (e-127) + 13 */
        uint32_t h = m >> shift, rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((ax >> 13) - (112u << 10));
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

static float f16_val(uint16_t h) {          /* exact half -> float */
    uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF, x;
    if (e == 0) {
        if (!m) { x = s; }
        else { float v = ldexpf((float)m, -24); return s ? -v : v; }
    } else if (e == 31) x = s | 0x7F800000u | (m << 13);
    else x = s | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &x, 4); return f;
}

static inline void put_f16(uint8_t *p, float v) { uint16_t h = ys_f32_to_f16(v); p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8); }
static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Q4_0 (18 B / 32): ggml's scale choice; Yule's nibble order: byte i holds
 * weight 2i (low) and 2i+1 (high) — yule-core/src/dequant.rs:77-86 */
static void quant_q4_0(const float *x, uint8_t *b) {
    float amax = 0.0f, maxv = 0.0f;
    for (int i = 0; i < 32; i++) if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); maxv = x[i]; }
    float d = maxv / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(b, d);
    for (int i = 0; i < 16; i++) {
        int q0 = clampi((int)(x[2 * i] * id + 8.5f), 0, 15);
        int q1 = clampi((int)(x[2 * i + 1] * id + 8.5f), 0, 15);
        b[2 + i] = (uint8_t)(q0 | (q1 << 4));
    }
}

/* Q8_0 (34 B / 32) */
static void quant_q8_0(const float *x, uint8_t *b) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(b, d);
    for (int i = 0; i < 32; i++) b[2 + i] = (uint8_t)(int8_t)clampi((int)lrintf(x[i] * id), -128, 127);
}

/* Q4_K (144 B / 256): per 32-weight sub-block an affine [min, max] grid of
 * 16 levels; 6-bit scales/mins relative to f16 d/dmin, packed in the
 * layout ggml's get_scale_min_k4 reads (dequant.rs:169-190). */
static void quant_q4_k(const float *x, uint8_t *b) {
    float scale[8], mins[8], smax = 0.0f, mmax = 0.0f;
    for (int s = 0; s < 8; s++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int i = 0; i < 32; i++) { lo = fminf(lo, x[32 * s + i]); hi = fmaxf(hi, x[32 * s + i]); }
        scale[s] = (hi - lo) / 15.0f;
        mins[s] = -lo;
        smax = fmaxf(smax, scale[s]);
        mmax = fmaxf(mmax, mins[s]);
    }
    put_f16(b, smax / 63.0f);
    put_f16(b + 2, mmax / 63.0f);
    float D = f16_val((uint16_t)(b[0] | (b[1] << 8))), DM = f16_val((uint16_t)(b[2] | (b[3] << 8)));
    uint8_t sc[8], mn[8];
    for (int s = 0; s < 8; s++) {
        sc[s] = (uint8_t)(D > 0.0f ? clampi((int)lrintf(scale[s] / D), 0, 63) : 0);
        mn[s] = (uint8_t)(DM > 0.0f ? clampi((int)lrintf(mins[s] / DM), 0, 63) : 0);
    }
    uint8_t *q = b + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    uint8_t lev[256];
    for (int s = 0; s < 8; s++) {
        float es = D * (float)sc[s], em = DM * (float)mn[s];
        for (int i = 0; i < 32; i++)
            lev[32 * s + i] = (uint8_t)(es > 0.0f ? clampi((int)lrintf((x[32 * s + i] + em) / es), 0, 15) : 0);
    }
    for (int j = 0; j < 4; j++)
        for (int l = 0; l < 32; l++)
            b[16 + 32 * j + l] = (uint8_t)(lev[64 * j + l] | (lev[64 * j + 32 + l] << 4));
}

/* Q5_K (176 B / 256): Q4_K's scheme with 32 levels; the 5th bit of weight
 * 64j+l (low-nibble sub-block 2j) is bit 2j of qh[l], of weight 64j+32+l
 * bit 2j+1 (dequant.rs:292-338). */
static void quant_q5_k(const float *x, uint8_t *b) {
    float scale[8], mins[8], smax = 0.0f, mmax = 0.0f;
    for (int s = 0; s < 8; s++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int i = 0; i < 32; i++) { lo = fminf(lo, x[32 * s + i]); hi = fmaxf(hi, x[32 * s + i]); }
        scale[s] = (hi - lo) / 31.0f;
        mins[s] = -lo;
        smax = fmaxf(smax, scale[s]);
        mmax = fmaxf(mmax, mins[s]);
    }
    put_f16(b, smax / 63.0f);
    put_f16(b + 2, mmax / 63.0f);
    float D = f16_val((uint16_t)(b[0] | (b[1] << 8))), DM = f16_val((uint16_t)(b[2] | (b[3] << 8)));
    uint8_t sc[8], mn[8];
    for (int s = 0; s < 8; s++) {
        sc[s] = (uint8_t)(D > 0.0f ? clampi((int)lrintf(scale[s] / D), 0, 63) : 0);
        mn[s] = (uint8_t)(DM > 0.0f ? clampi((int)lrintf(mins[s] / DM), 0, 63) : 0);
    }
    uint8_t *q = b + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    uint8_t lev[256];
    for (int s = 0; s < 8; s++) {
        float es = D * (float)sc[s], em = DM * (float)mn[s];
        for (int i = 0; i < 32; i++)
            lev[32 * s + i] = (uint8_t)(es > 0.0f ? clampi((int)lrintf((x[32 * s + i] + em) / es), 0, 31) : 0);
    }
    uint8_t *qh = b + 16;
    memset(qh, 0, 32);
    for (int j = 0; j < 4; j++)
        for (int l = 0; l < 32; l++) {
            const uint8_t a = lev[64 * j + l], c = lev[64 * j + 32 + l];
            b[48 + 32 * j + l] = (uint8_t)((a & 15) | ((c & 15) << 4));
            qh[l] |= (uint8_t)(((a >> 4) << (2 * j)) | ((c >> 4) << (2 * j + 1)));
        }
}

/* Q8_K (292 B / 256): f32 d = amax/127 (little-endian), 256 int8 quants,
 * then 16 int16 sums of consecutive 16 quants (ggml's bsums; dequant.rs
 * does not read them). */
static void quant_q8_k(const float *x, uint8_t *b) {
    float amax = 0.0f;
    for (int i = 0; i < 256; i++) amax = fmaxf(amax, fabsf(x[i]));
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    memcpy(b, &d, 4);
    for (int i = 0; i < 256; i++) b[4 + i] = (uint8_t)(int8_t)clampi((int)lrintf(x[i] * id), -128, 127);
    for (int g = 0; g < 16; g++) {
        int sum = 0;
        for (int i = 0; i < 16; i++) sum += (int8_t)b[4 + 16 * g + i];
        const int16_t s16 = (int16_t)sum;
        memcpy(b + 260 + 2 * g, &s16, 2);
    }
}

/* Q6_K (210 B / 256): 16 sub-blocks of 16 with int8 scales relative to an
 * f16 d; 6-bit quants biased by 32, split into ql nibbles and qh pairs in
 * the layout of dequant.rs:340-372. */
static void quant_q6_k(const float *x, uint8_t *b) {
    float scale[16], smax = 0.0f;
    for (int s = 0; s < 16; s++) {
        float amax = 0.0f;
        for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(x[16 * s + i]));
        scale[s] = amax / 31.0f;
        smax = fmaxf(smax, scale[s]);
    }
    put_f16(b + 208, smax / 127.0f);
    float D = f16_val((uint16_t)(b[208] | (b[209] << 8)));
    int8_t *sc = (int8_t *)(b + 192);
    int q[256];
    for (int s = 0; s < 16; s++) {
        sc[s] = (int8_t)(D > 0.0f ? clampi((int)lrintf(scale[s] / D), -128, 127) : 0);
        float es = D * (float)sc[s];
        for (int i = 0; i < 16; i++)
            q[16 * s + i] = es != 0.0f ? clampi((int)lrintf(x[16 * s + i] / es), -32, 31) + 32 : 32;
    }
    for (int h = 0; h < 2; h++) {
        uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
        const int *qq = q + 128 * h;
        for (int l = 0; l < 32; l++) {
            int q1 = qq[l], q2 = qq[l + 32], q3 = qq[l + 64], q4 = qq[l + 96];
            ql[l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
            ql[l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
            qh[l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    }
}

static int geom(int dtype, int *bs, int *bb) {
    switch (dtype) {
    case 2: *bs = 32; *bb = 18; return 0;
    case 8: *bs = 32; *bb = 34; return 0;
    case 12: *bs = 256; *bb = 144; return 0;
    case 13: *bs = 256; *bb = 176; return 0;
    case 14: *bs = 256; *bb = 210; return 0;
    case 15: *bs = 256; *bb = 292; return 0;
    default: return -1;
    }
}

static void quant_block(int dtype, const float *x, uint8_t *b) {
    switch (dtype) {
    case 2: quant_q4_0(x, b); break;
    case 8: quant_q8_0(x, b); break;
    case 12: quant_q4_k(x, b); break;
    case 13: quant_q5_k(x, b); break;
    case 14: quant_q6_k(x, b); break;
    case 15: quant_q8_k(x, b); break;
    }
}

/* quantize x[n_rows][n_cols] row-major into GGUF blocks (n_cols % block == 0) */
int ys_quantize(int dtype, const float *x, size_t n_rows, size_t n_cols, uint8_t *out) {
    int bs, bb;
    if (geom(dtype, &bs, &bb) || n_cols % (size_t)bs) return -1;
    size_t bpr = n_cols / (size_t)bs;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)n_rows; r++)
        for (size_t k = 0; k < bpr; k++)
            quant_block(dtype, x + (size_t)r * n_cols + k * bs, out + ((size_t)r * bpr + k) * bb);
    return 0;
}

/* generate N(0, sigma^2) rows with ys_gauss's streams and quantize them,
 * without materialising the whole f32 matrix */
int ys_gen_quant(int dtype, uint64_t seed, float sigma, size_t n_rows, size_t n_cols, uint8_t *out) {
    int bs, bb;
    if (geom(dtype, &bs, &bb) || n_cols % (size_t)bs) return -1;
    size_t bpr = n_cols / (size_t)bs;
    int bad = 0;
#pragma omp parallel
    {
        float *row = (float *)malloc(n_cols * sizeof(float) + 8);
        if (!row) {
#pragma omp atomic write
            bad = 1;
        }
#pragma omp for schedule(static)
        for (long r = 0; r < (long)n_rows; r++) {
            if (!row) continue;
            gauss_row(seed, (uint64_t)r, sigma, row, n_cols);
            for (size_t k = 0; k < bpr; k++) quant_block(dtype, row + k * bs, out + ((size_t)r * bpr + k) * bb);
        }
        free(row);
    }
    return bad ? -1 : 0;
}
