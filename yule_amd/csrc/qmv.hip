// qmv.hip — fused dequant+dot quantized matvec (decode, batch 1) for raw GGUF
// blocks on gfx950, and the bit-exact block dequant kernel.
//
// Semantics: yule-gpu ComputeBackend::quantized_matmul (yule-gpu/src/lib.rs:
// 116-131), i.e. y[r] = sum_b vec_dot(W[r,b], x[b*bs..]) with the block dots
// of yule-core/src/dequant.rs:902-1009.  Results agree with the reference to
// f32 rounding (the summation order differs); dequant is bit-exact.
//
// Work decomposition (all formats):
//  * A "unit" is the slice of one block that one lane owns: Q4_K 64 weights
//    (one 32-byte qs group = sub-blocks 2j and 2j+1), Q6_K 32 weights, Q8_0
//    and Q4_0 one whole 32-weight block.
//  * A team of TEAM lanes (16/32/64) owns a row; a wave64 carries 64/TEAM
//    teams ("slots") on consecutive rows, so one load instruction streams a
//    contiguous stretch of consecutive rows.
//  * Each wave owns R row-groups.  At each column step a lane loads its
//    activation slice once into registers and applies it to all R rows, so
//    activation traffic is 1/R of a per-row re-read; weight bytes are read
//    from HBM exactly once, with no dequantized copy anywhere.
//  * After the column loop the TEAM partial sums are combined with xor
//    shuffles and one lane per slot stores y.
//
// Nibble arithmetic: a 4-bit (or 6/8-bit, biased to unsigned) quant masked
// into one 16-bit half of a dword is an f16 *denormal* of value q * 2^-24.
// v_fma_mix_f32 multiplies that half by an f32 activation and accumulates in
// f32 exactly as an f32 FMA on q would, scaled by 2^-24 (f16 denormals are
// preserved: the kernels run with FP16 denorm mode on).  Two AND masks per
// 4 bytes thus replace per-weight unpack + convert; the 2^24 (and the x16 of
// high nibbles masked in place) fold into the block scale.  Biased formats
// (Q6_K q+32, Q8_0 q+128, Q4_0 nib-8) subtract bias * sum(x) per unit,
// where sum(x) is computed once per column step.
#include <type_traits>

#include "blocks.h"
#include "internal.h"
#include "qmv_common.h"

namespace yule {

__device__ __forceinline__ float mix_lo(uint32_t v, float x, float acc) {
    h2_t h = __builtin_bit_cast(h2_t, v);
    return __builtin_fmaf((float)h.x, x, acc);
}
__device__ __forceinline__ float mix_hi(uint32_t v, float x, float acc) {
    h2_t h = __builtin_bit_cast(h2_t, v);
    return __builtin_fmaf((float)h.y, x, acc);
}
// dword of bytes [s, s+4) of the little-endian pair {hi:lo}, s in 0..3
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbyte(hi, lo, s);
}
// bytes [s/8, s/8+4) of {hi:lo}, s in {16, 32}
__device__ __forceinline__ uint32_t shr64(uint32_t hi, uint32_t lo, uint32_t s) {
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> s);
}

// Weight loads (plain: the nontemporal hint measured slower here on gfx950).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldw16(const uint8_t *p) {
    const u32x4 v = *reinterpret_cast<const u32x4 *>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ldw4(const uint32_t *p) { return *p; }

// Activation accessors: float4 at element i (i % 4 == 0) of x, either from
// global memory or from the LDS copy, which pads 4 floats after every 32 so
// that lanes reading consecutive unit slices spread over the LDS banks.
struct XGlobal {
    const float *__restrict__ p;
    __device__ float4 operator()(uint32_t i) const { return *reinterpret_cast<const float4 *>(p + i); }
};
__host__ __device__ __forceinline__ uint32_t lds_pad(uint32_t i) { return i + ((i >> 5) << 2); }
struct XLds {
    const float *p;
    __device__ float4 operator()(uint32_t i) const { return *reinterpret_cast<const float4 *>(p + lds_pad(i)); }
};

// ---------------------------------------------------------------- Q4_K
// 144 B: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16 (dequant.rs:255-290)
struct Q4K {
    static constexpr uint32_t BS = 256, BB = 144, UPB = 4, NX = 64, NAUX = 2;
    struct Raw { uint4 h, qa, qb; };
    template <class X>
    __device__ static void load_x(const X &x, uint32_t k, uint32_t j, float *xs, float *aux) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float4 v = x(k * 256 + j * 64 + 4 * i);
            xs[4 * i] = v.x; xs[4 * i + 1] = v.y; xs[4 * i + 2] = v.z; xs[4 * i + 3] = v.w;
        }
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) { s0 += xs[i]; s1 += xs[32 + i]; }
        aux[0] = s0; aux[1] = s1;
    }
    __device__ static Raw load(const uint8_t *__restrict__ blk, uint32_t j) {
        Raw r;
        r.h = ldw16(blk);
        r.qa = ldw16(blk + 16 + 32 * j);
        r.qb = ldw16(blk + 32 + 32 * j);
        return r;
    }
    __device__ static float dot(const Raw &r, uint32_t j, const float *xs, const float *aux) {
        const float d = f16_bits(r.h.x), dmin = f16_bits(r.h.x >> 16);
        // 6-bit scales/mins of sub-blocks 2j, 2j+1 (get_scale_min_k4,
        // dequant.rs:176-190), two bytes at a time
        const uint32_t sh = (j & 1u) << 4;
        const bool low = j < 2;
        const uint32_t A = low ? r.h.y : r.h.w, Am = low ? r.h.z : (r.h.w >> 4);
        const uint32_t mA = low ? 0x3F3Fu : 0x0F0Fu, mB = low ? 0u : 0x3030u;
        const uint32_t scs = ((A >> sh) & mA) | ((r.h.y >> (sh + 2)) & mB);
        const uint32_t mns = ((Am >> sh) & mA) | ((r.h.z >> (sh + 2)) & mB);
        const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        float alo = 0.f, ahi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t w = q[i], s = w >> 8;
            const uint32_t a = w & 0x000F000Fu, b = s & 0x000F000Fu;   // low nibbles (x1)
            const uint32_t c = w & 0x00F000F0u, e = s & 0x00F000F0u;   // high nibbles (x16)
            alo = mix_lo(a, xs[4 * i + 0], alo);
            alo = mix_lo(b, xs[4 * i + 1], alo);
            alo = mix_hi(a, xs[4 * i + 2], alo);
            alo = mix_hi(b, xs[4 * i + 3], alo);
            ahi = mix_lo(c, xs[32 + 4 * i + 0], ahi);
            ahi = mix_lo(e, xs[32 + 4 * i + 1], ahi);
            ahi = mix_hi(c, xs[32 + 4 * i + 2], ahi);
            ahi = mix_hi(e, xs[32 + 4 * i + 3], ahi);
        }
        const float sc0 = (float)(scs & 0xFFu), sc1 = (float)(scs >> 8);
        const float mn0 = (float)(mns & 0xFFu), mn1 = (float)(mns >> 8);
        const float t = sc0 * alo + (sc1 * 0.0625f) * ahi;
        return (d * kTwo24) * t - dmin * (mn0 * aux[0] + mn1 * aux[1]);
    }
};

// ---------------------------------------------------------------- Q5_K
// 176 B: d f16 @0, dmin f16 @2, scales[12] @4, qh[32] @16, qs[128] @48
// (dequant.rs:292-338).  Q4_K's units (group j = sub-blocks 2j, 2j+1) with
// a 5th bit per weight: bit 2j (low nibble) / 2j+1 (high) of qh[l].  The bit
// is merged into the f16-denormal halves: bit 4 of a low-nibble half (+16),
// bit 8 of a high-nibble half, whose x16 is already in place (+16*16).
struct Q5K {
    static constexpr uint32_t BS = 256, BB = 176, UPB = 4, NX = 64, NAUX = 2;
    struct Raw { uint4 h, ha, hb, qa, qb; };
    template <class X>
    __device__ static void load_x(const X &x, uint32_t k, uint32_t j, float *xs, float *aux) {
        Q4K::load_x(x, k, j, xs, aux);
    }
    __device__ static Raw load(const uint8_t *__restrict__ blk, uint32_t j) {
        Raw r;
        r.h = ldw16(blk);
        r.ha = ldw16(blk + 16);
        r.hb = ldw16(blk + 32);
        r.qa = ldw16(blk + 48 + 32 * j);
        r.qb = ldw16(blk + 64 + 32 * j);
        return r;
    }
    __device__ static float dot(const Raw &r, uint32_t j, const float *xs, const float *aux) {
        const float d = f16_bits(r.h.x), dmin = f16_bits(r.h.x >> 16);
        const uint32_t sh = (j & 1u) << 4;
        const bool low = j < 2;
        const uint32_t A = low ? r.h.y : r.h.w, Am = low ? r.h.z : (r.h.w >> 4);
        const uint32_t mA = low ? 0x3F3Fu : 0x0F0Fu, mB = low ? 0u : 0x3030u;
        const uint32_t scs = ((A >> sh) & mA) | ((r.h.y >> (sh + 2)) & mB);
        const uint32_t mns = ((Am >> sh) & mA) | ((r.h.z >> (sh + 2)) & mB);
        const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        const uint32_t hq[8] = {r.ha.x, r.ha.y, r.ha.z, r.ha.w, r.hb.x, r.hb.y, r.hb.z, r.hb.w};
        float alo = 0.f, ahi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t w = q[i], s = w >> 8;
            const uint32_t hb = hq[i] >> (2 * j), hs = hb >> 8;   // bit 0: low, bit 1: high nibble's 5th bit
            const uint32_t a = (w & 0x000F000Fu) | ((hb & 0x00010001u) << 4);
            const uint32_t b = (s & 0x000F000Fu) | ((hs & 0x00010001u) << 4);
            const uint32_t c = (w & 0x00F000F0u) | ((hb & 0x00020002u) << 7);
            const uint32_t e = (s & 0x00F000F0u) | ((hs & 0x00020002u) << 7);
            alo = mix_lo(a, xs[4 * i + 0], alo);
            alo = mix_lo(b, xs[4 * i + 1], alo);
            alo = mix_hi(a, xs[4 * i + 2], alo);
            alo = mix_hi(b, xs[4 * i + 3], alo);
            ahi = mix_lo(c, xs[32 + 4 * i + 0], ahi);
            ahi = mix_lo(e, xs[32 + 4 * i + 1], ahi);
            ahi = mix_hi(c, xs[32 + 4 * i + 2], ahi);
            ahi = mix_hi(e, xs[32 + 4 * i + 3], ahi);
        }
        const float sc0 = (float)(scs & 0xFFu), sc1 = (float)(scs >> 8);
        const float mn0 = (float)(mns & 0xFFu), mn1 = (float)(mns >> 8);
        const float t = sc0 * alo + (sc1 * 0.0625f) * ahi;
        return (d * kTwo24) * t - dmin * (mn0 * aux[0] + mn1 * aux[1]);
    }
};

// ---------------------------------------------------------------- Q8_K
// 292 B: d f32 @0, qs int8[256] @4, bsums[16] @260 (not read;
// dequant.rs:374-384).  Rows are a multiple of 4 bytes, so every block is
// dword aligned.  Unit u = quants 32u..32u+31, read as q ^ 0x80 = q + 128
// into f16-denormal halves, minus 128 * sum(x).
struct Q8K {
    static constexpr uint32_t BS = 256, BB = 292, UPB = 8, NX = 32, NAUX = 1;
    struct Raw { uint32_t d, w[8]; };
    template <class X>
    __device__ static void load_x(const X &x, uint32_t k, uint32_t u, float *xs, float *aux) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 v = x(k * 256 + u * 32 + 4 * i);
            xs[4 * i] = v.x; xs[4 * i + 1] = v.y; xs[4 * i + 2] = v.z; xs[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 32; i++) s += xs[i];
        aux[0] = s;
    }
    __device__ static Raw load(const uint8_t *__restrict__ blk, uint32_t u) {
        Raw r;
        const uint32_t *p = reinterpret_cast<const uint32_t *>(blk);
        r.d = ldw4(p);
#pragma unroll
        for (int i = 0; i < 8; i++) r.w[i] = ldw4(p + 1 + 8 * u + i);
        return r;
    }
    __device__ static float dot(const Raw &r, uint32_t, const float *xs, const float *aux) {
        const float d = __builtin_bit_cast(float, r.d);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q = r.w[i] ^ 0x80808080u;   // q + 128
            const uint32_t ev = q & 0x00FF00FFu, od = (q >> 8) & 0x00FF00FFu;
            acc = mix_lo(ev, xs[4 * i + 0], acc);
            acc = mix_lo(od, xs[4 * i + 1], acc);
            acc = mix_hi(ev, xs[4 * i + 2], acc);
            acc = mix_hi(od, xs[4 * i + 3], acc);
        }
        return d * (acc * kTwo24 - 128.f * aux[0]);
    }
};

// ---------------------------------------------------------------- Q6_K
// 210 B: ql[128] @0, qh[64] @128, scales i8[16] @192, d f16 @208
// (dequant.rs:340-372).  Unit u (0..7) = half h = u/4, positions
// l in [8p, 8p+8) with p = u%4, all four quarters g: 32 weights
// 128h + 32g + l, scales sc[8h + p/2 + 2g].  Blocks are only 2-byte aligned,
// so each field is read through an aligned dword window and realigned.
struct Q6K {
    static constexpr uint32_t BS = 256, BB = 210, UPB = 8, NX = 32, NAUX = 4;
    struct Raw { uint32_t a[3], b[3], h[3], s[3], d; uint32_t ma; };
    template <class X>
    __device__ static void load_x(const X &x, uint32_t k, uint32_t u, float *xs, float *aux) {
        const uint32_t h = u >> 2, p = u & 3u;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint32_t o = k * 256 + h * 128 + g * 32 + p * 8;
            float4 v0 = x(o), v1 = x(o + 4);
            xs[8 * g + 0] = v0.x; xs[8 * g + 1] = v0.y; xs[8 * g + 2] = v0.z; xs[8 * g + 3] = v0.w;
            xs[8 * g + 4] = v1.x; xs[8 * g + 5] = v1.y; xs[8 * g + 6] = v1.z; xs[8 * g + 7] = v1.w;
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) s += xs[8 * g + i];
            aux[g] = s;
        }
    }
    __device__ static Raw load(const uint8_t *__restrict__ blk, uint32_t u) {
        const uint32_t h = u >> 2, p = u & 3u;
        Raw r;
        r.ma = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
        const uint8_t *b0 = blk - r.ma;
        const uint32_t *pa = reinterpret_cast<const uint32_t *>(b0 + 64 * h + 8 * p);
        const uint32_t *pb = reinterpret_cast<const uint32_t *>(b0 + 64 * h + 32 + 8 * p);
        const uint32_t *ph = reinterpret_cast<const uint32_t *>(b0 + 128 + 32 * h + 8 * p);
        const uint32_t so = 192 + 8 * h + (p >> 1) + r.ma;   // scale bytes, from b0
        const uint32_t *ps = reinterpret_cast<const uint32_t *>(b0 + (so & ~3u));
#pragma unroll
        for (int i = 0; i < 3; i++) { r.a[i] = ldw4(pa + i); r.b[i] = ldw4(pb + i); r.h[i] = ldw4(ph + i); r.s[i] = ldw4(ps + i); }
        r.d = ldw4(reinterpret_cast<const uint32_t *>(b0 + 208));
        return r;
    }
    __device__ static float dot(const Raw &r, uint32_t u, const float *xs, const float *aux) {
        const uint32_t ma = r.ma, ms = (ma + ((u & 3u) >> 1)) & 3u;
        const float d = f16_bits(r.d >> (8 * ma));
        const uint32_t s_lo = align_bytes(r.s[1], r.s[0], ms), s_hi = align_bytes(r.s[2], r.s[1], ms);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t qa = align_bytes(r.a[i + 1], r.a[i], ma);
            const uint32_t qb = align_bytes(r.b[i + 1], r.b[i], ma);
            const uint32_t hh = align_bytes(r.h[i + 1], r.h[i], ma);
            uint32_t q[4];
            q[0] = (qa & 0x0F0F0F0Fu) | ((hh & 0x03030303u) << 4);
            q[1] = (qb & 0x0F0F0F0Fu) | ((hh & 0x0C0C0C0Cu) << 2);
            q[2] = ((qa >> 4) & 0x0F0F0F0Fu) | (hh & 0x30303030u);
            q[3] = ((qb >> 4) & 0x0F0F0F0Fu) | ((hh >> 2) & 0x30303030u);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t ev = q[g] & 0x00FF00FFu, od = (q[g] >> 8) & 0x00FF00FFu;
                acc[g] = mix_lo(ev, xs[8 * g + 4 * i + 0], acc[g]);
                acc[g] = mix_lo(od, xs[8 * g + 4 * i + 1], acc[g]);
                acc[g] = mix_hi(ev, xs[8 * g + 4 * i + 2], acc[g]);
                acc[g] = mix_hi(od, xs[8 * g + 4 * i + 3], acc[g]);
            }
        }
        const float sc0 = (float)(int8_t)(s_lo & 0xFFu), sc1 = (float)(int8_t)((s_lo >> 16) & 0xFFu);
        const float sc2 = (float)(int8_t)(s_hi & 0xFFu), sc3 = (float)(int8_t)((s_hi >> 16) & 0xFFu);
        float t = sc0 * (acc[0] * kTwo24 - 32.f * aux[0]);
        t += sc1 * (acc[1] * kTwo24 - 32.f * aux[1]);
        t += sc2 * (acc[2] * kTwo24 - 32.f * aux[2]);
        t += sc3 * (acc[3] * kTwo24 - 32.f * aux[3]);
        return d * t;
    }
};

// ---------------------------------------------------------------- Q8_0
// 34 B: d f16 @0, qs i8[32] @2 (dequant.rs:139-150). One block per unit.
struct Q80 {
    static constexpr uint32_t BS = 32, BB = 34, UPB = 1, NX = 32, NAUX = 1;
    struct Raw { uint32_t w[9]; uint32_t ma; };
    template <class X>
    __device__ static void load_x(const X &x, uint32_t k, uint32_t, float *xs, float *aux) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 v = x(k * 32 + 4 * i);
            xs[4 * i] = v.x; xs[4 * i + 1] = v.y; xs[4 * i + 2] = v.z; xs[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 32; i++) s += xs[i];
        aux[0] = s;
    }
    __device__ static Raw load(const uint8_t *__restrict__ blk, uint32_t) {
        Raw r;
        r.ma = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
        const uint32_t *p = reinterpret_cast<const uint32_t *>(blk - r.ma);
#pragma unroll
        for (int i = 0; i < 9; i++) r.w[i] = ldw4(p + i);
        return r;
    }
    __device__ static float dot(const Raw &r, uint32_t, const float *xs, const float *aux) {
        const float d = f16_bits(r.w[0] >> (8 * r.ma));
        const uint32_t sh = 8 * (r.ma + 2);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q = shr64(r.w[i + 1], r.w[i], sh) ^ 0x80808080u;   // q + 128
            const uint32_t ev = q & 0x00FF00FFu, od = (q >> 8) & 0x00FF00FFu;
            acc = mix_lo(ev, xs[4 * i + 0], acc);
            acc = mix_lo(od, xs[4 * i + 1], acc);
            acc = mix_hi(ev, xs[4 * i + 2], acc);
            acc = mix_hi(od, xs[4 * i + 3], acc);
        }
        return d * (acc * kTwo24 - 128.f * aux[0]);
    }
};

// ---------------------------------------------------------------- Q4_0
// 18 B: d f16 @0, qs[16] @2, Yule's interleaved order: byte i holds weight
// 2i (low nibble) and 2i+1 (high nibble) (dequant.rs:77-86).
struct Q40 {
    static constexpr uint32_t BS = 32, BB = 18, UPB = 1, NX = 32, NAUX = 1;
    struct Raw { uint32_t w[5]; uint32_t ma; };
    template <class X>
    __device__ static void load_x(const X &x, uint32_t k, uint32_t u, float *xs, float *aux) {
        Q80::load_x(x, k, u, xs, aux);
    }
    __device__ static Raw load(const uint8_t *__restrict__ blk, uint32_t) {
        Raw r;
        r.ma = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
        const uint32_t *p = reinterpret_cast<const uint32_t *>(blk - r.ma);
#pragma unroll
        for (int i = 0; i < 5; i++) r.w[i] = ldw4(p + i);
        return r;
    }
    __device__ static float dot(const Raw &r, uint32_t, const float *xs, const float *aux) {
        const float d = f16_bits(r.w[0] >> (8 * r.ma));
        const uint32_t sh = 8 * (r.ma + 2);
        float a1 = 0.f, a16 = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = shr64(r.w[i + 1], r.w[i], sh), s = w >> 8;
            const uint32_t a = w & 0x000F000Fu, b = s & 0x000F000Fu;   // weights 8i+{0,4}, 8i+{2,6}
            const uint32_t c = w & 0x00F000F0u, e = s & 0x00F000F0u;   // 8i+{1,5}, 8i+{3,7} (x16)
            a1 = mix_lo(a, xs[8 * i + 0], a1);
            a1 = mix_lo(b, xs[8 * i + 2], a1);
            a1 = mix_hi(a, xs[8 * i + 4], a1);
            a1 = mix_hi(b, xs[8 * i + 6], a1);
            a16 = mix_lo(c, xs[8 * i + 1], a16);
            a16 = mix_lo(e, xs[8 * i + 3], a16);
            a16 = mix_hi(c, xs[8 * i + 5], a16);
            a16 = mix_hi(e, xs[8 * i + 7], a16);
        }
        return d * ((a1 + a16 * 0.0625f) * kTwo24 - 8.f * aux[0]);
    }
};

// ---------------------------------------------------------------- kernel
template <class F, int TEAM, int R>
__global__ __launch_bounds__(256) void qmv_kernel(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                  float *__restrict__ y, uint32_t n_rows, uint32_t bpr) {
    constexpr uint32_t SLOTS = 64 / TEAM;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
    const uint32_t slot = lane / TEAM, t = lane % TEAM;
    const uint32_t row0 = wave * (SLOTS * R) + slot;
    const uint32_t units = bpr * F::UPB;
    const size_t row_bytes = (size_t)bpr * F::BB;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

    for (uint32_t u0 = 0; u0 < units; u0 += TEAM) {
        const uint32_t u = u0 + t;
        if (u < units) {
            const uint32_t k = u / F::UPB, sub = u % F::UPB;
            float xs[F::NX], aux[F::NAUX];
            F::load_x(XGlobal{x}, k, sub, xs, aux);
            typename F::Raw raw[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                uint32_t row = row0 + r * SLOTS;
                row = row < n_rows ? row : n_rows - 1;   // rows past the end re-read the last row
                raw[r] = F::load(w + row * row_bytes + (size_t)k * F::BB, sub);
            }
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] += F::dot(raw[r], sub, xs, aux);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int off = TEAM / 2; off >= 1; off >>= 1) acc[r] += __shfl_xor(acc[r], off, 64);
    }
    if (t == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = row0 + r * SLOTS;
            if (row < n_rows) y[row] = acc[r];
        }
    }
}

template <class F, int TEAM, int R>
static void launch_one(hipStream_t s, const uint8_t *w, const float *x, float *y, uint32_t n_rows, uint32_t bpr) {
    constexpr uint32_t rows_per_wave = (64 / TEAM) * R;
    const uint32_t waves = (n_rows + rows_per_wave - 1) / rows_per_wave;
    const uint32_t blocks = (waves + 3) / 4;
    hipLaunchKernelGGL((qmv_kernel<F, TEAM, R>), dim3(blocks), dim3(256), 0, s, w, x, y, n_rows, bpr);
}

template <class F, int TEAM>
static void launch_team(hipStream_t s, const uint8_t *w, const float *x, float *y, uint32_t n_rows, uint32_t bpr) {
    constexpr uint32_t slots = 64 / TEAM;
    if ((uint64_t)n_rows >= 2048ull * slots * 8) launch_one<F, TEAM, 8>(s, w, x, y, n_rows, bpr);
    else if ((uint64_t)n_rows >= 2048ull * slots * 4) launch_one<F, TEAM, 4>(s, w, x, y, n_rows, bpr);
    else if ((uint64_t)n_rows >= 2048ull * slots * 2) launch_one<F, TEAM, 2>(s, w, x, y, n_rows, bpr);
    else launch_one<F, TEAM, 1>(s, w, x, y, n_rows, bpr);
}

// Team width of the column-looping kernel: the one of 64/32/16 lanes that
// wastes the fewest lanes on the row's last column step.
static uint32_t pick_team(uint32_t units) {
    uint32_t best = 64;
    double best_eff = -1.0;
    for (uint32_t team : {64u, 32u, 16u}) {
        const uint32_t steps = (units + team - 1) / team;
        const double eff = (double)units / (double)(steps * team);
        if (eff > best_eff + 1e-9) { best_eff = eff; best = team; }
    }
    return best;
}

// ---------------------------------------------------------------- streaming kernel
// Rows stream through persistent workgroups.  A team of W lanes (16..512)
// covers a whole row, one unit per lane, so each lane's activation slice is
// loaded into registers once for the life of the workgroup; the team then
// walks rows row0, row0 + stride, ... with the next row's blocks already in
// flight while the current one is computed.  With several teams per
// workgroup, x is staged once through LDS.  Teams wider than a wave combine
// their per-wave sums through LDS.
template <int W>
__device__ __forceinline__ float team_sum(float v) {
    // within rows of 16 lanes: xor 1, xor 2 (quad_perm), half-mirror, mirror
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    if (W >= 64) {
        // the four row sums straight into scalar registers (wave-uniform result)
        const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
        const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
        const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
        const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
        return (r0 + r1) + (r2 + r3);
    }
    if (W >= 32) v += __shfl_xor(v, 16, 64);
    return v;
}

template <class R>
struct RawPair {
    R g, u;
};

// PAIR: segments 0 and 1 are the gate and up matrices (equal row counts);
// a team computes row r of both and stores silu(g)*u into segment 0's
// output (model_runner.rs:963-972), so SwiGLU costs nothing extra.
template <class F, int W, int D, int NT, bool PAIR, bool TWO>
__global__ __launch_bounds__(NT) void qmv_stream_kernel(const Segs sg, const float *__restrict__ x, uint32_t bpr,
                                                        const QmvXf xf) {
    static_assert(!PAIR || W <= 64, "paired rows need single-wave teams");
    constexpr uint32_t RI = NT / W;                   // rows per workgroup iteration
    constexpr uint32_t NWV = NT / 64;                 // waves per workgroup
    constexpr uint32_t WPT = W >= 64 ? W / 64 : 1;    // waves per team
    using Buf = typename std::conditional<PAIR, RawPair<typename F::Raw>, typename F::Raw>::type;
    extern __shared__ float xl[];
    __shared__ float part[NWV];
    const uint32_t tid = threadIdx.x, team = tid / W, t = tid % W;
    const uint32_t units = bpr * F::UPB, n_rows = PAIR ? sg.start[1] : sg.total;
    const size_t row_bytes = (size_t)bpr * F::BB;
    const bool active = t < units;
    const uint32_t k = active ? t / F::UPB : 0, sub = t % F::UPB;
    const uint32_t stride = gridDim.x * RI;
    const uint32_t r0 = blockIdx.x * RI;
    if (r0 >= n_rows) return;   // uniform per workgroup

    // concatenated row -> weight row pointer / output slot.  vbase[i] is
    // segment i's weight base moved back by start[i] rows, so a row's
    // address is vbase[seg] + row * row_bytes.  With whole-wave teams the
    // row is wave-uniform and all of this runs on the scalar unit.
    auto uni = [&](uint32_t v) { return W >= 64 ? __builtin_amdgcn_readfirstlane(v) : v; };
    auto seg_of = [&](uint32_t row) {
        uint32_t s = 0;
#pragma unroll
        for (int i = 1; i < kMaxSegs; i++) s += row >= sg.start[i];
        return s;
    };
    auto fetch = [&](uint32_t rbase) -> Buf {
        uint32_t row = rbase + team;
        row = uni(row < n_rows ? row : n_rows - 1);
        if constexpr (PAIR) {
            const size_t off = (size_t)row * row_bytes + (size_t)k * F::BB;
            return {F::load(sg.w[0] + off, sub), F::load(sg.w[1] + off, sub)};
        } else {
            const uint32_t s = seg_of(row);
            const uint8_t *wb = sg.w[0] - (size_t)sg.start[0] * row_bytes;
#pragma unroll
            for (int i = 1; i < kMaxSegs; i++)
                wb = s == (uint32_t)i ? sg.w[i] - (size_t)sg.start[i] * row_bytes : wb;
            return F::load(wb + (size_t)row * row_bytes + (size_t)k * F::BB, sub);
        }
    };
    unsigned long long best = 0;   // kEpiArgmax: packed (order key << 32 | row), max wins
    // `row` may differ across the lanes of a wave (ring flushes); callers
    // with a wave-uniform row pass it through uni() first
    auto store = [&](uint32_t row, float v) {
        const uint32_t s = seg_of(row);
        float *yb = sg.y[0] - sg.start[0];
#pragma unroll
        for (int i = 1; i < kMaxSegs; i++) yb = s == (uint32_t)i ? sg.y[i] - sg.start[i] : yb;
        if (xf.epi == kEpiAdd) v = yb[row] + v;   // residual + projection (model_runner.rs:782-784)
        yb[row] = v;
        if (xf.epi == kEpiArgmax) {
            const unsigned long long key = argmax_pack(v, row);
            best = key > best ? key : best;
        }
    };

    // Prologue order: this thread's share of x, and of the fused input
    // transform's second operand (RMSNorm weight or SwiGLU up), is loaded
    // into registers first, then the first rows' weight loads are issued,
    // then x goes to LDS.  Loads complete in issue order, so waiting for x
    // does not wait for the weights, and HBM latency overlaps the whole
    // staging.
    // float4 of x per thread held in flight (K <= 32 * NT in one pass; paired
    // kernels hold fewer, keeping their register count)
    constexpr uint32_t kXPer = PAIR ? 4 : 8;
    Buf buf[D];
    uint32_t rpos = 0;
    float rcos = 0.f, rsin = 0.f;
    // TWO: a fused input transform is on (its operand is loaded with x); a
    // template parameter, so the plain kernels carry none of its code
    {
        const uint32_t n = bpr * F::BS, n4 = n / 4;
        const float4 *x4 = reinterpret_cast<const float4 *>(x), *a4 = reinterpret_cast<const float4 *>(xf.a);
        float4 xv[kXPer], av[kXPer];
#pragma unroll
        for (uint32_t q = 0; q < kXPer; q++) {
            const uint32_t i = tid + NT * q;
            if (i < n4) {
                xv[q] = x4[i];
                if constexpr (TWO) av[q] = a4[i];
            }
        }
#pragma unroll
        for (int j = 0; j < D - 1; j++)
            if (r0 + j * stride < n_rows) buf[j] = fetch(r0 + j * stride);
        if (W < 64) {
            // RoPE epilogue: lane l keeps cos / sin of pair l of the position's
            // table row (unconditional loads from a valid address either way)
            const bool rope = xf.epi == kEpiRope;
            rpos = rope ? xf.ctl[0] : 0u;
            const uint32_t half = rope ? xf.hd / 2 : 1u, li = (tid & 63u) % half;
            rcos = (rope ? xf.cos_t : x)[(size_t)rpos * half + li];
            rsin = (rope ? xf.sin_t : x)[(size_t)rpos * half + li];
        }
        float inv = 1.0f;
        if (TWO && xf.mode == kXfRmsNorm) {
            // rms_norm (model_runner.rs:246-275) computed by every workgroup
            float ss = 0.f;
#pragma unroll
            for (uint32_t q = 0; q < kXPer; q++)
                if (tid + NT * q < n4) {
                    const float4 v = xv[q];
                    ss += v.x * v.x; ss += v.y * v.y; ss += v.z * v.z; ss += v.w * v.w;
                }
            for (uint32_t i = tid + NT * kXPer; i < n4; i += NT) {
                const float4 v = x4[i];
                ss += v.x * v.x; ss += v.y * v.y; ss += v.z * v.z; ss += v.w * v.w;
            }
            ss = team_sum<64>(ss);
            if ((tid & 63) == 0) part[tid >> 6] = ss;
            __syncthreads();
            ss = 0.f;
#pragma unroll
            for (uint32_t i = 0; i < NWV; i++) ss += part[i];
            inv = 1.0f / sqrtf(ss / (float)n + xf.eps);
        }
        auto put = [&](uint32_t i, float4 v, float4 a) {
            if (TWO && xf.mode == kXfRmsNorm) {
                v.x = v.x * inv * a.x; v.y = v.y * inv * a.y; v.z = v.z * inv * a.z; v.w = v.w * inv * a.w;
            } else if (TWO && xf.mode == kXfSwiGlu) {
                // gate * sigmoid(gate) * up (model_runner.rs:967-972)
                v.x = v.x * (1.0f / (1.0f + expf(-v.x))) * a.x;
                v.y = v.y * (1.0f / (1.0f + expf(-v.y))) * a.y;
                v.z = v.z * (1.0f / (1.0f + expf(-v.z))) * a.z;
                v.w = v.w * (1.0f / (1.0f + expf(-v.w))) * a.w;
            }
            *reinterpret_cast<float4 *>(xl + lds_pad(4 * i)) = v;
        };
#pragma unroll
        for (uint32_t q = 0; q < kXPer; q++)
            if (tid + NT * q < n4) put(tid + NT * q, xv[q], TWO ? av[q] : xv[q]);
        for (uint32_t i = tid + NT * kXPer; i < n4; i += NT) put(i, x4[i], TWO ? a4[i] : x4[i]);
        __syncthreads();
    }
    float xs[F::NX], aux[F::NAUX];
    F::load_x(XLds{xl}, k, sub, xs, aux);

    // Teams wider than a wave park per-wave sums in a 16-slot LDS ring and
    // flush eight row iterations per barrier (all loop control is uniform).
    __shared__ float ring[16][NWV];
    auto finish = [&](float acc, uint32_t rbase, uint32_t it, bool last) {
        acc = team_sum<(W < 64 ? W : 64)>(active ? acc : 0.f);
        if (W < 64 && xf.epi == kEpiRope) {
            // rows 2i and 2i + 1 of a head are teams 2j and 2j + 1 of one wave
            // (row bases are even): the pair meets across lane W
            const float other = __shfl_xor(acc, W, 64);
            const uint32_t row = rbase + team;
            const uint32_t s = seg_of(row < n_rows ? row : n_rows - 1), loc = row - sg.start[s < kMaxSegs ? s : 0];
            const uint32_t i = (loc % xf.hd) / 2;
            const float c = __shfl(rcos, (int)i, 64), sn = __shfl(rsin, (int)i, 64);
            const bool even = (loc & 1u) == 0;
            const float x0 = even ? acc : other, x1 = even ? other : acc;
            float v = acc;
            if (s < 2) v = even ? x0 * c - x1 * sn : x0 * sn + x1 * c;
            if (t == 0 && row < n_rows) {
                const size_t kvd = (size_t)(sg.start[2] - sg.start[1]);
                if (s == 0) sg.y[0][loc] = v;
                else (s == 1 ? xf.kc : xf.vc)[(size_t)rpos * kvd + loc] = v;
            }
        } else if (WPT == 1) {
            const uint32_t row = uni(rbase + team);
            if (t == 0 && row < n_rows) store(row, acc);
        } else {
            if ((tid & 63) == 0) ring[it & 15][tid >> 6] = acc;
            if ((it & 7) == 7 || last) {
                __syncthreads();
                const uint32_t first = it & ~7u;
                if (tid < 8 * RI) {
                    const uint32_t iter = first + tid / RI, tm = tid % RI;
                    const uint32_t row = r0 + iter * stride + tm;
                    if (iter <= it && row < n_rows) {
                        float s = 0.f;
#pragma unroll
                        for (uint32_t i = 0; i < WPT; i++) s += ring[iter & 15][tm * WPT + i];
                        store(row, s);
                    }
                }
            }
        }
    };
    // D-deep ring of row buffers: before computing row r, the load of row
    // r + (D-1)*stride is issued into the slot the previous row freed.
    uint32_t it = 0;
    for (uint32_t base = r0; base < n_rows; base += D * stride) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            const uint32_t r = base + j * stride;
            if (r >= n_rows) break;
            const uint32_t rn = r + (D - 1) * stride;
            if (rn < n_rows) buf[(j + D - 1) % D] = fetch(rn);
            if constexpr (PAIR) {
                float g = F::dot(buf[j].g, sub, xs, aux), u = F::dot(buf[j].u, sub, xs, aux);
                g = team_sum<W>(active ? g : 0.f);
                u = team_sum<W>(active ? u : 0.f);
                const uint32_t row = r + team;
                if (t == 0 && row < n_rows) sg.y[0][row] = g * (1.0f / (1.0f + expf(-g))) * u;
                it++;
            } else {
                finish(F::dot(buf[j], sub, xs, aux), r, it, r + stride >= n_rows);
                it++;
            }
        }
    }
    if (xf.epi == kEpiArgmax) {   // uniform: the workgroup's best row into its own slot
        __shared__ unsigned long long wbest[NWV];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const unsigned long long o = __shfl_xor(best, off, 64);
            best = o > best ? o : best;
        }
        if ((tid & 63) == 0) wbest[tid >> 6] = best;
        __syncthreads();
        if (tid == 0) {
            unsigned long long b = wbest[0];
            for (uint32_t i = 1; i < NWV; i++) b = wbest[i] > b ? wbest[i] : b;
            xf.amax[blockIdx.x] = b;   // one slot per workgroup: no contended atomic
        }
    }
}

template <class F, int W, int D, int NT>
static void launch_stream_d(hipStream_t s, const Segs &sg, const float *x, uint32_t bpr, uint32_t blocks,
                            const QmvXf &xf) {
    const size_t lds = (size_t)lds_pad(bpr * F::BS) * sizeof(float);
    if constexpr (W <= 64) {
        if (xf.pair) {   // always with a transform (checked by launch_qmv_fused)
            hipLaunchKernelGGL((qmv_stream_kernel<F, W, D, NT, true, true>), dim3(blocks), dim3(NT), lds, s, sg, x,
                               bpr, xf);
            return;
        }
    }
    if (xf.mode != kXfNone)
        hipLaunchKernelGGL((qmv_stream_kernel<F, W, D, NT, false, true>), dim3(blocks), dim3(NT), lds, s, sg, x, bpr,
                           xf);
    else
        hipLaunchKernelGGL((qmv_stream_kernel<F, W, D, NT, false, false>), dim3(blocks), dim3(NT), lds, s, sg, x,
                           bpr, xf);
}

// Workgroup shape: NT threads (RI = NT / W teams) share one LDS copy of the
// activation vector; about 16 waves per CU are resident (4 per SIMD, the
// VGPR limit), as NT-thread workgroups up to the LDS each copy takes.
template <class F, int W, int NT>
static void launch_stream_nt(hipStream_t s, const Segs &sg, const float *x, uint32_t bpr, const QmvXf &xf) {
    constexpr uint32_t RI = NT / W;
    static const int waves_env = env_int("YULE_QMV_WAVES_PER_CU", 16);
    const size_t lds = (size_t)lds_pad(bpr * F::BS) * sizeof(float) + 512;
    const int wg_lds = (int)(kLdsPerCu / lds);
    const int wg_waves = waves_env / (NT / 64) > 0 ? waves_env / (NT / 64) : 1;
    const int wg = wg_waves < wg_lds ? wg_waves : (wg_lds > 0 ? wg_lds : 1);
    const uint32_t rows = xf.pair ? sg.start[1] : sg.total;
    const uint32_t iters = (rows + RI - 1) / RI;
    const uint32_t cap = (uint32_t)(device_cus() * wg);
    uint32_t blocks = iters < cap ? iters : cap;
    if (xf.epi == kEpiArgmax && blocks > kArgmaxSlots) blocks = kArgmaxSlots;   // one slot per workgroup
    launch_stream_d<F, W, 2, NT>(s, sg, x, bpr, blocks, xf);
}

template <class F, int W>
static void launch_stream(hipStream_t s, const Segs &sg, const float *x, uint32_t bpr, const QmvXf &xf) {
    // one-wave teams (the 4096-column projections) measured ~1% faster in
    // 512-thread workgroups; narrower teams (2048 columns) 6% slower there
    static const int nt_narrow = env_int("YULE_QMV_THREADS", 256), nt_wide = env_int("YULE_QMV_THREADS_WIDE", 1024);
    static const int nt_w64 = env_int("YULE_QMV_THREADS_W64", 512);
    const int nt = W >= 512 ? 1024 : W >= 128 ? nt_wide : W == 64 ? nt_w64 : nt_narrow;
    if (nt >= 1024) return launch_stream_nt<F, W, 1024>(s, sg, x, bpr, xf);
    if constexpr (W >= 512) return;   // unreachable: 512-lane teams only run in 1024-thread workgroups
    else
    if (nt >= 512) return launch_stream_nt<F, W, 512>(s, sg, x, bpr, xf);
    else launch_stream_nt<F, W, 256>(s, sg, x, bpr, xf);
}

// Largest activation vector staged in LDS by the streaming kernel (floats).
constexpr uint32_t kMaxStageCols = 32768;

template <class F>
static bool stream_ok(uint32_t n_cols) {
    static const bool v1 = getenv("YULE_QMV_V1") != nullptr;
    return !v1 && (n_cols / F::BS) * F::UPB <= 512 && n_cols <= kMaxStageCols;
}

template <class F>
static int launch_fmt(hipStream_t s, const QmvSeg *segs, uint32_t n_seg, const float *x, uint32_t n_cols,
                      const QmvXf &xf) {
    const uint32_t bpr = n_cols / F::BS, units = bpr * F::UPB;
    if (stream_ok<F>(n_cols)) {
        Segs sg{};
        uint32_t total = 0;
        for (uint32_t i = 0; i < kMaxSegs; i++) {
            sg.w[i] = segs[i < n_seg ? i : 0].w;
            sg.y[i] = segs[i < n_seg ? i : 0].y;
            sg.start[i] = total;
            if (i < n_seg) total += segs[i].n_rows;
        }
        for (uint32_t i = n_seg; i < kMaxSegs; i++) sg.start[i] = total;
        sg.total = total;
        if (units <= 16) return launch_stream<F, 16>(s, sg, x, bpr, xf), YULE_OK;
        if (units <= 32) return launch_stream<F, 32>(s, sg, x, bpr, xf), YULE_OK;
        if (units <= 64) return launch_stream<F, 64>(s, sg, x, bpr, xf), YULE_OK;
        if (units <= 128) return launch_stream<F, 128>(s, sg, x, bpr, xf), YULE_OK;
        if (units <= 256) return launch_stream<F, 256>(s, sg, x, bpr, xf), YULE_OK;
        return launch_stream<F, 512>(s, sg, x, bpr, xf), YULE_OK;
    }
    if (xf.mode != kXfNone || xf.epi != kEpiStore)
        return set_error(YULE_ERR_UNSUPPORTED, "quantized_matmul: fused transform needs the streaming kernel");
    for (uint32_t i = 0; i < n_seg; i++) {   // one column-looping launch per matrix
        switch (pick_team(units)) {
        case 64: launch_team<F, 64>(s, segs[i].w, x, segs[i].y, segs[i].n_rows, bpr); break;
        case 32: launch_team<F, 32>(s, segs[i].w, x, segs[i].y, segs[i].n_rows, bpr); break;
        default: launch_team<F, 16>(s, segs[i].w, x, segs[i].y, segs[i].n_rows, bpr); break;
        }
    }
    return YULE_OK;
}

bool qmv_pairable(uint32_t dtype, uint32_t n_cols) {
    if (!qmv_fusable(dtype, n_cols)) return false;
    uint32_t bs, bb;
    quant_geometry(dtype, &bs, &bb);
    const uint32_t units = (n_cols / bs) * (dtype == YULE_DTYPE_Q4_K || dtype == YULE_DTYPE_Q5_K   ? 4u
                                            : dtype == YULE_DTYPE_Q6_K || dtype == YULE_DTYPE_Q8_K ? 8u
                                                                                                  : 1u);
    return units <= 64;
}

// The Q/K/V launch can apply RoPE and write the cache itself (kEpiRope) when
// its teams are at most 32 lanes wide (the two rows of a rotation pair then
// sit in one wave) and a head's rotation pairs fit one wave's lanes.
bool qmv_rope_ok(uint32_t dtype, uint32_t n_cols, uint32_t hd) {
    if (!qmv_fusable(dtype, n_cols) || hd == 0 || hd % 2 || hd / 2 > 64) return false;
    return qmv_pairable(dtype, n_cols) && qmv_team_width(dtype, n_cols) <= 32;
}

uint32_t qmv_team_width(uint32_t dtype, uint32_t n_cols) {
    uint32_t bs, bb;
    if (!quant_geometry(dtype, &bs, &bb)) return 0;
    const uint32_t upb = dtype == YULE_DTYPE_Q4_K || dtype == YULE_DTYPE_Q5_K   ? 4u
                         : dtype == YULE_DTYPE_Q6_K || dtype == YULE_DTYPE_Q8_K ? 8u
                                                                               : 1u;
    const uint32_t units = (n_cols / bs) * upb;
    return units <= 16 ? 16 : units <= 32 ? 32 : units <= 64 ? 64 : units <= 128 ? 128 : units <= 256 ? 256 : 512;
}

bool qmv_fusable(uint32_t dtype, uint32_t n_cols) {
    switch (dtype) {
    case YULE_DTYPE_Q4_K: return stream_ok<Q4K>(n_cols);
    case YULE_DTYPE_Q5_K: return stream_ok<Q5K>(n_cols);
    case YULE_DTYPE_Q6_K: return stream_ok<Q6K>(n_cols);
    case YULE_DTYPE_Q8_K: return stream_ok<Q8K>(n_cols);
    case YULE_DTYPE_Q8_0: return stream_ok<Q80>(n_cols);
    case YULE_DTYPE_Q4_0: return stream_ok<Q40>(n_cols);
    default: return false;
    }
}

int launch_qmv_fused(hipStream_t s, uint32_t dtype, const QmvSeg *segs, uint32_t n_seg, const float *x,
                     uint32_t n_cols, const QmvXf &xf) {
    if (n_seg == 0 || n_seg > kMaxSegs) return set_error(YULE_ERR_INVALID, "quantized_matmul: bad segment count");
    if (xf.epi == kEpiArgmax && n_seg != 1)
        return set_error(YULE_ERR_INVALID, "quantized_matmul: argmax epilogue needs a single matrix");
    if (xf.epi == kEpiRope && (n_seg != 3 || !qmv_rope_ok(dtype, n_cols, xf.hd) || segs[1].n_rows != segs[2].n_rows ||
                               segs[0].n_rows % xf.hd || segs[1].n_rows % xf.hd || xf.pair))
        return set_error(YULE_ERR_INVALID, "quantized_matmul: RoPE epilogue needs q, k, v of whole heads on narrow teams");
    if (xf.pair && (n_seg != 2 || segs[0].n_rows != segs[1].n_rows || !qmv_pairable(dtype, n_cols) ||
                    xf.mode == kXfNone))
        return set_error(YULE_ERR_INVALID, "quantized_matmul: paired gate/up needs two equal single-wave matrices and an input transform");
    int rc;
    switch (dtype) {
    case YULE_DTYPE_Q4_K: rc = launch_fmt<Q4K>(s, segs, n_seg, x, n_cols, xf); break;
    case YULE_DTYPE_Q5_K: rc = launch_fmt<Q5K>(s, segs, n_seg, x, n_cols, xf); break;
    case YULE_DTYPE_Q6_K: rc = launch_fmt<Q6K>(s, segs, n_seg, x, n_cols, xf); break;
    case YULE_DTYPE_Q8_K: rc = launch_fmt<Q8K>(s, segs, n_seg, x, n_cols, xf); break;
    case YULE_DTYPE_Q8_0: rc = launch_fmt<Q80>(s, segs, n_seg, x, n_cols, xf); break;
    case YULE_DTYPE_Q4_0: rc = launch_fmt<Q40>(s, segs, n_seg, x, n_cols, xf); break;
    default: return set_error(YULE_ERR_UNSUPPORTED, "quantized_matmul: unsupported dtype");
    }
    return rc ? rc : check_launch("quantized_matmul");
}

int launch_qmv_multi(hipStream_t s, uint32_t dtype, const QmvSeg *segs, uint32_t n_seg, const float *x,
                     uint32_t n_cols) {
    return launch_qmv_fused(s, dtype, segs, n_seg, x, n_cols, QmvXf{});
}

int launch_qmv(hipStream_t s, uint32_t dtype, const uint8_t *w, const float *x, float *y, uint32_t n_rows,
               uint32_t n_cols) {
    const QmvSeg seg{w, y, n_rows};
    return launch_qmv_multi(s, dtype, &seg, 1, x, n_cols);
}

// ---------------------------------------------------------------- dequant
__global__ void dequant_kernel(uint32_t dtype, uint32_t bs, uint32_t bb, const uint8_t *__restrict__ src,
                               float *__restrict__ dst, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    dst[i] = dequant_one(dtype, src + (i / bs) * bb, (uint32_t)(i % bs));
}

__global__ void embed_kernel(uint32_t dtype, uint32_t bs, uint32_t bb, const uint8_t *__restrict__ table,
                             const uint32_t *__restrict__ token, uint32_t n_rows, float *__restrict__ dst,
                             uint32_t dim) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    uint32_t t = token[0];
    t = t < n_rows ? t : n_rows - 1;   // a host-checked token is always in range
    const uint8_t *row = table + (size_t)t * (dim / bs) * bb;
    dst[i] = dequant_one(dtype, row + (i / bs) * bb, i % bs);
}

int launch_dequant(hipStream_t s, uint32_t dtype, const uint8_t *src, float *dst, uint32_t n_blocks) {
    uint32_t bs, bb;
    if (!quant_geometry(dtype, &bs, &bb)) return set_error(YULE_ERR_UNSUPPORTED, "dequantize: unsupported dtype");
    const uint64_t n = (uint64_t)n_blocks * bs;
    if (n == 0) return YULE_OK;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dtype, bs, bb, src, dst, n);
    return check_launch("dequantize");
}

int launch_embed_rows(hipStream_t s, uint32_t dtype, const uint8_t *table, const uint32_t *token, uint32_t n_rows,
                      float *dst, uint32_t dim) {
    uint32_t bs, bb;
    if (!quant_geometry(dtype, &bs, &bb)) return set_error(YULE_ERR_UNSUPPORTED, "embedding: unsupported dtype");
    hipLaunchKernelGGL(embed_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, dtype, bs, bb, table, token, n_rows,
                       dst, dim);
    return check_launch("embedding");
}

}  // namespace yule
