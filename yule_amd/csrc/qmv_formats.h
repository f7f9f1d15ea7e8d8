// qmv_formats.h — per-format unit loads and dots of the fused dequant+dot
// matvec (one lane owns one unit: a slice of one block), used by the
// streaming and column-looping matvec kernels (qmv.hip).  The nibble
// arithmetic is described in qmv.hip.
#pragma once
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

// sum over a team of W lanes (W = 16, 32: every lane of the team receives
// it; W >= 64: the wave's sum, wave-uniform)
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

}  // namespace yule
