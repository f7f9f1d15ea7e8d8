// blocks.h — bit-exact scalar dequantization of one GGUF block element on the
// device, shared by the dequant, embedding and prefill kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/yule_hip.h"

namespace yule {

// One thread per output weight, exactly the reference's f32 operation order
// (no contraction): dequant.rs:77-86, 142-150, 260-290, 297-338, 346-372,
// 376-384.
__device__ __forceinline__ float f16_exact(const uint8_t *p) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(p[0] | (p[1] << 8)));
}

__device__ inline float dequant_one(uint32_t dtype, const uint8_t *__restrict__ blk, uint32_t e) {
#pragma clang fp contract(off)
    switch (dtype) {
    case YULE_DTYPE_Q4_0: {
        const uint8_t byte = blk[2 + e / 2];
        const uint32_t nib = (e & 1u) ? (byte >> 4) : (byte & 0x0Fu);
        return ((float)nib - 8.0f) * f16_exact(blk);
    }
    case YULE_DTYPE_Q8_0:
        return (float)(int8_t)blk[2 + e] * f16_exact(blk);
    case YULE_DTYPE_Q4_K: {
        const float d = f16_exact(blk), dmin = f16_exact(blk + 2);
        const uint32_t j = e / 64, hi = (e / 32) & 1u, l = e & 31u, sb = 2 * j + hi;
        const uint8_t *q = blk + 4;
        uint32_t sc, mn;
        if (sb < 4) { sc = q[sb] & 63u; mn = q[sb + 4] & 63u; }
        else {
            sc = (q[sb + 4] & 0xFu) | ((uint32_t)(q[sb - 4] >> 6) << 4);
            mn = (uint32_t)(q[sb + 4] >> 4) | ((uint32_t)(q[sb] >> 6) << 4);
        }
        const uint8_t qs = blk[16 + 32 * j + l];
        const uint32_t v = hi ? (qs >> 4) : (qs & 0x0Fu);
        const float scale = d * (float)sc, mnv = dmin * (float)mn;
        return (float)v * scale - mnv;
    }
    case YULE_DTYPE_Q6_K: {
        const float d = f16_exact(blk + 208);
        const uint32_t half = e / 128, rr = e % 128, g = rr / 32, l = rr % 32;
        const uint8_t *ql = blk + 64 * half, *qh = blk + 128 + 32 * half;
        uint32_t v;
        switch (g) {
        case 0: v = (ql[l] & 0xFu) | ((qh[l] & 3u) << 4); break;
        case 1: v = (ql[l + 32] & 0xFu) | (((qh[l] >> 2) & 3u) << 4); break;
        case 2: v = (uint32_t)(ql[l] >> 4) | (((qh[l] >> 4) & 3u) << 4); break;
        default: v = (uint32_t)(ql[l + 32] >> 4) | (((qh[l] >> 6) & 3u) << 4); break;
        }
        const int q = (int)v - 32;
        const int8_t sc = (int8_t)blk[192 + 8 * half + l / 16 + 2 * g];
        return d * (float)sc * (float)q;
    }
    case YULE_DTYPE_Q5_K: {
        // Q4_K's header and qs with a 5th bit per weight from qh[32]:
        // bit 2j (low-nibble sub-block) or 2j+1 (high) of qh[l]
        const float d = f16_exact(blk), dmin = f16_exact(blk + 2);
        const uint32_t j = e / 64, hi = (e / 32) & 1u, l = e & 31u, sb = 2 * j + hi;
        const uint8_t *q = blk + 4;
        uint32_t sc, mn;
        if (sb < 4) { sc = q[sb] & 63u; mn = q[sb + 4] & 63u; }
        else {
            sc = (q[sb + 4] & 0xFu) | ((uint32_t)(q[sb - 4] >> 6) << 4);
            mn = (uint32_t)(q[sb + 4] >> 4) | ((uint32_t)(q[sb] >> 6) << 4);
        }
        const uint8_t qs = blk[48 + 32 * j + l];
        const uint32_t v = (hi ? (qs >> 4) : (qs & 0x0Fu)) + (((blk[16 + l] >> sb) & 1u) << 4);
        const float scale = d * (float)sc, mnv = dmin * (float)mn;
        return (float)v * scale - mnv;
    }
    case YULE_DTYPE_Q8_K: {
        const uint32_t db = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) |
                            ((uint32_t)blk[3] << 24);
        return (float)(int8_t)blk[4 + e] * __builtin_bit_cast(float, db);
    }
    default:
        return 0.f;
    }
}

}  // namespace yule
