// qmv_common.h — pieces shared by the matvec kernels (qmv.hip).
#pragma once

#include <cstdlib>

#include "internal.h"

namespace yule {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float f16_bits(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu));
}
constexpr float kTwo24 = 16777216.0f;

// Order-preserving map of an f32 onto u32 (larger float -> larger key), so a
// 64-bit max over (key << 32 | index) is argmax with the last maximal index
// winning, as argmax_ct does (yule-infer/src/sampler.rs:150-163).
__device__ __forceinline__ uint32_t argmax_key(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// Keys of +inf and -inf.  argmax_ct's test is the sign of (v - best): equal
// finite values give +0 and the later index wins, but inf - inf is the
// default NaN, whose sign bit is set on x86, so among equal infinities the
// first index stays.  The packed key therefore carries ~row for infinite
// values (the first of them is the largest) and row otherwise.
constexpr uint32_t kKeyPosInf = 0xFF800000u, kKeyNegInf = 0x007FFFFFu;
__device__ __forceinline__ unsigned long long argmax_pack(float v, uint32_t row) {
    const uint32_t k = argmax_key(v);
    const bool inf = k == kKeyPosInf || k == kKeyNegInf;
    return ((unsigned long long)k << 32) | (inf ? ~row : row);
}
// the row of a packed key
__device__ __forceinline__ uint32_t argmax_row(unsigned long long key) {
    const uint32_t k = (uint32_t)(key >> 32), lo = (uint32_t)(key & 0xFFFFFFFFull);
    return k == kKeyPosInf || k == kKeyNegInf ? ~lo : lo;
}

// Matrices sharing one activation vector (same n_cols and format) run as
// one launch over their concatenated rows (Q/K/V, gate/up): up to
// kStreamSegs per streaming-kernel launch; the up to kMaxSegs of a request
// take two launches beyond that.
constexpr int kStreamSegs = 3;
struct Segs {
    const uint8_t *w[kMaxSegs];
    float *y[kMaxSegs];
    uint32_t start[kMaxSegs];   // first concatenated row of each segment (slots past the last: total)
    uint32_t total;
};

static inline int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0, n = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus = n;
    }
    return cus;
}

// positive integer from the environment, else dflt (tuning knobs)
static inline int env_int(const char *name, int dflt) {
    const char *e = getenv(name);
    const int v = e ? atoi(e) : dflt;
    return v > 0 ? v : dflt;
}

// on/off switch: unset gives dflt, any set value other than 0 turns it on
static inline bool env_flag(const char *name, bool dflt) {
    const char *e = getenv(name);
    return e ? atoi(e) != 0 : dflt;
}

// LDS per CU on gfx950
constexpr size_t kLdsPerCu = 160 * 1024;

}  // namespace yule
