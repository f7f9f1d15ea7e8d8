// gemm.hip — prefill dequant-GEMM on the MFMA units:
//   Y[m][r] = sum_c X[m][c] * W[r][c],  X bf16 [M][K], W raw GGUF blocks, Y f32 [M][N].
// No counterpart in the reference, whose prefill is token by token
// (yule-infer/src/model_runner.rs:1075-1081); each row of Y equals one
// quantized_matmul of the corresponding row of X (parity target).
//
// Exactness: weights enter the MFMA as f16 holding exact integers (times a
// power of two) and every scale is applied in f32, so the only roundings are
// f32 accumulations.
//  * Q4_K, w = d*sc*q - dmin*mn: the B operand is sc*q*2^-14 (sc*q <= 945,
//    exact in f16), made with one v_pk_mul_f16 per two weights: the nibble
//    pair masked into a dword is the f16 denormal pair q*2^-24, times
//    (sc*2^10, sc*2^10).  A 16x16 tile accumulates one super-block (256 k)
//    into a temporary, then final += (d*2^14) * tmp in f32.
//    The min term sum_sub (dmin*mn)*(sum of x over the sub-block) is a
//    second, small MFMA product over K/32 sub-blocks with both operands
//    split into hi + lo f16 pairs (dmin*mn is an exact 17-bit f32 value);
//    hi*hi + hi*lo + lo*hi reproduces it to ~2^-22.
//  * Q6_K, w = d*sc*(q-32): the B operand is sc*(q-32) (|.| <= 4064; exact
//    up to 2048, above that rounded to the nearest even integer, i.e.
//    < 2.5e-4 relative on those few weights), d applied per super-block.
//  * Q5_K: Q4_K with the fifth bit of each quant ORed in from qh before the
//    scale multiply (sc*q <= 63*31 = 1953, still exact); same min term.
//  * Q8_K, w = d*q: the B operand is q (int8, exact), f32 d per super-block.
//  * Q8_0 / Q4_0, w = d*q and d*(q-8): the B operand is the integer q or
//    q - 8 (exact in f16, made from 1024 + q with one packed subtract), d
//    applied per 32-weight block: a 32-k MFMA step is exactly one block, so
//    acc += d * (that step's product).
//  * X: a pre-pass (one workgroup per row) scales each row by a power of two
//    that puts its largest magnitude in [2^9, 2^10), converts it to f16 once
//    per call (not once per weight tile) and stores each group of four k in
//    the order {0,2,1,3}, the order in which the dword nibble masks deliver
//    weights, so neither side is shuffled in the main loop.  A scaled bf16
//    is exact in f16 down to 2^-26 of the row's maximum (everything a sum
//    against that maximum can resolve), nothing overflows, and the Q4_K
//    sub-block sums (at most 32 * 2^10) fit f16 too; the epilogue multiplies
//    each Y row by the inverse power of two, which is exact.  f32 X
//    (yule_hip_quantized_gemm_f32) is split the same way into f16 hi + lo
//    (x = hi + lo to ~2^-22) and each workgroup sweeps its K range twice,
//    against hi and then lo, into the same accumulators: the accuracy of the
//    f32 matvec, for callers that need it (prefill whose results must match
//    token-by-token decode), in one launch.
//
#include <mutex>
#include <type_traits>
#include <string>

#include "qmv_common.h"

namespace yule {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Tiling: a workgroup of 2*BN threads computes a BM (m) x BN (r) tile, BN
// 128 or 256; its waves, two along m and BN/64 along r, each a BM/2 x 64
// sub-tile of MFMA 16x16x32 tiles.  K advances in
// stages of 64 (a quarter super-block): X and weight bytes of stage s+2 are
// loaded into registers while stage s runs on the MFMAs out of one LDS buffer
// and stage s+1 is dequantized into the other, one barrier per stage.  LDS
// rows are padded (72 or 80 halves) so that the 16 rows one ds_read_b128
// reads spread over the banks.
constexpr int GSK = 64;
// Offset (halves) of 16-byte chunk c of row r in a swizzled 64-half-wide
// LDS tile: chunk c ^ f(r), f a permutation of r & 7.  A group of eight lanes
// of an MFMA operand read takes chunk c of eight consecutive rows (distinct
// f(r): distinct slots).  A weight store takes rows r..r+3 (r % 4 == 0) x
// the two threads of a row, at chunks (k, k + 2) for the Q4_K/Q5_K nibble
// halves and (k, k + 4) for the other formats; f = the bit order (0, 2, 1)
// of r & 7 for the first and the identity for the second keep those eight
// slots distinct too.  X stores take the eight chunks of one row.
template <bool Q4>
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) {
    const uint32_t f = Q4 ? ((r & 1u) | ((r >> 1) & 2u) | ((r << 1) & 4u)) : (r & 7u);
    return r * GSK + ((c ^ f) << 3);
}

__device__ __forceinline__ _Float16 bf16_to_f16(uint16_t b) {
    return (_Float16)__builtin_bit_cast(float, (uint32_t)b << 16);
}

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_scale(uint32_t pair, h2v s) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, pair) * s);
}

// n bytes starting at p (only 2-byte aligned) as n/4 little-endian dwords,
// from the raw 4-byte-aligned window raw[] (the backend pads every allocation).
template <int N>
__device__ __forceinline__ void load_raw(const uint8_t *p, uint32_t *raw, uint32_t &mis) {
    mis = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(p - mis);
#pragma unroll
    for (int i = 0; i < N / 4 + 1; i++) raw[i] = w[i];
}
template <int N>
__device__ __forceinline__ void align_raw(const uint32_t *raw, uint32_t mis, uint32_t *out) {
#pragma unroll
    for (int i = 0; i < N / 4; i++) out[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], mis);
}

// X pre-pass, one workgroup of 256 threads per row m (8-element chunks c =
// tid + 256 i).  Pass 1: the row's largest magnitude, which sets the power of
// two s = 2^(10 - e) with |x| max = f * 2^e, f in [0.5, 1), so that the
// scaled row lies below 2^10 (a row of zeros, or one holding inf or NaN,
// keeps s = 1).  Pass 2 (the row again, now from L2): xh = f16(x * s) in the
// {0,2,1,3} order; for f32 input also xl = f16(x * s - xh); the Q4_K min
// term's sub-block sums of x * s as f16 hi + lo; rowscale[m] = 1 / s.
template <bool F32>
// (inputs first: the leading 14 dwords arrive preloaded in SGPRs)
__global__ __launch_bounds__(256) void gemm_xprep_kernel(const void *xin, const float *__restrict__ nw,
                                                         uint32_t K, float eps, uint32_t glu,
                                                         _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                                                         _Float16 *__restrict__ hi, _Float16 *__restrict__ lo,
                                                         float *__restrict__ rowscale, const float *__restrict__ part,
                                                         uint32_t ks, uint32_t ny, uint32_t rows, uint32_t accumulate) {
    __shared__ float red[4], red2[4];
    const uint32_t m = blockIdx.x, tid = threadIdx.x, nch = K / 8;
    if (part) {
        // the previous product's split-K reduction of this row first (its
        // partials part[z][rows][ny] summed z ascending into xin's row, plus
        // the row itself with accumulate: the same operations, in the same
        // order, as gemm_reduce_kernel), then the row is this product's X
        // (xin is written here, so it carries no __restrict__)
        float *yrow = const_cast<float *>(static_cast<const float *>(xin)) + (size_t)m * ny;
        const size_t stride = (size_t)rows * ny;
        const float *prow = part + (size_t)m * ny;
        // float4 columns, four at a time per thread: every partial of them
        // loaded before the sums (per element the same order as above)
        const uint32_t n4 = ny / 4;
        float4 *y4 = reinterpret_cast<float4 *>(yrow);
        const float4 *p4 = reinterpret_cast<const float4 *>(prow);
        const size_t st4 = stride / 4;
        for (uint32_t i0 = tid; i0 < n4; i0 += 4 * 256) {
            float4 sum[4], base[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t i = i0 + 256 * u < n4 ? i0 + 256 * u : i0;
                sum[u] = p4[i];
                base[u] = accumulate ? y4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            for (uint32_t z = 1; z < ks; z++) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = p4[(size_t)z * st4 + (i0 + 256 * u < n4 ? i0 + 256 * u : i0)];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    sum[u].x += v[u].x; sum[u].y += v[u].y; sum[u].z += v[u].z; sum[u].w += v[u].w;
                }
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (i0 + 256 * u >= n4) break;
                float4 r = sum[u];
                if (accumulate) { r.x = base[u].x + r.x; r.y = base[u].y + r.y; r.z = base[u].z + r.z; r.w = base[u].w + r.w; }
                y4[i0 + 256 * u] = r;
            }
        }
        __threadfence_block();
        __syncthreads();
    }
    auto load8 = [&](uint32_t c, float *v) {
        if constexpr (F32) {
            if (glu) {
                // rows held as [gate | up] (2K wide): x = gate * sigmoid(gate) * up
                // (SwiGLU, model_runner.rs:967-972, as the eltwise form computes it)
                const float *g = static_cast<const float *>(xin) + (size_t)m * 2 * K + 8 * c;
                const float4 a = reinterpret_cast<const float4 *>(g)[0], b = reinterpret_cast<const float4 *>(g)[1];
                const float4 ua = reinterpret_cast<const float4 *>(g + K)[0], ub = reinterpret_cast<const float4 *>(g + K)[1];
                const float gv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                const float uv[8] = {ua.x, ua.y, ua.z, ua.w, ub.x, ub.y, ub.z, ub.w};
#pragma unroll
                for (int t = 0; t < 8; t++) v[t] = gv[t] * (1.0f / (1.0f + expf(-gv[t]))) * uv[t];
                return;
            }
            const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(xin) + (size_t)m * K + 8 * c);
            const float4 a = p[0], b = p[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(xin) + (size_t)m * K + 8 * c);
            const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                v[2 * t] = __builtin_bit_cast(float, wv[t] << 16);
                v[2 * t + 1] = __builtin_bit_cast(float, wv[t] & 0xFFFF0000u);
            }
        }
    };
    // nw: the row is x * inv * nw, inv = 1 / sqrt(mean(x^2) + eps) (RMSNorm,
    // model_runner.rs:246-275, fused here so that the projection reads the
    // residual stream itself)
    auto loadw8 = [&](uint32_t c, float *v) {
        const float4 *p = reinterpret_cast<const float4 *>(nw + 8 * c);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    };
    float amax = 0.f, ss = 0.f;
    for (uint32_t c = tid; c < nch; c += 256) {
        float v[8];
        load8(c, v);
        if (nw) {
            float wv[8];
            loadw8(c, wv);
#pragma unroll
            for (int t = 0; t < 8; t++) {
                ss += v[t] * v[t];
                amax = fmaxf(amax, fabsf(v[t] * wv[t]));
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; t++) amax = fmaxf(amax, fabsf(v[t]));   // NaN is dropped here, kept below
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off, 64));
        ss += __shfl_xor(ss, off, 64);
    }
    if ((tid & 63) == 0) {
        red[tid >> 6] = amax;
        red2[tid >> 6] = ss;
    }
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float inv = nw ? 1.0f / sqrtf(((red2[0] + red2[1]) + (red2[2] + red2[3])) / (float)K + eps) : 1.0f;
    amax *= inv;   // the normalised row's largest magnitude, to rounding (the scale only needs its exponent)
    int e = 0;
    (void)frexpf(amax, &e);
    const int es = 10 - e < 126 ? 10 - e : 126;   // rows below 2^-116 keep s = 2^126
    const bool scaled = amax > 0.f && amax <= 3.402823466e38f;
    const float sc = scaled ? ldexpf(1.0f, es) : 1.0f;
    const int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    // The next chunk's loads are issued before this chunk's stores: a load
    // issued after stores would wait for them (one counter for both).
    float nv[8], nwv[8];
    load8(tid < nch ? tid : 0u, nv);
    if (nw) loadw8(tid < nch ? tid : 0u, nwv);
    for (uint32_t c0 = 0; c0 < nch; c0 += 256) {   // uniform trip count: the quad sums below need every lane
        const uint32_t c = c0 + tid;
        const bool ok = c < nch;
        float v[8];
#pragma unroll
        for (int t = 0; t < 8; t++) v[t] = nv[t];
        if (nw) {
#pragma unroll
            for (int t = 0; t < 8; t++) v[t] = v[t] * inv * nwv[t];
        }
        if (c0 + 256 < nch) {
            const uint32_t cn = c + 256 < nch ? c + 256 : 0u;
            load8(cn, nv);
            if (nw) loadw8(cn, nwv);
        }
        float s = 0.f;
        uint32_t oh[4], ol[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float a = v[perm[2 * t]] * sc, b = v[perm[2 * t + 1]] * sc;
            const h2v h = {(_Float16)a, (_Float16)b};
            oh[t] = __builtin_bit_cast(uint32_t, h);
            if constexpr (F32) {
                const h2v l = {(_Float16)(a - (float)h.x), (_Float16)(b - (float)h.y)};
                ol[t] = __builtin_bit_cast(uint32_t, l);
            }
        }
#pragma unroll
        for (int t = 0; t < 8; t++) s += v[t] * sc;
        // the four chunks of a 32-element sub-block are lanes 4j..4j+3
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if (ok) {
            const size_t o = (size_t)m * K + 8 * c;
            *reinterpret_cast<uint4 *>(xh + o) = make_uint4(oh[0], oh[1], oh[2], oh[3]);
            if constexpr (F32) *reinterpret_cast<uint4 *>(xl + o) = make_uint4(ol[0], ol[1], ol[2], ol[3]);
            if (hi && (c & 3u) == 0) {
                const size_t j = (size_t)m * (K / 32) + c / 4;
                const _Float16 h = (_Float16)s;
                hi[j] = h;
                lo[j] = (_Float16)(s - (float)h);
            }
        }
    }
    if (tid == 0) rowscale[m] = scaled ? ldexpf(1.0f, -es) : 1.0f;
}

// Per-stage register staging of one thread: XCH 16-byte chunks of X and the
// thread's weight bytes (Q4_K: header + 16 qs bytes; Q6_K: raw dword windows
// of 32 ql bytes, 32 qh bytes, two scales and d).
template <uint32_t DT, int XCH>
struct GemmRegs {
    uint4 x[XCH];
    uint4 h, q, q5h;   // Q4_K / Q5_K: header, 16 quant bytes; Q5_K: the matching 16 qh bytes
    uint32_t ql[9], qh[9], sc[2], d[2];
    uint32_t mql, mqh, msc, md;
    uint32_t qb[10], mqb;   // Q8_0 / Q4_0: the thread's 32-weight block as raw dwords
};

// 32-weight-block formats: block bytes (2-byte d, then the quants)
template <uint32_t DT>
constexpr uint32_t block32_bytes() { return DT == YULE_DTYPE_Q8_0 ? 34u : 18u; }

// two f16 in a dword from two 8-bit fields (bits 0-7, 16-23; upper bits
// clear): 1024 + u is exact, so subtracting (1024 + bias) leaves u - bias
__device__ __forceinline__ uint32_t u8pair_to_f16(uint32_t v, _Float16 bias) {
    const h2v h = __builtin_bit_cast(h2v, v | 0x64006400u) - h2v{(_Float16)1024.0f + bias, (_Float16)1024.0f + bias};
    return __builtin_bit_cast(uint32_t, h);
}

// Weight matrices of one launch, stacked along Y's rows (one matrix: s1 = s2 = N)
struct GemmW {
    const uint8_t *w[3];
    uint32_t s1, s2;
};

// Split-K: split z of `splits` takes super-blocks [kb_lo, kb_hi) and,
// when splits > 1, writes its partial tile to y + z*M*N (summed in a
// fixed order by gemm_reduce_kernel, so results do not depend on timing).
// Two waves per SIMD, except the Q6_K kernels with f32 X (two sweeps) or a
// 128 x 128 tile, whose dequant state does not fit that register budget
// (the 64-row two-sweep one would, but measured slower in the runner's
// batched prefill: 3.53 against 3.39 ms): one wave per SIMD there.
constexpr int gemm_waves_per_simd(uint32_t dt, int bm, int bn, int sweeps) {
    return dt == YULE_DTYPE_Q6_K && (sweeps == 2 || (bm == 128 && bn == 128)) ? 1 : 2;
}

template <uint32_t DT, int BM, int BN, int SWEEPS>
__global__ __launch_bounds__(2 * BN) __attribute__((amdgpu_waves_per_eu(gemm_waves_per_simd(DT, BM, BN, SWEEPS)))) void gemm_kernel(
    // the first 14 dwords (what the first loads need) arrive preloaded in
    // SGPRs: no kernel-argument load delays them
    const _Float16 *__restrict__ xh, const uint8_t *w0, const uint8_t *w1, const uint8_t *w2, uint32_t s1,
    uint32_t s2, uint32_t M, uint32_t N, uint32_t K, uint32_t tail_ks, const _Float16 *__restrict__ xl,
    float *__restrict__ y, const _Float16 *__restrict__ xs_hi, const _Float16 *__restrict__ xs_lo,
    const float *__restrict__ rowscale, uint32_t accumulate) {
    constexpr bool Q5 = DT == YULE_DTYPE_Q5_K;
    constexpr bool Q4 = DT == YULE_DTYPE_Q4_K || Q5;   // Q5_K: Q4_K plus a fifth bit per weight from qh
    constexpr bool B32 = DT == YULE_DTYPE_Q8_0 || DT == YULE_DTYPE_Q4_0;   // 32-weight blocks, d per block
    constexpr bool Q8K = DT == YULE_DTYPE_Q8_K;   // 256 int8 weights, f32 d per super-block
    constexpr bool SBP = Q4 || Q8K;                // super-block passes of four stages
    constexpr uint32_t BB = Q5 ? 176 : Q4 ? 144 : Q8K ? 292 : DT == YULE_DTYPE_Q6_K ? 210 : block32_bytes<DT>();
    constexpr int TM = BM / 32;                 // 16-row MFMA tiles per wave along m
    constexpr uint32_t NTH = 2 * BN;            // threads: two per weight row of the tile
    constexpr uint32_t WNN = BN / 64;           // waves along n (two along m)
    constexpr int XCH = BM * GSK / 8 / NTH;     // 16-byte X chunks per thread per stage
    // LDS tiles: rows of GSK = 64 halves (128 bytes, eight 16-byte chunks),
    // XOR-swizzled (swz) instead of padded: each group of eight lanes of a
    // load or store covers the eight chunk positions of a 128-byte bank line
    // once, and the 64 x 128 tile keeps three workgroups per CU.
    constexpr int GLD = GSK;
    // the two X buffers as two objects: a copy into one (XDMA below) then
    // does not make the compiler wait before reads of the other
    __shared__ __align__(16) _Float16 sxa[BM * GLD];
    __shared__ __align__(16) _Float16 sxb[BM * GLD];
    auto xbuf = [&](int b) -> _Float16 * { return b ? sxb : sxa; };
    __shared__ __align__(16) _Float16 sw[2][BN * GLD];
    __shared__ float sd[2][B32 ? 2 : 1][BN];   // d per weight row: super-block slot, or the stage's two blocks
    // Q6_K with f32 X: the weight tile holds q - 32 and each row's four
    // sub-block scales of the stage sit here as f16 pairs (16 * (sc >> 4),
    // sc & 15); the MFMA B operand is then both halves of sc * (q - 32), each
    // exact in f16 (|16 * (sc >> 4) * (q - 32)| <= 4096 in steps of 16,
    // |(sc & 15) * (q - 32)| <= 480), accumulated by two MFMAs.  The single
    // product sc * (q - 32) reaches 4096 and rounds above 2048; that rounding
    // (<= 4.9e-4 relative on those weights) is kept for bf16 X.
    constexpr bool X6 = DT == YULE_DTYPE_Q6_K && SWEEPS == 2;
    __shared__ uint32_t ssc[X6 ? 2 : 1][X6 ? BN : 1][4];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WNN, wn = wave % WNN;
    // XDMA (the 256 x 256 Q4_K tile with bf16 X, whose registers are full):
    // X goes from memory straight into LDS (global_load_lds) one stage
    // ahead instead of through XCH staging registers per stage in flight
    constexpr bool XDMA = DT == YULE_DTYPE_Q4_K && BM == 256 && BN == 256 && SWEEPS == 1;
    // Tile of this workgroup.  The grid is one-dimensional over
    // (split, m tile, n tile), n fastest, in id order: workgroups go to the
    // eight XCDs round-robin by id, so the ones resident together at any
    // time cover a few whole m tiles across all XCDs.  xcd_remap instead
    // gives each XCD a contiguous range of ids (its workgroups then share
    // one m tile's X rows in its L2); that measured 2-10% slower on every
    // format at M = 1024 and 2048 and is off unless YULE_GEMM_XCD_REMAP=1.
    const uint32_t nt = (N + BN - 1) / BN, mt = (M + BM - 1) / BM, tiles = nt * mt;
    // With tail > 0 the grid is instead the first tiles - tail tiles whole,
    // then the last `tail` tiles as two K halves each, dispatched last: the
    // last round of resident workgroups then runs half as long.  Both
    // halves add into y, which the host zeroed: 0 + a + b is exact in
    // either order.
    // tail_ks = tail | K splits << 16 (the grid size comes from arguments,
    // not from the dispatch packet, whose load would delay the first loads)
    // bit 31: XCD-contiguous tile order (see below)
    const uint32_t tail = tail_ks & 0xffffu, ks = (tail_ks >> 16) & 0x7fffu, xcd_remap = tail_ks >> 31;
    const uint32_t whole = tiles - tail;
    const bool halves = tail && blockIdx.x >= whole;
    const uint32_t splits = tail ? (halves ? 2u : 1u) : ks;
    const uint32_t span = tail ? whole : ks * tiles;
    uint32_t t = blockIdx.x, zs;
    if (halves) {
        zs = (t - whole) & 1u;
        t = whole + ((t - whole) >> 1);
    } else {
        if (xcd_remap) {
            const uint32_t q = span / 8u, rmd = span % 8u, xcd = t % 8u;
            t = xcd * q + (xcd < rmd ? xcd : rmd) + t / 8u;
        }
        zs = t / tiles;
    }
    const uint32_t tm = (t % tiles) / nt, tn = t % nt;
    const uint32_t m0 = tm * BM, r0 = tn * BN;
    const uint32_t bpr = K / 256;
    const uint32_t kb_lo = (uint32_t)((uint64_t)bpr * zs / splits);
    const uint32_t kb_hi = (uint32_t)((uint64_t)bpr * (zs + 1) / splits);
    const uint32_t S = 4 * (kb_hi - kb_lo);     // stages of this split (>= 4)
    const size_t row_bytes = B32 ? (size_t)(K / 32) * BB : (size_t)bpr * BB;
    // this split's partial product (offset applied at the stores, so that
    // the load of y is not waited for ahead of the first stage's loads)
    const size_t y_off = splits > 1 && !tail ? (size_t)zs * M * N : 0;

    // RS (Q4_K, Q5_K, and Q6_K with bf16 X): the accumulators
    // are kept in units of the current super-block's d of their column (u):
    // before each super-block the column's acc is rescaled by u / d_new, then
    // the block's products accumulate straight into acc, with no second
    // accumulator set (one f32 rounding per super-block, ~2^-24 of the
    // partial sum).  A super-block with d = 0 keeps the unit, and its B
    // operand is zero.  Q8_0 / Q4_0 (d per 32-weight block) accumulate each
    // block into tmp and add d * tmp; so do Q8_K, whose kernel measured
    // 10-15% slower rescaled (M = 64-2048), and Q6_K with f32 X (the
    // runner's batched prefill 2% slower rescaled).
    constexpr bool RS = !B32 && !Q8K && !(DT == YULE_DTYPE_Q6_K && SWEEPS == 2);
    floatx4 acc[TM][4], tmp[TM][4];
    float unit[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) { acc[i][j] = floatx4{0, 0, 0, 0}; tmp[i][j] = floatx4{0, 0, 0, 0}; }

    // weight role: two threads per weight row (adjacent lanes: each pair
    // loads one 32-byte run), 32 weights of the stage each
    const uint32_t wr = tid >> 1, part = tid & 1u;
    // Rows past M or N load from a valid row (X rows clamped to M - 1, weight
    // rows to row 0) and are used as they are: a row of the product depends
    // only on its own X row and a column only on its own weight row, and the
    // epilogue stores neither, so no masking is needed.
    // the tile's weight matrix: rows [0, s1) of Y come from w[0], [s1, s2)
    // from w[1], [s2, N) from w[2] (a tile never straddles two), addressed
    // here by the tile's row in Y
    const uint32_t seg = r0 >= s2 ? 2u : r0 >= s1 ? 1u : 0u;
    const uint8_t *w = (seg == 2 ? w2 : seg == 1 ? w1 : w0) - (size_t)(seg == 2 ? s2 : seg == 1 ? s1 : 0u) * row_bytes;
    const uint8_t *wrow = w + (size_t)(r0 + wr < N ? r0 + wr : r0) * row_bytes;

    // stc: std::integral_constant<int, ST>, the stage's index in its
    // super-block when the caller knows it at compile time (ST >= 0), else -1
    // X of the current sweep: xh, then (f32 X) xl, both into the same
    // accumulators (the weight tile's second sweep reads it from L2)
    const _Float16 *xcur = xh;
    auto load_stage = [&](uint32_t s, GemmRegs<DT, XCH> &R, auto stc) {
        constexpr int STC = decltype(stc)::value;
        const uint32_t kb = kb_lo + (s >> 2), st = STC >= 0 ? (uint32_t)STC : (s & 3u), k0 = kb * 256u + st * GSK;
        if constexpr (!XDMA) {
#pragma unroll
            for (int i = 0; i < XCH; i++) {
                const uint32_t idx = tid + NTH * i, row = idx >> 3, c = idx & 7u;
                const uint32_t m = m0 + row < M ? m0 + row : M - 1u;
                R.x[i] = *reinterpret_cast<const uint4 *>(xcur + (size_t)m * K + k0 + 8u * c);
            }
        }
        if constexpr (B32) {
            // block 2 (kb*4 + st) + part of the row: k = 64 stage + 32 part
            const uint8_t *blk = wrow + (size_t)(8u * kb + 2u * st + part) * BB;
            R.mqb = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);   // 0 or 2: blocks are 2-byte aligned
            const uint32_t *w4 = reinterpret_cast<const uint32_t *>(blk - R.mqb);
#pragma unroll
            for (int i = 0; i < (DT == YULE_DTYPE_Q8_0 ? 10 : 6); i++) R.qb[i] = w4[i];
            return;
        }
        const uint8_t *blk = wrow + (size_t)kb * BB;
        if constexpr (Q8K) {
            // Q8_K (dequant.rs:376-384): f32 d at 0, int8 quants at 4 (dword aligned)
            const uint32_t *w4 = reinterpret_cast<const uint32_t *>(blk);
            R.d[0] = w4[0];
#pragma unroll
            for (int i = 0; i < 8; i++) R.qb[i] = w4[1u + 16u * st + 8u * part + i];
            return;
        }
        if constexpr (Q5) {
            // Q5_K (dequant.rs:297-338): qh at 16, quants at 48
            R.h = *reinterpret_cast<const uint4 *>(blk);
            R.q = *reinterpret_cast<const uint4 *>(blk + 48u + 32u * st + 16u * part);
            R.q5h = *reinterpret_cast<const uint4 *>(blk + 16u + 16u * part);
        } else if constexpr (Q4) {
            R.h = *reinterpret_cast<const uint4 *>(blk);
            R.q = *reinterpret_cast<const uint4 *>(blk + 16u + 32u * st + 16u * part);
        } else {
            const uint32_t h = st >> 1, g = 2u * (st & 1u) + part;
            load_raw<32>(blk + 64u * h + 32u * part, R.ql, R.mql);
            load_raw<32>(blk + 128u + 32u * h, R.qh, R.mqh);
            load_raw<4>(blk + 192u + 8u * h + 2u * g, R.sc, R.msc);
            load_raw<4>(blk + 208u, R.d, R.md);
        }
    };

    auto dequant_stage = [&](uint32_t s, const GemmRegs<DT, XCH> &R, int b, auto stc) {
        constexpr int STC = decltype(stc)::value;
        // kb relative to the split (LDS slot parity only)
        const uint32_t kb = s >> 2, st = STC >= 0 ? (uint32_t)STC : (s & 3u);
        if constexpr (!XDMA) {
#pragma unroll
            for (int i = 0; i < XCH; i++) {
                const uint32_t idx = tid + NTH * i, row = idx >> 3, c = idx & 7u;
                // copied element by element: storing R.x[i] whole kept the
                // register staging in scratch memory (80-450 bytes per lane)
                const uint4 v = R.x[i];
                *reinterpret_cast<uint4 *>(xbuf(b) + swz<Q4>(row, c)) = make_uint4(v.x, v.y, v.z, v.w);
            }
        }
        _Float16 *wt = sw[b];
        uint4 o[4];
        if constexpr (Q8K) {
            uint32_t outw[16];
#pragma unroll
            for (int t = 0; t < 8; t++) {   // signed bytes -> (q0, q2), (q1, q3): the X order {0,2,1,3}
                const uint32_t q = R.qb[t];
                outw[2 * t] = u8pair_to_f16((q & 0x00FF00FFu) ^ 0x00800080u, (_Float16)128.0f);
                outw[2 * t + 1] = u8pair_to_f16(((q >> 8) & 0x00FF00FFu) ^ 0x00800080u, (_Float16)128.0f);
            }
#pragma unroll
            for (int c = 0; c < 4; c++)
                *reinterpret_cast<uint4 *>(wt + swz<Q4>(wr, 4u * part + c)) =
                    make_uint4(outw[4 * c], outw[4 * c + 1], outw[4 * c + 2], outw[4 * c + 3]);
            if (st == 0 && part == 0) sd[kb & 1u][0][wr] = __builtin_bit_cast(float, R.d[0]);
        } else if constexpr (B32) {
            // d, then the quants from byte 2 of the block (mqb = 0: the block
            // starts at raw dword 0; mqb = 2: at its upper half)
            const bool up = R.mqb != 0;
            const uint32_t dbits = up ? R.qb[0] >> 16 : R.qb[0] & 0xFFFFu;
            uint32_t outw[16];
            if constexpr (DT == YULE_DTYPE_Q8_0) {
                // signed bytes q[4t..4t+3] -> (q0, q2), (q1, q3): the X order {0,2,1,3}
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const uint32_t q = up ? R.qb[t + 1] : __builtin_amdgcn_alignbyte(R.qb[t + 1], R.qb[t], 2);
                    outw[2 * t] = u8pair_to_f16((q & 0x00FF00FFu) ^ 0x00800080u, (_Float16)128.0f);
                    outw[2 * t + 1] = u8pair_to_f16(((q >> 8) & 0x00FF00FFu) ^ 0x00800080u, (_Float16)128.0f);
                }
            } else {
                // Q4_0 (dequant.rs:77-86): weight 2j is the low nibble of quant
                // byte j, 2j+1 its high nibble; bytes b0..b3 hold weights
                // 8t..8t+7 -> (lo b0, lo b1), (hi b0, hi b1), (lo b2, lo b3), (hi b2, hi b3)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint32_t q = up ? R.qb[t + 1] : __builtin_amdgcn_alignbyte(R.qb[t + 1], R.qb[t], 2);
                    const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
                    outw[4 * t] = u8pair_to_f16(__builtin_amdgcn_perm(0u, lo, 0x0C010C00u), (_Float16)8.0f);
                    outw[4 * t + 1] = u8pair_to_f16(__builtin_amdgcn_perm(0u, hi, 0x0C010C00u), (_Float16)8.0f);
                    outw[4 * t + 2] = u8pair_to_f16(__builtin_amdgcn_perm(0u, lo, 0x0C030C02u), (_Float16)8.0f);
                    outw[4 * t + 3] = u8pair_to_f16(__builtin_amdgcn_perm(0u, hi, 0x0C030C02u), (_Float16)8.0f);
                }
            }
#pragma unroll
            for (int c = 0; c < 4; c++)
                *reinterpret_cast<uint4 *>(wt + swz<Q4>(wr, 4u * part + c)) =
                    make_uint4(outw[4 * c], outw[4 * c + 1], outw[4 * c + 2], outw[4 * c + 3]);
            sd[b][part][wr] = f16_bits(dbits);
        } else if constexpr (Q4) {
            // 6-bit scales of sub-blocks 2st (low nibbles) and 2st+1 (high),
            // get_scale_min_k4 (dequant.rs:176-190)
            const uint4 hd = R.h;
            const uint32_t sh = (st & 1u) << 4;
            const bool low = st < 2;
            const uint32_t A = low ? hd.y : hd.w;
            const uint32_t mA = low ? 0x3F3Fu : 0x0F0Fu, mB = low ? 0u : 0x3030u;
            const uint32_t scs = ((A >> sh) & mA) | ((hd.y >> (sh + 2)) & mB);
            // high nibbles stay in place (16 q * 2^-24, still a denormal
            // pair) against sc * 2^6, so the product is again sc * q * 2^-14
            // (RS: a super-block with d = 0 contributes through its min term
            // only, so its B operand is zero)
            const uint32_t dz = RS && (hd.x & 0x7FFFu) == 0u ? 0u : 1u;
            const _Float16 f0 = (_Float16)(float)((scs & 0xFFu) * 1024u * dz);
            const _Float16 f1 = (_Float16)(float)((scs >> 8) * 64u * dz);
            const h2v S0 = {f0, f0}, S1 = {f1, f1};
            const uint32_t q[4] = {R.q.x, R.q.y, R.q.z, R.q.w};
            const uint32_t qb[4] = {R.q5h.x, R.q5h.y, R.q5h.z, R.q5h.w};
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t v = q[i], v8 = v >> 8;
                uint32_t l0 = v & 0x000F000Fu, l1 = v8 & 0x000F000Fu, h0 = v & 0x00F000F0u, h1 = v8 & 0x00F000F0u;
                if constexpr (Q5) {
                    // fifth bits: qh bit 2st for the low-nibble weights (into bit
                    // 4 of each half), bit 2st+1 for the high ones (held as 16 q:
                    // into bit 8); the pairs stay f16 denormals
                    const uint32_t b = qb[i], b8 = b >> 8;
                    l0 |= ((b >> (2u * st)) & 0x00010001u) << 4;
                    l1 |= ((b8 >> (2u * st)) & 0x00010001u) << 4;
                    h0 |= ((b >> (2u * st + 1u)) & 0x00010001u) << 8;
                    h1 |= ((b8 >> (2u * st + 1u)) & 0x00010001u) << 8;
                }
                lo[2 * i] = pk_scale(l0, S0);
                lo[2 * i + 1] = pk_scale(l1, S0);
                hi[2 * i] = pk_scale(h0, S1);
                hi[2 * i + 1] = pk_scale(h1, S1);
            }
            o[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            o[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
            o[2] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            o[3] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
            // this thread's 16 bytes: k = 16 part + 0..15 (low), 32 + 16 part + 0..15 (high)
            *reinterpret_cast<uint4 *>(wt + swz<Q4>(wr, 2u * part)) = o[0];
            *reinterpret_cast<uint4 *>(wt + swz<Q4>(wr, 2u * part + 1u)) = o[1];
            *reinterpret_cast<uint4 *>(wt + swz<Q4>(wr, 4u + 2u * part)) = o[2];
            *reinterpret_cast<uint4 *>(wt + swz<Q4>(wr, 5u + 2u * part)) = o[3];
            if (st == 0 && part == 0) sd[kb & 1u][0][wr] = f16_bits(hd.x) * 16384.0f;
        } else {
            // Q6_K (dequant.rs:340-372): k = 32 part + l, quarter g = 2(st&1)+part of half st/2
            uint32_t ql[8], qh[8], scw[1], dw[1];
            align_raw<32>(R.ql, R.mql, ql);
            align_raw<32>(R.qh, R.mqh, qh);
            align_raw<4>(R.sc, R.msc, scw);
            align_raw<4>(R.d, R.md, dw);
            const uint32_t g = 2u * (st & 1u) + part, nib = 4u * (st & 1u), qsh = 2u * g;
            const int dnz = !RS || (dw[0] & 0x7FFFu) ? 1 : 0;   // RS: d = 0 zeroes B
            const int isc0 = dnz * (int8_t)(scw[0] & 0xFFu), isc1 = dnz * (int8_t)((scw[0] >> 8) & 0xFFu);
            const _Float16 sc0 = (_Float16)(float)isc0, sc1 = (_Float16)(float)isc1;
            const h2v S0 = {sc0, sc0}, S1 = {sc1, sc1};
            if constexpr (X6) {   // the stage's sub-blocks 2 part and 2 part + 1 of this row
                auto pack = [](int sc) {
                    const h2v v = {(_Float16)(float)(sc - (sc & 15)), (_Float16)(float)(sc & 15)};
                    return __builtin_bit_cast(uint32_t, v);
                };
                ssc[b][wr][2u * part] = pack(isc0);
                ssc[b][wr][2u * part + 1u] = pack(isc1);
            }
            uint32_t outw[16];
            // four weights per dword: the 6-bit values q (byte lanes), paired
            // (q0, q2), (q1, q3) in the X order {0,2,1,3}, as f16 q - 32
            // (exact), times the sub-block scale in f16: the packed multiply
            // rounds the integer product to nearest even, as converting it does
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t q6 = ((ql[i] >> nib) & 0x0F0F0F0Fu) | (((qh[i] >> qsh) & 0x03030303u) << 4);
                const h2v sc = i < 4 ? S0 : S1;   // weights 0-15 / 16-31 of the quarter
                const uint32_t e = u8pair_to_f16(q6 & 0x00FF00FFu, (_Float16)32.0f);
                const uint32_t o = u8pair_to_f16((q6 >> 8) & 0x00FF00FFu, (_Float16)32.0f);
                outw[2 * i] = X6 ? e : pk_scale(e, sc);
                outw[2 * i + 1] = X6 ? o : pk_scale(o, sc);
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                *reinterpret_cast<uint4 *>(wt + swz<Q4>(wr, 4u * part + c)) =
                    make_uint4(outw[4 * c], outw[4 * c + 1], outw[4 * c + 2], outw[4 * c + 3]);
            }
            if (st == 0 && part == 0) sd[kb & 1u][0][wr] = f16_bits(dw[0]);
        }
    };

    // a new super-block: acc into units of its d (slot: its scale slot)
    auto rescale = [&](uint32_t slot) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float dn = sd[slot][0][wn * 64 + j * 16 + (lane & 15u)];
            const bool nz = dn != 0.f;
            const float f = nz ? unit[j] / dn : 1.f;
            unit[j] = nz ? dn : unit[j];
#pragma unroll
            for (int i = 0; i < TM; i++) acc[i][j] *= f;
        }
    };
    // first: this stage opens a super-block (RS: rescale first)
    auto compute = [&](int b, auto first_t, uint32_t slot = 0) {
        constexpr bool first = decltype(first_t)::value;
        if constexpr (RS && first) rescale(slot);
#pragma unroll
        for (int ks = 0; ks < GSK / 32; ks++) {
            half8 a[TM], bw[4];
#pragma unroll
            for (int i = 0; i < TM; i++)
                a[i] = *reinterpret_cast<const half8 *>(
                    xbuf(b) + swz<Q4>(wm * (BM / 2) + i * 16 + (lane & 15u), ks * 4 + (lane >> 4)));
#pragma unroll
            for (int j = 0; j < 4; j++)
                bw[j] = *reinterpret_cast<const half8 *>(sw[b] + swz<Q4>(wn * 64 + j * 16 + (lane & 15u), ks * 4 + (lane >> 4)));
            if constexpr (B32) {
                // one k-step is one block: acc += d[r][block] * (its MFMA from zero)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], bw[j], floatx4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float dr = sd[b][ks][wn * 64 + j * 16 + (lane & 15u)];
#pragma unroll
                    for (int i = 0; i < TM; i++) acc[i][j] += dr * tmp[i][j];
                }
            } else if constexpr (X6) {
                // this lane's 8 k lie in sub-block 2 ks + lane / 32 of the stage
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t sp = ssc[b][wn * 64 + j * 16 + (lane & 15u)][2 * ks + (lane >> 5)];
                    const h2v sh = {__builtin_bit_cast(h2v, sp).x, __builtin_bit_cast(h2v, sp).x};
                    const h2v sl = {__builtin_bit_cast(h2v, sp).y, __builtin_bit_cast(h2v, sp).y};
                    half8 b1, b2;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const h2v q = {bw[j][2 * e], bw[j][2 * e + 1]};
                        const h2v p1 = q * sh, p2 = q * sl;
                        b1[2 * e] = p1.x; b1[2 * e + 1] = p1.y;
                        b2[2 * e] = p2.x; b2[2 * e + 1] = p2.y;
                    }
#pragma unroll
                    for (int i = 0; i < TM; i++) {   // (X6 is never RS)
                        tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b1, tmp[i][j], 0, 0, 0);
                        tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b2, tmp[i][j], 0, 0, 0);
                    }
                }
            } else if constexpr (RS) {
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], bw[j], acc[i][j], 0, 0, 0);
            } else {   // not RS (Q8_K, Q6_K with f32 X): the super-block into tmp (SBP: its first k-step from zero)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            a[i], bw[j], first && ks == 0 ? floatx4{0, 0, 0, 0} : tmp[i][j], 0, 0, 0);
            }
        }
    };
    auto block_done = [&](uint32_t kb) {   // not RS: acc += d[r] * super-block partial
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float dr = sd[kb & 1u][0][wn * 64 + j * 16 + (lane & 15u)];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                acc[i][j] += dr * tmp[i][j];
                if constexpr (!SBP) tmp[i][j] = floatx4{0, 0, 0, 0};
            }
        }
    };

    // XDMA: stage s's X tile into buffer b.  Slot idx = tid + NTH i of the
    // buffer (the 1 KB of wave w's copy i are slots 64 w + 512 i onwards) is
    // row idx / 8, chunk position idx % 8, which swz<true> fills from X chunk
    // (idx % 8) ^ f(row).
    // The copy is issued as inline assembly, outside the compiler's memory
    // model: with the builtin, the compiler could not tell a copy into one
    // buffer from reads of the other (both live in the kernel's one LDS
    // block) and waited for every load in flight, the copy just issued
    // included, before every other stage's MFMAs.  Unseen by the compiler,
    // the copies only make its own load waits count fewer operations than
    // are in flight, i.e. stricter; none falls after a stage's copy, since
    // the stage's weight registers were already covered by the previous
    // stage's explicit wait, which the compiler does account for.
    // Scheduling barriers keep the copies first in their stage, ahead of the
    // weight loads whose count the waits rely on.
    typedef __attribute__((address_space(3))) _Float16 *lds_h;
    auto dma_x = [&](uint32_t s, int b) {
        const uint32_t k0 = (kb_lo + (s >> 2)) * 256u + (s & 3u) * GSK;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const uint32_t idx = tid + NTH * i, row = idx >> 3, r7 = row & 7u;
            const uint32_t c = (idx & 7u) ^ ((r7 & 1u) | ((r7 >> 1) & 2u) | ((r7 << 1) & 4u));
            const uint32_t m = m0 + row < M ? m0 + row : M - 1u;
            const _Float16 *src = xcur + (size_t)m * K + k0 + 8u * c;
            const uint32_t dst = __builtin_amdgcn_readfirstlane(
                (uint32_t)reinterpret_cast<uintptr_t>((lds_h)(xbuf(b) + (64u * wave + NTH * i) * 8u)));
            asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(dst) : "m0");
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // end of an XDMA stage: this thread's copy of the next stage's X landed
    // (the stage's two weight loads, issued after it, may stay in flight:
    // loads complete in issue order, so at most those two are outstanding
    // once it has; a split weight load only makes the wait stricter), its
    // LDS stores done, then the barrier.  No __syncthreads: its release
    // fence waits for every load, the weight loads two stages ahead included.
    auto stage_sync = [&]() {
        if constexpr (XDMA) {
            __builtin_amdgcn_s_waitcnt((int)(2u | (7u << 4)));   // vmcnt(2) lgkmcnt(0)
            asm volatile("s_barrier" ::: "memory");
        } else {
            __syncthreads();
        }
    };
    const std::integral_constant<int, -1> rt{};   // stage index known only at run time
    const std::integral_constant<bool, true> opens{};
    const std::integral_constant<bool, false> cont{};
    // one sweep over this split's K range (called once, or for f32 X twice:
    // xh, then xl, into the same accumulators)
    auto sweep = [&]() {
    GemmRegs<DT, XCH> R0, R1;
    load_stage(0, R0, std::integral_constant<int, 0>{});
    if constexpr (XDMA) dma_x(0, 0);
    load_stage(1, R1, std::integral_constant<int, 1>{});
    // argument loads the epilogue needs (y, ...) and their waits stay behind
    // the first two stages' loads
    __builtin_amdgcn_sched_barrier(0);
    dequant_stage(0, R0, 0, std::integral_constant<int, 0>{});
    load_stage(2, R0, std::integral_constant<int, 2>{});   // S >= 4
    if constexpr (XDMA) {
        // X of stage 0 landed (stage 1's and 2's weight loads, four or more
        // operations, were issued after it)
        __builtin_amdgcn_s_waitcnt((int)(4u | (7u << 4)));   // vmcnt(4) lgkmcnt(0)
        asm volatile("s_barrier" ::: "memory");
    } else {
        __syncthreads();
    }
    // Q4_K, Q5_K, Q8_K: one super-block (four stages) per pass; stage t computes out of
    // LDS buffer t & 1 while stage t + 1 is dequantized into the other and
    // the bytes of stage t + 3 load into the register set stage t + 1 freed.
    // The pass's first stage rescales the accumulators to the super-block's
    // d (compute(first)).  Q6_K, whose dequant state is larger, keeps a
    // two-stage pass (the longer one spills) and rescales every other pass.
    // The last pass's final dequant and load are unconditional (stage S does
    // not exist: its dequant writes LDS buffer 0 and scale slot (S/4) & 1,
    // which nothing reads any more, and the load re-reads stage S - 1): a
    // branch there would make the compiler wait for every load in flight at
    // the loop head instead of only for the stage about to be dequantized.
    if constexpr (SBP) {
        for (uint32_t s = 0; s < S; s += 4) {
            // (XDMA: each stage first copies the next stage's X into the
            // buffer the previous stage read; past the end, stage S - 1
            // again, into a buffer nothing reads any more)
            if constexpr (XDMA) dma_x(s + 1, 1);
            compute(0, opens, (s >> 2) & 1u);
            dequant_stage(s + 1, R1, 1, std::integral_constant<int, 1>{});
            load_stage(s + 3 < S ? s + 3 : S - 1, R1, std::integral_constant<int, 3>{});
            stage_sync();
            if constexpr (XDMA) dma_x(s + 2, 0);
            compute(1, cont);
            dequant_stage(s + 2, R0, 0, std::integral_constant<int, 2>{});
            load_stage(s + 4 < S ? s + 4 : S - 1, R0, std::integral_constant<int, 0>{});
            stage_sync();
            if constexpr (XDMA) dma_x(s + 3, 1);
            compute(0, cont);
            dequant_stage(s + 3, R1, 1, std::integral_constant<int, 3>{});
            load_stage(s + 5 < S ? s + 5 : S - 1, R1, std::integral_constant<int, 1>{});
            stage_sync();
            if constexpr (XDMA) dma_x(s + 4 < S ? s + 4 : S - 1, 0);
            compute(1, cont);
            if constexpr (!RS) block_done(s >> 2);
            dequant_stage(s + 4, R0, 0, std::integral_constant<int, 0>{});
            load_stage(s + 6 < S ? s + 6 : S - 1, R0, std::integral_constant<int, 2>{});
            stage_sync();
        }
    } else if constexpr (B32) {
        for (uint32_t s = 0; s < S; s += 2) {
            compute(0, cont);
            dequant_stage(s + 1, R1, 1, rt);
            load_stage(s + 3 < S ? s + 3 : S - 1, R1, rt);
            __syncthreads();
            compute(1, cont);
            dequant_stage(s + 2, R0, 0, rt);
            load_stage(s + 4 < S ? s + 4 : S - 1, R0, rt);
            __syncthreads();
        }
    } else {
        for (uint32_t s = 0; s < S; s += 2) {
            if constexpr (RS)
                if ((s & 3u) == 0u) rescale((s >> 2) & 1u);   // stage s opens a super-block
            compute(0, cont);
            dequant_stage(s + 1, R1, 1, rt);
            load_stage(s + 3 < S ? s + 3 : S - 1, R1, rt);
            __syncthreads();
            compute(1, cont);
            if constexpr (!RS)
                if (((s + 1) & 3u) == 3u) block_done((s + 1) >> 2);
            dequant_stage(s + 2, R0, 0, rt);
            load_stage(s + 4 < S ? s + 4 : S - 1, R0, rt);
            __syncthreads();
        }
    }
    };
    sweep();
    if constexpr (SWEEPS == 2) {
        xcur = xl;
        sweep();
    }
    if constexpr (RS) {   // back to absolute units
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] *= unit[j];
    }

    // the row scales of this lane's output rows, loaded now so that the
    // stores below wait on nothing (a load issued after stores would wait
    // for them too: loads and stores share one counter)
    // (the 256-row tile loads them at the stores instead: registers)
    constexpr bool RS_EARLY = BM < 256;
    float rs[TM][4];
    if constexpr (RS_EARLY) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t m = m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + e;
                rs[i][e] = rowscale[m < M ? m : M - 1u];
            }
    }
    if (Q4 && xs_hi) {   // (no sums: the second, lo, product of an f32 X)
        // min term: acc -= sum_j xsum[m][j] * (dmin*mn)[r][j] over the K/32
        // sub-blocks.  In chunks of four super-blocks the workgroup stages
        // the operands once into the LDS the main loop no longer needs: each
        // weight row's headers decoded to -(dmin * mn) split into f16 hi + lo
        // (exact in f32), and each X row's sub-block sums (hi, lo).  A k-step
        // of 32 then covers the chunk: lane quarter q takes super-block q's
        // eight sub-blocks, and hi*hi + hi*lo + lo*hi reproduce the product.
        // Loads come from clamped indices, with out-of-range operands zeroed.
        // (Per-wave loads and decodes, where both m-waves fetched every header
        // and all n-waves every X sum, were 1-4% slower; issuing several
        // chunks' loads at once was 7% slower.)
        const uint32_t nsub = K / 32;
        _Float16 *mb = &sw[0][0];                 // [BN rows][4 super-blocks][hi 8, lo 8]
        _Float16 *ma = mb + BN * 64;              // [BM rows][4 super-blocks][hi 8, lo 8]
        static_assert(BN * 64 + BM * 64 <= 2 * BN * GLD, "min-term staging fits the weight tile buffers");
        for (uint32_t kk = kb_lo; kk < kb_hi; kk += 4) {
#pragma unroll
            for (uint32_t it = 0; it < (uint32_t)(BN * 4) / NTH; it++) {
                const uint32_t idx = tid + NTH * it, row = idx >> 2, sbq = idx & 3u, sb = kk + sbq;
                const bool ok = r0 + row < N && sb < kb_hi;
                const uint32_t rc = r0 + row < N ? r0 + row : r0, sbc = sb < kb_hi ? sb : kb_hi - 1u;
                const uint4 h4 = *reinterpret_cast<const uint4 *>(w + (size_t)rc * row_bytes + (size_t)sbc * BB);
                const float dmin = f16_bits(h4.x >> 16);
                const uint32_t hd[3] = {h4.y, h4.z, h4.w};
                const uint8_t *q = reinterpret_cast<const uint8_t *>(hd);
                half8 h, l;
#pragma unroll
                for (int s = 0; s < 8; s++) {
                    const uint32_t mn = s < 4 ? (q[s + 4] & 63u)
                                              : ((uint32_t)(q[s + 4] >> 4) | ((uint32_t)(q[s] >> 6) << 4));
                    const float v = ok ? -(dmin * (float)mn) : 0.f;
                    const _Float16 vh = (_Float16)v;
                    h[s] = vh;
                    l[s] = (_Float16)(v - (float)vh);
                }
                *reinterpret_cast<half8 *>(mb + idx * 16) = h;
                *reinterpret_cast<half8 *>(mb + idx * 16 + 8) = l;
            }
#pragma unroll
            for (uint32_t it = 0; it < (uint32_t)(BM * 4 + NTH - 1) / NTH; it++) {
                const uint32_t idx = tid + NTH * it, row = idx >> 2, sbq = idx & 3u, sb = kk + sbq;
                if (idx < (uint32_t)BM * 4) {
                    const bool ok = m0 + row < M && sb < kb_hi;
                    const uint32_t mc = m0 + row < M ? m0 + row : M - 1u, sbc = sb < kb_hi ? sb : kb_hi - 1u;
                    const half8 xh8 = *reinterpret_cast<const half8 *>(xs_hi + (size_t)mc * nsub + 8 * sbc);
                    const half8 xl8 = *reinterpret_cast<const half8 *>(xs_lo + (size_t)mc * nsub + 8 * sbc);
                    const half8 zero = {};
                    *reinterpret_cast<half8 *>(ma + idx * 16) = ok ? xh8 : zero;
                    *reinterpret_cast<half8 *>(ma + idx * 16 + 8) = ok ? xl8 : zero;
                }
            }
            __syncthreads();
            const uint32_t q4 = lane >> 4;
            half8 bh[4], bl[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t nrow = wn * 64 + j * 16 + (lane & 15u);
                bh[j] = *reinterpret_cast<const half8 *>(mb + (nrow * 4 + q4) * 16);
                bl[j] = *reinterpret_cast<const half8 *>(mb + (nrow * 4 + q4) * 16 + 8);
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t mrow = wm * (BM / 2) + i * 16 + (lane & 15u);
                const half8 ah = *reinterpret_cast<const half8 *>(ma + (mrow * 4 + q4) * 16);
                const half8 al = *reinterpret_cast<const half8 *>(ma + (mrow * 4 + q4) * 16 + 8);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[j], acc[i][j], 0, 0, 0);
                }
            }
            __syncthreads();   // before the next chunk overwrites the staging
        }
    }

    // ---- store: lane holds rows 4*(lane/16)+e of column lane%16 of each tile
    float *const ysplit = y + y_off;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t r = r0 + wn * 64 + j * 16 + (lane & 15u);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t m = m0 + wm * (BM / 2) + i * 16 + 4 * (lane >> 4) + e;
                if (m < M && r < N) {
                    float *const y = ysplit;
                    const float sc = RS_EARLY ? rs[i][e] : rowscale[m];
                    const float v = acc[i][j][e] * sc;   // the row's power of two back out: exact
                    if (halves) unsafeAtomicAdd(y + (size_t)m * N + r, v);
                    else if (accumulate && splits == 1) y[(size_t)m * N + r] += v;
                    else y[(size_t)m * N + r] = v;
                }
            }
        }
}

// Q4_K with bf16 X for few rows of X (M <= 32): the weights stream once
// from memory straight into MFMA operands, no LDS round trip, so the launch
// runs at the weight stream's pace instead of the tile kernels' per-stage
// barrier/dequant/MFMA chain.  A workgroup takes 128 weight rows over a
// K range (blockIdx.y of gridDim.y equal ranges, partials summed by the
// split-K reduction) with four compute waves, 32 rows each as two MFMA A
// tiles: A = the weights (one row per lane group of 16, the quarter-block
// 32q..32q+31 bytes of qs per lane quad q), B = X rows 16t..16t+15 (MT
// tiles of 16), each B fragment read from LDS once for both A tiles (half
// the LDS bytes per weight row of one A tile per wave; the K splits, which
// the wider workgroups need to fill the CUs, also shorten each
// workgroup's serial super-block chain).  In a k-step j (h = j / 4,
// u = j % 4) quad q supplies the weights 64q + 32h + 8u + {0,2,1,3,4,6,5,7}
// (the nibble-pair order of two qs dwords, h the nibble half), and the f16 X
// pre-pass stores each four k in that order, so a lane's X operand is one
// 16-byte piece of a row.  Each super-block's product (sc*q*2^-14 exact
// integers times f16 X) accumulates in f32 and is added times d*2^14, as in
// gemm_kernel; the min term is the same hi/lo MFMA product over the X
// sub-block sums, four super-blocks (one per quad) per MFMA.
// A fifth wave only copies into LDS: X into a ring of XB buffers (XB - 1
// super-blocks ahead) and, per group of four super-blocks, the X sub-block
// sums into one of NSB buffers (global_load_lds).  A wave's loads complete
// in issue order, so copies issued by the compute waves would hold each
// weight load behind them and cap the weight stream at the X ring's depth;
// alone in their waves the weight loads run D super-blocks ahead (D a
// multiple of 4 that divides the range's super-block count), and the min
// term's weight header is the ring's (each quad keeps the header of its
// super-block of the group).  One barrier per super-block for all five waves.
template <int MT, int D, int XB>
__global__ __launch_bounds__(320) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemm_q4k_skinny_kernel(
    const _Float16 *__restrict__ xh, const uint8_t *w0, const uint8_t *w1, const uint8_t *w2, uint32_t s1,
    uint32_t s2, uint32_t M, uint32_t N, uint32_t K, float *__restrict__ y, const _Float16 *__restrict__ xs_hi,
    const _Float16 *__restrict__ xs_lo, const float *__restrict__ rowscale, uint32_t accumulate) {
    static_assert(D % 4 == 0, "weight ring a whole number of min-term groups");
    typedef __attribute__((address_space(3))) void *lds_p;
    typedef __attribute__((address_space(1))) void *glb_p;
    constexpr int RT = 2;                      // A tiles (16 weight rows each) per compute wave
    constexpr uint32_t BB = 144, XROWS = 16 * MT;
    constexpr uint32_t XP = XROWS * 32 / 64;   // X pieces (16 bytes) per producer lane per super-block
    constexpr uint32_t SP = XROWS * 8 / 64;    // sub-block-sum pieces per producer lane per group
    static_assert(XB >= 3, "X ring: at least 3 buffers");
    // sums buffers: a group's copy goes out with its first super-block's, up
    // to XB - 1 super-blocks before it is read, so while up to XB / 4 + 1
    // other groups' buffers are still to be read
    constexpr uint32_t NSB = XB <= 4 ? 2 : 4;
    __shared__ __align__(16) _Float16 xbuf[XB][XROWS * 256];
    __shared__ __align__(16) _Float16 sbuf[NSB][2 * XROWS * 32];   // [group % NSB][hi rows | lo rows][32 sums]
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsub = K / 32, bpr = K / 256;
    const uint32_t S = bpr / gridDim.y, kb0 = blockIdx.y * S;   // this workgroup's super-blocks [kb0, kb0 + S)

    if (wave == 4) {
        // producer.  X: slot idx = lane + 64 i of a buffer is row idx / 32,
        // 16-byte piece p = idx % 32, holding X piece p ^ (row & 7) of that
        // row.  Sums: slot idx is part idx / (4 XROWS) (hi, lo), row
        // (idx / 4) % XROWS, piece idx % 4 of the group's 32 sums.
        uint32_t xoff[XP];
#pragma unroll
        for (uint32_t i = 0; i < XP; i++) {
            const uint32_t idx = lane + 64u * i, row = idx >> 5, c = (idx & 31u) ^ (row & 7u);
            xoff[i] = (row < M ? row : M - 1u) * K + 8u * c;
        }
        auto dma = [&](uint32_t sb) {
            _Float16 *dst = xbuf[sb % XB];
#pragma unroll
            for (uint32_t i = 0; i < XP; i++)
                __builtin_amdgcn_global_load_lds((glb_p)(xh + (kb0 + sb) * 256u + xoff[i]), (lds_p)(dst + 64u * i * 8u),
                                                 16, 0, 0);
            if ((sb & 3u) == 0) {
                _Float16 *sd = sbuf[(sb >> 2) % NSB];
#pragma unroll
                for (uint32_t i = 0; i < SP; i++) {
                    const uint32_t idx = lane + 64u * i, part = idx / (4u * XROWS), row = (idx >> 2) % XROWS;
                    const _Float16 *src = (part ? xs_lo : xs_hi) + (size_t)(row < M ? row : M - 1u) * nsub +
                                          (kb0 + sb) * 8u + 8u * (idx & 3u);
                    __builtin_amdgcn_global_load_lds((glb_p)src, (lds_p)(sd + 64u * i * 8u), 16, 0, 0);
                }
            }
        };
        // before super-block sb's barrier: its copies landed; the XB - 2
        // later super-blocks' copies (at least (XB - 2) XP operations) may be
        // in flight
        constexpr uint32_t VM = (XB - 2) * XP < 63u ? (XB - 2) * XP : 63u;
        constexpr int WAIT = (int)((VM & 15u) | ((VM >> 4) << 14) | (7u << 4) | (15u << 8));
        for (uint32_t i = 0; i < XB - 1; i++) dma(i < S ? i : S - 1u);
        for (uint32_t sb = 0; sb < S; sb++) {
            __builtin_amdgcn_s_waitcnt(WAIT);
            asm volatile("s_barrier" ::: "memory");
            // the X buffer of sb + XB - 1 was last read at sb - 1 and the
            // sums buffer of its group (when it opens one) at sb - 2 or
            // earlier, by every compute wave before this barrier; past the
            // end, a copy of the last super-block (never a group's first) into
            // an unread buffer keeps the count fixed
            dma(sb + XB - 1 < S ? sb + XB - 1 : S - 1u);
        }
        __builtin_amdgcn_s_waitcnt((int)(0u | (7u << 4) | (15u << 8)));   // vmcnt(0): no copy left in flight
        return;
    }

    const uint32_t q = lane >> 4, rl = lane & 15u;
    const size_t row_bytes = (size_t)bpr * BB;
    const uint32_t rbase = blockIdx.x * (64u * RT) + wave * (16u * RT);
    const uint8_t *wrow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const uint32_t r = rbase + 16u * rt + rl, rr = r < N ? r : N - 1u;   // this lane's weight rows (clamped)
        const uint32_t seg = rr >= s2 ? 2u : rr >= s1 ? 1u : 0u;
        wrow[rt] = (seg == 2 ? w2 : seg == 1 ? w1 : w0) + (size_t)(rr - (seg == 2 ? s2 : seg == 1 ? s1 : 0u)) * row_bytes +
                   (size_t)kb0 * BB;
    }

    struct WR { uint4 h, qa, qb; };
    WR ring[D][RT];
    auto load_w = [&](uint32_t sb, WR *R) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const uint8_t *blk = wrow[rt] + (size_t)sb * BB;
            R[rt].h = *reinterpret_cast<const uint4 *>(blk);
            R[rt].qa = *reinterpret_cast<const uint4 *>(blk + 16u + 32u * q);
            R[rt].qb = *reinterpret_cast<const uint4 *>(blk + 32u + 32u * q);
        }
    };

    floatx4 acc[RT][MT];
    uint4 hm[RT];   // headers of super-block 4g + q of the current group g
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        hm[rt] = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < MT; t++) acc[rt][t] = floatx4{0, 0, 0, 0};
    }

    auto compute = [&](const WR *R, const _Float16 *xs, uint32_t u) {
        // 6-bit scales of sub-blocks 2q and 2q+1 (get_scale_min_k4,
        // dequant.rs:176-190) as f16 multipliers of the masked nibbles
        const bool low = q < 2u;
        const uint32_t sh = (q & 1u) << 4;
        h2v S0[RT], S1[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const uint4 hd = R[rt].h;
            if (q == (u & 3u)) hm[rt] = hd;
            const uint32_t A = low ? hd.y : hd.w;
            const uint32_t scs = ((A >> sh) & (low ? 0x3F3Fu : 0x0F0Fu)) | ((hd.y >> (sh + 2u)) & (low ? 0u : 0x3030u));
            const _Float16 f0 = (_Float16)(float)((scs & 0xFFu) * 1024u), f1 = (_Float16)(float)((scs >> 8) * 64u);
            S0[rt] = h2v{f0, f0};
            S1[rt] = h2v{f1, f1};
        }
        floatx4 tmp[RT][MT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int t = 0; t < MT; t++) tmp[rt][t] = floatx4{0, 0, 0, 0};
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            const uint32_t h = j >> 2, uu = j & 3u;
            const uint32_t mask = h ? 0x00F000F0u : 0x000F000Fu;
            half8 a[RT];
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const h2v Sc = h ? S1[rt] : S0[rt];
                const uint4 &qv = uu < 2 ? R[rt].qa : R[rt].qb;
                const uint32_t v0 = (uu & 1u) ? qv.z : qv.x, v1 = (uu & 1u) ? qv.w : qv.y;
                const u32x4 av = {pk_scale(v0 & mask, Sc), pk_scale((v0 >> 8) & mask, Sc), pk_scale(v1 & mask, Sc),
                                  pk_scale((v1 >> 8) & mask, Sc)};
                a[rt] = __builtin_bit_cast(half8, av);
            }
            const uint32_t c = 8u * q + 4u * h + uu;
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const uint32_t m = 16u * t + rl;
                const half8 b = *reinterpret_cast<const half8 *>(xs + m * 256u + 8u * (c ^ (m & 7u)));
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
                    tmp[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rt], b, tmp[rt][t], 0, 0, 0);
            }
        }
        // d of the output rows 4q + e of each A tile (their lanes' headers, quad 0)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            float dd[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                dd[e] = f16_bits((uint32_t)__builtin_amdgcn_ds_bpermute((int)((4u * q + e) * 4u), (int)R[rt].h.x)) *
                        16384.0f;
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[rt][t][e] += dd[e] * tmp[rt][t][e];
        }
    };
    auto min_term = [&](const _Float16 *sums) {
        // -(dmin * mn) of this lane's super-block 4g + q, split hi + lo f16
        half8 ah[RT], al[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const float dmin = f16_bits(hm[rt].x >> 16);
            const uint32_t hdw[3] = {hm[rt].y, hm[rt].z, hm[rt].w};
            const uint8_t *qb = reinterpret_cast<const uint8_t *>(hdw);
#pragma unroll
            for (int sbi = 0; sbi < 8; sbi++) {
                const uint32_t mn = sbi < 4 ? (qb[sbi + 4] & 63u) : ((uint32_t)(qb[sbi + 4] >> 4) | ((uint32_t)(qb[sbi] >> 6) << 4));
                const float v = -(dmin * (float)mn);
                const _Float16 vh = (_Float16)v;
                ah[rt][sbi] = vh;
                al[rt][sbi] = (_Float16)(v - (float)vh);
            }
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const uint32_t m = 16u * t + rl;
            const half8 bh = *reinterpret_cast<const half8 *>(sums + m * 32u + 8u * q);
            const half8 bl = *reinterpret_cast<const half8 *>(sums + (XROWS + m) * 32u + 8u * q);
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[rt], bh, acc[rt][t], 0, 0, 0);
                acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[rt], bl, acc[rt][t], 0, 0, 0);
                acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[rt], bh, acc[rt][t], 0, 0, 0);
            }
        }
    };

#pragma unroll
    for (int u = 0; u < D; u++) load_w(u, ring[u]);
    for (uint32_t sb0 = 0; sb0 < S; sb0 += D) {
#pragma unroll
        for (uint32_t u = 0; u < (uint32_t)D; u++) {
            const uint32_t sb = sb0 + u;
            asm volatile("s_barrier" ::: "memory");   // X(sb) (and its group's sums) in their buffers
            compute(ring[u], xbuf[sb % XB], u);
            load_w(sb + D < S ? sb + D : S - 1u, ring[u]);
            if ((u & 3u) == 3u) min_term(sbuf[(sb >> 2) % NSB]);
        }
    }

    // split z's partial into its own Y block (the split-K reduction sums them)
    float *const ys = y + (gridDim.y > 1 ? (size_t)blockIdx.y * M * N : 0);
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const uint32_t m = 16u * t + rl;
        if (m >= M) continue;
        const float rs = rowscale[m];
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t r = rbase + 16u * rt + 4u * q + e;
                if (r < N) {
                    const float v = acc[rt][t][e] * rs;   // the row's power of two back out: exact
                    if (accumulate && gridDim.y == 1) ys[(size_t)m * N + r] += v;
                    else ys[(size_t)m * N + r] = v;
                }
            }
    }
}

// zeroes the y blocks of tiles [first, first + gridDim.x / (bm / 8)): one
// workgroup per 8 rows of a tile, 32 lanes per row storing consecutive
// floats (bm is 64 or 128, bn 128 or 256)
__global__ void gemm_zero_tiles_kernel(float *__restrict__ y, uint32_t M, uint32_t N, uint32_t first, uint32_t nt,
                                       uint32_t bm, uint32_t bn) {
    const uint32_t per_tile = bm / 8, t = first + blockIdx.x / per_tile;
    const uint32_t m = (t / nt) * bm + (blockIdx.x % per_tile) * 8 + threadIdx.x / 32;
    if (m >= M) return;
    for (uint32_t c = threadIdx.x % 32; c < bn; c += 32) {
        const uint32_t r = (t % nt) * bn + c;
        if (r < N) y[(size_t)m * N + r] = 0.f;
    }
}

// y[i] = sum over z of part[z][i], z ascending (accumulate: y[i] + that sum)
__global__ void gemm_reduce_kernel(const float *__restrict__ part, float *__restrict__ y, uint64_t n, uint32_t ks,
                                   uint32_t accumulate) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = part[i];
    for (uint32_t z = 1; z < ks; z++) s += part[(uint64_t)z * n + i];
    y[i] = accumulate ? y[i] + s : s;
}

}  // namespace yule

using namespace yule;

namespace {

// Split count: none once the tiles alone fill every CU; below that, as many
// splits as fit in one round of resident workgroups (gemm_wgs_per_cu), so
// that small-M launches keep all CUs busy without a partial second round.
// Tile width along the weight rows: 256 (eight waves) halves the X bytes
// each weight tile is multiplied against and measured 5-30% faster once M
// fills the CUs with wide tiles (M >= 1024; Q6_K, whose dequant is dearer,
// from M >= 512); 128 (four waves) below that.  YULE_GEMM_BN overrides.
uint32_t gemm_bn(uint32_t m, uint32_t dtype) {
    static const int env = env_int("YULE_GEMM_BN", 0);
    if (env == 128 || env == 256) return (uint32_t)env;
    return m >= 1024 || (dtype == YULE_DTYPE_Q6_K && m >= 512) ? 256u : 128u;
}

// Tile height: 64 rows for M <= 64, and for f32 X up to M = 128 (its two
// sweeps make the 128-row tile spill; the 64-row one keeps three
// workgroups per CU and twice the workgroups); 128 otherwise.
// YULE_GEMM_F32_BM64 sets that f32 bound.
// Q4_K with bf16 X from M = YULE_GEMM_BM256 (default 1024) on: 256-row
// tiles of 256-wide ones, each wave a 128 x 64 sub-tile (its accumulators
// fit beside the stage registers because they need no second set), which
// halves the LDS bytes each wave reads per MFMA against 64 x 64 sub-tiles:
// M = 2048 +12-14% (14336 x 4096 and 4096 x 14336).
uint32_t gemm_bm(uint32_t m, bool f32x, uint32_t dtype, uint32_t bn) {
    static const int env = env_int("YULE_GEMM_F32_BM64", 128);
    static const int big = env_int("YULE_GEMM_BM256", 1024);
    if ((uint32_t)big <= m && !f32x && bn == 256 && dtype == YULE_DTYPE_Q4_K) return 256u;
    return m <= 64 || (f32x && m <= (uint32_t)env) ? 64u : 128u;
}

// Workgroups resident per CU: one for the 256-wide tiles and for Q6_K's
// 128-row and two-sweep kernels (one wave per SIMD), two otherwise.
uint32_t gemm_wgs_per_cu(uint32_t dtype, uint32_t bm, uint32_t bn, bool f32x) {
    return bn == 256 || (dtype == YULE_DTYPE_Q6_K && (bm == 128 || f32x)) ? 1u : 2u;
}

uint32_t gemm_splits(uint32_t m, uint32_t n, uint32_t k, uint32_t bn, uint32_t bm, uint32_t per_cu) {
    static const int env = env_int("YULE_GEMM_SPLITS", 0);
    if (env > 0) return (uint32_t)env < k / 256 ? (uint32_t)env : k / 256;
    const uint32_t tiles = ((n + bn - 1) / bn) * ((m + bm - 1) / bm);
    const uint32_t cus = (uint32_t)device_cus();
    if (tiles >= cus) return 1;
    uint32_t ks = per_cu * cus / tiles;
    const uint32_t bpr = k / 256;
    return ks < 1 ? 1 : ks > bpr ? bpr : ks;
}

// Q4_K with bf16 X and M <= 32 runs gemm_q4k_skinny_kernel (no tail; its
// own K splits) when each row's super-block count is a multiple of 4: 14-24%
// faster per call than the tile kernel at M = 1..16 on 14336x4096,
// 4096x14336 and 4096x4096, 9-13% at M = 32 (equal on 1024x4096).  At
// M = 64 it loses or ties (its waves, one per SIMD, serialize dequant, MFMA
// chain and four times the X bytes from LDS).  YULE_GEMM_SKINNY=0 turns it off.
bool gemm_skinny(uint32_t m, uint32_t k, uint32_t dtype, bool f32x) {
    static const bool env = env_flag("YULE_GEMM_SKINNY", true);
    return env && !f32x && dtype == YULE_DTYPE_Q4_K && m <= 32 && (k / 256) % 4 == 0;
}

// K splits of the few-rows kernel: as many as keep its 128-row workgroups
// (one per CU) within one round, each split a whole number of four-super-
// block groups.
uint32_t gemm_skinny_splits(uint32_t n, uint32_t k) {
    const uint32_t wgs = (n + 127) / 128, groups = k / 1024, cus = (uint32_t)device_cus();
    uint32_t best = 1;
    for (uint32_t d = 2; d <= groups; d++)
        if (groups % d == 0 && wgs * d <= cus) best = d;
    return best;
}

// Tail tiles split in two K halves (zero: none).  Without splits, the tiles
// past the last whole round of resident workgroups (one 256-wide or two
// 128-wide per CU) form a partial round nearly as long as a full one (a
// workgroup there ran 86-97% of its full-round time); when they fill at
// most half a round, running them as K halves fills it and ends the
// launch earlier (5% on 14336 x 4096 at M = 2048).  Needs two super-blocks
// per row.  YULE_GEMM_TAIL=0 turns it off.
uint32_t gemm_tail(uint32_t m, uint32_t n, uint32_t k, uint32_t bn, uint32_t bm, uint32_t ks) {
    static const bool env = env_flag("YULE_GEMM_TAIL", true);
    if (!env || ks > 1 || k / 256 < 2) return 0;
    const uint32_t tiles = ((n + bn - 1) / bn) * ((m + bm - 1) / bm);
    const uint32_t round = (uint32_t)device_cus() * (bn == 256 ? 1u : 2u);
    if (tiles <= round) return 0;
    const uint32_t r = tiles % round;
    return r <= round / 2 ? r : 0;
}

// One product over the tile grid: X in f16 (xh), or for f32 X its hi and lo
// halves (xh, xl) swept in turn into the same accumulators.  Y rows are
// scaled by rowscale.
struct GemmPass {
    GemmW w;
    const _Float16 *xh, *xl, *xs_hi, *xs_lo;
    const float *rowscale;
    float *y;
    uint32_t m, n, k, ks, bn, bm, tail, accumulate;
};

template <uint32_t DT, int BN>
void launch_gemm_bn(hipStream_t s, const GemmPass &p) {
    static const uint32_t remap = env_flag("YULE_GEMM_XCD_REMAP", false) ? 1u : 0u;
    const uint32_t nt = (p.n + BN - 1) / BN;
    const uint32_t bm = p.bm, tiles = nt * ((p.m + bm - 1) / bm);
    const uint32_t grid = p.tail ? tiles + p.tail : tiles * p.ks;
    if (p.tail)
        hipLaunchKernelGGL(gemm_zero_tiles_kernel, dim3(p.tail * (bm / 8)), dim3(256), 0, s, p.y, p.m, p.n,
                           tiles - p.tail, nt, bm, (uint32_t)BN);
#define YULE_GEMM_ARGS p.xh, p.w.w[0], p.w.w[1], p.w.w[2], p.w.s1, p.w.s2, p.m, p.n, p.k, p.tail | p.ks << 16 | remap << 31, p.xl, p.y, p.xs_hi, \
        p.xs_lo, p.rowscale, p.accumulate
    if (p.xl) {   // f32 X: the hi and lo sweeps
        if (bm == 64)
            hipLaunchKernelGGL((gemm_kernel<DT, 64, BN, 2>), dim3(grid), dim3(2 * BN), 0, s, YULE_GEMM_ARGS);
        else
            hipLaunchKernelGGL((gemm_kernel<DT, 128, BN, 2>), dim3(grid), dim3(2 * BN), 0, s, YULE_GEMM_ARGS);
    } else if (bm == 64) {
        hipLaunchKernelGGL((gemm_kernel<DT, 64, BN, 1>), dim3(grid), dim3(2 * BN), 0, s, YULE_GEMM_ARGS);
    } else if (bm == 256) {   // 128 x 64 wave tiles (Q4_K, 256-wide tiles; chosen by gemm_bm)
        if constexpr (DT == YULE_DTYPE_Q4_K && BN == 256)
            hipLaunchKernelGGL((gemm_kernel<DT, 256, BN, 1>), dim3(grid), dim3(2 * BN), 0, s, YULE_GEMM_ARGS);
    } else {
        hipLaunchKernelGGL((gemm_kernel<DT, 128, BN, 1>), dim3(grid), dim3(2 * BN), 0, s, YULE_GEMM_ARGS);
    }
#undef YULE_GEMM_ARGS
}

template <uint32_t DT>
void launch_gemm(hipStream_t s, const GemmPass &p) {
    if (p.bn == 256) launch_gemm_bn<DT, 256>(s, p);
    else launch_gemm_bn<DT, 128>(s, p);
}

int launch_gemm_dt(hipStream_t s, uint32_t dtype, const GemmPass &p) {
    switch (dtype) {
    case YULE_DTYPE_Q4_K: launch_gemm<YULE_DTYPE_Q4_K>(s, p); break;
    case YULE_DTYPE_Q6_K: launch_gemm<YULE_DTYPE_Q6_K>(s, p); break;
    case YULE_DTYPE_Q5_K: launch_gemm<YULE_DTYPE_Q5_K>(s, p); break;
    case YULE_DTYPE_Q8_K: launch_gemm<YULE_DTYPE_Q8_K>(s, p); break;
    case YULE_DTYPE_Q8_0: launch_gemm<YULE_DTYPE_Q8_0>(s, p); break;
    default: launch_gemm<YULE_DTYPE_Q4_0>(s, p); break;
    }
    return check_launch("quantized_gemm");
}

template <int MT>
void launch_skinny_mt(hipStream_t s, const GemmPass &p) {
    const dim3 grid((p.n + 127) / 128, p.ks);
    constexpr int XB = 8;   // X ring: MT x 8 KB per buffer
    hipLaunchKernelGGL((gemm_q4k_skinny_kernel<MT, 4, XB>), grid, dim3(320), 0, s, p.xh, p.w.w[0], p.w.w[1], p.w.w[2],
                       p.w.s1, p.w.s2, p.m, p.n, p.k, p.y, p.xs_hi, p.xs_lo, p.rowscale, p.accumulate);
}

int launch_gemm_skinny(hipStream_t s, const GemmPass &p) {
    if (p.m <= 16) launch_skinny_mt<1>(s, p);
    else launch_skinny_mt<2>(s, p);
    return check_launch("quantized_gemm (few X rows)");
}

bool gemm_dtype_ok(uint32_t dtype) {
    return dtype == YULE_DTYPE_Q4_K || dtype == YULE_DTYPE_Q6_K || dtype == YULE_DTYPE_Q8_0 ||
           dtype == YULE_DTYPE_Q4_0 || dtype == YULE_DTYPE_Q5_K || dtype == YULE_DTYPE_Q8_K;
}

}  // namespace

// Workspace of one call (bytes) and the pieces inside it: split-K partials,
// then X in f16 (hi, and lo for f32 X), the Q4_K/Q5_K sub-block sums (hi, lo)
// and the per-row scales.
struct GemmWork {
    size_t part_bytes, total;
    size_t n_x, n_sub, n_y;
    uint32_t ks, bn, bm, tail;
    bool q4, skinny;
};

static GemmWork gemm_work(uint32_t m, uint32_t n_rows, uint32_t n_cols, uint32_t dtype, bool f32x) {
    GemmWork g;
    g.q4 = dtype == YULE_DTYPE_Q4_K || dtype == YULE_DTYPE_Q5_K;   // min term: X sub-block sums
    g.bn = gemm_bn(m, dtype);
    g.bm = gemm_bm(m, f32x, dtype, g.bn);
    g.skinny = gemm_skinny(m, n_cols, dtype, f32x);
    g.ks = g.skinny ? gemm_skinny_splits(n_rows, n_cols) : gemm_splits(m, n_rows, n_cols, g.bn, g.bm, gemm_wgs_per_cu(dtype, g.bm, g.bn, f32x));
    g.tail = g.skinny ? 0u : gemm_tail(m, n_rows, n_cols, g.bn, g.bm, g.ks);
    g.n_x = (size_t)m * n_cols;
    g.n_sub = (size_t)m * (n_cols / 32);
    g.n_y = (size_t)m * n_rows;
    g.part_bytes = g.ks > 1 ? ((g.ks * g.n_y * sizeof(float) + 255) & ~(size_t)255) : 0;
    g.total = g.part_bytes + ((f32x ? 2 : 1) * g.n_x + (g.q4 ? 2 * g.n_sub : 0)) * sizeof(_Float16) + 256 +
              (size_t)m * sizeof(float) + 256;
    return g;
}

// Enqueue the pre-pass and the product(s) of one call into workspace ws.
static GemmW one_matrix(const uint8_t *w, uint32_t n_rows) { return GemmW{{w, w, w}, n_rows, n_rows}; }

// accumulate: Y += the product (no K-half tail then: its atomic adds would
// add into Y in either order)
static int gemm_enqueue(hipStream_t s, const GemmW &w, const void *x, bool f32x, float *y, uint32_t m,
                        uint32_t n_rows, uint32_t n_cols, uint32_t dtype, const GemmWork &g, void *ws,
                        bool accumulate = false, const float *norm_w = nullptr, float eps = 0.f, bool glu = false,
                        GemmRed *defer = nullptr, const GemmRed *pending = nullptr) {
    uint8_t *b = static_cast<uint8_t *>(ws);
    float *part = g.ks > 1 ? reinterpret_cast<float *>(b) : nullptr;
    _Float16 *xh = reinterpret_cast<_Float16 *>(b + g.part_bytes);
    _Float16 *xl = f32x ? xh + g.n_x : nullptr;
    _Float16 *xs_hi = g.q4 ? xh + (f32x ? 2 : 1) * g.n_x : nullptr, *xs_lo = g.q4 ? xs_hi + g.n_sub : nullptr;
    float *rowscale = reinterpret_cast<float *>(
        (reinterpret_cast<uintptr_t>(xh + (f32x ? 2 : 1) * g.n_x + (g.q4 ? 2 * g.n_sub : 0)) + 255) & ~(uintptr_t)255);
    const bool red = pending && pending->ks > 1;
    if (red && (!f32x || pending->y != x || pending->m != m || pending->ny != (glu ? 2 : 1) * n_cols))
        return set_error(YULE_ERR_INVALID, "quantized_gemm: pending reduction does not produce this X");
    if (f32x)
        hipLaunchKernelGGL(gemm_xprep_kernel<true>, dim3(m), dim3(256), 0, s, x, norm_w, n_cols, eps, glu ? 1u : 0u,
                           xh, xl, xs_hi, xs_lo, rowscale, red ? pending->part : nullptr, red ? pending->ks : 0u,
                           red ? pending->ny : 0u, m, red && pending->accumulate ? 1u : 0u);
    else
        hipLaunchKernelGGL(gemm_xprep_kernel<false>, dim3(m), dim3(256), 0, s, x, norm_w, n_cols, eps, 0u, xh, xl,
                           xs_hi, xs_lo, rowscale, nullptr, 0u, 0u, m, 0u);
    int rc = check_launch("quantized_gemm: x pre-pass");
    if (rc) return rc;
    const GemmPass p{w, xh, xl, xs_hi, xs_lo, rowscale, g.ks > 1 ? part : y, m, n_rows, n_cols, g.ks, g.bn, g.bm,
                     accumulate ? 0u : g.tail, accumulate ? 1u : 0u};
    if ((rc = g.skinny ? launch_gemm_skinny(s, p) : launch_gemm_dt(s, dtype, p))) return rc;
    if (defer) *defer = GemmRed{part, y, g.ks > 1 ? g.ks : 0u, n_rows, m, accumulate};
    if (g.ks > 1 && defer) return YULE_OK;   // summed by the next product's pre-pass
    if (g.ks > 1) {
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((g.n_y + 255) / 256)), dim3(256), 0, s, part, y,
                           (uint64_t)g.n_y, g.ks, accumulate ? 1u : 0u);
        if ((rc = check_launch("quantized_gemm: split-K reduction"))) return rc;
    }
    return YULE_OK;
}

// ---- static workspace of the allocation-free entry point
// One array per GPU, in the code object, alive until the process ends.  Its
// device address is looked up once per device, with that device current, at
// backend creation (gemm_static_workspace_init); host code uses that
// address, never the array's name.
constexpr size_t kStaticWorkspaceBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kStaticWorkspaceBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_static_mu;
static void *g_static_ptr[kMaxDevices];

int yule::gemm_static_workspace_init(int device) {
    if (device < 0 || device >= kMaxDevices)
        return set_error(YULE_ERR_NO_DEVICE, "static workspace: device index above " + std::to_string(kMaxDevices - 1));
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (g_static_ptr[device]) return YULE_OK;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress (static workspace)");
    if (!p) return set_error(YULE_ERR_HIP, "static workspace: null device address");
    g_static_ptr[device] = p;
    return YULE_OK;
}

static void *static_workspace(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_static_mu);
    return g_static_ptr[device];
}

static int gemm_entry(yule_hip_backend *be, yule_buffer weights, yule_buffer x, bool f32x, yule_buffer y, uint32_t m,
                      uint32_t n_rows, uint32_t n_cols, uint32_t dtype, const char *what, bool noalloc = false) {
    if (!be) return set_error(YULE_ERR_INVALID, "null backend");
    if (!gemm_dtype_ok(dtype))
        return set_error(YULE_ERR_UNSUPPORTED, std::string(what) + ": dtype " + std::to_string(dtype) +
                                                   " not supported (Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, Q8_K)");
    if (n_cols % 256) return set_error(YULE_ERR_INVALID, std::string(what) + ": n_cols must be a multiple of 256");
    uint32_t bs, bb;
    quant_geometry(dtype, &bs, &bb);
    void *pw, *px, *py;
    int rc;
    if ((rc = get_buffer(be, weights, (size_t)n_rows * (n_cols / bs) * bb, &pw, what)) ||
        (rc = get_buffer(be, x, (size_t)m * n_cols * (f32x ? 4 : 2), &px, what)) ||
        (rc = get_buffer(be, y, (size_t)m * n_rows * 4, &py, what)))
        return rc;
    if (x == y) return set_error(YULE_ERR_INVALID, std::string(what) + ": x and y alias");
    if (weights == y || weights == x) return set_error(YULE_ERR_INVALID, std::string(what) + ": weights alias x or y");
    if (!m || !n_rows) return YULE_OK;
    if (!n_cols) return launch_fill(be->stream, (float *)py, 0.f, (uint64_t)m * n_rows);
    const GemmWork g = gemm_work(m, n_rows, n_cols, dtype, f32x);
    if (noalloc) {
        if (g.total > kStaticWorkspaceBytes)
            return set_error(YULE_ERR_INVALID, std::string(what) + ": this call needs " + std::to_string(g.total) +
                                                   " bytes of workspace, above the static " +
                                                   std::to_string(kStaticWorkspaceBytes) + "-byte one");
        void *ws = static_workspace(be->device);
        if (!ws) return set_error(YULE_ERR_HIP, std::string(what) + ": static workspace not set up for this device");
        return gemm_enqueue(be->stream, one_matrix((const uint8_t *)pw, n_rows), px, f32x, (float *)py, m, n_rows,
                            n_cols, dtype, g, ws);
    }
    ScratchLease lease;   // held until every launch below is enqueued
    if ((rc = get_scratch(be, g.total, &lease))) return rc;
    return gemm_enqueue(be->stream, one_matrix((const uint8_t *)pw, n_rows), px, f32x, (float *)py, m, n_rows, n_cols,
                        dtype, g, lease.ptr);
}

// the f32-X product for library callers that own their workspace (the
// runner's batched prefill)
bool yule::gemm_supports(uint32_t dtype, uint32_t n_cols) { return gemm_dtype_ok(dtype) && n_cols % 256 == 0; }

size_t yule::gemm_f32_workspace_bytes(uint32_t m, uint32_t n_rows, uint32_t n_cols, uint32_t dtype) {
    return gemm_work(m, n_rows, n_cols, dtype, true).total;
}

int yule::launch_gemm_f32(hipStream_t s, const uint8_t *w, const float *x, float *y, uint32_t m, uint32_t n_rows,
                          uint32_t n_cols, uint32_t dtype, void *ws, bool accumulate, const float *norm_w, float eps,
                          bool glu, GemmRed *defer, const GemmRed *pending) {
    if (!gemm_dtype_ok(dtype) || n_cols % 256) return set_error(YULE_ERR_UNSUPPORTED, "gemm: format or shape");
    if (glu && norm_w) return set_error(YULE_ERR_INVALID, "gemm: SwiGLU input and RMSNorm together");
    if (defer) defer->ks = 0;
    if (!m || !n_rows) return YULE_OK;
    return gemm_enqueue(s, one_matrix(w, n_rows), x, true, y, m, n_rows, n_cols, dtype,
                        gemm_work(m, n_rows, n_cols, dtype, true), ws, accumulate, norm_w, eps, glu, defer, pending);
}

// Several matrices of one format and width that share X, as one product
// (Y = [M][sum of their rows], each matrix's rows a block of columns): one
// pre-pass, one launch, one split-K reduction.  Each matrix's row count must
// be a multiple of 256, so that no tile of either width straddles two.
bool yule::gemm_multi_ok(uint32_t dtype, uint32_t n_cols, const uint32_t *rows, uint32_t n_mat) {
    if (!gemm_supports(dtype, n_cols) || n_mat == 0 || n_mat > 3) return false;
    for (uint32_t i = 0; i < n_mat; i++)
        if (rows[i] == 0 || rows[i] % 256) return false;
    return true;
}

size_t yule::gemm_f32_multi_workspace_bytes(uint32_t m, const uint32_t *rows, uint32_t n_mat, uint32_t n_cols,
                                            uint32_t dtype) {
    uint32_t total = 0;
    for (uint32_t i = 0; i < n_mat; i++) total += rows[i];
    return gemm_work(m, total, n_cols, dtype, true).total;
}

int yule::launch_gemm_f32_multi(hipStream_t s, const uint8_t *const *w, const uint32_t *rows, uint32_t n_mat,
                                const float *x, float *y, uint32_t m, uint32_t n_cols, uint32_t dtype, void *ws,
                                const float *norm_w, float eps, GemmRed *defer, const GemmRed *pending) {
    if (!gemm_multi_ok(dtype, n_cols, rows, n_mat)) return set_error(YULE_ERR_UNSUPPORTED, "gemm: format or shape");
    if (defer) defer->ks = 0;
    if (!m) return YULE_OK;
    GemmW g{{w[0], n_mat > 1 ? w[1] : w[0], n_mat > 2 ? w[2] : w[0]}, 0, 0};
    const uint32_t total = rows[0] + (n_mat > 1 ? rows[1] : 0) + (n_mat > 2 ? rows[2] : 0);
    g.s1 = n_mat > 1 ? rows[0] : total;
    g.s2 = n_mat > 2 ? rows[0] + rows[1] : total;
    return gemm_enqueue(s, g, x, true, y, m, total, n_cols, dtype, gemm_work(m, total, n_cols, dtype, true), ws,
                        false, norm_w, eps, false, defer, pending);
}

extern "C" int yule_hip_quantized_gemm(yule_hip_backend *be, yule_buffer weights, yule_buffer x_bf16, yule_buffer y,
                                       uint32_t m, uint32_t n_rows, uint32_t n_cols, uint32_t dtype) {
    return gemm_entry(be, weights, x_bf16, false, y, m, n_rows, n_cols, dtype, "quantized_gemm");
}

extern "C" int yule_hip_quantized_gemm_f32(yule_hip_backend *be, yule_buffer weights, yule_buffer x_f32, yule_buffer y,
                                           uint32_t m, uint32_t n_rows, uint32_t n_cols, uint32_t dtype) {
    return gemm_entry(be, weights, x_f32, true, y, m, n_rows, n_cols, dtype, "quantized_gemm_f32");
}

extern "C" int yule_hip_quantized_gemm_noalloc(yule_hip_backend *be, yule_buffer weights, yule_buffer x_bf16,
                                               yule_buffer y, uint32_t m, uint32_t n_rows, uint32_t n_cols,
                                               uint32_t dtype) {
    return gemm_entry(be, weights, x_bf16, false, y, m, n_rows, n_cols, dtype, "quantized_gemm_noalloc", true);
}
