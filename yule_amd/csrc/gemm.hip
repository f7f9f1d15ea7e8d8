// gemm.hip — prefill dequant-GEMM on the MFMA units:
//   Y[m][r] = sum_c X[m][c] * W[r][c],  X bf16 [M][K], W raw GGUF blocks, Y f32 [M][N].
// No counterpart in the reference, whose prefill is token by token
// (yule-infer/src/model_runner.rs:1075-1081); each row of Y equals one
// quantized_matmul of the corresponding row of X (parity target).
//
// Exactness: weights enter the MFMA as f16 holding exact integers and every
// scale is applied in f32, so the only roundings are f32 accumulations.
//  * Q4_K, w = d*sc*q - dmin*mn: the B operand is sc*q (integers <= 945,
//    exact in f16; bf16 would round them).  A 16x16 tile accumulates one
//    super-block (256 k) into a temporary, then final += d * tmp in f32.
//    The min term sum_sub (dmin*mn)*(sum of x over the sub-block) is a
//    second, small MFMA product over K/32 sub-blocks with both operands
//    split into hi + lo f16 pairs (dmin*mn is an exact 17-bit f32 value);
//    hi*hi + hi*lo + lo*hi reproduces it to ~2^-22.
//  * Q6_K, w = d*sc*(q-32): the B operand is sc*(q-32) (|.| <= 4064; exact
//    up to 2048, above that rounded to the nearest even integer, i.e.
//    < 2.5e-4 relative on those few weights), d applied per super-block.
//  * X: bf16 -> f16 is exact for every bf16 in f16's normal range.
//
// Tiling: a 256-thread workgroup computes a 128 (m) x 128 (r) tile; each of
// its four waves a 64 x 64 sub-tile of 4 x 4 MFMA 16x16x32 tiles.  Per step
// of 128 k (half a super-block) the workgroup dequantizes its 128 weight
// rows into LDS as f16 and converts its 128 x 128 X tile into LDS; rows are
// padded by 16 bytes so the ds_read_b128 operand loads avoid bank conflicts.
#include <string>

#include "internal.h"

namespace yule {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int GBM = 128, GBN = 128, GBK = 128;
constexpr int LDW = GBK + 8;   // padded row stride in halves

__device__ __forceinline__ _Float16 bf16_to_f16(uint16_t b) {
    return (_Float16)__builtin_bit_cast(float, (uint32_t)b << 16);
}

// n bytes starting at p (only 2-byte aligned) as n/4 little-endian dwords,
// read through 4-byte-aligned loads (the backend pads every allocation).
template <int N>
__device__ __forceinline__ void load_words(const uint8_t *p, uint32_t *out) {
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(p - mis);
    uint32_t raw[N / 4 + 1];
#pragma unroll
    for (int i = 0; i < N / 4 + 1; i++) raw[i] = w[i];
#pragma unroll
    for (int i = 0; i < N / 4; i++) out[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], mis);
}

// sum over each 32-column sub-block of X, split into f16 hi + lo:
// xs_hi/lo[m][j] for j < K/32
__global__ void xsum_kernel(const uint16_t *__restrict__ x, _Float16 *__restrict__ hi, _Float16 *__restrict__ lo,
                            uint32_t M, uint32_t K) {
    const uint32_t nsub = K / 32;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)M * nsub) return;
    const uint32_t m = (uint32_t)(i / nsub), j = (uint32_t)(i % nsub);
    const uint16_t *p = x + (size_t)m * K + 32 * j;
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 32; c++) s += __builtin_bit_cast(float, (uint32_t)p[c] << 16);
    const _Float16 h = (_Float16)s;
    hi[i] = h;
    lo[i] = (_Float16)(s - (float)h);
}

template <uint32_t DT>
__global__ __launch_bounds__(256) void gemm_kernel(const uint8_t *__restrict__ w, const uint16_t *__restrict__ x,
                                                   float *__restrict__ y, const _Float16 *__restrict__ xs_hi,
                                                   const _Float16 *__restrict__ xs_lo, uint32_t M, uint32_t N,
                                                   uint32_t K) {
    constexpr uint32_t BB = DT == YULE_DTYPE_Q4_K ? 144 : 210;
    __shared__ __align__(16) _Float16 sx[GBM * LDW];
    __shared__ __align__(16) _Float16 sw[GBN * LDW];
    __shared__ float sd[GBN];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = blockIdx.y * GBM, r0 = blockIdx.x * GBN;
    const uint32_t bpr = K / 256;
    const size_t row_bytes = (size_t)bpr * BB;

    floatx4 acc[4][4], tmp[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) { acc[i][j] = floatx4{0, 0, 0, 0}; tmp[i][j] = floatx4{0, 0, 0, 0}; }

    // weight-dequant role: two threads per weight row, 64 weights each
    const uint32_t wr = tid >> 1, part = tid & 1;
    const bool wrow_ok = r0 + wr < N;
    const uint8_t *wrow = w + (size_t)(wrow_ok ? r0 + wr : 0) * row_bytes;

    for (uint32_t kb = 0; kb < bpr; kb++) {
        for (uint32_t hs = 0; hs < 2; hs++) {   // the two 128-k halves of super-block kb
            const uint32_t k0 = kb * 256 + hs * 128;
            // ---- X tile -> LDS (bf16 -> f16, exact)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t idx = tid + 256 * i;            // 2048 chunks of 8 halves
                const uint32_t mr = idx >> 4, c8 = idx & 15;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (m0 + mr < M) v = *reinterpret_cast<const uint4 *>(x + (size_t)(m0 + mr) * K + k0 + 8 * c8);
                half8 h;
                const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    h[2 * q] = bf16_to_f16((uint16_t)(wv[q] & 0xFFFFu));
                    h[2 * q + 1] = bf16_to_f16((uint16_t)(wv[q] >> 16));
                }
                *reinterpret_cast<half8 *>(sx + mr * LDW + 8 * c8) = h;
            }
            // ---- W tile -> LDS as exact integer f16
            const uint8_t *blk = wrow + (size_t)kb * BB;
            _Float16 *dst = sw + wr * LDW;
            if constexpr (DT == YULE_DTYPE_Q4_K) {
                // this thread: qs group j = 2*hs + part -> sub-blocks 2j (low) and 2j+1 (high)
                const uint32_t j = 2 * hs + part;
                uint32_t hd[4], qs[8];
                const uint4 h4 = *reinterpret_cast<const uint4 *>(blk);
                hd[0] = h4.x; hd[1] = h4.y; hd[2] = h4.z; hd[3] = h4.w;
                const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * j);
                const uint4 qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * j);
                qs[0] = qa.x; qs[1] = qa.y; qs[2] = qa.z; qs[3] = qa.w;
                qs[4] = qb.x; qs[5] = qb.y; qs[6] = qb.z; qs[7] = qb.w;
                const uint8_t *sb = reinterpret_cast<const uint8_t *>(hd) + 4;
                uint32_t sc0, sc1;
                const uint32_t s0 = 2 * j, s1 = 2 * j + 1;
                sc0 = s0 < 4 ? (sb[s0] & 63u) : ((sb[s0 + 4] & 0xFu) | ((uint32_t)(sb[s0 - 4] >> 6) << 4));
                sc1 = s1 < 4 ? (sb[s1] & 63u) : ((sb[s1 + 4] & 0xFu) | ((uint32_t)(sb[s1 - 4] >> 6) << 4));
                const _Float16 f0 = (_Float16)(float)sc0, f1 = (_Float16)(float)sc1;
                half8 lo8, hi8;
#pragma unroll
                for (int c = 0; c < 4; c++) {   // 4 chunks of 8 bytes -> 8 low + 8 high weights each
#pragma unroll
                    for (int b = 0; b < 8; b++) {
                        const uint32_t byte = (qs[2 * c + b / 4] >> (8 * (b & 3))) & 0xFFu;
                        lo8[b] = (_Float16)(float)(byte & 0xFu) * f0;
                        hi8[b] = (_Float16)(float)(byte >> 4) * f1;
                    }
                    *reinterpret_cast<half8 *>(dst + 64 * part + 8 * c) = wrow_ok ? lo8 : half8{};
                    *reinterpret_cast<half8 *>(dst + 64 * part + 32 + 8 * c) = wrow_ok ? hi8 : half8{};
                }
                if (part == 0) sd[wr] = wrow_ok ? (float)__builtin_bit_cast(_Float16, (uint16_t)(hd[0] & 0xFFFFu)) : 0.f;
            } else {
                // Q6_K half hs: part 0 -> quarters g = 0, 2 (ql[0..31]); part 1 -> g = 1, 3 (ql[32..63])
                uint32_t ql[8], qh[8], scw[2], dw[1];
                load_words<32>(blk + 64 * hs + 32 * part, ql);
                load_words<32>(blk + 128 + 32 * hs, qh);
                load_words<8>(blk + 192 + 8 * hs, scw);
                load_words<4>(blk + 208, dw);
                const int8_t *sc = reinterpret_cast<const int8_t *>(scw);
                const uint32_t ga = part, gb = part + 2;          // quarters from low / high nibbles
                const uint32_t sha = 2 * ga, shb = 2 * gb;        // qh bit pair position
#pragma unroll
                for (int c = 0; c < 4; c++) {                     // l = 8c .. 8c+7
                    half8 va, vb;
#pragma unroll
                    for (int b = 0; b < 8; b++) {
                        const uint32_t l = 8 * c + b;
                        const uint32_t qlb = (ql[l / 4] >> (8 * (l & 3))) & 0xFFu;
                        const uint32_t qhb = (qh[l / 4] >> (8 * (l & 3))) & 0xFFu;
                        const int qa = (int)((qlb & 0xFu) | (((qhb >> sha) & 3u) << 4)) - 32;
                        const int qb = (int)((qlb >> 4) | (((qhb >> shb) & 3u) << 4)) - 32;
                        const uint32_t is = l / 16;
                        va[b] = (_Float16)(float)(sc[is + 2 * ga] * qa);
                        vb[b] = (_Float16)(float)(sc[is + 2 * gb] * qb);
                    }
                    *reinterpret_cast<half8 *>(dst + 32 * ga + 8 * c) = wrow_ok ? va : half8{};
                    *reinterpret_cast<half8 *>(dst + 32 * gb + 8 * c) = wrow_ok ? vb : half8{};
                }
                if (part == 0) sd[wr] = wrow_ok ? (float)__builtin_bit_cast(_Float16, (uint16_t)(dw[0] & 0xFFFFu)) : 0.f;
            }
            __syncthreads();
            // ---- MFMA over the 128-k step
#pragma unroll
            for (int ks = 0; ks < GBK / 32; ks++) {
                half8 a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; i++)
                    a[i] = *reinterpret_cast<const half8 *>(sx + (wm * 64 + i * 16 + (lane & 15)) * LDW + ks * 32 +
                                                           8 * (lane >> 4));
#pragma unroll
                for (int j = 0; j < 4; j++)
                    b[j] = *reinterpret_cast<const half8 *>(sw + (wn * 64 + j * 16 + (lane & 15)) * LDW + ks * 32 +
                                                           8 * (lane >> 4));
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], tmp[i][j], 0, 0, 0);
            }
            if (hs == 1) {   // super-block done: final += d[r] * tmp
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float dr = sd[wn * 64 + j * 16 + (lane & 15)];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc[i][j] += dr * tmp[i][j];
                        tmp[i][j] = floatx4{0, 0, 0, 0};
                    }
                }
            }
            __syncthreads();
        }
    }

    if constexpr (DT == YULE_DTYPE_Q4_K) {
        // min term: acc -= sum_j xsum[m][j] * (dmin*mn)[r][j] over the K/32
        // sub-blocks; a k-step of 32 covers 4 super-blocks, lane quarter q
        // takes super-block 4*kk + q, i.e. its 8 sub-blocks.
        const uint32_t nsub = K / 32;
        for (uint32_t kk = 0; kk < bpr; kk += 4) {
            const uint32_t sbk = kk + (lane >> 4);          // super-block of this lane's 8 sub-blocks
            half8 bh[4], bl[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t r = r0 + wn * 64 + j * 16 + (lane & 15);
                half8 h = {}, l = {};
                if (r < N && sbk < bpr) {
                    const uint8_t *blk = w + (size_t)r * row_bytes + (size_t)sbk * BB;
                    const uint4 h4 = *reinterpret_cast<const uint4 *>(blk);
                    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(h4.x >> 16));
                    const uint32_t hd[3] = {h4.y, h4.z, h4.w};
                    const uint8_t *q = reinterpret_cast<const uint8_t *>(hd);
#pragma unroll
                    for (int s = 0; s < 8; s++) {
                        const uint32_t mn = s < 4 ? (q[s + 4] & 63u)
                                                  : ((uint32_t)(q[s + 4] >> 4) | ((uint32_t)(q[s] >> 6) << 4));
                        const float v = -(dmin * (float)mn);     // exact in f32
                        const _Float16 vh = (_Float16)v;
                        h[s] = vh;
                        l[s] = (_Float16)(v - (float)vh);
                    }
                }
                bh[j] = h;
                bl[j] = l;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t m = m0 + wm * 64 + i * 16 + (lane & 15);
                half8 ah = {}, al = {};
                if (m < M && sbk < bpr) {
                    ah = *reinterpret_cast<const half8 *>(xs_hi + (size_t)m * nsub + 8 * sbk);
                    al = *reinterpret_cast<const half8 *>(xs_lo + (size_t)m * nsub + 8 * sbk);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    }

    // ---- store: lane holds rows 4*(lane/16)+e of column lane%16 of each tile
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t r = r0 + wn * 64 + j * 16 + (lane & 15);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t m = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + e;
                if (m < M && r < N) y[(size_t)m * N + r] = acc[i][j][e];
            }
        }
}

}  // namespace yule

using namespace yule;

// Per-backend scratch for the sub-block sums of X (grown on demand).
namespace {
struct GemmScratch {
    yule_hip_backend *be = nullptr;
    void *p = nullptr;
    size_t size = 0;
};
GemmScratch g_scratch;
std::mutex g_scratch_mu;
}  // namespace

extern "C" int yule_hip_quantized_gemm(yule_hip_backend *be, yule_buffer weights, yule_buffer x_bf16, yule_buffer y,
                                       uint32_t m, uint32_t n_rows, uint32_t n_cols, uint32_t dtype) {
    if (!be) return set_error(YULE_ERR_INVALID, "null backend");
    if (dtype != YULE_DTYPE_Q4_K && dtype != YULE_DTYPE_Q6_K)
        return set_error(YULE_ERR_UNSUPPORTED, "quantized_gemm: dtype " + std::to_string(dtype) +
                                                   " not supported (Q4_K and Q6_K)");
    if (n_cols % 256) return set_error(YULE_ERR_INVALID, "quantized_gemm: n_cols must be a multiple of 256");
    uint32_t bs, bb;
    quant_geometry(dtype, &bs, &bb);
    void *pw, *px, *py;
    int rc;
    if ((rc = get_buffer(be, weights, (size_t)n_rows * (n_cols / bs) * bb, &pw, "quantized_gemm (weights)")) ||
        (rc = get_buffer(be, x_bf16, (size_t)m * n_cols * 2, &px, "quantized_gemm (x)")) ||
        (rc = get_buffer(be, y, (size_t)m * n_rows * 4, &py, "quantized_gemm (y)")))
        return rc;
    if (x_bf16 == y) return set_error(YULE_ERR_INVALID, "quantized_gemm: x and y alias");
    if (!m || !n_rows) return YULE_OK;
    if (!n_cols) return launch_fill(be->stream, (float *)py, 0.f, (uint64_t)m * n_rows);
    _Float16 *xs_hi = nullptr, *xs_lo = nullptr;
    if (dtype == YULE_DTYPE_Q4_K) {
        const size_t need = (size_t)m * (n_cols / 32) * 2 * sizeof(_Float16) + 256;
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (g_scratch.be != be || g_scratch.size < need) {
            if (g_scratch.p) {
                hipStreamSynchronize(be->stream);
                hipFree(g_scratch.p);
            }
            g_scratch = GemmScratch{};
            if ((rc = hip_error(hipMalloc(&g_scratch.p, need), "quantized_gemm: scratch"))) return rc;
            g_scratch.be = be;
            g_scratch.size = need;
        }
        xs_hi = static_cast<_Float16 *>(g_scratch.p);
        xs_lo = xs_hi + (size_t)m * (n_cols / 32);
        const uint64_t nx = (uint64_t)m * (n_cols / 32);
        hipLaunchKernelGGL(xsum_kernel, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, be->stream,
                           (const uint16_t *)px, xs_hi, xs_lo, m, n_cols);
        if ((rc = check_launch("quantized_gemm: x sums"))) return rc;
        hipLaunchKernelGGL(gemm_kernel<YULE_DTYPE_Q4_K>, dim3((n_rows + GBN - 1) / GBN, (m + GBM - 1) / GBM),
                           dim3(256), 0, be->stream, (const uint8_t *)pw, (const uint16_t *)px, (float *)py, xs_hi,
                           xs_lo, m, n_rows, n_cols);
    } else {
        hipLaunchKernelGGL(gemm_kernel<YULE_DTYPE_Q6_K>, dim3((n_rows + GBN - 1) / GBN, (m + GBM - 1) / GBM),
                           dim3(256), 0, be->stream, (const uint8_t *)pw, (const uint16_t *)px, (float *)py, nullptr,
                           nullptr, m, n_rows, n_cols);
    }
    return check_launch("quantized_gemm");
}
