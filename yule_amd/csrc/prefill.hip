// prefill.hip — the runner's batched prompt pass: the operations of a decode
// step applied to P prompt rows at once, so that each projection runs as one
// matrix-core GEMM (gemm.hip, f32 X) instead of P matvecs.  Yule prefills token
// by token (yule-infer/src/model_runner.rs:1075-1081); every row here computes
// exactly what that step computes for its token, to f32 rounding, and writes
// the same KV-cache rows:
//   embedding rows -> per layer [RMSNorm rows] [Q, K, V GEMMs] [RoPE + cache
//   rows] [causal attention] [O GEMM] [residual] [RMSNorm rows] [gate, up
//   GEMMs] [SwiGLU] [down GEMM] [residual].
#include "blocks.h"
#include "internal.h"

namespace yule {

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wsum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wmax(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
// sum over aligned groups of n lanes (n = 2, 4, 8 or 16), every lane of a
// group receiving the group's sum
__device__ __forceinline__ float gsum(float v, uint32_t n) {
    if (n >= 2) v += dpp<0xB1>(v);
    if (n >= 4) v += dpp<0x4E>(v);
    if (n >= 8) v += dpp<0x141>(v);
    if (n >= 16) v += dpp<0x140>(v);
    return v;
}

}  // namespace

// ---- embedding rows: out[p] = dequantized row tokens[p] of the table
// (the token lookup of model_runner.rs:543-560, gpu_runner.rs:309-343)
__global__ void embed_rows_kernel(uint32_t dtype, uint32_t bs, uint32_t bb, const uint8_t *__restrict__ table,
                                  const uint32_t *__restrict__ tokens, uint32_t vocab, float *__restrict__ out,
                                  uint32_t dim) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, p = blockIdx.y;
    if (i >= dim) return;
    uint32_t t = tokens[p];
    t = t < vocab ? t : vocab - 1;   // host-checked tokens are in range; the clamp keeps reads in the table
    const uint8_t *row = table + (size_t)t * (dim / bs) * bb;
    out[(size_t)p * dim + i] = dequant_one(dtype, row + (i / bs) * bb, i % bs);
}

int launch_embed_rows_batch(hipStream_t s, uint32_t dtype, const uint8_t *table, const uint32_t *tokens,
                            uint32_t vocab, float *out, uint32_t dim, uint32_t n) {
    uint32_t bs, bb;
    if (!quant_geometry(dtype, &bs, &bb)) return set_error(YULE_ERR_UNSUPPORTED, "embedding: unsupported dtype");
    hipLaunchKernelGGL(embed_rows_kernel, dim3((dim + 255) / 256, n), dim3(256), 0, s, dtype, bs, bb, table, tokens,
                       vocab, out, dim);
    return check_launch("embedding rows");
}

// ---- RoPE of row p's q (in place) and k with the table row of position
// pos0 + p, and k, v into cache row pos0 + p (model_runner.rs:277-293,
// 654-669; the same arithmetic as the decode step's Q/K/V epilogue).  Rows
// of q are ldq floats apart, rows of k and v ldkv (separate buffers: qd and
// kvd; one [q | k | v] buffer: qd + 2 kvd for all three).
__global__ void rope_rows_kernel(float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
                                 float *__restrict__ kc, float *__restrict__ vc, const float *__restrict__ cos_t,
                                 const float *__restrict__ sin_t, uint32_t pos0, uint32_t qd, uint32_t kvd,
                                 uint32_t hd, uint32_t ldq, uint32_t ldkv) {
    const uint32_t p = blockIdx.y, j = blockIdx.x * blockDim.x + threadIdx.x, half = hd / 2;
    const uint32_t pos = pos0 + p, nqp = qd / 2, nkp = kvd / 2;
    if (j < nqp) {   // rotation pair j of q
        const uint32_t i = j % half;
        const float c = cos_t[(size_t)pos * half + i], sn = sin_t[(size_t)pos * half + i];
        float *qr = q + (size_t)p * ldq + 2 * j;
        const float x0 = qr[0], x1 = qr[1];
        qr[0] = x0 * c - x1 * sn;
        qr[1] = x0 * sn + x1 * c;
    } else if (j < nqp + nkp) {   // pair j - nqp of k, and the matching v values
        const uint32_t jk = j - nqp, i = jk % half;
        const float c = cos_t[(size_t)pos * half + i], sn = sin_t[(size_t)pos * half + i];
        const float *kr = k + (size_t)p * ldkv + 2 * jk;
        const float x0 = kr[0], x1 = kr[1];
        float *krow = kc + (size_t)pos * kvd + 2 * jk, *vrow = vc + (size_t)pos * kvd + 2 * jk;
        krow[0] = x0 * c - x1 * sn;
        krow[1] = x0 * sn + x1 * c;
        const float *vr = v + (size_t)p * ldkv + 2 * jk;
        vrow[0] = vr[0];
        vrow[1] = vr[1];
    }
}

int launch_rope_rows(hipStream_t s, float *q, const float *k, const float *v, float *kc, float *vc, const float *cos_t,
                     const float *sin_t, uint32_t pos0, uint32_t n, uint32_t qd, uint32_t kvd, uint32_t hd, uint32_t ldq,
                     uint32_t ldkv) {
    const uint32_t pairs = (qd + kvd) / 2;
    hipLaunchKernelGGL(rope_rows_kernel, dim3((pairs + 255) / 256, n), dim3(256), 0, s, q, k, v, kc, vc, cos_t, sin_t,
                       pos0, qd, kvd, hd, ldq, ldkv);
    return check_launch("rope rows");
}

// ---- causal GQA attention of prompt row p (position pos0 + p) over cache
// rows 0..pos0 + p (model_runner.rs:679-758), one workgroup per (query
// head, row).  Positions run in chunks of C = 4096 / HD with an online
// softmax: per chunk the scores (HD / 16 lanes per position, four float4 of
// the row each), the chunk maximum, then the running (m, l, o) rescaled by
// exp(m_old - m_new).  Output lanes own a float4 of dims and four positions
// of each chunk; their partial sums meet through LDS at the end.
template <uint32_t HD>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const float *__restrict__ q, const float *__restrict__ kc,
                                                           const float *__restrict__ vc, float *__restrict__ out,
                                                           uint32_t pos0, uint32_t qd, uint32_t ldq,
                                                           uint32_t group, uint32_t n_kv) {
    constexpr uint32_t NT = 256, ND4 = HD / 4, LPP = HD / 16, C = NT / LPP, NG = NT / ND4;
    static_assert(C == 4 * NG && LPP >= 2 && LPP <= 16, "geometry");
    __shared__ float ps[C];
    __shared__ float red[8];
    __shared__ float4 ored[NT];
    const uint32_t h = blockIdx.x, p = blockIdx.y, tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
    const uint32_t kvh = h / group, kvs4 = n_kv * ND4, seq = pos0 + p + 1;
    const float4 *q4 = reinterpret_cast<const float4 *>(q + (size_t)p * ldq) + (size_t)h * ND4;
    const float4 *kc4 = reinterpret_cast<const float4 *>(kc) + (size_t)kvh * ND4;
    const float4 *vc4 = reinterpret_cast<const float4 *>(vc) + (size_t)kvh * ND4;
    const uint32_t t = tid / LPP, sub = tid % LPP, d4 = tid % ND4, pg = tid / ND4;
    float4 qv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) qv[u] = q4[sub + u * LPP];
    const float scale = 1.0f / sqrtf((float)HD);
    float m = -INFINITY, l = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t c0 = 0; c0 < seq; c0 += C) {
        const uint32_t row = c0 + t < seq ? c0 + t : seq - 1;
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float4 kv = kc4[(size_t)row * kvs4 + sub + u * LPP];
            acc += qv[u].x * kv.x;
            acc += qv[u].y * kv.y;
            acc += qv[u].z * kv.z;
            acc += qv[u].w * kv.w;
        }
        const bool valid = c0 + t < seq;
        const float sc = valid ? gsum(acc, LPP) * scale : -INFINITY;
        float cm = wmax(sc);
        if (lane == 0) red[w] = cm;
        __syncthreads();
        cm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float mn = fmaxf(m, cm), alpha = expf(m - mn);   // exp(-inf) = 0 on the first chunk
        const float e = valid ? expf(sc - mn) : 0.f;
        if (sub == 0) ps[t] = e;
        float ls = wsum(sub == 0 ? e : 0.f);
        __syncthreads();   // red[] read, ps[] complete
        if (lane == 0) red[4 + w] = ls;
        __syncthreads();
        ls = (red[4] + red[5]) + (red[6] + red[7]);
        l = l * alpha + ls;
        o.x *= alpha; o.y *= alpha; o.z *= alpha; o.w *= alpha;
#pragma unroll
        for (uint32_t u = 0; u < 4; u++) {
            const uint32_t tt = pg * 4 + u, r = c0 + tt < seq ? c0 + tt : seq - 1;
            const float4 vv = vc4[(size_t)r * kvs4 + d4];
            const float pw = ps[tt];   // 0 past the sequence
            o.x += pw * vv.x; o.y += pw * vv.y; o.z += pw * vv.z; o.w += pw * vv.w;
        }
        m = mn;
        __syncthreads();   // ps[] and red[] reused by the next chunk
    }
    ored[tid] = o;
    __syncthreads();
    if (tid < ND4) {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        for (uint32_t g = 0; g < NG; g++) {
            const float4 b = ored[g * ND4 + tid];
            a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        }
        const float inv = 1.0f / l;
        reinterpret_cast<float4 *>(out + (size_t)p * qd)[(size_t)h * ND4 + tid] =
            make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
    }
}

bool attn_prefill_supported(uint32_t hd) { return hd == 32 || hd == 64 || hd == 128 || hd == 256; }

int launch_attn_prefill(hipStream_t s, const float *q, const float *kc, const float *vc, float *out, uint32_t pos0,
                        uint32_t n, uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t ldq) {
    const dim3 grid(n_heads, n);
    const uint32_t qd = n_heads * hd, group = n_heads / n_kv;
    switch (hd) {
    case 32: hipLaunchKernelGGL(attn_prefill_kernel<32>, grid, dim3(256), 0, s, q, kc, vc, out, pos0, qd, ldq, group, n_kv); break;
    case 64: hipLaunchKernelGGL(attn_prefill_kernel<64>, grid, dim3(256), 0, s, q, kc, vc, out, pos0, qd, ldq, group, n_kv); break;
    case 128: hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, dim3(256), 0, s, q, kc, vc, out, pos0, qd, ldq, group, n_kv); break;
    case 256: hipLaunchKernelGGL(attn_prefill_kernel<256>, grid, dim3(256), 0, s, q, kc, vc, out, pos0, qd, ldq, group, n_kv); break;
    default: return set_error(YULE_ERR_UNSUPPORTED, "prefill attention: head size");
    }
    return check_launch("prefill attention");
}

}  // namespace yule
