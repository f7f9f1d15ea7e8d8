// ops.hip — the remaining ComputeBackend methods (yule-gpu/src/lib.rs:26-114)
// as gfx950 kernels, plus the fused GQA decode attention and the greedy
// argmax the HIP runner uses.  Semantics follow CpuBackend
// (yule-gpu/src/cpu.rs:163-539); f32 results agree to rounding, since
// reductions run as trees instead of the reference's sequential loops.
#include <cstdlib>
#include <string>

#include "blocks.h"
#include "internal.h"
#include "qmv_common.h"

namespace yule {

// ------------------------------------------------------------ reductions
// Wave reductions by DPP row permutations (VALU latency, unlike the LDS
// permute network a lane shuffle goes through): lane-xor 1 and 2 inside
// quads, then the half-row and row mirrors, which pair whole quads and
// whole half-rows once those hold equal values; the four row results are
// combined from readlanes.  Every lane returns the wave result; call them
// with all 64 lanes active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i of 8 <- lane 7 - i
constexpr int kDppMirror = 0x140;      // lane i of 16 <- lane 15 - i
__device__ __forceinline__ float lane_of(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<kDppXor1>(v);
    v += dpp_mov<kDppXor2>(v);
    v += dpp_mov<kDppHalfMirror>(v);
    v += dpp_mov<kDppMirror>(v);
    return (lane_of(v, 0) + lane_of(v, 16)) + (lane_of(v, 32) + lane_of(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<kDppXor1>(v));
    v = fmaxf(v, dpp_mov<kDppXor2>(v));
    v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_mov<kDppMirror>(v));
    return fmaxf(fmaxf(lane_of(v, 0), lane_of(v, 16)), fmaxf(lane_of(v, 32), lane_of(v, 48)));
}
// sum over the lanes i, i + n, i + 2n, ... of the wave (n a power of two up
// to 64), every lane receiving its class's sum: row rotations for strides
// inside a 16-lane row, lane shuffles across rows.  (The gfx950 row and
// half-wave swap builtins were tried for the cross-row steps: with both
// operands the same value the optimizer has folded the two swapped copies
// into one in some contexts, giving wrong sums, so they are not used.)
__device__ __forceinline__ float strided_sum(float v, uint32_t n) {
    if (n <= 1) v += dpp_mov<0x121>(v);   // row_ror:1
    if (n <= 2) v += dpp_mov<0x122>(v);   // row_ror:2
    if (n <= 4) v += dpp_mov<0x124>(v);   // row_ror:4
    if (n <= 8) v += dpp_mov<0x128>(v);   // row_ror:8
    if (n <= 16) v += __shfl_xor(v, 16, 64);
    if (n <= 32) v += __shfl_xor(v, 32, 64);
    return v;
}
// sum over aligned groups of n lanes (n = 1, 2, 4 or 8), every lane of a
// group receiving the group's sum
__device__ __forceinline__ float group_sum(float v, uint32_t n) {
    if (n >= 2) v += dpp_mov<kDppXor1>(v);
    if (n >= 4) v += dpp_mov<kDppXor2>(v);
    if (n >= 8) v += dpp_mov<kDppHalfMirror>(v);
    return v;
}
// block-wide reductions for blockDim.x a multiple of 64 and <= 1024
__device__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}
__device__ float block_max(float v, float *red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < nw; i++) t = fmaxf(t, red[i]);
    return t;
}

// ------------------------------------------------------------ elementwise
__global__ void fill_kernel(float *out, float v, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = v;
}

int launch_fill(hipStream_t s, float *out, float v, uint64_t n) {
    if (!n) return YULE_OK;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, v, n);
    return check_launch("fill");
}

__global__ void pad_kernel(const float *__restrict__ x, uint32_t n, float *__restrict__ out, uint32_t n_out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n_out) out[i] = i < n ? x[i] : 0.f;
}

int launch_pad(hipStream_t s, const float *x, uint32_t n, float *out, uint32_t n_out) {
    hipLaunchKernelGGL(pad_kernel, dim3((n_out + 255) / 256), dim3(256), 0, s, x, n, out, n_out);
    return check_launch("pad");
}

// op 0: silu (cpu.rs:339-357), 1: element_mul, 2: add, 3: silu_mul
// (model_runner.rs:967-972: g * (1/(1+exp(-g))) * u)
__global__ void eltwise_kernel(int op, const float *__restrict__ a, const float *__restrict__ b,
                               float *__restrict__ out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = a[i];
    switch (op) {
    case 0: out[i] = x * (1.0f / (1.0f + expf(-x))); break;
    case 1: out[i] = x * b[i]; break;
    case 2: out[i] = x + b[i]; break;
    default: out[i] = x * (1.0f / (1.0f + expf(-x))) * b[i]; break;
    }
}

int launch_eltwise(hipStream_t s, int op, const float *a, const float *b, float *out, uint32_t n) {
    if (!n) return YULE_OK;
    hipLaunchKernelGGL(eltwise_kernel, dim3((n + 255) / 256), dim3(256), 0, s, op, a, b, out, n);
    return check_launch("elementwise");
}

// ------------------------------------------------------------ rms_norm
// cpu.rs:263-295 / model_runner.rs:246-275: out = x * (1/sqrt(mean(x^2)+eps)) * w
__global__ __launch_bounds__(1024) void rms_norm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                        float *__restrict__ out, uint32_t n, float eps) {
    __shared__ float red[16];
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * inv * w[i];
}

int launch_rms_norm(hipStream_t s, const float *x, const float *w, float *out, uint32_t n, float eps) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(1024), 0, s, x, w, out, n, eps);
    return check_launch("rms_norm");
}

// ------------------------------------------------------------ softmax
// cpu.rs:226-258, single workgroup
__global__ __launch_bounds__(1024) void softmax_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                       uint32_t n) {
    __shared__ float red[16];
    float m = -INFINITY;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, in[i]);
    m = block_max(m, red);
    float sum = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float e = expf(in[i] - m);
        out[i] = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    const float inv = 1.0f / sum;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] *= inv;
}

// ------------------------------------------------------------ rope
// cpu.rs:300-335: interleaved pairs, freq = 1/base^(2i/hd), theta = pos*freq
__global__ void rope_kernel(float *__restrict__ q, float *__restrict__ k, uint32_t pos, uint32_t hd, float base,
                            uint32_t nq, uint32_t nk) {
    const uint32_t half = hd / 2;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t total = (nq + nk) * half;
    if (i >= total) return;
    const uint32_t head = i / half, p = i % half;
    float *v = head < nq ? q + head * hd : k + (head - nq) * hd;
    // f32 values of the reference's f32 formula, each evaluated in double and
    // rounded once, so they match the host libm's rounded f32 results
    const float freq = (float)(1.0 / pow((double)base, (double)(2.0f * (float)p / (float)hd)));
    const float theta = (float)pos * freq;
    const float c = (float)cos((double)theta), sn = (float)sin((double)theta);
    const float x0 = v[2 * p], x1 = v[2 * p + 1];
    v[2 * p] = x0 * c - x1 * sn;
    v[2 * p + 1] = x0 * sn + x1 * c;
}

// ------------------------------------------------------------ matmul (f32)
// cpu.rs:163-222: C[m,n] = A[m,k] * B[k,n]; one thread per output, f32 FMA
// over k.  Not on the quantized hot path (kept for trait completeness).
__global__ void matmul_kernel(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ c,
                              uint32_t m, uint32_t n, uint32_t k) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
    if (j >= n || i >= m) return;
    float acc = 0.f;
    for (uint32_t p = 0; p < k; p++) acc += a[(size_t)i * k + p] * b[(size_t)p * n + j];
    c[(size_t)i * n + j] = acc;
}

// ------------------------------------------------------------ attention (trait)
// cpu.rs:462-500: one wave per position, lanes over the head dimension
__global__ void attn_score_kernel(const float *__restrict__ q, const float *__restrict__ kc, float *__restrict__ sc,
                                  uint32_t hd, uint32_t seq, uint32_t ho, uint32_t kvo, uint32_t kvs) {
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= seq) return;
    float acc = 0.f;
    for (uint32_t d = lane; d < hd; d += 64) acc += q[ho + d] * kc[(size_t)t * kvs + kvo + d];
    acc = wave_sum(acc);
    if (lane == 0) sc[t] = acc * (1.0f / sqrtf((float)hd));
}

// cpu.rs:502-539: thread per output dimension, sequential over positions
__global__ void attn_value_kernel(const float *__restrict__ w, const float *__restrict__ vc, float *__restrict__ out,
                                  uint32_t hd, uint32_t seq, uint32_t kvo, uint32_t kvs, uint32_t oo) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= hd) return;
    float acc = 0.f;
    for (uint32_t t = 0; t < seq; t++) acc += w[t] * vc[(size_t)t * kvs + kvo + d];
    out[oo + d] = acc;
}

// ------------------------------------------------------------ GQA decode attention
constexpr uint32_t kMaxSeqLds = 16384;
constexpr uint32_t kMaxHeadDim = 256;
// cache row width bound of attn_step_kernel: its prefetched rows (below
// 8192) then sit at byte offsets below 2^32
constexpr uint64_t kAttnMaxKvDim = 1u << 17;

// ------------------------------------------------------------ argmax
// argmax_ct (sampler.rs:142-163): an element replaces the best when the
// sign bit of (v - best) is clear.  For equal finite values that is +0, so the
// last maximal index wins; for equal infinities inf - inf is the default NaN,
// sign bit set on x86, so the first one stays (an all -inf input gives 0).
// NaN logits are outside this rule (the sequential scan is then not a
// maximum over any order).
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && (__builtin_isinf(v) ? i < bi : i > bi));
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ in, uint32_t n,
                                                      uint32_t *__restrict__ out) {
    __shared__ float rv[16];
    __shared__ uint32_t ri[16];
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x)
        if (better(in[i], i, bv, bi)) { bv = in[i]; bi = i; }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const uint32_t oi = __shfl_xor(bi, off, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) { rv[w] = bv; ri[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < (int)(blockDim.x >> 6); k++)
            if (better(rv[k], ri[k], bv, bi)) { bv = rv[k]; bi = ri[k]; }
        out[0] = n ? bi : 0u;
    }
}

int launch_argmax(hipStream_t s, const float *in, uint32_t n, uint32_t *out) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, in, n, out);
    return check_launch("argmax");
}

}  // namespace yule

using namespace yule;

// ------------------------------------------------------------ read probe
// Streams `n16` 16-byte words from `src` (grid-stride, one load in flight
// per lane, the fastest single-launch read pattern measured on gfx950) and
// writes one XOR of every word each workgroup read to part[blockIdx.x], so
// that the reads are observable and the host can check them.
__global__ __launch_bounds__(256) void read_probe_kernel(const uint4 *__restrict__ src, uint64_t n16,
                                                         uint32_t *__restrict__ part, uint32_t grid) {
    __shared__ uint32_t red[4];
    const uint64_t T = (uint64_t)grid * 256;   // grid size as an argument: no dispatch-packet load
    uint32_t acc = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += T) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// Variants of the read probe, to map what a single launch can read:
//   P = 0  grid-stride 16-byte words, U independent loads in flight per lane
//          (word i + j*T for j < U, T = threads in the grid);
//   P = 1  per-lane runs of U consecutive words (a 16*U-byte run per lane),
//          runs grid-strided;
//   P = 2  one contiguous chunk of ceil(n16 / grid) words per workgroup,
//          read with consecutive words across its lanes, U loads in flight
//          (the layout of a matvec whose workgroups stream whole rows).
// Every word is read exactly once in each variant, and the per-workgroup
// XOR is written as in read_probe_kernel.
template <int P, int U>
__global__ __launch_bounds__(256) void read_probe_var_kernel(const uint4 *__restrict__ src, uint64_t n16,
                                                             uint32_t *__restrict__ part, uint32_t grid) {
    __shared__ uint32_t red[4];
    uint32_t acc = 0;
    uint64_t base, step, end = n16;
    uint32_t lstride;   // distance between a lane's U words
    if (P == 0) {
        base = (uint64_t)blockIdx.x * 256 + threadIdx.x;
        lstride = grid * 256u;
        step = (uint64_t)lstride * U;
    } else if (P == 1) {
        base = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * U;
        lstride = 1;
        step = (uint64_t)grid * 256u * U;
    } else {
        const uint64_t chunk = (n16 + grid - 1) / grid;
        const uint64_t c0 = chunk * blockIdx.x;
        end = c0 + chunk < n16 ? c0 + chunk : n16;
        base = c0 + threadIdx.x;
        lstride = 256;
        step = 256u * U;
    }
    for (uint64_t i = base; i < end; i += step) {
        uint4 v[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const uint64_t w = i + (uint64_t)j * lstride;
            v[j] = w < end ? src[w] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < U; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// MFMA issue-rate probe: CH independent accumulator chains per wave, no
// memory traffic inside the loop (operands come from `in`, so nothing folds),
// one result per lane to `out`.  SHAPE 0: v_mfma_f32_16x16x32_f16 (16384
// flops), 1: v_mfma_f32_32x32x16_f16 (32768 flops).
typedef _Float16 probe_half8 __attribute__((ext_vector_type(8)));
typedef float probe_f4 __attribute__((ext_vector_type(4)));
typedef float probe_f16v __attribute__((ext_vector_type(16)));
template <int SHAPE, int CH>
__global__ __launch_bounds__(256) void mfma_probe_kernel(const uint4 *__restrict__ in, float *__restrict__ out,
                                                         uint32_t iters) {
    const uint4 av = in[threadIdx.x & 63u], bv = in[64 + (threadIdx.x & 63u)];
    const probe_half8 a = __builtin_bit_cast(probe_half8, av), b = __builtin_bit_cast(probe_half8, bv);
    float s = 0.f;
    if constexpr (SHAPE == 0) {
        // chains as separate variables (an array of them made the compiler
        // rotate accumulators through copies inside the loop)
        // distinct starting values, so that no two chains are the same computation
        const float z = __builtin_bit_cast(float, av.x) * 0.f;
        probe_f4 c0 = {z, z, z, z}, c1 = c0 + 1.f, c2 = c0 + 2.f, c3 = c0 + 3.f, c4 = c0 + 4.f, c5 = c0 + 5.f,
                 c6 = c0 + 6.f, c7 = c0 + 7.f;
        for (uint32_t it = 0; it < iters; it++) {
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c0, 0, 0, 0);
            if (CH > 1) c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c1, 0, 0, 0);
            if (CH > 2) c2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c2, 0, 0, 0);
            if (CH > 2) c3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c3, 0, 0, 0);
            if (CH > 4) c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c4, 0, 0, 0);
            if (CH > 4) c5 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c5, 0, 0, 0);
            if (CH > 4) c6 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c6, 0, 0, 0);
            if (CH > 4) c7 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c7, 0, 0, 0);
        }
        const probe_f4 t = ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7));
        s = t[0] + t[3];
    } else {
        probe_f16v acc[CH];
        const float z = __builtin_bit_cast(float, av.x) * 0.f;
#pragma unroll
        for (int j = 0; j < CH; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[j][e] = z + (float)j;
        for (uint32_t it = 0; it < iters; it++)
#pragma unroll
            for (int j = 0; j < CH; j++) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < CH; j++) s += acc[j][0] + acc[j][15];
    }
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

namespace yule {
__global__ __launch_bounds__(64) void empty_kernel() {}

int launch_empty(hipStream_t s) {
    hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, s);
    return check_launch("empty kernel");
}
}  // namespace yule

#define BE_OR_FAIL(be) \
    if (!(be)) return set_error(YULE_ERR_INVALID, "null backend")

static int f32buf(yule_hip_backend *be, yule_buffer h, size_t n_floats, float **p, const char *what,
                  size_t off_floats = 0) {
    void *v;
    int rc = get_buffer(be, h, n_floats * 4, &v, what, off_floats * 4);
    *p = (float *)v;
    return rc;
}

extern "C" {

int yule_hip_matmul(yule_hip_backend *be, yule_buffer a, yule_buffer b, yule_buffer out, uint32_t m, uint32_t n,
                    uint32_t k) {
    BE_OR_FAIL(be);
    float *pa, *pb, *pc;
    int rc;
    if ((rc = f32buf(be, a, (size_t)m * k, &pa, "matmul (a)")) || (rc = f32buf(be, b, (size_t)k * n, &pb, "matmul (b)")) ||
        (rc = f32buf(be, out, (size_t)m * n, &pc, "matmul (out)")))
        return rc;
    if (!m || !n) return YULE_OK;
    hipLaunchKernelGGL(matmul_kernel, dim3((n + 255) / 256, m), dim3(256), 0, be->stream, pa, pb, pc, m, n, k);
    return check_launch("matmul");
}

int yule_hip_softmax(yule_hip_backend *be, yule_buffer in, yule_buffer out, uint32_t size) {
    BE_OR_FAIL(be);
    float *pi, *po;
    int rc;
    if ((rc = f32buf(be, in, size, &pi, "softmax (in)")) || (rc = f32buf(be, out, size, &po, "softmax (out)")))
        return rc;
    if (!size) return YULE_OK;
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(1024), 0, be->stream, pi, po, size);
    return check_launch("softmax");
}

int yule_hip_rms_norm(yule_hip_backend *be, yule_buffer in, yule_buffer weight, yule_buffer out, uint32_t size,
                      float eps) {
    BE_OR_FAIL(be);
    float *pi, *pw, *po;
    int rc;
    if ((rc = f32buf(be, in, size, &pi, "rms_norm (in)")) || (rc = f32buf(be, weight, size, &pw, "rms_norm (weight)")) ||
        (rc = f32buf(be, out, size, &po, "rms_norm (out)")))
        return rc;
    if (!size) return YULE_OK;
    return launch_rms_norm(be->stream, pi, pw, po, size, eps);
}

int yule_hip_rope(yule_hip_backend *be, yule_buffer q, yule_buffer k, uint32_t pos, uint32_t head_dim, float freq_base,
                  uint32_t n_heads_q, uint32_t n_heads_k) {
    BE_OR_FAIL(be);
    if (head_dim == 0 || head_dim % 2) return set_error(YULE_ERR_INVALID, "rope: head_dim must be even and > 0");
    if (q == k) return set_error(YULE_ERR_INVALID, "rope: q and k alias");
    float *pq, *pk;
    int rc;
    if ((rc = f32buf(be, q, (size_t)n_heads_q * head_dim, &pq, "rope (q)")) ||
        (rc = f32buf(be, k, (size_t)n_heads_k * head_dim, &pk, "rope (k)")))
        return rc;
    const uint32_t total = (n_heads_q + n_heads_k) * (head_dim / 2);
    if (!total) return YULE_OK;
    hipLaunchKernelGGL(rope_kernel, dim3((total + 255) / 256), dim3(256), 0, be->stream, pq, pk, pos, head_dim,
                       freq_base, n_heads_q, n_heads_k);
    return check_launch("rope");
}

static int eltwise_entry(yule_hip_backend *be, int op, yule_buffer a, yule_buffer b, yule_buffer out, uint32_t size,
                         const char *what) {
    BE_OR_FAIL(be);
    float *pa, *pb = nullptr, *po;
    int rc;
    if ((rc = f32buf(be, a, size, &pa, what)) || (rc = f32buf(be, out, size, &po, what))) return rc;
    if (op != 0 && (rc = f32buf(be, b, size, &pb, what))) return rc;
    return launch_eltwise(be->stream, op, pa, pb, po, size);
}

int yule_hip_silu(yule_hip_backend *be, yule_buffer in, yule_buffer out, uint32_t size) {
    return eltwise_entry(be, 0, in, 0, out, size, "silu");
}
int yule_hip_element_mul(yule_hip_backend *be, yule_buffer a, yule_buffer b, yule_buffer out, uint32_t size) {
    return eltwise_entry(be, 1, a, b, out, size, "element_mul");
}
int yule_hip_add(yule_hip_backend *be, yule_buffer a, yule_buffer b, yule_buffer out, uint32_t size) {
    return eltwise_entry(be, 2, a, b, out, size, "add");
}
int yule_hip_silu_mul(yule_hip_backend *be, yule_buffer gate, yule_buffer up, yule_buffer out, uint32_t size) {
    return eltwise_entry(be, 3, gate, up, out, size, "silu_mul");
}

int yule_hip_attn_score(yule_hip_backend *be, yule_buffer q, yule_buffer k_cache, yule_buffer scores,
                        uint32_t head_dim, uint32_t seq_len, uint32_t head_offset, uint32_t kv_offset,
                        uint32_t kv_stride) {
    BE_OR_FAIL(be);
    float *pq, *pk, *ps;
    int rc;
    if (seq_len && kv_offset + head_dim > kv_stride)
        return set_error(YULE_ERR_INVALID, "attn_score: kv_offset + head_dim exceeds kv_stride");
    if ((rc = f32buf(be, q, (size_t)head_offset + head_dim, &pq, "attn_score (q)")) ||
        (rc = f32buf(be, k_cache, (size_t)seq_len * kv_stride, &pk, "attn_score (k_cache)")) ||
        (rc = f32buf(be, scores, seq_len, &ps, "attn_score (scores)")))
        return rc;
    if (!seq_len) return YULE_OK;
    hipLaunchKernelGGL(attn_score_kernel, dim3((seq_len + 3) / 4), dim3(256), 0, be->stream, pq, pk, ps, head_dim,
                       seq_len, head_offset, kv_offset, kv_stride);
    return check_launch("attn_score");
}

int yule_hip_attn_value(yule_hip_backend *be, yule_buffer weights, yule_buffer v_cache, yule_buffer out,
                        uint32_t head_dim, uint32_t seq_len, uint32_t kv_offset, uint32_t kv_stride,
                        uint32_t out_offset) {
    BE_OR_FAIL(be);
    float *pw, *pv, *po;
    int rc;
    if (seq_len && kv_offset + head_dim > kv_stride)
        return set_error(YULE_ERR_INVALID, "attn_value: kv_offset + head_dim exceeds kv_stride");
    if ((rc = f32buf(be, weights, seq_len, &pw, "attn_value (weights)")) ||
        (rc = f32buf(be, v_cache, (size_t)seq_len * kv_stride, &pv, "attn_value (v_cache)")) ||
        (rc = f32buf(be, out, (size_t)out_offset + head_dim, &po, "attn_value (out)")))
        return rc;
    if (!head_dim) return YULE_OK;
    hipLaunchKernelGGL(attn_value_kernel, dim3((head_dim + 255) / 256), dim3(256), 0, be->stream, pw, pv, po,
                       head_dim, seq_len, kv_offset, kv_stride, out_offset);
    return check_launch("attn_value");
}

int yule_hip_gqa_decode_attn(yule_hip_backend *be, yule_buffer q, yule_buffer k_cache, yule_buffer v_cache,
                             yule_buffer out, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                             uint32_t seq_len) {
    BE_OR_FAIL(be);
    if (!n_kv_heads || n_heads % n_kv_heads)
        return set_error(YULE_ERR_INVALID, "gqa_decode_attn: n_heads must be a multiple of n_kv_heads");
    if (!head_dim || head_dim > kMaxHeadDim)
        return set_error(YULE_ERR_INVALID, "gqa_decode_attn: head_dim must be in 1..256");
    const bool split = seq_len >= attn_split_min_seq() || seq_len > kMaxSeqLds;
    if (!seq_len || seq_len > 262144u)
        return set_error(YULE_ERR_INVALID, "gqa_decode_attn: seq_len must be in 1..262144");
    if (split && !split_attn_supported(n_heads, n_kv_heads, head_dim) && seq_len > kMaxSeqLds)
        return set_error(YULE_ERR_UNSUPPORTED, "gqa_decode_attn: above 16384 positions needs <= 8 query heads per KV head");
    if (!(split && split_attn_supported(n_heads, n_kv_heads, head_dim)) && (uint64_t)n_kv_heads * head_dim > kAttnMaxKvDim)
        return set_error(YULE_ERR_UNSUPPORTED, "gqa_decode_attn: n_kv_heads * head_dim above 131072");
    float *pq, *pk, *pv, *po;
    int rc;
    const size_t kv = (size_t)seq_len * n_kv_heads * head_dim;
    if ((rc = f32buf(be, q, (size_t)n_heads * head_dim, &pq, "gqa_decode_attn (q)")) ||
        (rc = f32buf(be, k_cache, kv, &pk, "gqa_decode_attn (k_cache)")) ||
        (rc = f32buf(be, v_cache, kv, &pv, "gqa_decode_attn (v_cache)")) ||
        (rc = f32buf(be, out, (size_t)n_heads * head_dim, &po, "gqa_decode_attn (out)")))
        return rc;
    if (head_dim % 4) return set_error(YULE_ERR_INVALID, "gqa_decode_attn: head_dim must be a multiple of 4");
    if (split && split_attn_supported(n_heads, n_kv_heads, head_dim)) {
        ScratchLease ws;   // held until both launches are enqueued
        if ((rc = get_scratch(be, split_scratch_bytes(n_heads, head_dim, seq_len), &ws))) return rc;
        return launch_attn_split(be->stream, pq, nullptr, nullptr, pk, pv, nullptr, nullptr, nullptr, po, ws.ptr,
                                 n_heads, n_kv_heads, head_dim, seq_len);
    }
    return launch_gqa_attn(be->stream, pq, pk, pv, po, n_heads, n_kv_heads, head_dim, seq_len);
}

int yule_hip_read_probe(yule_hip_backend *be, yule_buffer src, uint64_t bytes, yule_buffer partials,
                        uint32_t n_partials) {
    BE_OR_FAIL(be);
    if (bytes % 16 || n_partials == 0 || n_partials > 65536)
        return set_error(YULE_ERR_INVALID, "read_probe: bytes must be a multiple of 16, n_partials in 1..65536");
    void *ps, *pp;
    int rc;
    if ((rc = get_buffer(be, src, bytes, &ps, "read_probe (src)")) ||
        (rc = get_buffer(be, partials, (size_t)n_partials * 4, &pp, "read_probe (partials)")))
        return rc;
    hipLaunchKernelGGL(read_probe_kernel, dim3(n_partials), dim3(256), 0, be->stream, (const uint4 *)ps, bytes / 16,
                       (uint32_t *)pp, n_partials);
    return check_launch("read_probe");
}

int yule_hip_read_probe_variant(yule_hip_backend *be, yule_buffer src, uint64_t bytes, yule_buffer partials,
                                uint32_t n_partials, uint32_t pattern, uint32_t loads) {
    BE_OR_FAIL(be);
    if (bytes % 16 || n_partials == 0 || n_partials > 65536 || pattern > 2 ||
        (loads != 1 && loads != 2 && loads != 4 && loads != 8))
        return set_error(YULE_ERR_INVALID, "read_probe_variant: bytes a multiple of 16, n_partials in 1..65536, "
                                           "pattern 0..2, loads 1, 2, 4 or 8");
    void *ps, *pp;
    int rc;
    if ((rc = get_buffer(be, src, bytes, &ps, "read_probe_variant (src)")) ||
        (rc = get_buffer(be, partials, (size_t)n_partials * 4, &pp, "read_probe_variant (partials)")))
        return rc;
    typedef void (*Kern)(const uint4 *, uint64_t, uint32_t *, uint32_t);
    static const Kern k[3][4] = {
        {read_probe_var_kernel<0, 1>, read_probe_var_kernel<0, 2>, read_probe_var_kernel<0, 4>, read_probe_var_kernel<0, 8>},
        {read_probe_var_kernel<1, 1>, read_probe_var_kernel<1, 2>, read_probe_var_kernel<1, 4>, read_probe_var_kernel<1, 8>},
        {read_probe_var_kernel<2, 1>, read_probe_var_kernel<2, 2>, read_probe_var_kernel<2, 4>, read_probe_var_kernel<2, 8>}};
    const int li = loads == 1 ? 0 : loads == 2 ? 1 : loads == 4 ? 2 : 3;
    hipLaunchKernelGGL(k[pattern][li], dim3(n_partials), dim3(256), 0, be->stream, (const uint4 *)ps, bytes / 16,
                       (uint32_t *)pp, n_partials);
    return check_launch("read_probe_variant");
}

int yule_hip_mfma_probe(yule_hip_backend *be, yule_buffer in, yule_buffer out, uint32_t shape, uint32_t chains,
                        uint32_t n_wg, uint32_t iters) {
    BE_OR_FAIL(be);
    if (shape > 1 || (chains != 1 && chains != 2 && chains != 4 && chains != 8) || n_wg == 0 || n_wg > 65536 ||
        iters == 0)
        return set_error(YULE_ERR_INVALID, "mfma_probe: shape 0 or 1, chains 1, 2, 4 or 8, n_wg in 1..65536, iters > 0");
    void *pi, *po;
    int rc;
    if ((rc = get_buffer(be, in, 128 * 16, &pi, "mfma_probe (in)")) ||
        (rc = get_buffer(be, out, (size_t)n_wg * 256 * 4, &po, "mfma_probe (out)")))
        return rc;
    typedef void (*Kern)(const uint4 *, float *, uint32_t);
    static const Kern k[2][4] = {
        {mfma_probe_kernel<0, 1>, mfma_probe_kernel<0, 2>, mfma_probe_kernel<0, 4>, mfma_probe_kernel<0, 8>},
        {mfma_probe_kernel<1, 1>, mfma_probe_kernel<1, 2>, mfma_probe_kernel<1, 4>, mfma_probe_kernel<1, 8>}};
    const int ci = chains == 1 ? 0 : chains == 2 ? 1 : chains == 4 ? 2 : 3;
    hipLaunchKernelGGL(k[shape][ci], dim3(n_wg), dim3(256), 0, be->stream, (const uint4 *)pi, (float *)po, iters);
    return check_launch("mfma_probe");
}

int yule_hip_argmax(yule_hip_backend *be, yule_buffer in, uint32_t n, yule_buffer out) {
    BE_OR_FAIL(be);
    float *pi;
    void *po;
    int rc;
    if ((rc = f32buf(be, in, n, &pi, "argmax (in)")) || (rc = get_buffer(be, out, 4, &po, "argmax (out)"))) return rc;
    return launch_argmax(be->stream, pi, n, (uint32_t *)po);
}

}  // extern "C"

// ------------------------------------------------------------ runner kernels
namespace yule {

// Device control block of the decode runner: ctl[0] = position, ctl[1] =
// next input token (written by argmax_advance), ctl[2] = prompt length.
// Token of this step: prompt[pos] while pos < prompt length, else ctl[1].
__device__ __forceinline__ uint32_t step_token(const uint32_t *ctl, const uint32_t *prompt) {
    const uint32_t p = ctl[0];
    return p < ctl[2] ? prompt[p] : ctl[1];
}

__global__ void embed_step_kernel(uint32_t dtype, uint32_t bs, uint32_t bb, const uint8_t *__restrict__ table,
                                  const uint32_t *__restrict__ ctl, const uint32_t *__restrict__ prompt,
                                  uint32_t vocab, float *__restrict__ dst, uint32_t dim) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    uint32_t t = step_token(ctl, prompt);
    t = t < vocab ? t : vocab - 1;   // host-checked tokens are in range; clamp keeps reads inside the table
    const uint8_t *row = table + (size_t)t * (dim / bs) * bb;
    dst[i] = dequant_one(dtype, row + (i / bs) * bb, i % bs);
}

int launch_embed_step(hipStream_t s, uint32_t dtype, const uint8_t *table, const uint32_t *ctl, const uint32_t *prompt,
                      uint32_t vocab, float *dst, uint32_t dim) {
    uint32_t bs, bb;
    if (!quant_geometry(dtype, &bs, &bb)) return set_error(YULE_ERR_UNSUPPORTED, "embedding: unsupported dtype");
    hipLaunchKernelGGL(embed_step_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, dtype, bs, bb, table, ctl, prompt,
                       vocab, dst, dim);
    return check_launch("embedding");
}

// Fused decode attention step for one layer: RoPE of q and of the new k
// with the table row of the current position, the cache write of the new k
// and v (model_runner.rs:654-669), then GQA attention over positions
// 0..pos (model_runner.rs:679-758).  One workgroup per query head; the
// first head of each KV group writes that group's cache row, and every
// workgroup uses its own rotated copy of the new k / v for position pos, so
// no workgroup reads a cache row another one is writing.  Scores: a few
// lanes per position (float4 loads of the K row, shuffle-reduced); softmax
// over LDS; output: lanes over the head dimension, positions split across
// 4·NT/hd lane groups and combined through LDS.
// Without a control block (ctl == nullptr) it is plain GQA attention of the
// already-rotated q over cache rows 0..seq_host-1 (the ABI entry point).
// its workgroup size (256 measured 6.0 / 9.7 us at 64 / 384 positions against
// 6.4 / 7.5 us for 1024, TinyLlama shapes)
constexpr int kAttnThreads = 1024;

template <int NT>
__global__ __launch_bounds__(NT) void attn_step_kernel(const float *__restrict__ q, const float *__restrict__ k,
                                                       const float *__restrict__ v, float *__restrict__ kc,
                                                       float *__restrict__ vc, const float *__restrict__ cos_t,
                                                       const float *__restrict__ sin_t,
                                                       const uint32_t *__restrict__ ctl, float *__restrict__ out,
                                                       uint32_t group, uint32_t n_kv, uint32_t hd,
                                                       uint32_t seq_host) {
    constexpr int PRE = 8;                              // V rows per lane loaded before the softmax
    constexpr int KPRE = 8;                             // float4 of a K row per lane
    constexpr uint32_t NW = NT / 64;
    static_assert(kMaxHeadDim <= NT, "one lane per head dimension");
    extern __shared__ float scores[];                   // [pos + 1]
    __shared__ __align__(16) float qs[kMaxHeadDim], kn[kMaxHeadDim], vn[kMaxHeadDim];
    __shared__ __align__(16) float part[4 * NT];        // partial outputs: at most ng * hd = 4 * NT
    __shared__ float red[16], wstat[2 * NW];
    const uint32_t h = blockIdx.x, kvh = h / group, kvs = n_kv * hd, half = hd / 2, tid = threadIdx.x;
    const uint32_t lane = tid & 63, w = tid >> 6;
    const bool step = ctl != nullptr;
    const uint32_t seq = step ? ctl[0] + 1 : seq_host;
    const uint32_t pos = step ? seq - 1 : 0xFFFFFFFFu;   // row served from the local copy
    const float *kbase = kc + (size_t)kvh * hd, *vbase = vc + (size_t)kvh * hd;
    // output layout: each lane owns 4 consecutive dims (float4 of V) and the
    // positions g, g + ng, ...; the first PRE of them are loaded now, so
    // their latency overlaps the K loads and the softmax (the row at pos is
    // loaded and not used: it comes from the local copy).  Cache rows are
    // buffer loads whose range ends at row seq (lanes past it read zeros),
    // and a wave skips a prefetch whose positions all lie past seq (a
    // uniform branch): every issued load costs L1 address cycles, in range
    // or not.  The RoPE inputs are loaded last; the rotation then waits for
    // every prefetch too, which all fly at once.
    const uint32_t nd4 = hd / 4, ng = NT / nd4, d4 = tid % nd4, g = tid / nd4;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(w);
    // rows 0..seq-1 of this KV head (prefetched rows are below PRE * ng <=
    // 8192; the host keeps their offsets below 2^32 bytes)
    const uint64_t row_bytes = (uint64_t)kvs * sizeof(float);
    const uint64_t rec = (uint64_t)seq * row_bytes;
    const int nrec = (int)(rec < 0xFFFFFF00ull ? rec : 0xFFFFFF00ull);   // offset 0xFFFFFFF0 stays outside
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(kbase), (short)0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(vbase), (short)0, nrec, 0x00020000);
    auto row_load = [&](const __amdgpu_buffer_rsrc_t &rs_, uint32_t off) {
        const auto r = __builtin_amdgcn_raw_buffer_load_b128(rs_, off, 0, 0);
        return make_float4(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[2]), __uint_as_float(r[3]));
    };
    const uint32_t rb = (uint32_t)row_bytes, vstep = ng * rb, g0 = wv * 64 / nd4;   // g0: the wave's first group
    uint32_t voff = g * rb + d4 * 16u;
    asm("" : "+v"(voff));   // keeps the sums below from being re-associated into multiply-adds
    float4 vpre[PRE];
#pragma unroll
    for (int u = 0; u < PRE; u++) {
        vpre[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (g0 + u * ng < seq) vpre[u] = row_load(vrs, voff + u * vstep);
    }
    // scores: kl lanes per position (the smallest power of two giving each
    // lane at most KPRE float4 of the K row), NT / kl positions per pass; the
    // first pass's K rows are loaded now, before q is rotated
    uint32_t kl = 1;
    while (kl * KPRE < nd4) kl *= 2;
    const uint32_t kpass = NT / kl, kt = tid / kl, kp = tid % kl;
    float4 kpre[KPRE];
    uint32_t koff = kt * rb;
    asm("" : "+v"(koff));
#pragma unroll
    for (int u = 0; u < KPRE; u++) kpre[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (wv * 64 / kl < seq) {
#pragma unroll
        for (int u = 0; u < KPRE; u++) {
            const uint32_t c4 = kp + u * kl;   // columns past the row read zeros
            kpre[u] = row_load(krs, c4 < nd4 ? koff + c4 * 16u : 0xFFFFFFF0u);
        }
    }
    const float *qh = q + (size_t)h * hd;
    const float *kh = step ? k + (size_t)kvh * hd : qh, *vh = step ? v + (size_t)kvh * hd : qh;
    const float *ct = step ? cos_t + (size_t)pos * half : qh, *st = step ? sin_t + (size_t)pos * half : qh;
    const uint32_t ri = tid < half ? tid : half - 1, vi = tid < hd ? tid : hd - 1;
    const float rc = ct[ri], rs = st[ri], qx0 = qh[2 * ri], qx1 = qh[2 * ri + 1];
    const float kx0 = kh[2 * ri], kx1 = kh[2 * ri + 1], vx = vh[vi];
    if (step && tid < half) {
        qs[2 * tid] = qx0 * rc - qx1 * rs;
        qs[2 * tid + 1] = qx0 * rs + qx1 * rc;
        kn[2 * tid] = kx0 * rc - kx1 * rs;
        kn[2 * tid + 1] = kx0 * rs + kx1 * rc;
    }
    if (tid < hd) (step ? vn : qs)[tid] = vx;
    __syncthreads();
    if (step && h % group == 0) {
        float *krow = kc + (size_t)pos * kvs + kvh * hd, *vrow = vc + (size_t)pos * kvs + kvh * hd;
        for (uint32_t i = tid; i < hd; i += NT) { krow[i] = kn[i]; vrow[i] = vn[i]; }
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const float4 *qs4 = reinterpret_cast<const float4 *>(qs), *kn4 = reinterpret_cast<const float4 *>(kn);
    const float4 *vn4 = reinterpret_cast<const float4 *>(vn);
    // the registers holding row pos take the local copy (the cache row may
    // not be written yet); the loops below are then free of branches
    if (step) {
        if (kt == pos) {
#pragma unroll
            for (int u = 0; u < KPRE; u++) {
                const uint32_t c4 = kp + u * kl;
                kpre[u] = c4 < nd4 ? kn4[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int u = 0; u < PRE; u++)
            if (g + u * ng == pos) vpre[u] = vn4[d4];
    }
    // softmax weights: p_t = scores[t] * f[wave of t] * inv.  One pass:
    // scores hold exp(s_t - m_w) with m_w the max of wave w's positions, and
    // f[w] = exp(m_w - M) (lane w of every wave holds f[w]).  Several passes:
    // block-wide max and sum, f = 1.
    float fl = 1.f, inv;
    if (seq <= kpass) {
        // q . K_t over this lane's float4s kp + u * kl of the row (zeros past
        // it), summed over the kl lanes
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < KPRE; u++) {
            const uint32_t c4 = kp + u * kl;
            const float4 qv = qs4[c4 < nd4 ? c4 : nd4 - 1], kr = kpre[u];
            acc += qv.x * kr.x;
            acc += qv.y * kr.y;
            acc += qv.z * kr.z;
            acc += qv.w * kr.w;
        }
        const bool valid = kt < seq;
        const float sc = group_sum(acc, kl) * scale;
        const float mw = wave_max(valid ? sc : -INFINITY);
        const float e = valid ? expf(sc - mw) : 0.f;
        const float lw = wave_sum(kp == 0 ? e : 0.f);
        if (valid && kp == 0) scores[kt] = e;
        if (lane == 0) { wstat[2 * w] = mw; wstat[2 * w + 1] = lw; }
        __syncthreads();
        const float ml = lane < NW ? wstat[2 * lane] : -INFINITY;
        const float mx = wave_max(ml);
        fl = lane < NW ? expf(ml - mx) : 0.f;
        inv = 1.0f / wave_sum(lane < NW ? fl * wstat[2 * lane + 1] : 0.f);
    } else {
        float m = -INFINITY;
        for (uint32_t base = 0; base < seq; base += kpass) {
            const uint32_t t = base + kt;
            const float4 *kr = reinterpret_cast<const float4 *>(kbase + (size_t)(t < seq ? t : seq - 1) * kvs);
            float acc = 0.f;
#pragma unroll
            for (int u = 0; u < KPRE; u++) {
                const uint32_t c4 = kp + u * kl;
                if (c4 < nd4) {
                    const float4 kv = t == pos ? kn4[c4] : kr[c4], qv = qs4[c4];
                    acc += qv.x * kv.x;
                    acc += qv.y * kv.y;
                    acc += qv.z * kv.z;
                    acc += qv.w * kv.w;
                }
            }
            const float sc = group_sum(acc, kl) * scale;
            if (t < seq) {
                if (kp == 0) scores[t] = sc;
                m = fmaxf(m, sc);
            }
        }
        m = block_max(m, red);
        float sum = 0.f;
        for (uint32_t t = tid; t < seq; t += NT) {
            const float e = expf(scores[t] - m);
            scores[t] = e;
            sum += e;
        }
        inv = 1.0f / block_sum(sum, red);   // its barriers also publish scores[]
    }
    // the prefetched positions (lanes of groups g >= ng, which exist only when
    // hd / 4 does not divide NT, accumulate what is never written out)
    float4 o[4];
#pragma unroll
    for (int u = 0; u < 4; u++) o[u] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < PRE; u++) {
        const uint32_t t = g + u * ng, wt = t * kl / 64;
        const float f = __shfl(fl, wt < NW ? wt : NW - 1, 64);   // 1 beyond the first pass
        const float sv = scores[t < seq ? t : seq - 1];
        const float p = t < seq ? sv * f * inv : 0.f;
        const float4 vv = vpre[u];
        float4 &a = o[u & 3];
        a.x += p * vv.x; a.y += p * vv.y; a.z += p * vv.z; a.w += p * vv.w;
    }
    // positions past the preloaded ones (several passes only): four
    // independent accumulators keep four V loads in flight per lane
    if (g < ng) {
        uint32_t t = g + PRE * ng;
        for (; t + 3 * ng < seq; t += 4 * ng) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t tt = t + u * ng;
                const float *vr = tt == pos ? vn : vbase + (size_t)tt * kvs;
                const float4 vv = reinterpret_cast<const float4 *>(vr)[d4];
                const float p = scores[tt] * inv;
                o[u].x += p * vv.x; o[u].y += p * vv.y; o[u].z += p * vv.z; o[u].w += p * vv.w;
            }
        }
        for (; t < seq; t += ng) {
            const float *vr = t == pos ? vn : vbase + (size_t)t * kvs;
            const float4 vv = reinterpret_cast<const float4 *>(vr)[d4];
            const float p = scores[t] * inv;
            o[0].x += p * vv.x; o[0].y += p * vv.y; o[0].z += p * vv.z; o[0].w += p * vv.w;
        }
    }
    float4 acc4;
    acc4.x = (o[0].x + o[1].x) + (o[2].x + o[3].x);
    acc4.y = (o[0].y + o[1].y) + (o[2].y + o[3].y);
    acc4.z = (o[0].z + o[1].z) + (o[2].z + o[3].z);
    acc4.w = (o[0].w + o[1].w) + (o[2].w + o[3].w);
    // combine the lane groups: when hd / 4 divides 64, the groups inside a
    // wave first by shuffles, leaving NW partials per dim; otherwise all ng
    const bool in_wave = 64 % nd4 == 0;
    if (in_wave) {
        acc4.x = strided_sum(acc4.x, nd4);
        acc4.y = strided_sum(acc4.y, nd4);
        acc4.z = strided_sum(acc4.z, nd4);
        acc4.w = strided_sum(acc4.w, nd4);
        if (lane < nd4) reinterpret_cast<float4 *>(part)[w * nd4 + d4] = acc4;
    } else if (g < ng) {
        reinterpret_cast<float4 *>(part)[g * nd4 + d4] = acc4;
    }
    __syncthreads();
    const uint32_t nparts = in_wave ? NW : ng;
    for (uint32_t i = tid; i < hd; i += NT) {
        float acc = 0.f;
#pragma unroll 16
        for (uint32_t j = 0; j < nparts; j++) acc += part[j * hd + i];
        out[(size_t)h * hd + i] = acc;
    }
}

// ------------------------------------------------------------ split-KV attention
// Flash-decoding for long contexts (the reference's flash_decode_split.comp /
// flash_decode_reduce.comp, vulkan/mod.rs:179-263): phase 1 runs one
// workgroup per (KV head, chunk of positions) and serves all G query heads
// of the group from one pass over the chunk's K and V rows, writing per head
// the chunk maximum m_c, the sum l_c = sum_t exp(s_t - m_c) and the
// unnormalised output o_c = sum_t exp(s_t - m_c) V_t; phase 2 combines the
// chunks: out = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c.
// The chunk length is a function of the sequence length alone (split_chunk),
// evaluated on the device in decode steps, so a captured graph sized for
// max_seq serves every position; workgroups past the last chunk exit.
constexpr uint32_t kSplitMaxGroup = 8;      // query heads per KV head
constexpr uint32_t kSplitMinChunk = 64;
constexpr uint32_t kSplitMaxChunks = 4096;  // chunks per head the combine handles (262144 positions)

// 256 positions per chunk once that still gives two workgroups per CU, else
// 128, else 64
__host__ __device__ inline uint32_t split_chunk(uint32_t seq, uint32_t n_kv) {
    const uint32_t target = 512;
    if (n_kv * ((seq + 255) / 256) >= target) return 256;
    if (n_kv * ((seq + 127) / 128) >= target) return 128;
    return 64;
}

template <uint32_t G>
__global__ __launch_bounds__(256) void attn_split_kernel(const float *__restrict__ q, const float *__restrict__ k,
                                                         const float *__restrict__ v, float *__restrict__ kc,
                                                         float *__restrict__ vc, const float *__restrict__ cos_t,
                                                         const float *__restrict__ sin_t,
                                                         const uint32_t *__restrict__ ctl, float *__restrict__ part,
                                                         float2 *__restrict__ ml, uint32_t n_kv, uint32_t hd,
                                                         uint32_t seq_host, uint32_t max_chunks) {
    __shared__ __align__(16) float qs[G * kMaxHeadDim];
    __shared__ __align__(16) float kn[kMaxHeadDim], vn[kMaxHeadDim];
    __shared__ float pl[G * 256];
    __shared__ __align__(16) float acc_lds[G * 1024];
    __shared__ float red[4 * G];
    const uint32_t kvh = blockIdx.x, chunk = blockIdx.y, tid = threadIdx.x;
    const bool step = ctl != nullptr;
    const uint32_t seq = step ? ctl[0] + 1 : seq_host;
    const uint32_t pos = step ? seq - 1 : 0xFFFFFFFFu;
    const uint32_t C = split_chunk(seq, n_kv), c0 = chunk * C;
    if (c0 >= seq) return;   // uniform over the workgroup
    const uint32_t len = min(C, seq - c0), kvs = n_kv * hd, half = hd / 2, h0 = kvh * G;
    const bool own = step && pos - c0 < len;   // this chunk holds the new row
    if (!step) {
        for (uint32_t i = tid; i < G * hd; i += 256) qs[i] = q[(size_t)h0 * hd + i];
    } else {
        for (uint32_t i = tid; i < G * half; i += 256) {
            const uint32_t g = i / half, j = i % half;
            const float c = cos_t[(size_t)pos * half + j], sn = sin_t[(size_t)pos * half + j];
            const float *qh = q + (size_t)(h0 + g) * hd;
            const float x0 = qh[2 * j], x1 = qh[2 * j + 1];
            qs[g * hd + 2 * j] = x0 * c - x1 * sn;
            qs[g * hd + 2 * j + 1] = x0 * sn + x1 * c;
        }
        if (own) {
            const float *kh = k + (size_t)kvh * hd, *vh = v + (size_t)kvh * hd;
            for (uint32_t j = tid; j < half; j += 256) {
                const float c = cos_t[(size_t)pos * half + j], sn = sin_t[(size_t)pos * half + j];
                const float x0 = kh[2 * j], x1 = kh[2 * j + 1];
                kn[2 * j] = x0 * c - x1 * sn;
                kn[2 * j + 1] = x0 * sn + x1 * c;
            }
            for (uint32_t j = tid; j < hd; j += 256) vn[j] = vh[j];
        }
    }
    __syncthreads();
    if (own) {   // the only workgroup that touches row pos of this KV head
        float *krow = kc + (size_t)pos * kvs + kvh * hd, *vrow = vc + (size_t)pos * kvs + kvh * hd;
        for (uint32_t j = tid; j < hd; j += 256) { krow[j] = kn[j]; vrow[j] = vn[j]; }
    }
    // scores: LP = 256 / C adjacent lanes per position, each over a residue
    // class of the row's float4s, combined by lane shuffles
    const uint32_t LP = 256 / C, t = tid / LP, sub = tid % LP, nd4 = hd / 4;
    const bool valid = t < len;
    const uint32_t p = c0 + t;
    float acc[G];
#pragma unroll
    for (uint32_t g = 0; g < G; g++) acc[g] = 0.f;
    if (valid) {
        const float4 *kr = reinterpret_cast<const float4 *>(p == pos ? kn : kc + (size_t)p * kvs + kvh * hd);
        for (uint32_t c4 = sub; c4 < nd4; c4 += LP) {
            const float4 kv = kr[c4];
#pragma unroll
            for (uint32_t g = 0; g < G; g++) {
                const float4 qv = reinterpret_cast<const float4 *>(qs + g * hd)[c4];
                acc[g] += qv.x * kv.x;
                acc[g] += qv.y * kv.y;
                acc[g] += qv.z * kv.z;
                acc[g] += qv.w * kv.w;
            }
        }
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const uint32_t lane = tid & 63, w = tid >> 6;
    float sc[G], m[G], l[G];
#pragma unroll
    for (uint32_t g = 0; g < G; g++) {
        for (uint32_t off = 1; off < LP; off <<= 1) acc[g] += __shfl_xor(acc[g], off, 64);
        sc[g] = valid ? acc[g] * scale : -INFINITY;
        m[g] = wave_max(sc[g]);
    }
    if (lane == 0) {
#pragma unroll
        for (uint32_t g = 0; g < G; g++) red[w * G + g] = m[g];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t g = 0; g < G; g++) {
        m[g] = fmaxf(fmaxf(red[g], red[G + g]), fmaxf(red[2 * G + g], red[3 * G + g]));
        const float e = valid ? expf(sc[g] - m[g]) : 0.f;
        if (valid && sub == 0) pl[g * 256 + t] = e;
        l[g] = wave_sum(sub == 0 ? e : 0.f);
    }
    __syncthreads();   // every lane has read red[] (maxima); pl[] is complete
    if (lane == 0) {
#pragma unroll
        for (uint32_t g = 0; g < G; g++) red[w * G + g] = l[g];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t g = 0; g < G; g++) l[g] = (red[g] + red[G + g]) + (red[2 * G + g] + red[3 * G + g]);
    // unnormalised output: lanes own a float4 of dims and a residue class of
    // the chunk's positions; every V row loaded serves all G heads
    const uint32_t ng = 256 / nd4, d4 = tid % nd4, gi = tid / nd4;
    float4 o[G];
#pragma unroll
    for (uint32_t g = 0; g < G; g++) o[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (gi < ng) {
        uint32_t tt = gi;
        for (; tt + ng < len; tt += 2 * ng) {
            const uint32_t pa = c0 + tt, pb = pa + ng;
            const float4 va = reinterpret_cast<const float4 *>(pa == pos ? vn : vc + (size_t)pa * kvs + kvh * hd)[d4];
            const float4 vb = reinterpret_cast<const float4 *>(pb == pos ? vn : vc + (size_t)pb * kvs + kvh * hd)[d4];
#pragma unroll
            for (uint32_t g = 0; g < G; g++) {
                const float wa = pl[g * 256 + tt], wb = pl[g * 256 + tt + ng];
                o[g].x += wa * va.x; o[g].y += wa * va.y; o[g].z += wa * va.z; o[g].w += wa * va.w;
                o[g].x += wb * vb.x; o[g].y += wb * vb.y; o[g].z += wb * vb.z; o[g].w += wb * vb.w;
            }
        }
        if (tt < len) {
            const uint32_t pa = c0 + tt;
            const float4 va = reinterpret_cast<const float4 *>(pa == pos ? vn : vc + (size_t)pa * kvs + kvh * hd)[d4];
#pragma unroll
            for (uint32_t g = 0; g < G; g++) {
                const float wa = pl[g * 256 + tt];
                o[g].x += wa * va.x; o[g].y += wa * va.y; o[g].z += wa * va.z; o[g].w += wa * va.w;
            }
        }
#pragma unroll
        for (uint32_t g = 0; g < G; g++) reinterpret_cast<float4 *>(acc_lds + (gi * G + g) * hd)[d4] = o[g];
    }
    __syncthreads();
    for (uint32_t i = tid; i < G * hd; i += 256) {
        const uint32_t g = i / hd, d = i % hd;
        float a = 0.f;
        for (uint32_t j = 0; j < ng; j++) a += acc_lds[(j * G + g) * hd + d];
        part[((size_t)(h0 + g) * max_chunks + chunk) * hd + d] = a;
    }
    if (tid < G) ml[(size_t)(h0 + tid) * max_chunks + chunk] = make_float2(m[tid], l[tid]);
}

// Phase 2: one workgroup per query head.
__global__ __launch_bounds__(256) void attn_combine_kernel(const float *__restrict__ part,
                                                           const float2 *__restrict__ ml,
                                                           const uint32_t *__restrict__ ctl, float *__restrict__ out,
                                                           uint32_t n_kv, uint32_t hd, uint32_t seq_host,
                                                           uint32_t max_chunks) {
    __shared__ float wt[kSplitMaxChunks];
    __shared__ float red[16];
    const uint32_t h = blockIdx.x, tid = threadIdx.x;
    const uint32_t seq = ctl ? ctl[0] + 1 : seq_host;
    const uint32_t C = split_chunk(seq, n_kv), n_ch = (seq + C - 1) / C;
    const float2 *mh = ml + (size_t)h * max_chunks;
    float mx = -INFINITY;
    for (uint32_t c = tid; c < n_ch; c += 256) mx = fmaxf(mx, mh[c].x);
    mx = block_max(mx, red);
    float lsum = 0.f;
    for (uint32_t c = tid; c < n_ch; c += 256) {
        const float2 v = mh[c];
        const float e = expf(v.x - mx);
        wt[c] = e;
        lsum += e * v.y;
    }
    lsum = block_sum(lsum, red);   // its barriers also publish wt[]
    const float inv = 1.0f / lsum;
    const float *ph = part + (size_t)h * max_chunks * hd;
    for (uint32_t d = tid; d < hd; d += 256) {
        float a0 = 0.f, a1 = 0.f;
        uint32_t c = 0;
        for (; c + 1 < n_ch; c += 2) {
            a0 += wt[c] * ph[(size_t)c * hd + d];
            a1 += wt[c + 1] * ph[(size_t)(c + 1) * hd + d];
        }
        if (c < n_ch) a0 += wt[c] * ph[(size_t)c * hd + d];
        out[(size_t)h * hd + d] = (a0 + a1) * inv;
    }
}

// ------------------------------------------------------------ chunked attention
// Decode-step attention over an already-rotated q and a cache that already
// holds row pos (the Q/K/V launch applied RoPE and wrote it, kEpiRope):
// GQA attention of query head h over positions 0..pos (model_runner.rs:
// 679-758), spread over one workgroup per (query head, chunk of C = 4096/HD
// positions) so that short contexts occupy many CUs, with the chunks of a
// head combined inside the same launch: each workgroup writes its chunk's
// maximum m_c, sum l_c = sum exp(s - m_c) and unnormalised output
// o_c = sum exp(s - m_c) V, then takes a ticket from the head's counter; the
// last one combines out = sum exp(m_c - M) o_c / sum exp(m_c - M) l_c over
// the chunks in order and resets the counter (so a replayed graph finds it
// at zero).  A sequence of one chunk writes out directly.
// The cache rows of the chunk, q and the V rows are loaded before the
// control block is read: every load is in flight at once, from clamped row
// indices (rows past max_rows are never touched).
constexpr uint32_t kChunkMaxCombine = 1024;   // chunks per head (the runner uses it below 16384 positions)
// one head's ticket per 128-byte line: the heads' atomics do not queue on one
// line; likewise each chunk's (m, l) pair
constexpr uint32_t kTicketStride = 32, kMlStride = 16;

// threads per chunk workgroup (128, 256 or 512; YULE_ATTN_CHUNK_THREADS):
// the chunk length follows, 16 NT / HD positions
static uint32_t chunk_threads() {
    static const int env = env_int("YULE_ATTN_CHUNK_THREADS", 256);
    return env == 128 || env == 512 ? (uint32_t)env : 256u;
}

template <uint32_t HD, uint32_t NT>
__global__ __launch_bounds__(NT) void attn_chunk_kernel(
    // the leading 14 dwords arrive preloaded in SGPRs
    const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
    const uint32_t *__restrict__ ctl, uint32_t group, uint32_t n_kv, uint32_t seq_host, uint32_t max_rows,
    float *__restrict__ out, float *__restrict__ part, float2 *__restrict__ ml, uint32_t *__restrict__ ticket,
    uint32_t max_chunks) {
    constexpr uint32_t ND4 = HD / 4, NW = NT / 64;
    constexpr uint32_t LPP = HD / 16;          // lanes per position in the scores, four float4 each
    constexpr uint32_t C = NT / LPP;           // positions per chunk
    constexpr uint32_t NG = NT / ND4;          // position groups in the output
    constexpr uint32_t PPG = C / NG;           // positions per group
    static_assert(C % NG == 0 && LPP >= 2 && LPP <= 8, "chunk geometry");
    __shared__ float ps[C];
    __shared__ float red[8];
    __shared__ float4 ored[NW][ND4];
    __shared__ uint32_t last;
    __shared__ float fcs[kChunkMaxCombine], lcs[kChunkMaxCombine];
    const uint32_t h = blockIdx.x, ch = blockIdx.y, tid = threadIdx.x;
    const uint32_t kvh = h / group, kvs4 = n_kv * ND4, c0 = ch * C;
    const float4 *q4 = reinterpret_cast<const float4 *>(q) + (size_t)h * ND4;
    const float4 *kc4 = reinterpret_cast<const float4 *>(kc) + (size_t)kvh * ND4;
    const float4 *vc4 = reinterpret_cast<const float4 *>(vc) + (size_t)kvh * ND4;
    // scores: position t of the chunk, float4s sub, sub + LPP, ... of the row
    const uint32_t t = tid / LPP, sub = tid % LPP;
    const uint32_t krow = c0 + t < max_rows ? c0 + t : max_rows - 1;
    float4 kv[4], qv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        kv[u] = kc4[(size_t)krow * kvs4 + sub + u * LPP];
        qv[u] = q4[sub + u * LPP];
    }
    // output: float4 d4 of the dims, positions pg * PPG + u
    const uint32_t d4 = tid % ND4, pg = tid / ND4;
    float4 vv[PPG];
#pragma unroll
    for (uint32_t u = 0; u < PPG; u++) {
        const uint32_t r = c0 + pg * PPG + u;
        vv[u] = vc4[(size_t)(r < max_rows ? r : max_rows - 1) * kvs4 + d4];
    }
    const uint32_t seq = ctl ? ctl[0] + 1 : seq_host;
    if (c0 >= seq) return;   // uniform: a chunk past the sequence (the grid covers max_rows)
    const uint32_t n_ch = (seq + C - 1) / C;
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        acc += qv[u].x * kv[u].x;
        acc += qv[u].y * kv[u].y;
        acc += qv[u].z * kv[u].z;
        acc += qv[u].w * kv[u].w;
    }
    const bool valid = c0 + t < seq;
    const float sc = valid ? group_sum(acc, LPP) * (1.0f / sqrtf((float)HD)) : -INFINITY;
    const float m = block_max(sc, red);
    const float e = valid ? expf(sc - m) : 0.f;
    if (sub == 0) ps[t] = e;
    const float l = block_sum(sub == 0 ? e : 0.f, red);   // its barriers also publish ps[]
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (uint32_t u = 0; u < PPG; u++) {
        const float p = ps[pg * PPG + u];
        o.x += p * vv[u].x; o.y += p * vv[u].y; o.z += p * vv[u].z; o.w += p * vv[u].w;
    }
    // groups inside a wave (lanes d4 + ND4 * j), then the waves
#pragma unroll
    for (uint32_t off = ND4; off < 64; off <<= 1) {
        o.x += __shfl_xor(o.x, off, 64); o.y += __shfl_xor(o.y, off, 64);
        o.z += __shfl_xor(o.z, off, 64); o.w += __shfl_xor(o.w, off, 64);
    }
    const uint32_t lane = tid & 63u, w = tid >> 6;
    if (lane < ND4) ored[w][lane] = o;
    __syncthreads();
    // the waves' sums in a fixed order: pairwise for four waves, then on in
    // wave order
    auto wave_total = [&](uint32_t d) {
        float4 t;
        if constexpr (NW >= 4) {
            const float4 a = ored[0][d], b = ored[1][d], c = ored[2][d], e = ored[3][d];
            t = make_float4((a.x + b.x) + (c.x + e.x), (a.y + b.y) + (c.y + e.y), (a.z + b.z) + (c.z + e.z),
                            (a.w + b.w) + (c.w + e.w));
        } else {
            const float4 a = ored[0][d], b = ored[1][d];
            t = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
        }
#pragma unroll
        for (uint32_t i = 4; i < NW; i++) {
            const float4 c = ored[i][d];
            t.x += c.x; t.y += c.y; t.z += c.z; t.w += c.w;
        }
        return t;
    };
    if (n_ch == 1) {   // the whole sequence in this chunk
        if (tid < ND4) {
            const float inv = 1.0f / l;
            const float4 a = wave_total(tid);
            reinterpret_cast<float4 *>(out)[(size_t)h * ND4 + tid] = make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
        }
        return;
    }
    // Cross-workgroup hand-off without cache-wide fences: the partials are
    // written and read with device-scope atomic stores and loads (coherent at
    // device scope, i.e. not held in one XCD's L2), the writing wave waits for
    // those stores to complete before the ticket (a device-scope atomic) is
    // taken, and the last workgroup reads the other chunks' partials with
    // device-scope loads after its ticket: the device-scope release and
    // acquire sequences minus their cache-wide writeback and invalidate,
    // which only non-atomic data would need.  (Agent-scope
    // fences here write back and invalidate the whole L2 of the XCD: measured
    // 1130 against 1510 decode tok/s.)
    auto st = [](float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto ld = [](const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    if (tid < ND4) {
        const float4 a = wave_total(tid);
        float *pp = part + ((size_t)h * max_chunks + ch) * HD + 4 * tid;
        st(pp + 0, a.x);
        st(pp + 1, a.y);
        st(pp + 2, a.z);
        st(pp + 3, a.w);
    }
    float *mlp = reinterpret_cast<float *>(ml + ((size_t)h * max_chunks + ch) * kMlStride);
    if (tid == 0) {
        st(mlp, m);
        st(mlp + 1, l);
    }
    // every store above is from wave 0 (HD / 4 <= 32 lanes, and lane 0), as
    // is the ticket: that wave waits until its stores have completed, then
    // takes the ticket (the signal fences keep the compiler from moving
    // memory operations across the wait)
    if (tid < 64) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (tid == 0)
            last = __hip_atomic_fetch_add(ticket + h * kTicketStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   n_ch - 1;
    }
    __syncthreads();
    if (!last) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // combine: every (m, l) pair and, for up to kPre chunks, the thread's
    // partial outputs are loaded at once (one memory round trip)
    const float *mh = reinterpret_cast<const float *>(ml + (size_t)h * max_chunks * kMlStride);
    const float *ph = part + (size_t)h * max_chunks * HD;
    constexpr uint32_t kPre = 8;
    const uint32_t dd = tid < HD ? tid : 0u;
    float pv[kPre];
#pragma unroll
    for (uint32_t c = 0; c < kPre; c++) pv[c] = ld(ph + (size_t)(c < n_ch ? c : 0u) * HD + dd);
    float mm = -INFINITY;
    for (uint32_t c = tid; c < n_ch; c += NT) {
        const float mc = ld(mh + 2 * kMlStride * c), lc = ld(mh + 2 * kMlStride * c + 1);
        fcs[c] = mc;
        lcs[c] = lc;
        mm = fmaxf(mm, mc);
    }
    const float M = block_max(mm, red);
    float lsum = 0.f;
    for (uint32_t c = tid; c < n_ch; c += NT) {
        const float f = expf(fcs[c] - M);
        fcs[c] = f;
        lsum += f * lcs[c];
    }
    const float L = block_sum(lsum, red);   // its barriers also publish fcs[]
    if (tid < HD) {
        float a = 0.f;
#pragma unroll
        for (uint32_t c = 0; c < kPre; c++)
            if (c < n_ch) a += fcs[c] * pv[c];
        for (uint32_t c = kPre; c < n_ch; c++) a += fcs[c] * ld(ph + (size_t)c * HD + tid);
        out[(size_t)h * HD + tid] = a / L;
    }
    if (tid == 0) __hip_atomic_store(ticket + h * kTicketStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// chunk length of attn_chunk_kernel for a head size (0: not served)
uint32_t attn_chunk_len(uint32_t hd) { return hd == 64 || hd == 128 ? chunk_threads() * 16u / hd : 0u; }

size_t attn_chunk_scratch_bytes(uint32_t n_heads, uint32_t hd, uint32_t max_rows) {
    const uint32_t C = attn_chunk_len(hd);
    if (!C) return 0;
    const size_t mc = (max_rows + C - 1) / C;
    return (size_t)n_heads * mc * hd * sizeof(float) + (size_t)n_heads * mc * kMlStride * sizeof(float2) +
           (size_t)n_heads * kTicketStride * sizeof(uint32_t) + 256;
}

// scratch: partials, (m, l) pairs, then the per-head tickets, which must be
// zero before the first launch (they return to zero after every launch)
int launch_attn_chunks(hipStream_t s, const float *q, const float *kc, const float *vc, const uint32_t *ctl,
                       float *out, void *scratch, uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t max_rows,
                       uint32_t seq_host) {
    const uint32_t C = attn_chunk_len(hd);
    if (!C || !n_kv || n_heads % n_kv) return set_error(YULE_ERR_UNSUPPORTED, "chunked attention: head size");
    const uint32_t mc = (max_rows + C - 1) / C;
    if (mc > kChunkMaxCombine) return set_error(YULE_ERR_INVALID, "chunked attention: sequence too long");
    float *part = static_cast<float *>(scratch);
    float2 *ml = reinterpret_cast<float2 *>(part + (size_t)n_heads * mc * hd);
    uint32_t *ticket = reinterpret_cast<uint32_t *>(ml + (size_t)n_heads * mc * kMlStride);
    const dim3 grid(n_heads, mc);
#define YULE_CHUNK_LAUNCH(HD, NT)                                                                                  \
    hipLaunchKernelGGL((attn_chunk_kernel<HD, NT>), grid, dim3(NT), 0, s, q, kc, vc, ctl, n_heads / n_kv, n_kv,   \
                       seq_host, max_rows, out, part, ml, ticket, mc)
    const uint32_t nt = chunk_threads();
    if (hd == 64) {
        if (nt == 128) YULE_CHUNK_LAUNCH(64, 128);
        else if (nt == 512) YULE_CHUNK_LAUNCH(64, 512);
        else YULE_CHUNK_LAUNCH(64, 256);
    } else {
        if (nt == 128) YULE_CHUNK_LAUNCH(128, 128);
        else if (nt == 512) YULE_CHUNK_LAUNCH(128, 512);
        else YULE_CHUNK_LAUNCH(128, 256);
    }
#undef YULE_CHUNK_LAUNCH
    return check_launch("attn_chunks");
}

bool split_attn_supported(uint32_t n_heads, uint32_t n_kv, uint32_t hd) {
    return n_kv && n_heads % n_kv == 0 && n_heads / n_kv <= kSplitMaxGroup && hd % 4 == 0 && hd <= kMaxHeadDim;
}

// Sequence length from which attention runs split-KV (environment
// YULE_ATTN_SPLIT_MIN, default 512); shorter sequences run one workgroup
// per query head (attn_step_kernel).
uint32_t attn_split_min_seq() {
    const char *e = getenv("YULE_ATTN_SPLIT_MIN");
    const long v = e ? strtol(e, nullptr, 10) : 0;
    return v > 0 ? (uint32_t)v : 512u;
}

// grid chunks for a launch whose sequence length is at most `seq_cap`
uint32_t split_max_chunks(uint32_t seq_cap) { return (seq_cap + kSplitMinChunk - 1) / kSplitMinChunk; }

size_t split_scratch_bytes(uint32_t n_heads, uint32_t hd, uint32_t seq_cap) {
    const size_t mc = split_max_chunks(seq_cap);
    return (size_t)n_heads * mc * hd * sizeof(float) + (size_t)n_heads * mc * sizeof(float2) + 256;
}

int launch_attn_split(hipStream_t s, const float *q, const float *k, const float *v, float *kc, float *vc,
                      const float *cos_t, const float *sin_t, const uint32_t *ctl, float *out, void *scratch,
                      uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t seq_cap) {
    const uint32_t mc = split_max_chunks(seq_cap);
    if (mc > kSplitMaxChunks) return set_error(YULE_ERR_INVALID, "split attention: sequence too long");
    float *part = static_cast<float *>(scratch);
    float2 *ml = reinterpret_cast<float2 *>(part + (size_t)n_heads * mc * hd);
    const uint32_t seq_host = ctl ? 0u : seq_cap;
    const dim3 grid(n_kv, ctl ? mc : (seq_cap + split_chunk(seq_cap, n_kv) - 1) / split_chunk(seq_cap, n_kv));
#define YULE_SPLIT_CASE(G)                                                                                       \
    case G:                                                                                                      \
        hipLaunchKernelGGL(attn_split_kernel<G>, grid, dim3(256), 0, s, q, k, v, kc, vc, cos_t, sin_t, ctl, part, \
                           ml, n_kv, hd, seq_host, mc);                                                          \
        break;
    switch (n_heads / n_kv) {
        YULE_SPLIT_CASE(1) YULE_SPLIT_CASE(2) YULE_SPLIT_CASE(3) YULE_SPLIT_CASE(4)
        YULE_SPLIT_CASE(5) YULE_SPLIT_CASE(6) YULE_SPLIT_CASE(7) YULE_SPLIT_CASE(8)
    default: return set_error(YULE_ERR_UNSUPPORTED, "split attention: more than 8 query heads per KV head");
    }
#undef YULE_SPLIT_CASE
    int rc = check_launch("attn_split");
    if (rc) return rc;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads), dim3(256), 0, s, part, ml, ctl, out, n_kv, hd, seq_host,
                       mc);
    return check_launch("attn_combine");
}

int launch_attn_step(hipStream_t s, const float *q, const float *k, const float *v, float *kc, float *vc,
                     const float *cos_t, const float *sin_t, const uint32_t *ctl, float *out, uint32_t n_heads,
                     uint32_t n_kv, uint32_t hd, uint32_t max_seq) {
    if ((uint64_t)n_kv * hd > kAttnMaxKvDim)
        return set_error(YULE_ERR_UNSUPPORTED, "attention: n_kv_heads * head_dim above 131072");
    const size_t lds = (size_t)max_seq * sizeof(float);
    hipLaunchKernelGGL(attn_step_kernel<kAttnThreads>, dim3(n_heads), dim3(kAttnThreads), lds, s, q, k, v, kc, vc,
                       cos_t, sin_t, ctl, out, n_heads / n_kv, n_kv, hd, 0u);
    return check_launch("attn_step");
}

int launch_gqa_attn(hipStream_t s, const float *q, const float *kc, const float *vc, float *out, uint32_t n_heads,
                    uint32_t n_kv, uint32_t hd, uint32_t seq) {
    if ((uint64_t)n_kv * hd > kAttnMaxKvDim)
        return set_error(YULE_ERR_UNSUPPORTED, "gqa_decode_attn: n_kv_heads * head_dim above 131072");
    const size_t lds = (size_t)seq * sizeof(float);
    float *kcw = const_cast<float *>(kc), *vcw = const_cast<float *>(vc);
    hipLaunchKernelGGL(attn_step_kernel<kAttnThreads>, dim3(n_heads), dim3(kAttnThreads), lds, s, q, nullptr, nullptr,
                       kcw, vcw, nullptr, nullptr, nullptr, out, n_heads / n_kv, n_kv, hd, seq);
    return check_launch("gqa_decode_attn");
}

// RoPE of q (in place) and k with the precomputed table row of the current
// position (model_runner.rs:277-293), then k and v written into the layer's
// cache row (model_runner.rs:665-669).
__global__ void rope_kv_kernel(float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
                               float *__restrict__ kc, float *__restrict__ vc, const float *__restrict__ cos_t,
                               const float *__restrict__ sin_t, const uint32_t *__restrict__ ctl, uint32_t nq,
                               uint32_t nk, uint32_t hd) {
    const uint32_t half = hd / 2, kvd = nk * hd;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t pos = ctl[0];
    const uint32_t nqp = nq * half, nkp = nk * half;
    if (i < nqp + nkp) {
        const uint32_t head = i / half, p = i % half;
        const float c = cos_t[(size_t)pos * half + p], sn = sin_t[(size_t)pos * half + p];
        if (head < nq) {
            float *h = q + head * hd;
            const float x0 = h[2 * p], x1 = h[2 * p + 1];
            h[2 * p] = x0 * c - x1 * sn;
            h[2 * p + 1] = x0 * sn + x1 * c;
        } else {
            const uint32_t kh = head - nq;
            const float x0 = k[kh * hd + 2 * p], x1 = k[kh * hd + 2 * p + 1];
            float *dst = kc + (size_t)pos * kvd + kh * hd;
            dst[2 * p] = x0 * c - x1 * sn;
            dst[2 * p + 1] = x0 * sn + x1 * c;
        }
    } else if (i < nqp + nkp + kvd) {
        const uint32_t j = i - nqp - nkp;
        vc[(size_t)pos * kvd + j] = v[j];
    }
}

int launch_rope_kv(hipStream_t s, float *q, const float *k, const float *v, float *kc, float *vc, const float *cos_t,
                   const float *sin_t, const uint32_t *ctl, uint32_t nq, uint32_t nk, uint32_t hd) {
    const uint32_t total = (nq + nk) * (hd / 2) + nk * hd;
    hipLaunchKernelGGL(rope_kv_kernel, dim3((total + 255) / 256), dim3(256), 0, s, q, k, v, kc, vc, cos_t, sin_t, ctl,
                       nq, nk, hd);
    return check_launch("rope_kv");
}

// argmax_ct over the logits (last maximal index wins), then advance the
// control block: the winner becomes the next input token, is recorded at
// out_tokens[pos], and the position moves on.
__global__ __launch_bounds__(1024) void argmax_advance_kernel(const float *__restrict__ in, uint32_t n,
                                                              uint32_t *__restrict__ ctl,
                                                              uint32_t *__restrict__ out_tokens) {
    __shared__ float rv[16];
    __shared__ uint32_t ri[16];
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x)
        if (better(in[i], i, bv, bi)) { bv = in[i]; bi = i; }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const uint32_t oi = __shfl_xor(bi, off, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) { rv[w] = bv; ri[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < (int)(blockDim.x >> 6); k++)
            if (better(rv[k], ri[k], bv, bi)) { bv = rv[k]; bi = ri[k]; }
        const uint32_t pos = ctl[0];
        ctl[1] = bi;
        out_tokens[pos] = bi;
        ctl[0] = pos + 1;
    }
}

// Advance the control block from the lm_head matvec's argmax: the maximum of
// the packed keys (key << 32 | row) its workgroups left in their slots (slots
// no workgroup of the launch owns stay 0 and never win); the low 32 bits are
// the winning row, the last one among equal maxima.
__global__ __launch_bounds__(1024) void advance_kernel(const unsigned long long *__restrict__ slots,
                                                       uint32_t *__restrict__ ctl, uint32_t *__restrict__ out_tokens) {
    static_assert(kArgmaxSlots == 2 * 1024, "two slots per thread");
    __shared__ unsigned long long wbest[16];
    const unsigned long long s0 = slots[threadIdx.x], s1 = slots[threadIdx.x + 1024];
    unsigned long long b = s0 > s1 ? s0 : s1;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(b, off, 64);
        b = o > b ? o : b;
    }
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; w++) b = wbest[w] > b ? wbest[w] : b;
        const uint32_t tok = argmax_row(b), pos = ctl[0];
        ctl[1] = tok;
        out_tokens[pos] = tok;
        ctl[0] = pos + 1;
    }
}

int launch_advance(hipStream_t s, const unsigned long long *slots, uint32_t *ctl, uint32_t *out_tokens) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1024), 0, s, slots, ctl, out_tokens);
    return check_launch("advance");
}

int launch_argmax_advance(hipStream_t s, const float *logits, uint32_t n, uint32_t *ctl, uint32_t *out_tokens) {
    hipLaunchKernelGGL(argmax_advance_kernel, dim3(1), dim3(1024), 0, s, logits, n, ctl, out_tokens);
    return check_launch("argmax_advance");
}

}  // namespace yule
