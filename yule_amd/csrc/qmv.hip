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
#include "qmv_formats.h"

namespace yule {

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
// Rows stream through persistent workgroups.  A team of W lanes (16..512;
// 192 = three waves, so rows of 129-192 units leave no wave idle)
// covers a whole row, one unit per lane, so each lane's activation slice is
// loaded into registers once for the life of the workgroup; the team then
// walks rows row0, row0 + stride, ... with the next row's blocks already in
// flight while the current one is computed.  With several teams per
// workgroup, x is staged once through LDS.  Teams wider than a wave combine
// their per-wave sums through LDS.

template <class R>
struct RawPair {
    R g, u;
};

// PAIR: segments 0 and 1 are the gate and up matrices (equal row counts);
// a team computes row r of both and stores silu(g)*u into segment 0's
// output (model_runner.rs:963-972), so SwiGLU costs nothing extra.
// EXACT: the row loop holds no branch around a memory operation, so the
// compiler's wait before each row covers that row's loads only (with a
// branch it waits for every load in flight, the next row's prefetch
// included: loads complete in issue order).  The next row's fetch is
// unconditional (rows past the end re-read the last row); a one-wave team
// stores with every lane (the same value to one address; a team past the
// last row stores that row's value again); teams wider than a wave flush
// their LDS ring once after the loop, where the residual of kEpiAdd is
// loaded too; a duplicate last row leaves the argmax unchanged (same value,
// same row).  The host picks it for one-wave-or-narrower teams without an
// input transform and with the store epilogue, and for the argmax epilogue
// behind a transform (the lm_head: several rows per team) (decode's narrow fused
// launches measured slower in this form: Q/K/V with RoPE 4.61 -> 4.96 us,
// paired gate/up 5.78 -> 5.92, O + residual 3.27 -> 3.38), and for wider
// teams with at most 16 row iterations each.
// ADD (with EXACT, one-wave teams, no input transform): the residual-add
// epilogue with its load of y[row] unconditional; the host picks it only
// when the rows divide evenly over the workgroups' teams, so that no team
// computes a duplicate of the last row (two read-modify-writes of one y
// element would race).
template <class F, int W, int D, int NT, bool PAIR, bool TWO, bool EXACT = false, bool ADD = false>
__global__ __launch_bounds__(NT) void qmv_stream_kernel(const uint8_t *vb0, const uint8_t *vb1, const uint8_t *vb2,
                                                        const float *__restrict__ x, uint32_t st1, uint32_t st2,
                                                        uint32_t n_rows, uint32_t bpr_pf,
                                                        const uint32_t *__restrict__ rope_ctl, const Segs sg,
                                                        const QmvXf xf) {
    static_assert(!PAIR || W <= 64, "paired rows need single-wave teams");
    constexpr uint32_t RI = NT / W;                   // rows per workgroup iteration
    constexpr uint32_t NWV = NT / 64;                 // waves per workgroup
    constexpr uint32_t WPT = W >= 64 ? W / 64 : 1;    // waves per team
    using Buf = typename std::conditional<PAIR, RawPair<typename F::Raw>, typename F::Raw>::type;
    extern __shared__ float xl[];
    __shared__ float part[NWV];
    const uint32_t tid = threadIdx.x, team = tid / W, t = tid % W;
    // The leading scalar arguments (segment bases, x, row starts, row count,
    // bpr, the RoPE control block: 14 dwords) arrive preloaded in SGPRs
    // (-amdgpu-kernarg-preload-count), so the first weight and x loads issue
    // without waiting for a kernel-argument load.  vbI = segment I's weights
    // moved back by its first row (PAIR: the gate and up weights themselves);
    // stI = first concatenated row of segment I.  At most kStreamSegs
    // segments.  rope_ctl: the control block of a kEpiRope launch, else null.
    const uint8_t *const vbv[kStreamSegs] = {vb0, vb1, vb2};
    const uint32_t stv[kStreamSegs] = {0u, st1, st2};
    // bpr_pf: blocks per row | compute workgroups << 16 (any further
    // workgroups prefetch)
    const uint32_t bpr = bpr_pf & 0xffffu, nblk = bpr_pf >> 16;
    if (blockIdx.x >= nblk) {
        const uint32_t pfw = gridDim.x - nblk;
        // prefetch workgroup: one dword of every 128-byte line of the row
        // groups that the next launch runs on this workgroup's XCD
        for (uint32_t i = 0; i < (xf.pf_delay & 0x7fffffffu); i++) __builtin_amdgcn_s_sleep(8);
        const uint32_t xcd = blockIdx.x & 7u, rank = (blockIdx.x - nblk) >> 3, nr = pfw >> 3;
        const uint32_t lpg = (xf.pf_gbytes + 127) / 128, nseg = xf.pf_w[1] ? 2u : 1u;
        const uint32_t mine = xf.pf_groups > xcd + 8 * rank ? (xf.pf_groups - xcd - 8 * rank + 8 * nr - 1) / (8 * nr) : 0;
        uint32_t acc = 0;
        for (uint32_t j = tid; j < mine * lpg * nseg; j += NT) {
            const uint32_t gi = j / (lpg * nseg), rem = j % (lpg * nseg), sgi = rem / lpg, line = rem % lpg;
            const size_t off = (size_t)(xcd + 8 * (rank + gi * nr)) * xf.pf_gbytes + (size_t)line * 128;
            if (off < xf.pf_total) acc ^= *reinterpret_cast<const uint32_t *>((sgi ? xf.pf_w[1] : xf.pf_w[0]) + off);
        }
        if ((xf.pf_delay >> 31) && rope_ctl) {
            // (pf_delay bit 31, a Q/K/V launch with the RoPE epilogue) this
            // layer's K and V cache rows before the current position, for the
            // attention launch that follows: its workgroups on every XCD read
            // all of them, so each XCD's prefetch workgroups read them all
            const uint32_t pos = rope_ctl[0];
            const uint32_t lines = (uint32_t)(((size_t)pos * (st2 - st1) * sizeof(float) + 127) / 128);
            for (uint32_t j = rank * NT + tid; j < 2 * lines; j += nr * NT) {
                const float *base = j < lines ? xf.kc : xf.vc;
                acc ^= __builtin_bit_cast(uint32_t, base[(size_t)(j < lines ? j : j - lines) * 32]);
            }
        }
        if (acc == 0x9E3779B9u && n_rows == 0) sg.y[0][0] = 0.f;   // keeps the loads; never true
        return;
    }
    const uint32_t units = bpr * F::UPB;
    const size_t row_bytes = (size_t)bpr * F::BB;
    const bool active = t < units;
    const uint32_t k = active ? t / F::UPB : 0, sub = t % F::UPB;
    const uint32_t stride = nblk * RI;
    const uint32_t r0 = blockIdx.x * RI;
    if (r0 >= n_rows) return;   // uniform per workgroup

    // concatenated row -> weight row pointer / output slot: a row's address
    // is vbv[seg] + row * row_bytes.  With whole-wave teams the row is
    // wave-uniform and all of this runs on the scalar unit.
    auto uni = [&](uint32_t v) { return W >= 64 ? __builtin_amdgcn_readfirstlane(v) : v; };
    auto seg_of = [&](uint32_t row) {
        uint32_t s = 0;
#pragma unroll
        for (int i = 1; i < kStreamSegs; i++) s += row >= stv[i];
        return s;
    };
    auto fetch = [&](uint32_t rbase) -> Buf {
        uint32_t row = rbase + team;
        row = uni(row < n_rows ? row : n_rows - 1);
        if constexpr (PAIR) {
            const size_t off = (size_t)row * row_bytes + (size_t)k * F::BB;
            return {F::load(vb0 + off, sub), F::load(vb1 + off, sub)};
        } else {
            const uint32_t s = seg_of(row);
            const uint8_t *wb = vb0;
#pragma unroll
            for (int i = 1; i < kStreamSegs; i++) wb = s == (uint32_t)i ? vbv[i] : wb;
            return F::load(wb + (size_t)row * row_bytes + (size_t)k * F::BB, sub);
        }
    };
    unsigned long long best = 0;   // kEpiArgmax: packed (order key << 32 | row), max wins
    // `row` may differ across the lanes of a wave (ring flushes); callers
    // with a wave-uniform row pass it through uni() first
    auto store = [&](uint32_t row, float v) {
        const uint32_t s = seg_of(row);
        float *yb = sg.y[0];
#pragma unroll
        for (int i = 1; i < kStreamSegs; i++) yb = s == (uint32_t)i ? sg.y[i] - stv[i] : yb;
        // (the one-wave EXACT kernels run the store epilogue only, and with
        // an input transform also the argmax one: no load under a branch;
        // argmax adds register work alone)
        constexpr bool STORE_ONLY = EXACT && WPT == 1;
        if (ADD || (!STORE_ONLY && xf.epi == kEpiAdd)) v = yb[row] + v;   // residual + projection (model_runner.rs:782-784)
        yb[row] = v;
        if ((!STORE_ONLY || TWO) && xf.epi == kEpiArgmax) {
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
        // kEpiRope: the position first of all, so that the table loads below,
        // which need it, wait for it alone and not for the x and weight loads
        // behind it (loads complete in issue order)
        uint32_t pos_early = 0;
        if (TWO && W < 64 && rope_ctl) pos_early = rope_ctl[0];
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
            if (EXACT || r0 + j * stride < n_rows) buf[j] = fetch(r0 + j * stride);
        // nothing below (the RoPE block's argument loads and their wait)
        // is scheduled ahead of the first rows' weight loads
        __builtin_amdgcn_sched_barrier(0);
        if (TWO && W < 64) {   // kEpiRope comes with an input transform (checked on the host)
            // RoPE epilogue: lane l keeps cos / sin of pair l of the position's
            // table row (unconditional loads from a valid address either way)
            const bool rope = xf.epi == kEpiRope;
            rpos = rope ? pos_early : 0u;
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
        if (TWO && W < 64 && !EXACT && xf.epi == kEpiRope) {   // (RoPE launches never run EXACT)
            // rows 2i and 2i + 1 of a head are teams 2j and 2j + 1 of one wave
            // (row bases are even): the pair meets across lane W
            const float other = __shfl_xor(acc, W, 64);
            const uint32_t row = rbase + team;
            const uint32_t s = seg_of(row < n_rows ? row : n_rows - 1), loc = row - stv[s < kStreamSegs ? s : 0];
            const uint32_t i = (loc % xf.hd) / 2;
            const float c = __shfl(rcos, (int)i, 64), sn = __shfl(rsin, (int)i, 64);
            const bool even = (loc & 1u) == 0;
            const float x0 = even ? acc : other, x1 = even ? other : acc;
            float v = acc;
            if (s < 2) v = even ? x0 * c - x1 * sn : x0 * sn + x1 * c;
            if (t == 0 && row < n_rows) {
                const size_t kvd = (size_t)(st2 - st1);
                if (s == 0) sg.y[0][loc] = v;
                else (s == 1 ? xf.kc : xf.vc)[(size_t)rpos * kvd + loc] = v;
            }
        } else if (WPT == 1) {
            const uint32_t row = uni(rbase + team);
            if constexpr (EXACT) {
                // every lane of the team stores (the same value, one address);
                // a team past the last row (store epilogue only) stores the
                // last row again: its clamped fetch computed that row, so the
                // value is identical
                store(row < n_rows ? row : n_rows - 1, acc);
            } else if (t == 0 && row < n_rows) {
                store(row, acc);
            }
        } else {
            if ((tid & 63) == 0) ring[it & 15][tid >> 6] = acc;
            // (EXACT: at most 16 row iterations per team, checked on the host;
            // the ring is flushed once after the loop, so the loop holds no
            // barrier and no global store)
            if (!EXACT && ((it & 7) == 7 || last)) {
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
            // (EXACT: unconditional, rows past the end re-read the last row, so
            // that no branch merges before the next row's wait)
            if (EXACT || rn < n_rows) buf[(j + D - 1) % D] = fetch(rn);
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
    if constexpr (EXACT && WPT > 1) {   // the ring's iterations 0 .. it - 1 (it <= 16)
        __syncthreads();
        if (tid < 16 * RI) {
            const uint32_t iter = tid / RI, tm = tid % RI;
            const uint32_t row = r0 + iter * stride + tm;
            if (iter < it && row < n_rows) {
                float s = 0.f;
#pragma unroll
                for (uint32_t i = 0; i < WPT; i++) s += ring[iter][tm * WPT + i];
                store(row, s);
            }
        }
    }
    if ((!(EXACT && WPT == 1) || TWO) && xf.epi == kEpiArgmax) {   // uniform: the workgroup's best row into its own slot
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
    const size_t row_bytes = (size_t)bpr * F::BB;
    const uint8_t *vb[kStreamSegs];
    for (int i = 0; i < kStreamSegs; i++) vb[i] = xf.pair ? sg.w[i] : sg.w[i] - (size_t)sg.start[i] * row_bytes;
    const uint32_t n_rows = xf.pair ? sg.start[1] : sg.total;
    const uint32_t *rope_ctl = xf.epi == kEpiRope ? xf.ctl : nullptr;
    const uint32_t bpr_pf = bpr | blocks << 16;
    // EXACT kernel (see qmv_stream_kernel) when every computed row is real or
    // a duplicate that stores the same value, and wide teams' rings hold all
    // their row iterations; YULE_QMV_EXACT=0 turns it off (comparison)
    static const bool exact_on = env_flag("YULE_QMV_EXACT", true);
    constexpr uint32_t RI = NT / W;
    const uint64_t iters = (n_rows + (uint64_t)blocks * RI - 1) / ((uint64_t)blocks * RI);
    // (narrow teams: the plain store epilogue, and the argmax one behind an
    // input transform, the lm_head's, whose launches give each team several
    // rows: decode 1762 -> 1828 tok/s)
    const bool exact = exact_on && (W > 64 ? iters <= 16
                                           : (xf.mode == kXfNone && xf.epi == kEpiStore) ||
                                                 (xf.mode != kXfNone && xf.epi == kEpiArgmax));
    blocks += xf.pf_wgs;
#define YULE_QMV_ARGS vb[0], vb[1], vb[2], x, sg.start[1], sg.start[2], n_rows, bpr_pf, rope_ctl, sg, xf
#define YULE_QMV_LAUNCH(P, T)                                                                                        \
    do {                                                                                                             \
        if (exact)                                                                                                   \
            hipLaunchKernelGGL((qmv_stream_kernel<F, W, D, NT, P, T, true>), dim3(blocks), dim3(NT), lds, s,         \
                               YULE_QMV_ARGS);                                                                       \
        else                                                                                                         \
            hipLaunchKernelGGL((qmv_stream_kernel<F, W, D, NT, P, T, false>), dim3(blocks), dim3(NT), lds, s,        \
                               YULE_QMV_ARGS);                                                                       \
    } while (0)
    if constexpr (W <= 64) {
        if (xf.pair) {   // always with a transform (checked by launch_qmv_fused)
            hipLaunchKernelGGL((qmv_stream_kernel<F, W, D, NT, true, true>), dim3(blocks), dim3(NT), lds, s,
                               YULE_QMV_ARGS);
            return;
        }
    }
    if (xf.mode != kXfNone) {
        YULE_QMV_LAUNCH(false, true);
    } else if (W <= 64 && exact_on && xf.epi == kEpiAdd && n_rows % ((uint64_t)(blocks - xf.pf_wgs) * RI) == 0) {
        // residual add with no duplicate rows: the EXACT loop with the add
        // (decode's O + residual)
        hipLaunchKernelGGL((qmv_stream_kernel<F, W, D, NT, false, false, true, W <= 64>), dim3(blocks), dim3(NT), lds,
                           s, YULE_QMV_ARGS);
    } else {
        YULE_QMV_LAUNCH(false, false);
    }
#undef YULE_QMV_LAUNCH
#undef YULE_QMV_ARGS
}

// Compute workgroups of a streaming launch: about waves_env waves per CU, no
// more than the LDS copies of x allow, no more than the row iterations.
static uint32_t stream_blocks(uint32_t W, uint32_t NT, uint32_t bs, uint32_t bpr, uint32_t rows, bool pair,
                              bool argmax) {
    const uint32_t RI = NT / W;
    static const int waves_all = env_int("YULE_QMV_WAVES_PER_CU", 16);
    static const int waves_pair = env_int("YULE_QMV_PAIR_WAVES", 8);
    const int waves_env = pair ? waves_pair : waves_all;
    const size_t lds = (size_t)lds_pad(bpr * bs) * sizeof(float) + 512;
    const int wg_lds = (int)(kLdsPerCu / lds);
    const int wg_waves = waves_env / (int)(NT / 64) > 0 ? waves_env / (int)(NT / 64) : 1;
    const int wg = wg_waves < wg_lds ? wg_waves : (wg_lds > 0 ? wg_lds : 1);
    const uint32_t iters = (rows + RI - 1) / RI;
    const uint32_t cap = (uint32_t)(device_cus() * wg);
    uint32_t blocks = iters < cap ? iters : cap;
    if (argmax && blocks > kArgmaxSlots) blocks = kArgmaxSlots;   // one slot per workgroup
    return blocks;
}

// Workgroup shape: NT threads (RI = NT / W teams) share one LDS copy of the
// activation vector; about 16 waves per CU are resident (4 per SIMD, the
// VGPR limit), as NT-thread workgroups up to the LDS each copy takes.
template <class F, int W, int NT>
static void launch_stream_nt(hipStream_t s, const Segs &sg, const float *x, uint32_t bpr, const QmvXf &xf) {
    // paired gate/up launches are sized for 8 waves per CU: TinyLlama's 5632
    // gate/up row pairs as 512 workgroups (two rounds for some) decode
    // 1663 -> 1684 tok/s against 704 (4 or 6 waves: 1618)
    const uint32_t rows = xf.pair ? sg.start[1] : sg.total;
    const uint32_t blocks = stream_blocks(W, NT, F::BS, bpr, rows, xf.pair, xf.epi == kEpiArgmax);
    // the argmax epilogue's launches (the lm_head: ~8 rows per team at
    // 32000 rows) keep three rows in flight per team, the others two
    static const bool deep = env_flag("YULE_QMV_ARGMAX_DEEP", true);
    if (deep && xf.epi == kEpiArgmax) return launch_stream_d<F, W, 3, NT>(s, sg, x, bpr, blocks, xf);
    launch_stream_d<F, W, 2, NT>(s, sg, x, bpr, blocks, xf);
}

template <class F, int W>
static void launch_stream(hipStream_t s, const Segs &sg, const float *x, uint32_t bpr, const QmvXf &xf) {
    // one-wave teams (the 4096-column projections) measured ~1% faster in
    // 512-thread workgroups; narrower teams (2048 columns) 6% slower there
    static const int nt_narrow = env_int("YULE_QMV_THREADS", 256), nt_wide = env_int("YULE_QMV_THREADS_WIDE", 1024);
    static const int nt_w64 = env_int("YULE_QMV_THREADS_W64", 512);
    if constexpr (W == 192) return launch_stream_nt<F, W, 768>(s, sg, x, bpr, xf);   // four three-wave teams
    else {
    const int nt = W >= 512 ? 1024 : W >= 128 ? nt_wide : W == 64 ? nt_w64 : nt_narrow;
    if (nt >= 1024) return launch_stream_nt<F, W, 1024>(s, sg, x, bpr, xf);
    if constexpr (W >= 512) return;   // unreachable: 512-lane teams only run in 1024-thread workgroups
    else
    if (nt >= 512) return launch_stream_nt<F, W, 512>(s, sg, x, bpr, xf);
    else launch_stream_nt<F, W, 256>(s, sg, x, bpr, xf);
    }
}

// Largest activation vector staged in LDS by the streaming kernel (floats).
constexpr uint32_t kMaxStageCols = 32768;

template <class F>
static bool stream_ok(uint32_t n_cols) {
    static const bool v1 = getenv("YULE_QMV_V1") != nullptr;
    return !v1 && (n_cols / F::BS) * F::UPB <= 512 && n_cols <= kMaxStageCols;
}

// team width and workgroup size launch_fmt / launch_stream pick for a row of `units`
static uint32_t stream_team(uint32_t units) {
    return units <= 16 ? 16 : units <= 32 ? 32 : units <= 64 ? 64 : units <= 128 ? 128 : units <= 192 ? 192
         : units <= 256 ? 256 : 512;
}
static uint32_t stream_threads(uint32_t W) {
    static const int nt_narrow = env_int("YULE_QMV_THREADS", 256), nt_wide = env_int("YULE_QMV_THREADS_WIDE", 1024);
    static const int nt_w64 = env_int("YULE_QMV_THREADS_W64", 512);
    if (W == 192) return 768;
    const int nt = W >= 512 ? 1024 : W >= 128 ? nt_wide : W == 64 ? nt_w64 : nt_narrow;
    return nt >= 1024 ? 1024 : nt >= 512 ? 512 : 256;
}

template <class F>
static bool group_plan(uint32_t n_rows, uint32_t n_cols, bool pair, uint32_t *gb, uint32_t *groups, uint32_t *rpg) {
    if (!stream_ok<F>(n_cols) || n_cols % F::BS) return false;
    const uint32_t bpr = n_cols / F::BS, W = stream_team(bpr * F::UPB), NT = stream_threads(W), RI = NT / W;
    if (pair && W > 64) return false;
    const uint32_t blocks = stream_blocks(W, NT, F::BS, bpr, n_rows, pair, false);
    if (blocks % 8) return false;   // then group g would not map to XCD g % 8
    *gb = RI * bpr * F::BB;
    *groups = (n_rows + RI - 1) / RI;
    *rpg = RI;
    return true;
}

bool qmv_group_plan(uint32_t dtype, uint32_t n_rows, uint32_t n_cols, bool pair, uint32_t *gb, uint32_t *groups,
                    uint32_t *rpg) {
    switch (dtype) {
    case YULE_DTYPE_Q4_K: return group_plan<Q4K>(n_rows, n_cols, pair, gb, groups, rpg);
    case YULE_DTYPE_Q5_K: return group_plan<Q5K>(n_rows, n_cols, pair, gb, groups, rpg);
    case YULE_DTYPE_Q6_K: return group_plan<Q6K>(n_rows, n_cols, pair, gb, groups, rpg);
    case YULE_DTYPE_Q8_K: return group_plan<Q8K>(n_rows, n_cols, pair, gb, groups, rpg);
    case YULE_DTYPE_Q8_0: return group_plan<Q80>(n_rows, n_cols, pair, gb, groups, rpg);
    case YULE_DTYPE_Q4_0: return group_plan<Q40>(n_rows, n_cols, pair, gb, groups, rpg);
    default: return false;
    }
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
        if (n_seg > (uint32_t)kStreamSegs) {   // as two launches (no fused epilogue spans matrices here)
            const int rc = launch_fmt<F>(s, segs, kStreamSegs, x, n_cols, xf);
            return rc ? rc : launch_fmt<F>(s, segs + kStreamSegs, n_seg - kStreamSegs, x, n_cols, xf);
        }
        if (units <= 16) return launch_stream<F, 16>(s, sg, x, bpr, xf), YULE_OK;
        if (units <= 32) return launch_stream<F, 32>(s, sg, x, bpr, xf), YULE_OK;
        if (units <= 64) return launch_stream<F, 64>(s, sg, x, bpr, xf), YULE_OK;
        if (units <= 128) return launch_stream<F, 128>(s, sg, x, bpr, xf), YULE_OK;
        if (units <= 192) return launch_stream<F, 192>(s, sg, x, bpr, xf), YULE_OK;
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
                               segs[0].n_rows % xf.hd || segs[1].n_rows % xf.hd || xf.pair || xf.mode == kXfNone))
        return set_error(YULE_ERR_INVALID,
                         "quantized_matmul: RoPE epilogue needs q, k, v of whole heads on narrow teams and an input transform");
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
