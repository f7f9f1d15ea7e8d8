// internal.h — shared host-side state of libyule_hip.so (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/yule_hip.h"

namespace yule {

// Every allocation carries this many bytes of slack past its requested size:
// the matvec kernels read 2-byte-aligned GGUF blocks (Q4_0 18 B, Q8_0 34 B,
// Q6_K 210 B) through 4-byte-aligned dword loads, so the last block of a
// buffer may be fetched up to 4 bytes past its end.
constexpr size_t kAllocSlack = 64;

struct Buffer {
    void *ptr = nullptr;
    size_t size = 0;  // bytes requested by the caller (validation bound)
};

}  // namespace yule

struct yule_hip_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    hipDeviceProp_t props{};
    std::mutex mu;  // guards `buffers`; ComputeBackend is Send + Sync
    std::unordered_map<uint64_t, yule::Buffer> buffers;
    hipEvent_t timer[2] = {nullptr, nullptr};
    // harness capture of the calls between capture_begin and capture_end
    hipGraph_t cap_graph = nullptr;
    hipGraphExec_t cap_exec = nullptr;
    // device workspace shared by the ops that need one (GEMM staging and
    // split-K partials, split-KV attention partials); grown on demand,
    // freed with the backend
    std::mutex scratch_mu;
    void *scratch = nullptr;
    size_t scratch_size = 0;
};

namespace yule {

// thread-local last error, returned by yule_hip_last_error()
int set_error(int code, const std::string &msg);
int hip_error(hipError_t e, const char *what);

// Look up a handle and check that [offset, offset+need) lies inside it.
int get_buffer(yule_hip_backend *be, uint64_t h, size_t need, void **ptr, const char *what,
               size_t offset = 0);

// The backend's workspace for one call.  The lease holds the workspace lock
// until it is destroyed, so a call enqueues every launch that uses the
// workspace before another thread's call can get it: launches on the one
// backend stream then never interleave over it.  Growing it waits for the
// stream (earlier launches may still read the old one).
struct ScratchLease {
    std::unique_lock<std::mutex> lock;
    void *ptr = nullptr;
};
int get_scratch(yule_hip_backend *be, size_t need, ScratchLease *lease);

// Launch failures surface through hipGetLastError after a kernel launch.
int check_launch(const char *what);

// Block geometry of the supported GGUF formats (dtype.rs:62-118); false if
// unsupported by the quantized kernels.
bool quant_geometry(uint32_t dtype, uint32_t *block_size, uint32_t *block_bytes);

// One matrix of a multi-matrix matvec launch (all share input and n_cols).
constexpr int kMaxSegs = 4;
struct QmvSeg {
    const uint8_t *w;
    float *y;
    uint32_t n_rows;
};

// Optional fusions of the streaming matvec: a transform applied to the
// activation vector while it is staged, and an epilogue.
constexpr uint32_t kXfNone = 0, kXfRmsNorm = 1, kXfSwiGlu = 2;
constexpr uint32_t kEpiStore = 0, kEpiAdd = 1, kEpiArgmax = 2, kEpiRope = 3;
// argmax epilogue slots (one per workgroup of the launch; zero-filled once)
constexpr uint32_t kArgmaxSlots = 2048;
struct QmvXf {
    uint32_t mode = kXfNone;         // kXfRmsNorm: x*inv_rms*a; kXfSwiGlu: x*sigmoid(x)*a
    const float *a = nullptr;        // norm weight or up vector, n_cols floats
    float eps = 0.f;
    uint32_t epi = kEpiStore;        // kEpiAdd: y += result; kEpiArgmax: store, and each workgroup's
    unsigned long long *amax = nullptr;  // best (key << 32 | row) into amax[blockIdx.x] (kArgmaxSlots)
    bool pair = false;               // gate/up pair: segment 0 output = silu(gate)*up
    // kEpiRope (the Q/K/V launch of a decode step; segments q, k, v, teams of
    // at most 32 lanes): RoPE with the table row of position ctl[0] applied to
    // q (stored to segment 0's output) and k, and k and v stored straight into
    // the KV cache row ctl[0] (model_runner.rs:654-669, 277-293)
    const uint32_t *ctl = nullptr;
    const float *cos_t = nullptr, *sin_t = nullptr;   // [max_seq][hd / 2]
    float *kc = nullptr, *vc = nullptr;               // [max_seq][n_kv * hd]
    uint32_t hd = 0;
    // prefetch: pf_wgs extra workgroups (a multiple of 8, after the compute
    // grid) read the following launch's matrix pf_w[0] (and pf_w[1], the up
    // half of a gate/up pair, same rows) into the L2 of the XCD whose
    // workgroups will read them: that launch's row group g (pf_gbytes bytes
    // of each matrix, pf_total bytes in all) belongs to XCD g % 8
    // (pf_delay: sleep iterations before the reads; bit 31 set on a Q/K/V
    // launch with the RoPE epilogue: the layer's K/V cache rows before the
    // current position too, for the attention launch)
    const uint8_t *pf_w[2] = {nullptr, nullptr};
    uint32_t pf_wgs = 0, pf_gbytes = 0, pf_groups = 0, pf_delay = 0;
    size_t pf_total = 0;
};

// Kernel launchers (device code in qmv.hip / ops.hip / attn.hip / gemm.hip).
// Arguments are already validated; all enqueue on `stream`.
int launch_qmv(hipStream_t stream, uint32_t dtype, const uint8_t *w, const float *x, float *y,
               uint32_t n_rows, uint32_t n_cols);
int launch_qmv_multi(hipStream_t stream, uint32_t dtype, const QmvSeg *segs, uint32_t n_seg, const float *x,
                     uint32_t n_cols);
// true when (dtype, n_cols) runs on the streaming kernel, i.e. fusions apply
bool qmv_fusable(uint32_t dtype, uint32_t n_cols);
// true when gate/up of this shape can run as one paired launch (xf.pair)
bool qmv_pairable(uint32_t dtype, uint32_t n_cols);
// row-group size (bytes) and group count of a streaming launch of this shape
// whose group g runs on XCD g % 8; false when its grid gives no such mapping
bool qmv_group_plan(uint32_t dtype, uint32_t n_rows, uint32_t n_cols, bool pair, uint32_t *group_bytes,
                    uint32_t *groups, uint32_t *rows_per_group);
// lanes per row of the streaming matvec for this shape
uint32_t qmv_team_width(uint32_t dtype, uint32_t n_cols);
// true when the Q/K/V launch can apply RoPE and write the KV cache (kEpiRope)
bool qmv_rope_ok(uint32_t dtype, uint32_t n_cols, uint32_t hd);
int launch_qmv_fused(hipStream_t stream, uint32_t dtype, const QmvSeg *segs, uint32_t n_seg, const float *x,
                     uint32_t n_cols, const QmvXf &xf);
int launch_dequant(hipStream_t stream, uint32_t dtype, const uint8_t *src, float *dst,
                   uint32_t n_blocks);
// dequantize row token[0] (clamped to n_rows-1) of a [n_rows][dim] quantized
// table; the token is read on the device so the launch can sit in a graph
int launch_embed_rows(hipStream_t stream, uint32_t dtype, const uint8_t *table, const uint32_t *token,
                      uint32_t n_rows, float *dst, uint32_t dim);
// device address of the allocation-free GEMM's static workspace on `device`,
// looked up once with that device current (yule_hip_create)
int gemm_static_workspace_init(int device);
// decode-step attention over a cache that already holds row ctl[0] and a
// rotated q (after a kEpiRope Q/K/V launch): one workgroup per (query head,
// chunk), chunks combined in-launch; hd 64 or 128 (attn_chunk_len != 0)
uint32_t attn_chunk_len(uint32_t hd);
size_t attn_chunk_scratch_bytes(uint32_t n_heads, uint32_t hd, uint32_t max_rows);
int launch_attn_chunks(hipStream_t stream, const float *q, const float *kc, const float *vc, const uint32_t *ctl,
                       float *out, void *scratch, uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t max_rows,
                       uint32_t seq_host);
// f32-X prefill GEMM into a caller-owned workspace (gemm.hip)
// A split-K reduction left for the next product's X pre-pass (defer): the
// partials part[ks][m][ny] of y, summed into y (accumulate: added to it) by
// the pre-pass of the product whose X is y (pending), row by row before it
// reads the row.  ks = 0: nothing left.  The partials live in the first
// product's workspace, so the second needs another.
struct GemmRed {
    const float *part;
    float *y;
    uint32_t ks, ny, m;
    bool accumulate;
};
bool gemm_supports(uint32_t dtype, uint32_t n_cols);
size_t gemm_f32_workspace_bytes(uint32_t m, uint32_t n_rows, uint32_t n_cols, uint32_t dtype);
// up to three matrices of one format sharing X as one f32-X product into
// Y [m][sum of rows] (each row count a multiple of 256)
bool gemm_multi_ok(uint32_t dtype, uint32_t n_cols, const uint32_t *rows, uint32_t n_mat);
size_t gemm_f32_multi_workspace_bytes(uint32_t m, const uint32_t *rows, uint32_t n_mat, uint32_t n_cols,
                                      uint32_t dtype);
int launch_gemm_f32_multi(hipStream_t stream, const uint8_t *const *w, const uint32_t *rows, uint32_t n_mat,
                          const float *x, float *y, uint32_t m, uint32_t n_cols, uint32_t dtype, void *ws,
                          const float *norm_w = nullptr, float eps = 0.f, GemmRed *defer = nullptr,
                          const GemmRed *pending = nullptr);
// accumulate: Y += X W (the residual add of the output and down projections);
// norm_w: X's rows RMS-normalised and scaled by norm_w (eps) on the way in;
// glu: x holds [gate | up] rows (2 n_cols wide) and X = gate * sigmoid(gate)
// * up, formed on the way in (the down projection after a gate|up product)
int launch_gemm_f32(hipStream_t stream, const uint8_t *w, const float *x, float *y, uint32_t m, uint32_t n_rows,
                    uint32_t n_cols, uint32_t dtype, void *ws, bool accumulate = false, const float *norm_w = nullptr,
                    float eps = 0.f, bool glu = false, GemmRed *defer = nullptr, const GemmRed *pending = nullptr);
// batched prompt pass (prefill.hip)
int launch_embed_rows_batch(hipStream_t stream, uint32_t dtype, const uint8_t *table, const uint32_t *tokens,
                            uint32_t vocab, float *out, uint32_t dim, uint32_t n);
// rows of q ldq floats apart, rows of k and v ldkv
int launch_rope_rows(hipStream_t stream, float *q, const float *k, const float *v, float *kc, float *vc,
                     const float *cos_t, const float *sin_t, uint32_t pos0, uint32_t n, uint32_t qd, uint32_t kvd,
                     uint32_t hd, uint32_t ldq, uint32_t ldkv);
bool attn_prefill_supported(uint32_t hd);
int launch_attn_prefill(hipStream_t stream, const float *q, const float *kc, const float *vc, float *out, uint32_t pos0,
                        uint32_t n, uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t ldq);
// one launch of an empty kernel (launch-overhead probe)
int launch_empty(hipStream_t stream);
// out[i] = value for i < n
int launch_fill(hipStream_t stream, float *out, float value, uint64_t n);
// out[i] = i < n ? x[i] : 0 for i < n_out (a row staged zero-padded)
int launch_pad(hipStream_t stream, const float *x, uint32_t n, float *out, uint32_t n_out);
// op 0 silu, 1 mul, 2 add, 3 silu(a)*b
int launch_eltwise(hipStream_t stream, int op, const float *a, const float *b, float *out, uint32_t n);
int launch_rms_norm(hipStream_t stream, const float *x, const float *w, float *out, uint32_t n, float eps);
// GQA decode attention of rotated q over cache rows 0..seq-1
int launch_gqa_attn(hipStream_t stream, const float *q, const float *kc, const float *vc, float *out, uint32_t n_heads,
                    uint32_t n_kv, uint32_t hd, uint32_t seq);
int launch_argmax(hipStream_t stream, const float *in, uint32_t n, uint32_t *out);
// decode-runner steps driven by the device control block ctl = {pos, token, prompt_len}
int launch_embed_step(hipStream_t stream, uint32_t dtype, const uint8_t *table, const uint32_t *ctl,
                      const uint32_t *prompt, uint32_t vocab, float *dst, uint32_t dim);
// reduce the lm_head's kArgmaxSlots workgroup slots, then advance the control block
int launch_advance(hipStream_t stream, const unsigned long long *slots, uint32_t *ctl, uint32_t *out_tokens);
int launch_rope_kv(hipStream_t stream, float *q, const float *k, const float *v, float *kc, float *vc,
                   const float *cos_t, const float *sin_t, const uint32_t *ctl, uint32_t nq, uint32_t nk,
                   uint32_t hd);
// RoPE + KV-cache write + GQA attention of one decode step (one launch)
int launch_attn_step(hipStream_t stream, const float *q, const float *k, const float *v, float *kc, float *vc,
                     const float *cos_t, const float *sin_t, const uint32_t *ctl, float *out, uint32_t n_heads,
                     uint32_t n_kv, uint32_t hd, uint32_t max_seq);
// Split-KV (flash-decoding) attention: phase 1 over (KV head, chunk) and a
// combine; with ctl it is the decode step (RoPE + KV write, sequence length
// ctl[0] + 1 <= seq_cap), without it plain GQA over seq_cap rotated rows.
// `scratch` holds split_scratch_bytes(n_heads, hd, seq_cap) bytes.
bool split_attn_supported(uint32_t n_heads, uint32_t n_kv, uint32_t hd);
uint32_t attn_split_min_seq();
size_t split_scratch_bytes(uint32_t n_heads, uint32_t hd, uint32_t seq_cap);
int launch_attn_split(hipStream_t stream, const float *q, const float *k, const float *v, float *kc, float *vc,
                      const float *cos_t, const float *sin_t, const uint32_t *ctl, float *out, void *scratch,
                      uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t seq_cap);
int launch_argmax_advance(hipStream_t stream, const float *logits, uint32_t n, uint32_t *ctl, uint32_t *out_tokens);

}  // namespace yule
