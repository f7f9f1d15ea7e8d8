/*
 * yule_hip.h — C ABI of libyule_hip.so, the MI355X (gfx950) HIP backend for
 * Yule.  It mirrors the yule-gpu ComputeBackend trait
 * (yule-gpu/src/lib.rs:21-132) one entry point per trait method, so a Rust
 * `impl ComputeBackend for HipBackend` can forward each method to one call
 * (binding shown in INTEGRATION.md).
 *
 * Conventions
 *  - Every call returns 0 (YULE_OK) or a YULE_ERR_* code; the message of the
 *    last failure on the calling thread is yule_hip_last_error().  This is
 *    the trait's Result<()> / YuleError::Gpu(String)
 *    (yule-core/src/error.rs:44).
 *  - Buffers are opaque 64-bit handles (BufferHandle(pub u64),
 *    yule-gpu/src/lib.rs:135), zero-initialised on allocation
 *    (yule-gpu/src/cpu.rs:157).
 *  - Kernels are enqueued on one stream owned by the backend, in call order.
 *    copy_from_device and synchronize block; copy_to_device returns after the
 *    host bytes have been consumed.  This matches the CUDA backend's
 *    ordering (yule-gpu/src/cuda/mod.rs, cuda/memory.rs:75-78).
 *  - Sizes that would read or write outside a buffer are rejected with
 *    YULE_ERR_INVALID before any kernel is launched.
 *  - dtype values are GGUF type ids (yule-core/src/dtype.rs:21-33).
 */
#ifndef YULE_HIP_H
#define YULE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define YULE_OK 0
#define YULE_ERR_INVALID 1     /* bad argument, size or handle */
#define YULE_ERR_UNSUPPORTED 2 /* dtype / op not supported (trait default Err) */
#define YULE_ERR_NO_DEVICE 3   /* no usable gfx950 device */
#define YULE_ERR_OOM 4         /* device allocation failed */
#define YULE_ERR_HIP 5         /* HIP runtime error */
#define YULE_ERR_PARSE 6       /* malformed GGUF file (YuleError::Parse and friends) */
#define YULE_ERR_IO 7          /* file could not be opened or mapped */

#define YULE_DTYPE_F32 0
#define YULE_DTYPE_F16 1
#define YULE_DTYPE_Q4_0 2
#define YULE_DTYPE_Q8_0 8
#define YULE_DTYPE_Q4_K 12
#define YULE_DTYPE_Q5_K 13
#define YULE_DTYPE_Q6_K 14
#define YULE_DTYPE_Q8_K 15

typedef struct yule_hip_backend yule_hip_backend;
typedef uint64_t yule_buffer;

/* DeviceInfo, yule-gpu/src/lib.rs:137-143; backend is always 4 (HIP) here */
typedef struct {
    char name[256];
    uint32_t backend;
    uint64_t memory_bytes;
    uint32_t compute_units;
} yule_device_info;

const char *yule_hip_last_error(void);

/* Vulkan/CUDA is_available() probes (yule-gpu/src/vulkan/device.rs:150);
 * 1 when a gfx950 device is present, else 0. */
int yule_hip_is_available(void);

/* create_backend(BackendKind) (yule-gpu/src/lib.rs:175-189) */
int yule_hip_create(int device, yule_hip_backend **out);
int yule_hip_destroy(yule_hip_backend *be);

/* ComputeBackend::name (lib.rs:22) -> "hip" */
const char *yule_hip_name(const yule_hip_backend *be);
/* ComputeBackend::device_info (lib.rs:23) */
int yule_hip_device_info(yule_hip_backend *be, yule_device_info *out);

/* ComputeBackend::allocate / free (lib.rs:24-25) */
int yule_hip_allocate(yule_hip_backend *be, size_t size_bytes, yule_buffer *out);
int yule_hip_free(yule_hip_backend *be, yule_buffer h);

/* copy_to_device / copy_from_device / copy_buffer / copy_buffer_offset /
 * synchronize (lib.rs:68-80) */
int yule_hip_copy_to_device(yule_hip_backend *be, const void *data, size_t size, yule_buffer h);
int yule_hip_copy_from_device(yule_hip_backend *be, yule_buffer h, void *data, size_t size);
int yule_hip_copy_buffer(yule_hip_backend *be, yule_buffer src, yule_buffer dst, size_t size);
int yule_hip_copy_buffer_offset(yule_hip_backend *be, yule_buffer src, yule_buffer dst,
                                size_t src_offset, size_t dst_offset, size_t size);
int yule_hip_synchronize(yule_hip_backend *be);

/* ComputeBackend::matmul (lib.rs:26-34): C[m,n] = A[m,k] * B[k,n], f32 row-major */
int yule_hip_matmul(yule_hip_backend *be, yule_buffer a, yule_buffer b, yule_buffer out,
                    uint32_t m, uint32_t n, uint32_t k);
/* ComputeBackend::softmax (lib.rs:35) */
int yule_hip_softmax(yule_hip_backend *be, yule_buffer in, yule_buffer out, uint32_t size);
/* ComputeBackend::rms_norm (lib.rs:36-43): out = in / sqrt(mean(in^2)+eps) * weight */
int yule_hip_rms_norm(yule_hip_backend *be, yule_buffer in, yule_buffer weight, yule_buffer out,
                      uint32_t size, float eps);
/* ComputeBackend::rope (lib.rs:44-53): in place on q and k, interleaved pairs,
 * freq_i = 1/freq_base^(2i/head_dim), every head of each buffer. */
int yule_hip_rope(yule_hip_backend *be, yule_buffer q, yule_buffer k, uint32_t pos,
                  uint32_t head_dim, float freq_base, uint32_t n_heads_q, uint32_t n_heads_k);
/* ComputeBackend::silu (lib.rs:54): out = in * sigmoid(in) (the trait's and
 * CpuBackend's meaning, yule-gpu/src/cpu.rs:339-357) */
int yule_hip_silu(yule_hip_backend *be, yule_buffer in, yule_buffer out, uint32_t size);
/* ComputeBackend::element_mul (lib.rs:55-61): out = a * b */
int yule_hip_element_mul(yule_hip_backend *be, yule_buffer a, yule_buffer b, yule_buffer out,
                         uint32_t size);
/* ComputeBackend::add (lib.rs:62-68): out = a + b */
int yule_hip_add(yule_hip_backend *be, yule_buffer a, yule_buffer b, yule_buffer out, uint32_t size);

/* ComputeBackend::attn_score (lib.rs:82-96):
 * scores[t] = (q[head_offset..+hd] . k[t*kv_stride+kv_offset..+hd]) / sqrt(hd) */
int yule_hip_attn_score(yule_hip_backend *be, yule_buffer q, yule_buffer k_cache, yule_buffer scores,
                        uint32_t head_dim, uint32_t seq_len, uint32_t head_offset,
                        uint32_t kv_offset, uint32_t kv_stride);
/* ComputeBackend::attn_value (lib.rs:98-114):
 * out[out_offset+d] = sum_t w[t] * v[t*kv_stride+kv_offset+d] */
int yule_hip_attn_value(yule_hip_backend *be, yule_buffer weights, yule_buffer v_cache,
                        yule_buffer out, uint32_t head_dim, uint32_t seq_len,
                        uint32_t kv_offset, uint32_t kv_stride, uint32_t out_offset);

/* ComputeBackend::quantized_matmul (lib.rs:116-131) — the hot path.
 * y[r] = sum_b vec_dot(W[r, b], x[b*bs .. (b+1)*bs]) for r < n_rows.
 * weights: raw GGUF blocks, row-major, ceil(n_cols/bs) blocks per row;
 * input: f32[n_cols]; output: f32[n_rows], fully overwritten.  When n_cols
 * is not a block multiple the last block's columns >= n_cols are skipped,
 * as in the reference's GPU kernels (cuda/mod.rs:311-313, qmv_*.cu).
 * dtype: Q4_0, Q8_0, Q4_K or Q6_K (the reference's GPU set), plus Q5_K
 * (the CPU path's vec_dot_q5_k, dequant.rs:1088-1140) and Q8_K (the
 * reference has its dequant only, dequant.rs:376-384; here it runs through
 * the same matvec).  Other dtypes -> YULE_ERR_UNSUPPORTED, as the Vulkan
 * backend's Err (yule-gpu/src/vulkan/mod.rs:333-343). */
int yule_hip_quantized_matmul(yule_hip_backend *be, yule_buffer weights, yule_buffer input,
                              yule_buffer output, uint32_t n_rows, uint32_t n_cols, uint32_t dtype);

/* ---- extensions beyond the trait (used by the HIP runner) ---- */

/* quantized_matmul of n_mats (1..4) matrices that share one input vector,
 * n_cols and dtype, in a single launch over their concatenated rows:
 * outputs[i][r] = sum_b vec_dot(weights[i][r, b], input[b*bs..]).  The
 * Q/K/V and gate/up projections of a decode step (yule-infer/src/
 * model_runner.rs:636-638, :963-964; gpu_runner.rs:392-419) each become
 * one launch.  Same validation and results as n_mats separate calls. */
int yule_hip_quantized_matmul_multi(yule_hip_backend *be, uint32_t n_mats, const yule_buffer *weights,
                                    const yule_buffer *outputs, const uint32_t *n_rows, yule_buffer input,
                                    uint32_t n_cols, uint32_t dtype);

/* dequant_block over n_blocks consecutive blocks starting src_offset bytes
 * into src (yule-core/src/dequant.rs:1232-1275), bit-exact, f32 out.
 * Replaces the CPU embedding dequant + upload of
 * yule-infer/src/gpu_runner.rs:309-343. */
int yule_hip_dequantize(yule_hip_backend *be, yule_buffer src, size_t src_offset, yule_buffer dst,
                        uint32_t n_blocks, uint32_t dtype);

/* The fused SwiGLU the GPU backends run under the names silu/element_mul
 * (yule-gpu/src/vulkan/mod.rs:397-428, cuda/mod.rs:173-208) and the CPU
 * runner inlines (yule-infer/src/model_runner.rs:967-972):
 * out[i] = gate[i] * sigmoid(gate[i]) * up[i]. */
int yule_hip_silu_mul(yule_hip_backend *be, yule_buffer gate, yule_buffer up, yule_buffer out,
                      uint32_t size);

/* Fused GQA decode attention for one token over an f32 KV cache, replacing
 * the per-head attn_score + softmax + attn_value sequence
 * (yule-infer/src/model_runner.rs:679-758, shaders/multihead_attn.comp):
 * for each query head h (kv head h / (n_heads/n_kv_heads)):
 *   s_t = q_h . K_t / sqrt(hd); p = softmax(s); out_h = sum_t p_t V_t
 * k_cache/v_cache: [seq][n_kv_heads*head_dim] f32 rows, t < seq_len.
 * head_dim a multiple of 4, <= 256; seq_len <= 262144.  From 512 positions
 * (environment YULE_ATTN_SPLIT_MIN) it runs split-KV (flash-decoding,
 * shaders/flash_decode_split.comp + flash_decode_reduce.comp) when a KV
 * head serves <= 8 query heads; above 16384 positions that is required.
 * Below the split threshold n_kv_heads*head_dim must be <= 131072.
 * The split partials live in a backend-owned workspace. */
int yule_hip_gqa_decode_attn(yule_hip_backend *be, yule_buffer q, yule_buffer k_cache,
                             yule_buffer v_cache, yule_buffer out, uint32_t n_heads,
                             uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq_len);

/* Greedy argmax over f32[n] written as one u32 into out (argmax_ct,
 * yule-infer/src/sampler.rs:150-163: the last maximal index wins). */
int yule_hip_argmax(yule_hip_backend *be, yule_buffer in, uint32_t n, yule_buffer out);

/* Prefill dequant-GEMM (no counterpart in the reference, whose prefill runs
 * token by token, yule-infer/src/model_runner.rs:1075-1081):
 * Y[m][r] = sum_c X[m][c] * W[r][c] for m < M, with X bf16 [M][n_cols]
 * (row-major), W raw GGUF blocks as in quantized_matmul, Y f32 [M][n_rows].
 * Runs on the MFMA units; Q4_0, Q4_K, Q5_K, Q6_K, Q8_0 and Q8_K (other
 * dtypes return YULE_ERR_UNSUPPORTED), n_cols a multiple of 256, M any
 * positive size.  Any finite bf16 row is accepted: each row is scaled by a
 * power of two into f16 range for the matrix cores and the scale is undone
 * exactly on Y (rows holding inf or NaN give inf/NaN outputs, as the f32 sum
 * would).  Each row of Y meets the matvec bar against the f32 matvec of the
 * same (bf16-valued) row.  Weights aliasing x or y are rejected. */
int yule_hip_quantized_gemm(yule_hip_backend *be, yule_buffer weights, yule_buffer x_bf16,
                            yule_buffer y, uint32_t m, uint32_t n_rows, uint32_t n_cols,
                            uint32_t dtype);

/* The same product for f32 X [M][n_cols] (no counterpart in the reference):
 * each row is split into f16 hi + lo after its power-of-two scale
 * (x = hi + lo to ~2^-22) and Y = X_hi W + X_lo W, both products swept
 * into the same accumulators in one launch, so
 * each row matches the f32 matvec of the same row to the matvec bar at f32
 * accuracy (the batched prefill of the runner, whose KV cache must equal
 * token-by-token decode's).  Same formats, shapes, aliasing rules and
 * workspace use as yule_hip_quantized_gemm. */
int yule_hip_quantized_gemm_f32(yule_hip_backend *be, yule_buffer weights, yule_buffer x_f32,
                                yule_buffer y, uint32_t m, uint32_t n_rows, uint32_t n_cols,
                                uint32_t dtype);

/* Allocation-free variant of yule_hip_quantized_gemm (no counterpart in the
 * reference; for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * It runs the same kernels with its workspace in a static 32 MiB device
 * array per GPU (the library holds it until the process ends) instead of
 * the backend's grown-on-demand workspace; it calls no allocator.  Calls
 * whose workspace would exceed 32 MiB (X in f16 plus split-K partials, e.g.
 * M = 2048 at n_cols = 14336) return YULE_ERR_INVALID.  Every call on a GPU
 * shares that GPU's array: calls that can overlap on one GPU (other streams,
 * other backends on the same device) race; calls on one stream are ordered.
 * The array needs no clearing between calls (every byte a call reads was
 * written by that call). */
int yule_hip_quantized_gemm_noalloc(yule_hip_backend *be, yule_buffer weights, yule_buffer x_bf16,
                                    yule_buffer y, uint32_t m, uint32_t n_rows, uint32_t n_cols,
                                    uint32_t dtype);

/* ---- decode runner (yule-infer GpuTransformerRunner counterpart) ---- */

/* One transformer layer's tensors as host pointers to raw GGUF data
 * (weight_loader.rs:158-199 names: blk.N.attn_norm, attn_q, attn_k, attn_v,
 * attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down).  Matrices are
 * [rows][cols] blocks of a quantized dtype; norms are F32 or F16. */
typedef struct {
    const void *attn_norm;
    uint32_t attn_norm_dtype;
    const void *wq, *wk, *wv, *wo;
    uint32_t wq_dtype, wk_dtype, wv_dtype, wo_dtype;
    const void *ffn_norm;
    uint32_t ffn_norm_dtype;
    const void *w_gate, *w_up, *w_down;
    uint32_t w_gate_dtype, w_up_dtype, w_down_dtype;
} yule_layer_desc;

/* Dense Llama-family model (RunnerConfig, model_runner.rs:384-465):
 * head_dim = dim / n_heads, RoPE over the full head dimension, SwiGLU FFN. */
typedef struct {
    uint32_t n_layers, dim, n_heads, n_kv_heads, ff_dim, vocab, max_seq;
    float norm_eps, rope_base;
    const void *token_embd;
    uint32_t token_embd_dtype;
    const void *output_norm;
    uint32_t output_norm_dtype;
    const void *output;
    uint32_t output_dtype;
    const yule_layer_desc *layers; /* n_layers entries */
} yule_model_desc;

typedef struct yule_hip_runner yule_hip_runner;

/* TransformerRunner::new (model_runner.rs:384-531): uploads every tensor
 * once (gpu_runner.rs:171-254), allocates the f32 KV cache
 * [n_layers][max_seq][n_kv_heads*head_dim] and the RoPE table.  The host
 * tensors may be released after the call. */
int yule_hip_runner_create(yule_hip_backend *be, const yule_model_desc *model, yule_hip_runner **out);
int yule_hip_runner_destroy(yule_hip_runner *r);
/* ModelRunner::reset (model_runner.rs:1087-1092): position back to 0. */
int yule_hip_runner_reset(yule_hip_runner *r);
uint32_t yule_hip_runner_pos(const yule_hip_runner *r);
/* ModelRunner::decode_step (model_runner.rs:1083-1085): forward one token
 * at the current position; logits (f32[vocab]) copied out when non-null.
 * Fails with "context length exceeded" at pos == max_seq (:538-540). */
int yule_hip_runner_decode_step(yule_hip_runner *r, uint32_t token, float *logits);
/* ModelRunner::prefill (model_runner.rs:1075-1081): token by token; logits
 * of the last token when non-null. */
int yule_hip_runner_prefill(yule_hip_runner *r, const uint32_t *tokens, uint32_t n, float *logits);
/* The same prefill with the n tokens as one batch (no counterpart in the
 * reference, which prefills token by token): each layer runs its projections
 * as f32-X GEMMs on the matrix cores (yule_hip_quantized_gemm_f32), RoPE and
 * the KV-cache rows for all n positions, and causal attention per row; the
 * last row then goes through the final norm, lm_head and argmax as the
 * token-by-token prefill's last step would.  KV cache and logits equal the
 * token-by-token ones to f32 rounding.  Needs every projection in a GEMM
 * format with columns a multiple of 256 and head_dim 32, 64, 128 or 256;
 * otherwise YULE_ERR_UNSUPPORTED.  generate_greedy prefills this way whenever
 * it can (environment YULE_RUNNER_TOKEN_PREFILL at runner creation: token by
 * token). */
int yule_hip_runner_prefill_batched(yule_hip_runner *r, const uint32_t *tokens, uint32_t n, float *logits);
/* Milliseconds the prompt pass of the last generate_greedy took (HIP events). */
float yule_hip_runner_last_prefill_ms(const yule_hip_runner *r);
/* Greedy generation from position 0 entirely on the device: n_prompt
 * prompt tokens, then n_decode decode steps fed by argmax_ct
 * (sampler.rs:150-163).  out_tokens receives n_decode + 1 ids: the argmax
 * after the last prompt token and after each decode step.  When non-null,
 * ms_per_decode_step is the mean of the decode steps, from HIP events on
 * the backend stream (the yule-validate/src/performance.rs:303-337
 * tokens/s method: 1000 / ms). */
int yule_hip_runner_generate_greedy(yule_hip_runner *r, const uint32_t *prompt, uint32_t n_prompt,
                                    uint32_t n_decode, uint32_t *out_tokens, float *ms_per_decode_step);

/* ---- GGUF v3 files (yule-core/src/gguf.rs) ---- */

typedef struct yule_gguf yule_gguf;

/* TensorInfo (yule-core/src/tensor.rs) of one tensor of a mapped file. */
typedef struct {
    const char *name;     /* owned by the yule_gguf */
    uint32_t dtype;       /* GGUF type id (dtype.rs:155-190) */
    uint32_t n_dims;
    uint64_t dims[8];     /* GGUF order: dims[0] is the row length; unused = 1 */
    uint64_t offset;      /* relative to the data section */
    uint64_t size_bytes;
    const void *data;     /* mapped bytes, valid until yule_hip_gguf_close */
} yule_gguf_tensor;

/* GgufParser::parse_file (gguf.rs:255-432): read-only mapping, magic and
 * version 3, the reference's limits (strings <= 1 MiB, <= 100k tensors and
 * metadata pairs, arrays <= 10M, <= 8 dims), data section at the header end
 * rounded up to general.alignment (default 32), tensors inside the file and
 * not overlapping.  Errors: YULE_ERR_IO, YULE_ERR_PARSE. */
int yule_hip_gguf_open(const char *path, yule_gguf **out);
int yule_hip_gguf_close(yule_gguf *g);
int yule_hip_gguf_header(const yule_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset,
                         uint64_t *n_tensors, uint64_t *n_kv);
int yule_hip_gguf_tensor(const yule_gguf *g, uint64_t index, yule_gguf_tensor *out);
int yule_hip_gguf_find(const yule_gguf *g, const char *name, yule_gguf_tensor *out);
/* metadata lookups with GgufValue::as_u32 / as_f64 / as_str semantics
 * (gguf.rs:50-90); YULE_ERR_INVALID when absent or of another type */
int yule_hip_gguf_get_u32(const yule_gguf *g, const char *key, uint32_t *out);
int yule_hip_gguf_get_f64(const yule_gguf *g, const char *key, double *out);
int yule_hip_gguf_get_str(const yule_gguf *g, const char *key, const char **out);
int yule_hip_gguf_get_array_len(const yule_gguf *g, const char *key, uint64_t *out);

/* yule_hip_runner_create from a GGUF file of a dense Llama model
 * (general.architecture llama or mistral): llama.* metadata and blk.N.*
 * tensor names (weight_loader.rs:78-199), RunnerConfig defaults
 * (model_runner.rs:384-465).  max_seq 0 takes llama.context_length. */
int yule_hip_runner_create_from_gguf(yule_hip_backend *be, const char *path, uint32_t max_seq,
                                     yule_hip_runner **out);

/* ---- timing helpers for harnesses (no trait counterpart) ---- */

/* One quantized_matmul (n_mats == 1) or quantized_matmul_multi call, for
 * the timing helper below. */
typedef struct {
    uint32_t n_mats;
    yule_buffer weights[4], outputs[4];
    uint32_t n_rows[4];
    yule_buffer input;
    uint32_t n_cols, dtype;
} yule_qmv_op;

/* Run the list `ops` `iters` times on the backend stream and report the
 * elapsed milliseconds between two HIP events recorded on that stream
 * around all iterations.  With use_graph != 0 the list is captured once
 * into a HIP graph and replayed, so host launch latency does not enter the
 * measurement.  Callers cycle distinct weight copies through `ops` so that
 * no launch re-reads a matrix left in the 256 MB last-level cache. */
int yule_hip_time_qmv_ops(yule_hip_backend *be, const yule_qmv_op *ops, uint32_t n_ops, uint32_t iters,
                          int use_graph, float *ms_total);

/* Roofline probe: one launch that streams `bytes` (a multiple of 16) of
 * `src` with n_partials 256-thread workgroups (grid-stride 16-byte loads)
 * and writes, per workgroup, the XOR of every 32-bit word it read to
 * partials[i] (the XOR of all partials is the XOR of the whole range).  It
 * measures what a single launch that only reads the same bytes achieves,
 * beside the quantized kernels' own rates.  No reference counterpart. */
int yule_hip_read_probe(yule_hip_backend *be, yule_buffer src, uint64_t bytes, yule_buffer partials,
                        uint32_t n_partials);

/* Variants of the read probe (same arguments, same partials), to map the
 * single-launch read rate against the access pattern: pattern 0 =
 * grid-stride 16-byte words with `loads` (1, 2, 4 or 8) independent loads in
 * flight per lane; 1 = a run of `loads` consecutive 16-byte words per lane
 * (16, 32, 64 or 128-byte runs), runs grid-strided; 2 = one contiguous chunk
 * per workgroup, consecutive words across its lanes, `loads` in flight.
 * No reference counterpart. */
/* MFMA issue-rate probe (no reference counterpart): n_wg workgroups of 256
 * threads (four waves), each wave running `chains` (1, 2, 4 or 8)
 * independent accumulator chains of `iters` MFMAs with no memory traffic in
 * the loop: shape 0 = v_mfma_f32_16x16x32_f16 (16384 flops each), 1 =
 * v_mfma_f32_32x32x16_f16 (32768 flops).  Operands are the 128 16-byte words
 * of `in` (f16 values); one float per thread goes to `out` (n_wg * 1 KiB).
 * Time it with timer_start / timer_stop. */
int yule_hip_mfma_probe(yule_hip_backend *be, yule_buffer in, yule_buffer out, uint32_t shape, uint32_t chains,
                        uint32_t n_wg, uint32_t iters);

int yule_hip_read_probe_variant(yule_hip_backend *be, yule_buffer src, uint64_t bytes, yule_buffer partials,
                                uint32_t n_partials, uint32_t pattern, uint32_t loads);

/* Launch-overhead probe: n_kernels launches of an empty kernel (one
 * workgroup of 64 threads that returns at once), run `iters` times, captured
 * into one HIP graph when use_graph != 0; writes the elapsed milliseconds
 * between HIP events on the backend stream around all iterations.  It
 * measures the fixed cost of a kernel boundary that every launch of a
 * decode step pays.  No reference counterpart. */
int yule_hip_time_empty_launches(yule_hip_backend *be, uint32_t n_kernels, uint32_t iters, int use_graph,
                                 float *ms_total);

/* Event timer on the backend stream: timer_start records a start event;
 * timer_stop records a stop event after everything enqueued since, waits
 * for it and writes the elapsed milliseconds. */
int yule_hip_timer_start(yule_hip_backend *be);
int yule_hip_timer_stop(yule_hip_backend *be, float *ms);

/* Graph-capture harness (no reference counterpart): capture_begin starts a
 * HIP stream capture of the backend stream (thread-local mode: only calls
 * from this thread are captured, and they are recorded, not run);
 * capture_end ends it and instantiates the graph (replacing any earlier
 * one); capture_replay launches the instantiated graph on the backend
 * stream.  Used to check that an entry point enqueues cleanly under
 * capture (no allocation, no synchronization) and that replays give the
 * eager result. */
int yule_hip_capture_begin(yule_hip_backend *be);
int yule_hip_capture_end(yule_hip_backend *be);
int yule_hip_capture_replay(yule_hip_backend *be);

#ifdef __cplusplus
}
#endif
#endif
