// runner.cpp — decode runner over the HIP backend: the counterpart of
// yule-infer's GpuTransformerRunner (yule-infer/src/gpu_runner.rs:171-695)
// with the CPU TransformerRunner's forward-pass semantics
// (yule-infer/src/model_runner.rs:533-1036; dense Llama branch).
//
// Device-resident decode: weights are uploaded once as raw GGUF blocks;
// embedding lookup, every projection, RoPE, the KV-cache write, attention,
// SwiGLU, the residual adds, the final norm, the lm_head and the greedy
// argmax all run on the GPU.  The step reads its position and input token
// from a device control block (ctl = {pos, token, prompt_len}), so one HIP
// graph captured once replays every step, prefill and decode alike; the
// argmax kernel writes the next token and advances the position.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "internal.h"

using namespace yule;

// most decode steps captured into one replayed graph
constexpr long kMaxGraphSteps = 64;

struct yule_hip_runner {
    yule_hip_backend *be = nullptr;
    uint32_t n_layers = 0, dim = 0, n_heads = 0, n_kv = 0, hd = 0, ff = 0, vocab = 0, max_seq = 0;
    float eps = 1e-5f, rope_base = 10000.f;
    std::vector<void *> allocs;
    struct Layer {
        float *attn_norm, *ffn_norm;
        const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
        uint32_t tq, tk, tv, to, tg, tu, td;
        float *kc, *vc;
    };
    std::vector<Layer> layers;
    const uint8_t *embd = nullptr, *out_w = nullptr;
    uint32_t embd_t = 0, out_t = 0;
    float *out_norm = nullptr, *cos_t = nullptr, *sin_t = nullptr;
    float *hidden, *normed, *q, *k, *v, *attn, *proj, *gate, *up, *ffn, *logits;
    uint32_t *ctl = nullptr, *prompt = nullptr, *tokens = nullptr;
    uint32_t *ctl_host = nullptr;  // pinned staging for ctl updates
    unsigned long long *amax = nullptr;  // lm_head argmax slots, one per workgroup (packed key | row)
    bool fused = false;            // every matrix runs on the streaming matvec
    // attention of steps whose sequence length (pos + 1) reaches split_min
    // runs split-KV (attn_split_kernel + combine, partials in attn_ws);
    // shorter ones run one workgroup per query head.  One captured graph
    // per variant: [0] short, [1] split.
    uint32_t split_min = 0;
    void *attn_ws = nullptr;
    // shorter steps, when the Q/K/V launch can rotate and write the cache
    // itself (kEpiRope): chunked attention with in-launch combine (partials
    // and per-head tickets in chunk_ws, zeroed at creation)
    void *chunk_ws = nullptr;
    // batched prefill (prefill_rows): row buffers for max_seq rows and the
    // GEMM workspace, allocated at the first batched prefill
    bool batchable = false;
    float *bx = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr, *ba = nullptr, *bg = nullptr,
          *bu = nullptr;
    // [q | k | v] and [gate | up] rows of the layers whose projections share
    // a format (one GEMM each)
    float *bqkv = nullptr, *bgu = nullptr;
    void *bws = nullptr;
    size_t bws_size = 0;
    float last_prefill_ms = 0.f;
    hipGraph_t graph[2] = {nullptr, nullptr};
    hipGraphExec_t exec[2] = {nullptr, nullptr};
    // multi_steps of the same step per graph: generate_greedy replays these
    // over runs of decode steps of one variant (one graph launch per
    // multi_steps tokens: each launch of a graph costs ~7 us of idle GPU)
    uint32_t multi_steps = 8;   // at most kMaxGraphSteps
    // experimental: launches carry extra workgroups that read the next
    // launch's weights into its XCDs' L2 (bit 1: O -> gate/up, 2: gate/up ->
    // down, 4: Q/K/V -> O)
    uint32_t pf_mask = 4 | 8, pf_wgs = 256, pf_delay = 0;
    hipGraph_t graph_n[2] = {nullptr, nullptr};
    hipGraphExec_t exec_n[2] = {nullptr, nullptr};
    uint32_t pos = 0;  // host mirror of ctl[0]
};

namespace {


int set_ctl(yule_hip_runner *r, uint32_t pos, uint32_t token, uint32_t prompt_len);
int enqueue_head(yule_hip_runner *r);

int dev_alloc(yule_hip_runner *r, size_t bytes, void **p) {
    int rc = hip_error(hipMalloc(p, bytes + kAllocSlack), "runner: allocate");
    if (rc) return rc;
    r->allocs.push_back(*p);
    return hip_error(hipMemset(*p, 0, bytes + kAllocSlack), "runner: zero-fill");
}

int upload(yule_hip_runner *r, const void *src, size_t bytes, void **dst) {
    int rc = dev_alloc(r, bytes, dst);
    if (rc) return rc;
    return hip_error(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice), "runner: upload");
}

// f32 copy of a norm weight given as F32 or F16 (f16_to_f32 is exact;
// model_runner.rs:257-271 reads either)
int upload_norm(yule_hip_runner *r, const void *src, uint32_t dtype, uint32_t n, float **dst) {
    if (!src) return set_error(YULE_ERR_INVALID, "runner: missing norm weight");
    std::vector<float> tmp(n);
    if (dtype == YULE_DTYPE_F32) {
        std::memcpy(tmp.data(), src, (size_t)n * 4);
    } else if (dtype == YULE_DTYPE_F16) {
        const uint16_t *h = static_cast<const uint16_t *>(src);
        for (uint32_t i = 0; i < n; i++) {
            const uint32_t s = (h[i] >> 15) & 1u, e = (h[i] >> 10) & 0x1Fu, m = h[i] & 0x3FFu;
            uint32_t bits;
            if (e == 0) {
                if (m == 0) bits = s << 31;
                else {
                    uint32_t mm = m;
                    int ee = -14;
                    while (!(mm & 0x400u)) { mm <<= 1; ee--; }
                    bits = (s << 31) | ((uint32_t)(ee + 127) << 23) | ((mm & 0x3FFu) << 13);
                }
            } else if (e == 31) bits = (s << 31) | (0xFFu << 23) | (m << 13);
            else bits = (s << 31) | ((e - 15 + 127) << 23) | (m << 13);
            std::memcpy(&tmp[i], &bits, 4);
        }
    } else {
        return set_error(YULE_ERR_UNSUPPORTED, "runner: norm weights must be F32 or F16");
    }
    return upload(r, tmp.data(), (size_t)n * 4, reinterpret_cast<void **>(dst));
}

int upload_matrix(yule_hip_runner *r, const void *src, uint32_t dtype, uint32_t rows, uint32_t cols, const char *name,
                  const uint8_t **dst) {
    uint32_t bs, bb;
    if (!src) return set_error(YULE_ERR_INVALID, std::string("runner: missing tensor ") + name);
    if (!quant_geometry(dtype, &bs, &bb))
        return set_error(YULE_ERR_UNSUPPORTED, std::string("runner: ") + name + " has unsupported dtype " +
                                                   std::to_string(dtype));
    if (cols % bs)
        return set_error(YULE_ERR_INVALID, std::string("runner: ") + name + " columns not a block multiple");
    return upload(r, src, (size_t)rows * (cols / bs) * bb, reinterpret_cast<void **>(const_cast<uint8_t **>(dst)));
}

// Final norm + lm_head + argmax over r->hidden, then advance the control
// block (model_runner.rs:1008-1025, sampler.rs:150-163).
int enqueue_head(yule_hip_runner *r) {
    hipStream_t s = r->be->stream;
    int rc;
    if (r->fused) {
        QmvXf head;
        head.mode = kXfRmsNorm;
        head.a = r->out_norm;
        head.eps = r->eps;
        head.epi = kEpiArgmax;
        head.amax = r->amax;
        const QmvSeg so{r->out_w, r->logits, r->vocab};
        if ((rc = launch_qmv_fused(s, r->out_t, &so, 1, r->hidden, r->dim, head))) return rc;
        return launch_advance(s, r->amax, r->ctl, r->tokens);
    }
    if ((rc = launch_rms_norm(s, r->hidden, r->out_norm, r->normed, r->dim, r->eps))) return rc;
    if ((rc = launch_qmv(s, r->out_t, r->out_w, r->normed, r->logits, r->vocab, r->dim))) return rc;
    return launch_argmax_advance(s, r->logits, r->vocab, r->ctl, r->tokens);
}

// One decode step for the token selected by ctl, entirely on r->be->stream.
// Per layer, when every matrix runs on the streaming matvec (fusable):
//   [rms_norm + Q/K/V] [RoPE + KV write + attention] [O + residual]
//   [rms_norm + gate/up + SwiGLU] [down + residual]
// (SwiGLU moves into the down launch's staging when gate/up cannot pair)
// and at the end [rms_norm + lm_head + argmax] [advance]; otherwise the
// same operations as separate kernels.
// Point xf's prefetch workgroups at the weights of a following launch: one
// matrix of n_rows x n_cols, or a gate/up pair (w1 = up) of that shape;
// nothing when that launch's grid gives no group-to-XCD mapping.
static void plan_prefetch(const yule_hip_runner *r, QmvXf &xf, uint32_t dtype, const uint8_t *w0, const uint8_t *w1,
                          uint32_t n_rows, uint32_t n_cols) {
    uint32_t gb = 0, groups = 0, rpg = 0, bs = 0, bb = 0;
    if (!r->pf_wgs || !qmv_group_plan(dtype, n_rows, n_cols, w1 != nullptr, &gb, &groups, &rpg) ||
        !quant_geometry(dtype, &bs, &bb))
        return;
    xf.pf_w[0] = w0;
    xf.pf_w[1] = w1;
    xf.pf_wgs = r->pf_wgs;
    xf.pf_gbytes = gb;
    xf.pf_groups = groups;
    xf.pf_delay = r->pf_delay;
    xf.pf_total = (size_t)n_rows * (n_cols / bs) * bb;
}

int enqueue_step(yule_hip_runner *r, bool split) {
    hipStream_t s = r->be->stream;
    const uint32_t qd = r->n_heads * r->hd, kvd = r->n_kv * r->hd;
    int rc;
    const bool fuse = r->fused;
    if ((rc = launch_embed_step(s, r->embd_t, r->embd, r->ctl, r->prompt, r->vocab, r->hidden, r->dim)))
        return rc;
    for (const auto &L : r->layers) {
        // attention block (model_runner.rs:619-784)
        QmvXf norm;
        norm.mode = kXfRmsNorm;
        norm.a = L.attn_norm;
        norm.eps = r->eps;
        const float *xin = r->normed;
        if (!fuse) {
            if ((rc = launch_rms_norm(s, r->hidden, L.attn_norm, r->normed, r->dim, r->eps))) return rc;
            norm = QmvXf{};
        } else {
            xin = r->hidden;
        }
        const bool chunked = fuse && !split && r->chunk_ws && L.tq == L.tk && L.tk == L.tv &&
                             qmv_rope_ok(L.tq, r->dim, r->hd);
        if (chunked) {   // RoPE and the cache write in the Q/K/V launch's epilogue
            norm.epi = kEpiRope;
            norm.ctl = r->ctl;
            norm.cos_t = r->cos_t;
            norm.sin_t = r->sin_t;
            norm.kc = L.kc;
            norm.vc = L.vc;
            norm.hd = r->hd;
        }
        if ((r->pf_mask & 4) && fuse) plan_prefetch(r, norm, L.to, L.wo, nullptr, r->dim, qd);
        // bit 8: those prefetch workgroups also read the layer's K/V cache
        // rows before the position, for the chunked attention launch
        if ((r->pf_mask & 8) && chunked && norm.pf_wgs) norm.pf_delay |= 1u << 31;
        if (L.tq == L.tk && L.tk == L.tv) {
            const QmvSeg segs[3] = {{L.wq, r->q, qd}, {L.wk, r->k, kvd}, {L.wv, r->v, kvd}};
            if ((rc = launch_qmv_fused(s, L.tq, segs, 3, xin, r->dim, norm))) return rc;
        } else {
            const QmvSeg sq{L.wq, r->q, qd}, sk{L.wk, r->k, kvd}, sv{L.wv, r->v, kvd};
            if ((rc = launch_qmv_fused(s, L.tq, &sq, 1, xin, r->dim, norm)) ||
                (rc = launch_qmv_fused(s, L.tk, &sk, 1, xin, r->dim, norm)) ||
                (rc = launch_qmv_fused(s, L.tv, &sv, 1, xin, r->dim, norm)))
                return rc;
        }
        if (chunked)
            rc = launch_attn_chunks(s, r->q, L.kc, L.vc, r->ctl, r->attn, r->chunk_ws, r->n_heads, r->n_kv, r->hd,
                                    std::min(r->max_seq, r->split_min), 0u);
        else if (split)
            rc = launch_attn_split(s, r->q, r->k, r->v, L.kc, L.vc, r->cos_t, r->sin_t, r->ctl, r->attn, r->attn_ws,
                                   r->n_heads, r->n_kv, r->hd, r->max_seq);
        else
            rc = launch_attn_step(s, r->q, r->k, r->v, L.kc, L.vc, r->cos_t, r->sin_t, r->ctl, r->attn, r->n_heads,
                                  r->n_kv, r->hd, std::min(r->max_seq, r->split_min));
        if (rc) return rc;
        if (fuse) {
            QmvXf add;
            add.epi = kEpiAdd;
            if ((r->pf_mask & 1) && L.tg == L.tu && qmv_pairable(L.tg, r->dim))
                plan_prefetch(r, add, L.tg, L.wg, L.wu, r->ff, r->dim);
            const QmvSeg so{L.wo, r->hidden, r->dim};
            if ((rc = launch_qmv_fused(s, L.to, &so, 1, r->attn, qd, add))) return rc;
        } else {
            if ((rc = launch_qmv(s, L.to, L.wo, r->attn, r->proj, r->dim, qd))) return rc;
            if ((rc = launch_eltwise(s, 2, r->hidden, r->proj, r->hidden, r->dim))) return rc;
        }
        // feed-forward block (model_runner.rs:792-1004)
        norm = QmvXf{};
        if (fuse) {
            norm.mode = kXfRmsNorm;
            norm.a = L.ffn_norm;
            norm.eps = r->eps;
        } else if ((rc = launch_rms_norm(s, r->hidden, L.ffn_norm, r->normed, r->dim, r->eps))) {
            return rc;
        }
        const bool pair = fuse && L.tg == L.tu && qmv_pairable(L.tg, r->dim);
        if (pair) {   // gate/up + SwiGLU in one launch; act lands in r->gate
            norm.pair = true;
            if (r->pf_mask & 2) plan_prefetch(r, norm, L.td, L.wd, nullptr, r->dim, r->ff);
            const QmvSeg segs[2] = {{L.wg, r->gate, r->ff}, {L.wu, r->up, r->ff}};
            if ((rc = launch_qmv_fused(s, L.tg, segs, 2, xin, r->dim, norm))) return rc;
        } else if (L.tg == L.tu) {
            const QmvSeg segs[2] = {{L.wg, r->gate, r->ff}, {L.wu, r->up, r->ff}};
            if ((rc = launch_qmv_fused(s, L.tg, segs, 2, xin, r->dim, norm))) return rc;
        } else {
            const QmvSeg sg{L.wg, r->gate, r->ff}, su{L.wu, r->up, r->ff};
            if ((rc = launch_qmv_fused(s, L.tg, &sg, 1, xin, r->dim, norm)) ||
                (rc = launch_qmv_fused(s, L.tu, &su, 1, xin, r->dim, norm)))
                return rc;
        }
        if (fuse) {
            QmvXf sw;
            sw.mode = pair ? kXfNone : kXfSwiGlu;
            sw.a = pair ? nullptr : r->up;
            sw.epi = kEpiAdd;
            const QmvSeg sd{L.wd, r->hidden, r->dim};
            if ((rc = launch_qmv_fused(s, L.td, &sd, 1, r->gate, r->ff, sw))) return rc;
        } else {
            if ((rc = launch_eltwise(s, 3, r->gate, r->up, r->gate, r->ff))) return rc;
            if ((rc = launch_qmv(s, L.td, L.wd, r->gate, r->ffn, r->dim, r->ff))) return rc;
            if ((rc = launch_eltwise(s, 2, r->hidden, r->ffn, r->hidden, r->dim))) return rc;
        }
    }
    return enqueue_head(r);
}

// Capture `steps` decode steps into *graph and instantiate *exec.  On any
// failure after the capture began, the graph is destroyed and both slots are
// left null, so a later call captures afresh without leaking the old graph.
static int capture_steps(yule_hip_runner *r, bool split, uint32_t steps, hipGraph_t *graph, hipGraphExec_t *exec) {
    if (*graph) {   // a graph whose instantiation failed earlier
        (void)hipGraphDestroy(*graph);
        *graph = nullptr;
    }
    hipStream_t s = r->be->stream;
    int rc = hip_error(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "runner: begin capture");
    if (rc) return rc;
    int erc = YULE_OK;
    for (uint32_t i = 0; i < steps && !erc; i++) erc = enqueue_step(r, split);
    rc = hip_error(hipStreamEndCapture(s, graph), "runner: end capture");
    if (!erc && !rc)
        rc = hip_error(hipGraphInstantiate(exec, *graph, nullptr, nullptr, 0), "runner: graph instantiate");
    if (erc || rc) {
        if (*graph) (void)hipGraphDestroy(*graph);
        *graph = nullptr;
        *exec = nullptr;
        return erc ? erc : rc;
    }
    return YULE_OK;
}

int ensure_graph(yule_hip_runner *r, bool split) {
    if (r->exec[split]) return YULE_OK;
    return capture_steps(r, split, 1, &r->graph[split], &r->exec[split]);
}

// generate_greedy's runs of decode steps replay multi-step graphs (not with
// YULE_RUNNER_NO_GRAPH, and not when the runner's multi_steps is 1)
bool multi_ok(const yule_hip_runner *r) {
    static const bool direct = getenv("YULE_RUNNER_NO_GRAPH") != nullptr;
    return !direct && r->multi_steps > 1;
}

int ensure_graph_n(yule_hip_runner *r, bool split) {
    if (r->exec_n[split]) return YULE_OK;
    return capture_steps(r, split, r->multi_steps, &r->graph_n[split], &r->exec_n[split]);
}

// Replay the captured step for position `pos`, or (YULE_RUNNER_NO_GRAPH set,
// for tracing profilers that do not follow graph launches) enqueue its
// kernels directly.
int run_step(yule_hip_runner *r, uint32_t pos) {
    static const bool direct = getenv("YULE_RUNNER_NO_GRAPH") != nullptr;
    const bool split = pos + 1 >= r->split_min;
    if (direct) return enqueue_step(r, split);
    int rc = ensure_graph(r, split);
    if (rc) return rc;
    return hip_error(hipGraphLaunch(r->exec[split], r->be->stream), "runner: graph launch");
}

// Q/K/V (gate/up) of a layer as one GEMM: one format, rows multiples of 256
bool qkv_one(const yule_hip_runner *r, const yule_hip_runner::Layer &L) {
    const uint32_t qd = r->n_heads * r->hd, kvd = r->n_kv * r->hd, rows[3] = {qd, kvd, kvd};
    return L.tq == L.tk && L.tk == L.tv && gemm_multi_ok(L.tq, r->dim, rows, 3);
}
bool gu_one(const yule_hip_runner *r, const yule_hip_runner::Layer &L) {
    const uint32_t rows[2] = {r->ff, r->ff};
    return L.tg == L.tu && gemm_multi_ok(L.tg, r->dim, rows, 2);
}

// GEMM workspace the batched pass over n rows needs (the largest of its
// products)
size_t batch_workspace(const yule_hip_runner *r, uint32_t n) {
    const uint32_t qd = r->n_heads * r->hd, kvd = r->n_kv * r->hd;
    size_t need = 0;
    for (const auto &L : r->layers) {
        const size_t w[7] = {gemm_f32_workspace_bytes(n, qd, r->dim, L.tq), gemm_f32_workspace_bytes(n, kvd, r->dim, L.tk),
                             gemm_f32_workspace_bytes(n, kvd, r->dim, L.tv), gemm_f32_workspace_bytes(n, r->dim, qd, L.to),
                             gemm_f32_workspace_bytes(n, r->ff, r->dim, L.tg), gemm_f32_workspace_bytes(n, r->ff, r->dim, L.tu),
                             gemm_f32_workspace_bytes(n, r->dim, r->ff, L.td)};
        for (size_t v : w) need = std::max(need, v);
        const uint32_t qkv[3] = {qd, kvd, kvd}, gu[2] = {r->ff, r->ff};
        if (qkv_one(r, L)) need = std::max(need, gemm_f32_multi_workspace_bytes(n, qkv, 3, r->dim, L.tq));
        if (gu_one(r, L)) need = std::max(need, gemm_f32_multi_workspace_bytes(n, gu, 2, r->dim, L.tg));
    }
    return need;
}

int ensure_batch(yule_hip_runner *r, uint32_t n) {
    const uint32_t qd = r->n_heads * r->hd, kvd = r->n_kv * r->hd;
    int rc;
    if (!r->bx) {
        struct { float **p; size_t n; } bufs[] = {
            {&r->bx, r->dim}, {&r->bq, qd}, {&r->bk, kvd}, {&r->bv, kvd},
            {&r->ba, qd}, {&r->bg, r->ff}, {&r->bu, r->ff}, {&r->bqkv, qd + 2 * kvd},
            {&r->bgu, 2 * r->ff}};
        for (auto &b : bufs)
            if ((rc = dev_alloc(r, (size_t)r->max_seq * b.n * 4, reinterpret_cast<void **>(b.p)))) return rc;
    }
    // two workspaces: a product whose split-K reduction is left to the next
    // product's pre-pass keeps its partials in one while the next runs in
    // the other
    const size_t need = 2 * ((batch_workspace(r, n) + 255) & ~(size_t)255);
    if (need > r->bws_size) {
        if (r->bws) {
            if ((rc = hip_error(hipStreamSynchronize(r->be->stream), "runner: synchronize"))) return rc;
            hipFree(r->bws);
            r->bws = nullptr;
            r->bws_size = 0;
        }
        if ((rc = hip_error(hipMalloc(&r->bws, need), "runner: prefill workspace"))) return rc;
        r->bws_size = need;
    }
    return YULE_OK;
}

// The prompt tokens at r->prompt[pos0, pos0 + n) through every layer as n
// rows at once (prefill.hip; projections as f32-X GEMMs: RMSNorm folded into
// the GEMM's X pre-pass, Q/K/V and gate/up one product each where they share
// a format, the residual adds in the O and down products), writing KV rows
// pos0.. pos0 + n - 1; then the head over the last row, as the decode step
// for position pos0 + n - 1 would run it, with ctl = {pos0 + n - 1, -,
// prompt_len}: the argmax lands in tokens[pos0 + n - 1] and ctl[1], and ctl[0]
// moves to pos0 + n.  ctl_ready: the caller has already written that control
// block (set_ctl synchronizes the stream, so a timed caller does it first).
int prefill_rows(yule_hip_runner *r, uint32_t pos0, uint32_t n, uint32_t prompt_len, bool ctl_ready = false) {
    hipStream_t s = r->be->stream;
    const uint32_t qd = r->n_heads * r->hd, kvd = r->n_kv * r->hd;
    int rc;
    if ((rc = ensure_batch(r, n))) return rc;
    // the control block only feeds the head and advance at the end
    if (!ctl_ready && (rc = set_ctl(r, pos0 + n - 1, 0, prompt_len))) return rc;
    // products alternate between the two workspaces; the O, gate/up and down
    // products leave their split-K reduction to the next product's pre-pass
    // (red), which reads their X right after (except the last down: the head
    // reads its rows)
    void *wsv[2] = {r->bws, static_cast<uint8_t *>(r->bws) + r->bws_size / 2};
    uint32_t wi = 0;
    auto next_ws = [&]() { return wsv[wi ^= 1]; };
    GemmRed red{}, none{};
    if ((rc = launch_embed_rows_batch(s, r->embd_t, r->embd, r->prompt + pos0, r->vocab, r->bx, r->dim, n))) return rc;
    const uint32_t qkv_rows[3] = {qd, kvd, kvd}, gu_rows[2] = {r->ff, r->ff};
    for (size_t li = 0; li < r->layers.size(); li++) {
        const auto &L = r->layers[li];
        const bool last = li + 1 == r->layers.size();
        // q, k, v rows: one [q | k | v] product when the three share a format
        const float *q = r->bq, *k = r->bk, *v = r->bv;
        uint32_t ldq = qd, ldkv = kvd;
        if (qkv_one(r, L)) {
            const uint8_t *w[3] = {L.wq, L.wk, L.wv};
            if ((rc = launch_gemm_f32_multi(s, w, qkv_rows, 3, r->bx, r->bqkv, n, r->dim, L.tq, next_ws(), L.attn_norm,
                                            r->eps, nullptr, &red)))
                return rc;
            q = r->bqkv;
            k = r->bqkv + qd;
            v = r->bqkv + qd + kvd;
            ldq = ldkv = qd + 2 * kvd;
        } else if ((rc = launch_gemm_f32(s, L.wq, r->bx, r->bq, n, qd, r->dim, L.tq, next_ws(), false, L.attn_norm,
                                         r->eps, false, nullptr, &red)) ||
                   (rc = launch_gemm_f32(s, L.wk, r->bx, r->bk, n, kvd, r->dim, L.tk, next_ws(), false, L.attn_norm,
                                         r->eps)) ||
                   (rc = launch_gemm_f32(s, L.wv, r->bx, r->bv, n, kvd, r->dim, L.tv, next_ws(), false, L.attn_norm,
                                         r->eps))) {
            return rc;
        }
        red = none;
        if ((rc = launch_rope_rows(s, const_cast<float *>(q), k, v, L.kc, L.vc, r->cos_t, r->sin_t, pos0, n, qd, kvd,
                                   r->hd, ldq, ldkv)) ||
            (rc = launch_attn_prefill(s, q, L.kc, L.vc, r->ba, pos0, n, r->n_heads, r->n_kv, r->hd, ldq)) ||
            (rc = launch_gemm_f32(s, L.wo, r->ba, r->bx, n, r->dim, qd, L.to, next_ws(), true, nullptr, 0.f, false,
                                  &red)))   // residual += O
            return rc;
        // gate and up: one [gate | up] product when they share a format
        // (one [gate | up] product: SwiGLU is formed in the down product's X
        // pre-pass)
        const bool gu = gu_one(r, L);
        if (gu) {
            const uint8_t *w[2] = {L.wg, L.wu};
            const GemmRed in = red;
            if ((rc = launch_gemm_f32_multi(s, w, gu_rows, 2, r->bx, r->bgu, n, r->dim, L.tg, next_ws(), L.ffn_norm,
                                            r->eps, &red, &in)))
                return rc;
        } else {
            if ((rc = launch_gemm_f32(s, L.wg, r->bx, r->bg, n, r->ff, r->dim, L.tg, next_ws(), false, L.ffn_norm, r->eps,
                                      false, nullptr, &red)) ||
                (rc = launch_gemm_f32(s, L.wu, r->bx, r->bu, n, r->ff, r->dim, L.tu, next_ws(), false, L.ffn_norm, r->eps)) ||
                (rc = launch_eltwise(s, 3, r->bg, r->bu, r->bg, n * r->ff)))
                return rc;
            red = none;
        }
        const GemmRed in = red;
        if ((rc = launch_gemm_f32(s, L.wd, gu ? r->bgu : r->bg, r->bx, n, r->dim, r->ff, L.td, next_ws(), true, nullptr,
                                  0.f, gu, last ? nullptr : &red, &in)))   // residual += down
            return rc;
        if (last) red = none;
    }
    if ((rc = hip_error(hipMemcpyAsync(r->hidden, r->bx + (size_t)(n - 1) * r->dim, (size_t)r->dim * 4,
                                       hipMemcpyDeviceToDevice, s),
                        "runner: last prompt row")))
        return rc;
    return enqueue_head(r);
}

int set_ctl(yule_hip_runner *r, uint32_t pos, uint32_t token, uint32_t prompt_len) {
    // the pinned staging buffer may still feed a queued copy
    int rc = hip_error(hipStreamSynchronize(r->be->stream), "runner: synchronize");
    if (rc) return rc;
    r->ctl_host[0] = pos;
    r->ctl_host[1] = token;
    r->ctl_host[2] = prompt_len;
    return hip_error(hipMemcpyAsync(r->ctl, r->ctl_host, 3 * sizeof(uint32_t), hipMemcpyHostToDevice, r->be->stream),
                     "runner: control update");
}

}  // namespace

extern "C" {

int yule_hip_runner_create(yule_hip_backend *be, const yule_model_desc *d, yule_hip_runner **out) {
    if (!be || !d || !out) return set_error(YULE_ERR_INVALID, "runner_create: null argument");
    *out = nullptr;
    if (!d->n_layers || !d->dim || !d->n_heads || !d->n_kv_heads || !d->ff_dim || !d->vocab || !d->max_seq || !d->layers)
        return set_error(YULE_ERR_INVALID, "runner_create: zero-sized configuration");
    if (d->dim % d->n_heads || d->n_heads % d->n_kv_heads)
        return set_error(YULE_ERR_INVALID, "runner_create: dim/n_heads/n_kv_heads inconsistent");
    const uint32_t hd = d->dim / d->n_heads;
    if (hd % 4 || hd > 256)
        return set_error(YULE_ERR_INVALID, "runner_create: head_dim must be a multiple of 4 and <= 256");
    const bool can_split = split_attn_supported(d->n_heads, d->n_kv_heads, hd);
    if (d->max_seq > (can_split ? 262144u : 16384u))
        return set_error(YULE_ERR_INVALID, can_split ? "runner_create: max_seq above 262144"
                                                     : "runner_create: max_seq above 16384 (more than 8 query heads "
                                                       "per KV head)");
    auto *r = new yule_hip_runner();
    r->be = be;
    r->n_layers = d->n_layers; r->dim = d->dim; r->n_heads = d->n_heads; r->n_kv = d->n_kv_heads; r->hd = hd;
    r->ff = d->ff_dim; r->vocab = d->vocab; r->max_seq = d->max_seq; r->eps = d->norm_eps; r->rope_base = d->rope_base;
    r->split_min = can_split ? std::min(attn_split_min_seq(), 16384u) : 0xFFFFFFFFu;
    const uint32_t qd = r->n_heads * hd, kvd = r->n_kv * hd;
    int rc = YULE_OK;
    auto fail = [&](int code) { yule_hip_runner_destroy(r); return code; };
    if ((rc = hip_error(hipSetDevice(be->device), "runner: set device"))) return fail(rc);
    if ((rc = upload_matrix(r, d->token_embd, d->token_embd_dtype, r->vocab, r->dim, "token_embd", &r->embd)))
        return fail(rc);
    r->embd_t = d->token_embd_dtype;
    if ((rc = upload_norm(r, d->output_norm, d->output_norm_dtype, r->dim, &r->out_norm))) return fail(rc);
    if ((rc = upload_matrix(r, d->output, d->output_dtype, r->vocab, r->dim, "output", &r->out_w))) return fail(rc);
    r->out_t = d->output_dtype;
    r->layers.resize(r->n_layers);
    for (uint32_t i = 0; i < r->n_layers; i++) {
        const yule_layer_desc &ld = d->layers[i];
        auto &L = r->layers[i];
        L.tq = ld.wq_dtype; L.tk = ld.wk_dtype; L.tv = ld.wv_dtype; L.to = ld.wo_dtype;
        L.tg = ld.w_gate_dtype; L.tu = ld.w_up_dtype; L.td = ld.w_down_dtype;
        if ((rc = upload_norm(r, ld.attn_norm, ld.attn_norm_dtype, r->dim, &L.attn_norm)) ||
            (rc = upload_norm(r, ld.ffn_norm, ld.ffn_norm_dtype, r->dim, &L.ffn_norm)) ||
            (rc = upload_matrix(r, ld.wq, L.tq, qd, r->dim, "attn_q", &L.wq)) ||
            (rc = upload_matrix(r, ld.wk, L.tk, kvd, r->dim, "attn_k", &L.wk)) ||
            (rc = upload_matrix(r, ld.wv, L.tv, kvd, r->dim, "attn_v", &L.wv)) ||
            (rc = upload_matrix(r, ld.wo, L.to, r->dim, qd, "attn_output", &L.wo)) ||
            (rc = upload_matrix(r, ld.w_gate, L.tg, r->ff, r->dim, "ffn_gate", &L.wg)) ||
            (rc = upload_matrix(r, ld.w_up, L.tu, r->ff, r->dim, "ffn_up", &L.wu)) ||
            (rc = upload_matrix(r, ld.w_down, L.td, r->dim, r->ff, "ffn_down", &L.wd)) ||
            (rc = dev_alloc(r, (size_t)r->max_seq * kvd * 4, reinterpret_cast<void **>(&L.kc))) ||
            (rc = dev_alloc(r, (size_t)r->max_seq * kvd * 4, reinterpret_cast<void **>(&L.vc))))
            return fail(rc);
    }
    // RoPE table with RopeTable::new's f32 formula (model_runner.rs:77-100)
    const uint32_t half = hd / 2;
    std::vector<float> ct((size_t)r->max_seq * half), st((size_t)r->max_seq * half);
    for (uint32_t p = 0; p < r->max_seq; p++)
        for (uint32_t i = 0; i < half; i++) {
            const float freq = 1.0f / powf(r->rope_base, 2.0f * (float)i / (float)hd);
            const float theta = (float)p * freq;
            ct[(size_t)p * half + i] = cosf(theta);
            st[(size_t)p * half + i] = sinf(theta);
        }
    if ((rc = upload(r, ct.data(), ct.size() * 4, reinterpret_cast<void **>(&r->cos_t))) ||
        (rc = upload(r, st.data(), st.size() * 4, reinterpret_cast<void **>(&r->sin_t))))
        return fail(rc);
    struct { float **p; size_t n; } bufs[] = {
        {&r->hidden, r->dim}, {&r->normed, r->dim}, {&r->q, qd}, {&r->k, kvd}, {&r->v, kvd}, {&r->attn, qd},
        {&r->proj, r->dim}, {&r->gate, r->ff}, {&r->up, r->ff}, {&r->ffn, r->dim}, {&r->logits, r->vocab}};
    for (auto &b : bufs)
        if ((rc = dev_alloc(r, b.n * 4, reinterpret_cast<void **>(b.p)))) return fail(rc);
    if ((rc = dev_alloc(r, 4 * sizeof(uint32_t), reinterpret_cast<void **>(&r->ctl))) ||
        (rc = dev_alloc(r, (size_t)r->max_seq * 4, reinterpret_cast<void **>(&r->prompt))) ||
        (rc = dev_alloc(r, (size_t)r->max_seq * 4, reinterpret_cast<void **>(&r->tokens))))
        return fail(rc);
    if ((rc = dev_alloc(r, kArgmaxSlots * sizeof(unsigned long long), reinterpret_cast<void **>(&r->amax))))
        return fail(rc);
    // chunked attention for steps below the split threshold (YULE_ATTN_CHUNKS=0
    // at creation: the one-workgroup-per-head kernel instead)
    const char *ce = getenv("YULE_ATTN_CHUNKS");
    if ((!ce || atoi(ce) != 0) && attn_chunk_len(hd) &&
        (rc = dev_alloc(r, attn_chunk_scratch_bytes(r->n_heads, hd, std::min(r->max_seq, r->split_min)), &r->chunk_ws)))
        return fail(rc);
    if (r->max_seq >= r->split_min &&
        (rc = dev_alloc(r, split_scratch_bytes(r->n_heads, hd, r->max_seq), &r->attn_ws)))
        return fail(rc);
    r->fused = getenv("YULE_RUNNER_UNFUSED") == nullptr && qmv_fusable(r->out_t, r->dim);
    // decode steps per replayed graph in generate_greedy (1: one per step)
    // tuning knobs, each clamped to a documented range: at most 64 decode steps
    // per captured graph, 2048 prefetch workgroups and 4096 sleep rounds
    auto knob = [](const char *name, long lo, long hi, long dflt) {
        const char *e = getenv(name);
        if (!e) return dflt;
        const long v = atol(e);
        return v < lo ? lo : v > hi ? hi : v;
    };
    r->multi_steps = (uint32_t)knob("YULE_RUNNER_GRAPH_STEPS", 1, kMaxGraphSteps, r->multi_steps);
    r->pf_mask = (uint32_t)knob("YULE_RUNNER_PREFETCH", 0, 15, r->pf_mask);
    r->pf_wgs = (uint32_t)knob("YULE_RUNNER_PREFETCH_WGS", 0, 2048, r->pf_wgs) & ~7u;
    r->pf_delay = (uint32_t)knob("YULE_RUNNER_PREFETCH_DELAY", 0, 4096, r->pf_delay);
    for (const auto &L : r->layers)
        r->fused = r->fused && qmv_fusable(L.tq, r->dim) && qmv_fusable(L.tk, r->dim) && qmv_fusable(L.tv, r->dim) &&
                   qmv_fusable(L.to, qd) && qmv_fusable(L.tg, r->dim) && qmv_fusable(L.tu, r->dim) &&
                   qmv_fusable(L.td, r->ff);
    // batched prefill: every projection on the GEMM, attention head size served,
    // unless YULE_RUNNER_TOKEN_PREFILL is set (then prompts go token by token)
    r->batchable = getenv("YULE_RUNNER_TOKEN_PREFILL") == nullptr && attn_prefill_supported(hd);
    for (const auto &L : r->layers)
        r->batchable = r->batchable && gemm_supports(L.tq, r->dim) && gemm_supports(L.tk, r->dim) &&
                       gemm_supports(L.tv, r->dim) && gemm_supports(L.to, qd) && gemm_supports(L.tg, r->dim) &&
                       gemm_supports(L.tu, r->dim) && gemm_supports(L.td, r->ff);
    if ((rc = hip_error(hipHostMalloc(reinterpret_cast<void **>(&r->ctl_host), 4 * sizeof(uint32_t), 0),
                        "runner: pinned control block")))
        return fail(rc);
    *out = r;
    return YULE_OK;
}

int yule_hip_runner_destroy(yule_hip_runner *r) {
    if (!r) return YULE_OK;
    if (r->be) hipStreamSynchronize(r->be->stream);
    for (int i = 0; i < 2; i++) {
        if (r->exec[i]) hipGraphExecDestroy(r->exec[i]);
        if (r->exec_n[i]) hipGraphExecDestroy(r->exec_n[i]);
        if (r->graph_n[i]) hipGraphDestroy(r->graph_n[i]);
        if (r->graph[i]) hipGraphDestroy(r->graph[i]);
    }
    for (void *p : r->allocs) hipFree(p);
    if (r->bws) hipFree(r->bws);
    if (r->ctl_host) hipHostFree(r->ctl_host);
    delete r;
    return YULE_OK;
}

// ModelRunner::reset (model_runner.rs:1087-1092)
int yule_hip_runner_reset(yule_hip_runner *r) {
    if (!r) return set_error(YULE_ERR_INVALID, "runner_reset: null runner");
    r->pos = 0;
    return YULE_OK;
}

uint32_t yule_hip_runner_pos(const yule_hip_runner *r) { return r ? r->pos : 0; }

// ModelRunner::decode_step (model_runner.rs:1083-1085): one forward pass at
// the current position; logits copied out when `logits` is non-null.
int yule_hip_runner_decode_step(yule_hip_runner *r, uint32_t token, float *logits) {
    if (!r) return set_error(YULE_ERR_INVALID, "runner: null runner");
    if (r->pos >= r->max_seq) return set_error(YULE_ERR_INVALID, "context length exceeded");
    if (token >= r->vocab) return set_error(YULE_ERR_INVALID, "token id out of range");
    int rc;
    if ((rc = set_ctl(r, r->pos, token, 0))) return rc;
    if ((rc = run_step(r, r->pos))) return rc;
    r->pos++;
    if (logits &&
        (rc = hip_error(hipMemcpyAsync(logits, r->logits, (size_t)r->vocab * 4, hipMemcpyDeviceToHost, r->be->stream),
                        "runner: logits copy")))
        return rc;
    return hip_error(hipStreamSynchronize(r->be->stream), "runner: synchronize");
}

// ModelRunner::prefill (model_runner.rs:1075-1081): token by token; logits
// of the last token.
int yule_hip_runner_prefill(yule_hip_runner *r, const uint32_t *tokens, uint32_t n, float *logits) {
    if (!r || (!tokens && n)) return set_error(YULE_ERR_INVALID, "runner_prefill: null argument");
    for (uint32_t i = 0; i < n; i++) {
        int rc = yule_hip_runner_decode_step(r, tokens[i], i + 1 == n ? logits : nullptr);
        if (rc) return rc;
    }
    return YULE_OK;
}

int yule_hip_runner_generate_greedy(yule_hip_runner *r, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_decode,
                                    uint32_t *out_tokens, float *ms_per_decode_step) {
    if (!r || !prompt || !out_tokens || n_prompt == 0)
        return set_error(YULE_ERR_INVALID, "runner_generate: null argument or empty prompt");
    if ((uint64_t)n_prompt + n_decode > r->max_seq)
        return set_error(YULE_ERR_INVALID, "runner_generate: prompt + decode steps exceed the context length");
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= r->vocab) return set_error(YULE_ERR_INVALID, "runner_generate: token id out of range");
    hipStream_t s = r->be->stream;
    int rc;
    // every graph the run needs is captured before the timed loop
    if ((rc = ensure_graph(r, false))) return rc;
    if (n_prompt + n_decode >= r->split_min && (rc = ensure_graph(r, true))) return rc;
    if (multi_ok(r) && n_decode >= r->multi_steps) {
        if (n_prompt + r->multi_steps < r->split_min && (rc = ensure_graph_n(r, false))) return rc;
        if (n_prompt + n_decode >= r->split_min && (rc = ensure_graph_n(r, true))) return rc;
    }
    if ((rc = hip_error(hipMemcpyAsync(r->prompt, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, s),
                        "runner: prompt upload")))
        return rc;
    hipEvent_t e0 = nullptr, e1 = nullptr, p0 = nullptr;
    const bool batched = r->batchable && n_prompt >= 2;
    if ((rc = hip_error(hipEventCreate(&e0), "hipEventCreate")) || (rc = hip_error(hipEventCreate(&e1), "hipEventCreate")) ||
        (rc = hip_error(hipEventCreate(&p0), "hipEventCreate")))
        goto done;
    if (r->batchable && n_prompt >= 2 && (rc = ensure_batch(r, n_prompt))) goto done;
    // the control block is written (a host synchronization) before p0, so the
    // prefill time holds GPU work only
    if ((rc = set_ctl(r, batched ? n_prompt - 1 : 0, 0, n_prompt))) goto done;
    if ((rc = hip_error(hipEventRecord(p0, s), "hipEventRecord"))) goto done;
    if (batched) {   // the prompt as one batched pass
        if ((rc = prefill_rows(r, 0, n_prompt, n_prompt, true))) goto done;
    } else {
        for (uint32_t i = 0; i < n_prompt && !rc; i++) rc = run_step(r, i);
        if (rc) goto done;
    }
    if ((rc = hip_error(hipEventRecord(e0, s), "hipEventRecord"))) goto done;
    for (uint32_t i = 0; i < n_decode && !rc;) {
        const uint32_t pos = n_prompt + i, K = r->multi_steps;
        const bool split = pos + 1 >= r->split_min;
        if (multi_ok(r) && i + K <= n_decode && (pos + K >= r->split_min) == split) {
            rc = hip_error(hipGraphLaunch(r->exec_n[split], r->be->stream), "runner: graph launch");
            i += K;
        } else {
            rc = run_step(r, pos);
            i++;
        }
    }
    if (rc || (rc = hip_error(hipEventRecord(e1, s), "hipEventRecord"))) goto done;
    if ((rc = hip_error(hipEventSynchronize(e1), "hipEventSynchronize"))) goto done;
    if (ms_per_decode_step) {
        float ms = 0.f;
        if ((rc = hip_error(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime"))) goto done;
        *ms_per_decode_step = n_decode ? ms / (float)n_decode : 0.f;
    }
    if ((rc = hip_error(hipEventElapsedTime(&r->last_prefill_ms, p0, e0), "hipEventElapsedTime"))) goto done;
    // the argmax after the last prompt token and after every decode step
    rc = hip_error(hipMemcpy(out_tokens, r->tokens + (n_prompt - 1), (size_t)(n_decode + 1) * 4,
                             hipMemcpyDeviceToHost),
                   "runner: token copy");
    r->pos = n_prompt + n_decode;
done:
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (p0) hipEventDestroy(p0);
    return rc;
}

// Batched counterpart of yule_hip_runner_prefill: the n tokens through every
// layer at once (each projection one GEMM), from the current position.
int yule_hip_runner_prefill_batched(yule_hip_runner *r, const uint32_t *tokens, uint32_t n, float *logits) {
    if (!r || !tokens || !n) return set_error(YULE_ERR_INVALID, "runner_prefill_batched: null argument or no tokens");
    if (!r->batchable) return set_error(YULE_ERR_UNSUPPORTED, "runner_prefill_batched: a projection format or head "
                                                                "size has no batched path (use runner_prefill)");
    if ((uint64_t)r->pos + n > r->max_seq) return set_error(YULE_ERR_INVALID, "context length exceeded");
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] >= r->vocab) return set_error(YULE_ERR_INVALID, "token id out of range");
    hipStream_t s = r->be->stream;
    int rc;
    if ((rc = hip_error(hipMemcpyAsync(r->prompt + r->pos, tokens, (size_t)n * 4, hipMemcpyHostToDevice, s),
                        "runner: prompt upload")) ||
        (rc = hip_error(hipStreamSynchronize(s), "runner: synchronize")))   // `tokens` is pageable host memory
        return rc;
    if ((rc = prefill_rows(r, r->pos, n, 0))) return rc;
    r->pos += n;
    if (logits &&
        (rc = hip_error(hipMemcpyAsync(logits, r->logits, (size_t)r->vocab * 4, hipMemcpyDeviceToHost, s),
                        "runner: logits copy")))
        return rc;
    return hip_error(hipStreamSynchronize(s), "runner: synchronize");
}

float yule_hip_runner_last_prefill_ms(const yule_hip_runner *r) { return r ? r->last_prefill_ms : 0.f; }

}  // extern "C"
