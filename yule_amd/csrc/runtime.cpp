// runtime.cpp — backend object, buffer handles, copies and the validated
// quantized_matmul entry point of libyule_hip.so.
//
// Mirrors the ComputeBackend trait's host-side contract
// (yule-gpu/src/lib.rs:21-132): opaque u64 handles from a global counter
// (yule-gpu/src/buffer.rs:5-9), zero-initialised buffers
// (yule-gpu/src/cpu.rs:157), Result<()> as status code + message.
#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "internal.h"

namespace {
thread_local std::string g_last_error;
std::atomic<uint64_t> g_next_handle{1};
}  // namespace

namespace yule {

int set_error(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int hip_error(hipError_t e, const char *what) {
    if (e == hipSuccess) return YULE_OK;
    return set_error(e == hipErrorOutOfMemory ? YULE_ERR_OOM : YULE_ERR_HIP,
                     std::string(what) + ": " + hipGetErrorString(e));
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? YULE_OK : hip_error(e, what);
}

int get_scratch(yule_hip_backend *be, size_t need, ScratchLease *lease) {
    std::unique_lock<std::mutex> lk(be->scratch_mu);
    if (be->scratch_size < need) {
        int rc;
        if (be->scratch) {
            if ((rc = hip_error(hipStreamSynchronize(be->stream), "scratch: synchronize"))) return rc;
            (void)hipFree(be->scratch);
            be->scratch = nullptr;
            be->scratch_size = 0;
        }
        const size_t sz = (need + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
        if ((rc = hip_error(hipMalloc(&be->scratch, sz), "scratch: allocate"))) return rc;
        be->scratch_size = sz;
    }
    lease->ptr = be->scratch;
    lease->lock = std::move(lk);
    return YULE_OK;
}

int get_buffer(yule_hip_backend *be, uint64_t h, size_t need, void **ptr, const char *what, size_t offset) {
    std::lock_guard<std::mutex> lk(be->mu);
    auto it = be->buffers.find(h);
    if (it == be->buffers.end())
        return set_error(YULE_ERR_INVALID, std::string(what) + ": buffer " + std::to_string(h) + " not found");
    if (offset > it->second.size || need > it->second.size - offset)
        return set_error(YULE_ERR_INVALID, std::string(what) + ": access of " + std::to_string(need) +
                                               " bytes at offset " + std::to_string(offset) +
                                               " exceeds buffer " + std::to_string(h) + " of " +
                                               std::to_string(it->second.size) + " bytes");
    *ptr = static_cast<uint8_t *>(it->second.ptr) + offset;
    return YULE_OK;
}

bool quant_geometry(uint32_t dtype, uint32_t *bs, uint32_t *bb) {
    switch (dtype) {  // yule-core/src/dtype.rs:62-118
    case YULE_DTYPE_Q4_0: *bs = 32; *bb = 18; return true;
    case YULE_DTYPE_Q8_0: *bs = 32; *bb = 34; return true;
    case YULE_DTYPE_Q4_K: *bs = 256; *bb = 144; return true;
    case YULE_DTYPE_Q5_K: *bs = 256; *bb = 176; return true;
    case YULE_DTYPE_Q6_K: *bs = 256; *bb = 210; return true;
    case YULE_DTYPE_Q8_K: *bs = 256; *bb = 292; return true;
    default: return false;
    }
}

}  // namespace yule

using namespace yule;

#define YULE_CHECK_BE(be)                                                         \
    do {                                                                          \
        if (!(be)) return set_error(YULE_ERR_INVALID, "null backend");            \
    } while (0)

extern "C" {

const char *yule_hip_last_error(void) { return g_last_error.c_str(); }

static bool is_gfx950(const hipDeviceProp_t &p) { return std::strncmp(p.gcnArchName, "gfx950", 6) == 0; }

int yule_hip_is_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) == hipSuccess && is_gfx950(p)) return 1;
    }
    return 0;
}

int yule_hip_create(int device, yule_hip_backend **out) {
    if (!out) return set_error(YULE_ERR_INVALID, "create: null out pointer");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return set_error(YULE_ERR_NO_DEVICE, "create: no HIP device present");
    if (device < 0 || device >= n)
        return set_error(YULE_ERR_NO_DEVICE, "create: device " + std::to_string(device) + " out of range");
    auto *be = new yule_hip_backend();
    be->device = device;
    int rc;
    if ((rc = hip_error(hipSetDevice(device), "hipSetDevice")) ||
        (rc = hip_error(hipGetDeviceProperties(&be->props, device), "hipGetDeviceProperties"))) {
        delete be;
        return rc;
    }
    if (!is_gfx950(be->props)) {
        std::string arch = be->props.gcnArchName;
        delete be;
        return set_error(YULE_ERR_NO_DEVICE, "create: device is " + arch + ", this build targets gfx950");
    }
    if ((rc = gemm_static_workspace_init(device))) {   // with `device` current
        delete be;
        return rc;
    }
    // default-priority stream (no priority games); non-blocking w.r.t. the null stream
    if ((rc = hip_error(hipStreamCreateWithFlags(&be->stream, hipStreamNonBlocking), "hipStreamCreate"))) {
        delete be;
        return rc;
    }
    *out = be;
    return YULE_OK;
}

int yule_hip_destroy(yule_hip_backend *be) {
    if (!be) return YULE_OK;
    hipSetDevice(be->device);
    hipStreamSynchronize(be->stream);
    for (auto &kv : be->buffers) hipFree(kv.second.ptr);
    be->buffers.clear();
    if (be->scratch) hipFree(be->scratch);
    for (hipEvent_t e : be->timer)
        if (e) hipEventDestroy(e);
    if (be->cap_exec) hipGraphExecDestroy(be->cap_exec);
    if (be->cap_graph) hipGraphDestroy(be->cap_graph);
    hipStreamDestroy(be->stream);
    delete be;
    return YULE_OK;
}

const char *yule_hip_name(const yule_hip_backend *) { return "hip"; }

int yule_hip_device_info(yule_hip_backend *be, yule_device_info *out) {
    YULE_CHECK_BE(be);
    if (!out) return set_error(YULE_ERR_INVALID, "device_info: null out");
    std::memset(out, 0, sizeof(*out));
    // the runtime's device name can be empty (seen on MI355X); ask the driver, else say "AMD GPU"
    char name[256] = {0};
    if (be->props.name[0]) std::snprintf(name, sizeof(name), "%s", be->props.name);
    else if (hipDeviceGetName(name, sizeof(name), be->device) != hipSuccess || !name[0])
        std::snprintf(name, sizeof(name), "AMD GPU");
    std::snprintf(out->name, sizeof(out->name), "%s (%s)", name, be->props.gcnArchName);
    out->backend = 4;
    out->memory_bytes = be->props.totalGlobalMem;
    out->compute_units = (uint32_t)be->props.multiProcessorCount;
    return YULE_OK;
}

int yule_hip_allocate(yule_hip_backend *be, size_t size, yule_buffer *out) {
    YULE_CHECK_BE(be);
    if (!out) return set_error(YULE_ERR_INVALID, "allocate: null out");
    void *p = nullptr;
    int rc = hip_error(hipMalloc(&p, size + kAllocSlack), "allocate");
    if (rc) return rc;
    // zero-initialised like the reference backends; ordered before any later
    // work on the same stream
    if ((rc = hip_error(hipMemsetAsync(p, 0, size + kAllocSlack, be->stream), "allocate: zero-fill"))) {
        hipFree(p);
        return rc;
    }
    const uint64_t h = g_next_handle.fetch_add(1);
    {
        std::lock_guard<std::mutex> lk(be->mu);
        be->buffers[h] = Buffer{p, size};
    }
    *out = h;
    return YULE_OK;
}

int yule_hip_free(yule_hip_backend *be, yule_buffer h) {
    YULE_CHECK_BE(be);
    void *p = nullptr;
    {
        std::lock_guard<std::mutex> lk(be->mu);
        auto it = be->buffers.find(h);
        if (it == be->buffers.end()) return YULE_OK;  // CpuBackend::free ignores unknown handles
        p = it->second.ptr;
        be->buffers.erase(it);
    }
    // queued kernels may still read the buffer
    int rc = hip_error(hipStreamSynchronize(be->stream), "free: synchronize");
    hipFree(p);
    return rc;
}

int yule_hip_copy_to_device(yule_hip_backend *be, const void *data, size_t size, yule_buffer h) {
    YULE_CHECK_BE(be);
    if (!data && size) return set_error(YULE_ERR_INVALID, "copy_to_device: null data");
    void *p;
    int rc = get_buffer(be, h, size, &p, "copy_to_device");
    if (rc || !size) return rc;
    if ((rc = hip_error(hipMemcpyAsync(p, data, size, hipMemcpyHostToDevice, be->stream), "copy_to_device")))
        return rc;
    return hip_error(hipStreamSynchronize(be->stream), "copy_to_device: synchronize");
}

int yule_hip_copy_from_device(yule_hip_backend *be, yule_buffer h, void *data, size_t size) {
    YULE_CHECK_BE(be);
    if (!data && size) return set_error(YULE_ERR_INVALID, "copy_from_device: null data");
    void *p;
    int rc = get_buffer(be, h, size, &p, "copy_from_device");
    if (rc || !size) return rc;
    if ((rc = hip_error(hipMemcpyAsync(data, p, size, hipMemcpyDeviceToHost, be->stream), "copy_from_device")))
        return rc;
    return hip_error(hipStreamSynchronize(be->stream), "copy_from_device: synchronize");
}

// yule-gpu/src/cpu.rs:425-434: copies min(size, src_len, dst_len) bytes
int yule_hip_copy_buffer(yule_hip_backend *be, yule_buffer src, yule_buffer dst, size_t size) {
    YULE_CHECK_BE(be);
    size_t ssz = 0, dsz = 0;
    void *ps = nullptr, *pd = nullptr;
    {
        std::lock_guard<std::mutex> lk(be->mu);
        auto a = be->buffers.find(src), b = be->buffers.find(dst);
        if (a == be->buffers.end() || b == be->buffers.end())
            return set_error(YULE_ERR_INVALID, "copy_buffer: buffer not found");
        ps = a->second.ptr; ssz = a->second.size;
        pd = b->second.ptr; dsz = b->second.size;
    }
    size_t n = size < ssz ? size : ssz;
    n = n < dsz ? n : dsz;
    if (!n) return YULE_OK;
    return hip_error(hipMemcpyAsync(pd, ps, n, hipMemcpyDeviceToDevice, be->stream), "copy_buffer");
}

// yule-gpu/src/cpu.rs:436-452: dst[dst_off..dst_off+size] = src[src_off..src_off+size]
int yule_hip_copy_buffer_offset(yule_hip_backend *be, yule_buffer src, yule_buffer dst, size_t src_offset,
                                size_t dst_offset, size_t size) {
    YULE_CHECK_BE(be);
    void *ps, *pd;
    int rc;
    if ((rc = get_buffer(be, src, size, &ps, "copy_buffer_offset (src)", src_offset))) return rc;
    if ((rc = get_buffer(be, dst, size, &pd, "copy_buffer_offset (dst)", dst_offset))) return rc;
    if (!size) return YULE_OK;
    return hip_error(hipMemcpyAsync(pd, ps, size, hipMemcpyDeviceToDevice, be->stream), "copy_buffer_offset");
}

int yule_hip_synchronize(yule_hip_backend *be) {
    YULE_CHECK_BE(be);
    return hip_error(hipStreamSynchronize(be->stream), "synchronize");
}

// Shared validation of the quantized entry points.
static int check_qmv_args(yule_hip_backend *be, yule_buffer weights, yule_buffer input, yule_buffer output,
                          uint32_t n_rows, uint32_t n_cols, uint32_t dtype, const char *what, const uint8_t **w,
                          const float **x, float **y, bool *empty_rows) {
    uint32_t bs, bb;
    if (!quant_geometry(dtype, &bs, &bb))
        return set_error(YULE_ERR_UNSUPPORTED,
                         std::string(what) + ": dtype " + std::to_string(dtype) + " not supported on this backend");
    if (input == output) return set_error(YULE_ERR_INVALID, std::string(what) + ": input and output alias");
    // kernels of other workgroups still read the weights while y is written
    if (weights == output || weights == input)
        return set_error(YULE_ERR_INVALID, std::string(what) + ": weights alias the input or the output");
    void *pw, *px, *py;
    int rc;
    // ceil(n_cols / bs) blocks per row, as the reference's GPU backends
    // launch them (cuda/mod.rs:311-313; vulkan/mod.rs:324-351)
    const size_t wbytes = (size_t)n_rows * ((n_cols + bs - 1) / bs) * bb;
    if ((rc = get_buffer(be, weights, wbytes, &pw, what))) return rc;
    if ((rc = get_buffer(be, input, (size_t)n_cols * 4, &px, what))) return rc;
    if ((rc = get_buffer(be, output, (size_t)n_rows * 4, &py, what))) return rc;
    *w = (const uint8_t *)pw; *x = (const float *)px; *y = (float *)py;
    *empty_rows = n_cols == 0;
    return YULE_OK;
}

// Validate a multi-matrix call: every matrix checked like quantized_matmul,
// and no output may alias the input or another output.
static int prepare_multi(yule_hip_backend *be, uint32_t n_mats, const yule_buffer *weights, const yule_buffer *outputs,
                         const uint32_t *n_rows, yule_buffer input, uint32_t n_cols, uint32_t dtype, const char *what,
                         QmvSeg *segs, const float **x) {
    if (n_mats == 0 || n_mats > (uint32_t)kMaxSegs || !weights || !outputs || !n_rows)
        return set_error(YULE_ERR_INVALID, std::string(what) + ": n_mats must be 1..4 with non-null arrays");
    for (uint32_t i = 0; i < n_mats; i++) {
        for (uint32_t j = 0; j < i; j++)
            if (outputs[i] == outputs[j]) return set_error(YULE_ERR_INVALID, std::string(what) + ": outputs alias");
        bool empty;
        float *y;
        int rc = check_qmv_args(be, weights[i], input, outputs[i], n_rows[i], n_cols, dtype, what, &segs[i].w, x, &y,
                                &empty);
        if (rc) return rc;
        segs[i].y = y;
        segs[i].n_rows = n_rows[i];
    }
    return YULE_OK;
}

// A row length that is not a multiple of the block size: the reference's
// GPU kernels run ceil(n_cols / bs) blocks per row and skip the columns
// >= n_cols (kernels/cuda/qmv_*.cu, shaders/qmv_*.comp column checks).
// Here x is staged in the backend workspace zero-padded to the block
// multiple, so the last block's extra columns contribute exactly 0 and the
// kernels run unchanged.  (The CPU path floors instead, cpu.rs:544-590; the
// GPU backends' semantics are the ones a GPU drop-in keeps.)
static int pad_input(yule_hip_backend *be, uint32_t dtype, const float *x, uint32_t n_cols, const float **xp,
                     uint32_t *n_cols_p, ScratchLease *ws) {
    uint32_t bs, bb;
    quant_geometry(dtype, &bs, &bb);
    const uint32_t np = (n_cols + bs - 1) / bs * bs;
    *xp = x;
    *n_cols_p = np;
    if (np == n_cols) return YULE_OK;
    int rc = get_scratch(be, (size_t)np * sizeof(float), ws);
    if (rc) return rc;
    *xp = static_cast<const float *>(ws->ptr);
    return launch_pad(be->stream, x, n_cols, static_cast<float *>(ws->ptr), np);
}

int yule_hip_quantized_matmul(yule_hip_backend *be, yule_buffer weights, yule_buffer input, yule_buffer output,
                              uint32_t n_rows, uint32_t n_cols, uint32_t dtype) {
    YULE_CHECK_BE(be);
    const uint8_t *w; const float *x; float *y; bool empty;
    int rc = check_qmv_args(be, weights, input, output, n_rows, n_cols, dtype, "quantized_matmul", &w, &x, &y, &empty);
    if (rc) return rc;
    if (n_rows == 0) return YULE_OK;
    if (empty) return launch_fill(be->stream, y, 0.0f, n_rows);  // zero blocks per row -> y = 0
    const float *xp;
    uint32_t np;
    ScratchLease ws;   // held until the matvec is enqueued
    if ((rc = pad_input(be, dtype, x, n_cols, &xp, &np, &ws))) return rc;
    return launch_qmv(be->stream, dtype, w, xp, y, n_rows, np);
}

int yule_hip_quantized_matmul_multi(yule_hip_backend *be, uint32_t n_mats, const yule_buffer *weights,
                                    const yule_buffer *outputs, const uint32_t *n_rows, yule_buffer input,
                                    uint32_t n_cols, uint32_t dtype) {
    YULE_CHECK_BE(be);
    QmvSeg segs[kMaxSegs];
    const float *x = nullptr;
    int rc = prepare_multi(be, n_mats, weights, outputs, n_rows, input, n_cols, dtype, "quantized_matmul_multi", segs,
                           &x);
    if (rc) return rc;
    uint32_t n = 0;
    for (uint32_t i = 0; i < n_mats; i++)
        if (segs[i].n_rows) segs[n++] = segs[i];
    if (n == 0) return YULE_OK;
    if (n_cols == 0) {
        for (uint32_t i = 0; i < n; i++)
            if ((rc = launch_fill(be->stream, segs[i].y, 0.0f, segs[i].n_rows))) return rc;
        return YULE_OK;
    }
    const float *xp;
    uint32_t np;
    ScratchLease ws;   // held until the matvec is enqueued
    if ((rc = pad_input(be, dtype, x, n_cols, &xp, &np, &ws))) return rc;
    return launch_qmv_multi(be->stream, dtype, segs, n, xp, np);
}

int yule_hip_dequantize(yule_hip_backend *be, yule_buffer src, size_t src_offset, yule_buffer dst,
                        uint32_t n_blocks, uint32_t dtype) {
    YULE_CHECK_BE(be);
    uint32_t bs, bb;
    if (!quant_geometry(dtype, &bs, &bb))
        return set_error(YULE_ERR_UNSUPPORTED, "dequantize: dtype " + std::to_string(dtype) + " not supported");
    void *ps, *pd;
    int rc;
    if ((rc = get_buffer(be, src, (size_t)n_blocks * bb, &ps, "dequantize (src)", src_offset))) return rc;
    if ((rc = get_buffer(be, dst, (size_t)n_blocks * bs * 4, &pd, "dequantize (dst)"))) return rc;
    return launch_dequant(be->stream, dtype, (const uint8_t *)ps, (float *)pd, n_blocks);
}

int yule_hip_time_qmv_ops(yule_hip_backend *be, const yule_qmv_op *ops, uint32_t n_ops, uint32_t iters,
                          int use_graph, float *ms_total) {
    YULE_CHECK_BE(be);
    if (!ops || !ms_total || n_ops == 0 || iters == 0)
        return set_error(YULE_ERR_INVALID, "time_qmv_ops: bad arguments");
    struct Launch { uint32_t dtype, n_cols, n; QmvSeg segs[kMaxSegs]; const float *x; };
    std::vector<Launch> L(n_ops);
    for (uint32_t i = 0; i < n_ops; i++) {
        int rc = prepare_multi(be, ops[i].n_mats, ops[i].weights, ops[i].outputs, ops[i].n_rows, ops[i].input,
                               ops[i].n_cols, ops[i].dtype, "time_qmv_ops", L[i].segs, &L[i].x);
        if (rc) return rc;
        if (ops[i].n_cols == 0) return set_error(YULE_ERR_INVALID, "time_qmv_ops: empty matrix");
        uint32_t bs, bb;
        quant_geometry(ops[i].dtype, &bs, &bb);
        if (ops[i].n_cols % bs)
            return set_error(YULE_ERR_INVALID, "time_qmv_ops: n_cols must be a multiple of the block size");
        for (uint32_t j = 0; j < ops[i].n_mats; j++)
            if (!ops[i].n_rows[j]) return set_error(YULE_ERR_INVALID, "time_qmv_ops: empty matrix");
        L[i].dtype = ops[i].dtype; L[i].n_cols = ops[i].n_cols; L[i].n = ops[i].n_mats;
    }
    auto enqueue = [&]() -> int {
        for (const Launch &l : L) {
            int rc = launch_qmv_multi(be->stream, l.dtype, l.segs, l.n, l.x, l.n_cols);
            if (rc) return rc;
        }
        return YULE_OK;
    };
    int rc = YULE_OK;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (use_graph) {
        if ((rc = hip_error(hipStreamBeginCapture(be->stream, hipStreamCaptureModeThreadLocal), "begin capture")))
            return rc;
        int erc = enqueue();
        rc = hip_error(hipStreamEndCapture(be->stream, &graph), "end capture");
        if (erc) rc = erc;
        if (!rc) rc = hip_error(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "graph instantiate");
        if (!rc) rc = hip_error(hipGraphLaunch(exec, be->stream), "graph warm-up launch");
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc) rc = hip_error(hipEventCreate(&e0), "hipEventCreate");
    if (!rc) rc = hip_error(hipEventCreate(&e1), "hipEventCreate");
    if (!rc) rc = hip_error(hipEventRecord(e0, be->stream), "hipEventRecord");
    for (uint32_t it = 0; it < iters && !rc; it++)
        rc = use_graph ? hip_error(hipGraphLaunch(exec, be->stream), "graph launch") : enqueue();
    if (!rc) rc = hip_error(hipEventRecord(e1, be->stream), "hipEventRecord");
    if (!rc) rc = hip_error(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.f;
    if (!rc) rc = hip_error(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (exec) hipGraphExecDestroy(exec);
    if (graph) hipGraphDestroy(graph);
    if (!rc) *ms_total = ms;
    return rc;
}

int yule_hip_time_empty_launches(yule_hip_backend *be, uint32_t n_kernels, uint32_t iters, int use_graph,
                                 float *ms_total) {
    YULE_CHECK_BE(be);
    if (!ms_total || n_kernels == 0 || n_kernels > 100000 || iters == 0)
        return set_error(YULE_ERR_INVALID, "time_empty_launches: bad arguments");
    auto enqueue = [&]() -> int {
        for (uint32_t i = 0; i < n_kernels; i++) {
            int rc = launch_empty(be->stream);
            if (rc) return rc;
        }
        return YULE_OK;
    };
    int rc = YULE_OK;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (use_graph) {
        if ((rc = hip_error(hipStreamBeginCapture(be->stream, hipStreamCaptureModeThreadLocal), "begin capture")))
            return rc;
        int erc = enqueue();
        rc = hip_error(hipStreamEndCapture(be->stream, &graph), "end capture");
        if (erc) rc = erc;
        if (!rc) rc = hip_error(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "graph instantiate");
        if (!rc) rc = hip_error(hipGraphLaunch(exec, be->stream), "graph warm-up launch");
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc) rc = hip_error(hipEventCreate(&e0), "hipEventCreate");
    if (!rc) rc = hip_error(hipEventCreate(&e1), "hipEventCreate");
    if (!rc) rc = hip_error(hipEventRecord(e0, be->stream), "hipEventRecord");
    for (uint32_t it = 0; it < iters && !rc; it++)
        rc = use_graph ? hip_error(hipGraphLaunch(exec, be->stream), "graph launch") : enqueue();
    if (!rc) rc = hip_error(hipEventRecord(e1, be->stream), "hipEventRecord");
    if (!rc) rc = hip_error(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.f;
    if (!rc) rc = hip_error(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (exec) hipGraphExecDestroy(exec);
    if (graph) hipGraphDestroy(graph);
    if (!rc) *ms_total = ms;
    return rc;
}

int yule_hip_timer_start(yule_hip_backend *be) {
    YULE_CHECK_BE(be);
    int rc;
    for (hipEvent_t &e : be->timer)
        if (!e && (rc = hip_error(hipEventCreate(&e), "timer: event create"))) return rc;
    return hip_error(hipEventRecord(be->timer[0], be->stream), "timer: record start");
}

int yule_hip_timer_stop(yule_hip_backend *be, float *ms) {
    YULE_CHECK_BE(be);
    if (!ms || !be->timer[0]) return set_error(YULE_ERR_INVALID, "timer_stop: no timer_start");
    int rc;
    if ((rc = hip_error(hipEventRecord(be->timer[1], be->stream), "timer: record stop")) ||
        (rc = hip_error(hipEventSynchronize(be->timer[1]), "timer: synchronize")))
        return rc;
    return hip_error(hipEventElapsedTime(ms, be->timer[0], be->timer[1]), "timer: elapsed");
}

static void drop_capture(yule_hip_backend *be) {
    if (be->cap_exec) (void)hipGraphExecDestroy(be->cap_exec);
    if (be->cap_graph) (void)hipGraphDestroy(be->cap_graph);
    be->cap_exec = nullptr;
    be->cap_graph = nullptr;
}

int yule_hip_capture_begin(yule_hip_backend *be) {
    YULE_CHECK_BE(be);
    drop_capture(be);
    return hip_error(hipStreamBeginCapture(be->stream, hipStreamCaptureModeThreadLocal), "capture: begin");
}

int yule_hip_capture_end(yule_hip_backend *be) {
    YULE_CHECK_BE(be);
    int rc = hip_error(hipStreamEndCapture(be->stream, &be->cap_graph), "capture: end");
    if (!rc) rc = hip_error(hipGraphInstantiate(&be->cap_exec, be->cap_graph, nullptr, nullptr, 0), "capture: instantiate");
    if (rc) drop_capture(be);
    return rc;
}

int yule_hip_capture_replay(yule_hip_backend *be) {
    YULE_CHECK_BE(be);
    if (!be->cap_exec) return set_error(YULE_ERR_INVALID, "capture_replay: nothing captured");
    return hip_error(hipGraphLaunch(be->cap_exec, be->stream), "capture: replay");
}

}  // extern "C"
