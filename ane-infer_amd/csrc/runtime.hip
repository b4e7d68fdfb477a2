// runtime.hip — context, errors, device memory and timing of libanehip.
//
// Replaces GpuContext (crates/engine/src/metal_graph.rs:49-260): one device,
// one stream (the reference's one MTLCommandQueue), and a workspace allocated
// once.  Unlike the reference, failures are reported as status codes with a
// message instead of being ignored (gpu_full_decode.rs:1030-1043).
#include "common.h"

#include <cstring>

namespace anehip {

ErrorSlot &global_error() {
    static thread_local ErrorSlot slot;
    return slot;
}

int set_error(ErrorSlot &slot, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    slot.msg = buf;
    return code;
}

int ensure_workspace(anehip_ctx *ctx, size_t floats) {
    Workspace &ws = ctx->ws;
    if (floats <= ws.partial_floats) return ANEHIP_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    ANEHIP_HIP_TRY(ctx->err, hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return set_error(ctx->err, ANEHIP_ESTATE,
                         "workspace must grow to %zu floats during capture: make the same call once before "
                         "anehip_capture_begin",
                         floats);
    if (ws.partial) {
        // queued kernels may still read the old buffer
        ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
        (void)hipFree(ws.partial);
    }
    ws.partial = nullptr;
    ws.partial_floats = 0;
    size_t want = floats < (1u << 20) ? (1u << 20) : floats;
    if (hipMalloc(&ws.partial, want * sizeof(float)) != hipSuccess)
        return set_error(ctx->err, ANEHIP_ENOMEM, "workspace: cannot allocate %zu floats", want);
    ws.partial_floats = want;
    return ANEHIP_OK;
}

}  // namespace anehip

using namespace anehip;

extern "C" {

int anehip_init(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return set_error(global_error(), ANEHIP_ENODEV, "no HIP device visible");
    for (int d = 0; d < n; d++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, d) == hipSuccess && std::strncmp(p.gcnArchName, "gfx950", 6) == 0)
            return ANEHIP_OK;
    }
    return set_error(global_error(), ANEHIP_ENODEV, "no gfx950 device among %d HIP devices", n);
}

const char *anehip_last_error(const anehip_ctx *ctx) {
    return ctx ? ctx->err.msg.c_str() : global_error().msg.c_str();
}

int anehip_model_setup(anehip_ctx *ctx, const anehip_model_desc *desc);  // decode.hip
void anehip_model_teardown(anehip_ctx *ctx);                             // decode.hip

int anehip_ctx_create(int device, const anehip_model_desc *desc, anehip_ctx **out) {
    if (!out) return set_error(global_error(), ANEHIP_EINVAL, "ctx_create: out is NULL");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
        return set_error(global_error(), ANEHIP_ENODEV, "ctx_create: device %d not present (%d visible)", device, n);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess || std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return set_error(global_error(), ANEHIP_ENODEV, "ctx_create: device %d is %s, not gfx950", device,
                         p.gcnArchName);
    if (hipSetDevice(device) != hipSuccess)
        return set_error(global_error(), ANEHIP_EHIP, "ctx_create: hipSetDevice(%d) failed", device);
    anehip_ctx *ctx = new anehip_ctx();
    ctx->device = device;
    ctx->cu_count = p.multiProcessorCount;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&ctx->ev_start) != hipSuccess || hipEventCreate(&ctx->ev_stop) != hipSuccess) {
        anehip_ctx_destroy(ctx);
        return set_error(global_error(), ANEHIP_EHIP, "ctx_create: stream/event creation failed");
    }
    if (hipMalloc(&ctx->dn_count, kDnCounters * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(ctx->dn_count, 0, kDnCounters * sizeof(uint32_t)) != hipSuccess) {
        anehip_ctx_destroy(ctx);
        return set_error(global_error(), ANEHIP_ENOMEM, "ctx_create: counter allocation failed");
    }
    int rc = ensure_workspace(ctx, 0);
    if (rc == ANEHIP_OK) rc = noalloc_setup(ctx);
    if (rc == ANEHIP_OK && desc) rc = anehip_model_setup(ctx, desc);
    if (rc != ANEHIP_OK) {
        set_error(global_error(), rc, "ctx_create: %s", ctx->err.msg.c_str());
        anehip_ctx_destroy(ctx);
        return rc;
    }
    *out = ctx;
    return ANEHIP_OK;
}

void anehip_ctx_destroy(anehip_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    anehip_model_teardown(ctx);
    for (void *p : ctx->user_allocs) (void)hipFree(p);
    if (ctx->ws.partial) (void)hipFree(ctx->ws.partial);
    if (ctx->inv_freq) (void)hipFree(ctx->inv_freq);
    if (ctx->dn_count) (void)hipFree(ctx->dn_count);
    if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
    if (ctx->ev_stop) (void)hipEventDestroy(ctx->ev_stop);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int anehip_sync(anehip_ctx *ctx) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "sync: ctx is NULL");
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    return ANEHIP_OK;
}

int anehip_dev_alloc(anehip_ctx *ctx, size_t nbytes, void **dptr) {
    if (!ctx || !dptr || nbytes == 0) return set_error(ctx ? ctx->err : global_error(), ANEHIP_EINVAL, "dev_alloc: bad argument");
    (void)hipSetDevice(ctx->device);
    void *p = nullptr;
    if (hipMalloc(&p, nbytes) != hipSuccess) {
        (void)hipGetLastError();
        return set_error(ctx->err, ANEHIP_ENOMEM, "dev_alloc: hipMalloc(%zu) failed", nbytes);
    }
    ctx->user_allocs.push_back(p);
    *dptr = p;
    return ANEHIP_OK;
}

int anehip_dev_free(anehip_ctx *ctx, void *dptr) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "dev_free: ctx is NULL");
    for (size_t i = 0; i < ctx->user_allocs.size(); i++) {
        if (ctx->user_allocs[i] == dptr) {
            ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
            ANEHIP_HIP_TRY(ctx->err, hipFree(dptr));
            ctx->user_allocs.erase(ctx->user_allocs.begin() + i);
            return ANEHIP_OK;
        }
    }
    return set_error(ctx->err, ANEHIP_EINVAL, "dev_free: %p was not allocated by this context", dptr);
}

int anehip_h2d(anehip_ctx *ctx, void *dst, const void *src, size_t nbytes) {
    if (!ctx || (!dst && nbytes) || (!src && nbytes)) return set_error(ctx ? ctx->err : global_error(), ANEHIP_EINVAL, "h2d: bad argument");
    if (!nbytes) return ANEHIP_OK;
    ANEHIP_HIP_TRY(ctx->err, hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, ctx->stream));
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    return ANEHIP_OK;
}

int anehip_d2h(anehip_ctx *ctx, void *dst, const void *src, size_t nbytes) {
    if (!ctx || (!dst && nbytes) || (!src && nbytes)) return set_error(ctx ? ctx->err : global_error(), ANEHIP_EINVAL, "d2h: bad argument");
    if (!nbytes) return ANEHIP_OK;
    ANEHIP_HIP_TRY(ctx->err, hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, ctx->stream));
    ANEHIP_HIP_TRY(ctx->err, hipStreamSynchronize(ctx->stream));
    return ANEHIP_OK;
}

int anehip_dev_memset(anehip_ctx *ctx, void *dst, int value, size_t nbytes) {
    if (!ctx || (!dst && nbytes)) return set_error(ctx ? ctx->err : global_error(), ANEHIP_EINVAL, "memset: bad argument");
    if (!nbytes) return ANEHIP_OK;
    // a memset node recorded into a graph is refused (a fill kernel is the
    // capturable way to clear memory)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    ANEHIP_HIP_TRY(ctx->err, hipStreamIsCapturing(ctx->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return set_error(ctx->err, ANEHIP_ESTATE, "memset: not allowed while the stream is being captured");
    ANEHIP_HIP_TRY(ctx->err, hipMemsetAsync(dst, value, nbytes, ctx->stream));
    return ANEHIP_OK;
}

int anehip_d2d(anehip_ctx *ctx, void *dst, const void *src, size_t nbytes) {
    if (!ctx || (!dst && nbytes) || (!src && nbytes)) return set_error(ctx ? ctx->err : global_error(), ANEHIP_EINVAL, "d2d: bad argument");
    if (!nbytes) return ANEHIP_OK;
    ANEHIP_HIP_TRY(ctx->err, hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, ctx->stream));
    return ANEHIP_OK;
}

int anehip_timer_start(anehip_ctx *ctx) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "timer_start: ctx is NULL");
    ANEHIP_HIP_TRY(ctx->err, hipEventRecord(ctx->ev_start, ctx->stream));
    return ANEHIP_OK;
}

int anehip_timer_stop(anehip_ctx *ctx, float *ms) {
    if (!ctx || !ms) return set_error(ctx ? ctx->err : global_error(), ANEHIP_EINVAL, "timer_stop: bad argument");
    ANEHIP_HIP_TRY(ctx->err, hipEventRecord(ctx->ev_stop, ctx->stream));
    ANEHIP_HIP_TRY(ctx->err, hipEventSynchronize(ctx->ev_stop));
    ANEHIP_HIP_TRY(ctx->err, hipEventElapsedTime(ms, ctx->ev_start, ctx->ev_stop));
    return ANEHIP_OK;
}

int anehip_quant_gemm(anehip_ctx *ctx, uint32_t ggml_type, const void *w, uint32_t m, uint32_t n,
                      const float *x, uint32_t batch, float *y) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "quant_gemm: ctx is NULL");
    if (!w || !x || !y) return set_error(ctx->err, ANEHIP_EINVAL, "quant_gemm: null pointer");
    if (ggml_type != ANEHIP_GGML_Q8_0 && ggml_type != ANEHIP_GGML_Q4_0)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "quant_gemm: ggml type %u (only Q4_0=2, Q8_0=8)", ggml_type);
    if (m == 0 || n == 0 || n % 32 != 0)
        return set_error(ctx->err, ANEHIP_ESHAPE, "quant_gemm: n=%u must be a positive multiple of 32 (m=%u)", n, m);
    if (n % 256 != 0)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "quant_gemm: n=%u is not a multiple of 256", n);
    if (batch == 0 || batch > 32)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "quant_gemm: batch=%u outside 1..32", batch);
    return launch_quant_gemm(ctx, ctx->stream, ggml_type, w, m, n, x, batch, y);
}

int anehip_quant_gemm_packed(anehip_ctx *ctx, uint32_t ggml_type, const void *wp, uint32_t m, uint32_t n,
                             const float *x, uint32_t batch, float *y) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "quant_gemm_packed: ctx is NULL");
    if (!wp || !x || !y) return set_error(ctx->err, ANEHIP_EINVAL, "quant_gemm_packed: null pointer");
    if (ggml_type != ANEHIP_GGML_Q8_0 && ggml_type != ANEHIP_GGML_Q4_0)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "quant_gemm_packed: ggml type %u (only Q4_0=2, Q8_0=8)",
                         ggml_type);
    if (m == 0 || n == 0 || n % 256)
        return set_error(ctx->err, ANEHIP_ESHAPE, "quant_gemm_packed: n=%u must be a positive multiple of 256", n);
    if (batch == 0 || batch > 256)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "quant_gemm_packed: batch=%u outside 1..256", batch);
    if (batch == 1) return anehip_quant_gemv_packed(ctx, ggml_type, wp, m, n, x, y);
    const int ksplit = gemm_rows_ksplit(ctx, m, n, batch);
    if (m % 4)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "quant_gemm_packed: m=%u must be a multiple of 4 for batch > 1",
                         m);
    // batch > 32: one 32-row group of planes per 32 rows (the prefill GEMM)
    const size_t groups = (batch + 31) / 32;
    const size_t count = (size_t)batch * m, xcount = groups * xf_plane_len(n);
    // The x-stationary kernels read the fp32 rows themselves and split them
    // into hi / lo fragments in each workgroup: at batch <= 16 (gemm_xs16)
    // and for splits of at most 2 panels.  Wider splits at batch 17-32
    // (lm_head: one split of 8 panels on gemm_xsh, whose 8 waves each split
    // a quarter of the row) first split x into planes with one launch.
    // Measured on MI355X (graphs of back-to-back calls, weights rotated):
    // lm_head 151936 x 2048 at batch 4 / 16 / 32 57.1-57.3 / 63.6-65.7 /
    // 72.9-74.2 us on the rows against 59.2-62.1 / 64.5-66.4 / 71.4-74.1 us
    // split first; 6144 x 2048 and 2048 x 6144 (2-panel splits) 9.2-14.5 us on
    // the rows against 0.2-1.4 us more split first.
    const int nsb = (int)(n / 256);
    if (batch <= 32 && gemm_is_xs(ctx, m, n, batch) && (batch <= 16 || nsb / ksplit <= 2)) {
        // the x-stationary kernels read the fp32 rows themselves: partials, then their sum
        if (ksplit == 1) return launch_gemm_xs_rows(ctx, ctx->stream, ggml_type, wp, m, n, x, batch, y);
        int rc = ensure_workspace(ctx, (size_t)ksplit * count);
        if (rc) return rc;
        if ((rc = launch_gemm_xs_rows(ctx, ctx->stream, ggml_type, wp, m, n, x, batch, ctx->ws.partial))) return rc;
        return launch_sum_partials(ctx, ctx->stream, ctx->ws.partial, y, count, ksplit);
    }
    // workspace: [x hi plane][x lo plane] (fp16, xcount each), the group
    // exponents, then the partials
    const size_t planes = xcount + (groups * xe_bytes(n) + 3) / 4;  // floats holding both planes and the exponents
    int rc = ensure_workspace(ctx, planes + (ksplit > 1 ? (size_t)ksplit * count : 0));
    if (rc) return rc;
    Planes xp;
    xp.hi = reinterpret_cast<_Float16 *>(ctx->ws.partial);
    xp.lo = xp.hi + xcount;
    xp.xe = reinterpret_cast<int8_t *>(xp.lo + xcount);
    if ((rc = launch_split_x(ctx, ctx->stream, x, batch, n, xp))) return rc;
    if (ksplit == 1) return launch_gemm_rows(ctx, ctx->stream, ggml_type, wp, m, n, xp, batch, y, 1);
    float *part = ctx->ws.partial + planes;
    if ((rc = launch_gemm_rows(ctx, ctx->stream, ggml_type, wp, m, n, xp, batch, part, ksplit))) return rc;
    return launch_sum_partials(ctx, ctx->stream, part, y, count, ksplit);
}

struct anehip_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

int anehip_capture_begin(anehip_ctx *ctx) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "capture_begin: ctx is NULL");
    ANEHIP_HIP_TRY(ctx->err, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    return ANEHIP_OK;
}

int anehip_capture_end(anehip_ctx *ctx, anehip_graph **out) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "capture_end: ctx is NULL");
    if (!out) return set_error(ctx->err, ANEHIP_EINVAL, "capture_end: out is NULL");
    *out = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return set_error(ctx->err, ANEHIP_EHIP, "capture_end: %s", hipGetErrorString(e));
    }
    anehip_graph *G = new anehip_graph();
    G->graph = g;
    e = hipGraphInstantiate(&G->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        anehip_graph_destroy(G);
        return set_error(ctx->err, ANEHIP_EHIP, "capture_end: instantiate: %s", hipGetErrorString(e));
    }
    *out = G;
    return ANEHIP_OK;
}

int anehip_graph_launch(anehip_ctx *ctx, anehip_graph *graph) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "graph_launch: ctx is NULL");
    if (!graph || !graph->exec) return set_error(ctx->err, ANEHIP_EINVAL, "graph_launch: no graph");
    ANEHIP_HIP_TRY(ctx->err, hipGraphLaunch(graph->exec, ctx->stream));
    return ANEHIP_OK;
}

void anehip_graph_destroy(anehip_graph *graph) {
    if (!graph) return;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
}

size_t anehip_quant_packed_bytes(uint32_t ggml_type, uint32_t m, uint32_t n) {
    if ((ggml_type != ANEHIP_GGML_Q8_0 && ggml_type != ANEHIP_GGML_Q4_0) || m == 0 || n == 0 || n % 256) return 0;
    return packed_bytes(ggml_type, m, n);
}

static int check_packed_args(anehip_ctx *ctx, const char *what, uint32_t ggml_type, uint32_t m, uint32_t n) {
    if (ggml_type != ANEHIP_GGML_Q8_0 && ggml_type != ANEHIP_GGML_Q4_0)
        return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "%s: ggml type %u (only Q4_0=2, Q8_0=8)", what, ggml_type);
    if (m == 0 || n == 0 || n % 256)
        return set_error(ctx->err, ANEHIP_ESHAPE, "%s: n=%u must be a positive multiple of 256 (m=%u)", what, n, m);
    return ANEHIP_OK;
}

int anehip_quant_pack(anehip_ctx *ctx, uint32_t ggml_type, const void *w, uint32_t m, uint32_t n, void *dst) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "quant_pack: ctx is NULL");
    if (!w || !dst) return set_error(ctx->err, ANEHIP_EINVAL, "quant_pack: null pointer");
    int rc = check_packed_args(ctx, "quant_pack", ggml_type, m, n);
    if (rc) return rc;
    return launch_repack(ctx, ctx->stream, ggml_type, w, m, n, dst);
}

int anehip_quant_gemv_packed(anehip_ctx *ctx, uint32_t ggml_type, const void *wp, uint32_t m, uint32_t n,
                             const float *x, float *y) {
    if (!ctx) return set_error(global_error(), ANEHIP_EINVAL, "quant_gemv_packed: ctx is NULL");
    if (!wp || !x || !y) return set_error(ctx->err, ANEHIP_EINVAL, "quant_gemv_packed: null pointer");
    int rc = check_packed_args(ctx, "quant_gemv_packed", ggml_type, m, n);
    if (rc) return rc;
    // few row tiles and n <= 8192: one launch with no K split
    if (const int H = gemv_rows_split(ctx, m, n)) return launch_gemv_rows(ctx, ctx->stream, ggml_type, wp, m, n, x, y, H);
    const int ksplit = gemv_packed_ksplit(ctx, m, n);  // the decode step's choice (<= 8 splits)
    GemvInput in;
    in.x = x;
    if (ksplit == 1) return launch_gemv_packed(ctx, ctx->stream, ggml_type, wp, m, n, in, y, 1);
    if ((rc = ensure_workspace(ctx, (size_t)ksplit * m))) return rc;
    if ((rc = launch_gemv_packed(ctx, ctx->stream, ggml_type, wp, m, n, in, ctx->ws.partial, ksplit))) return rc;
    return launch_sum_partials(ctx, ctx->stream, ctx->ws.partial, y, m, ksplit);
}

}  // extern "C"
