// Context, device memory and stream plumbing behind the C-ABI.
// Replaces the reference's Vulkan runtime (src/gpu/context.zig,
// src/gpu/buffer.zig, src/gpu/kernels.zig:185-194): one device, one stream,
// explicit copies in place of host-mapped UMA buffers.
#include "chn_internal.h"

#include <cstring>

namespace chn {

static thread_local std::string g_init_err;

int set_err(chn_ctx *ctx, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf; else g_init_err = buf;
    return code;
}

int hip_fail(chn_ctx *ctx, hipError_t e, const char *what) {
    int code = (e == hipErrorOutOfMemory) ? CHN_E_OUT_OF_MEMORY
             : (e == hipErrorNoDevice || e == hipErrorInvalidDevice) ? CHN_E_NO_DEVICE
             : CHN_E_HIP;
    return set_err(ctx, code, "%s: %s", what, hipGetErrorString(e));
}

int ensure_workspace(chn_ctx *ctx, size_t bytes) {
    if (ctx->ws_bytes >= bytes) return CHN_OK;
    if (ctx->recording)
        return set_err(ctx, CHN_E_UNSUPPORTED,
                       "the workspace (%zu bytes) must grow to %zu bytes: make one unrecorded call of this shape "
                       "before recording",
                       ctx->ws_bytes, bytes);
    ++ctx->ws_gen;
    if (ctx->ws) {
        CHN_HIP(ctx, hipStreamSynchronize(ctx->stream));
        CHN_HIP(ctx, hipFree(ctx->ws));
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    CHN_HIP(ctx, hipMalloc(&ctx->ws, want));
    ctx->ws_bytes = want;
    return CHN_OK;
}

__global__ void k_fill_u32(uint32_t *dst, uint32_t value, size_t count) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < count; i += stride) dst[i] = value;
}

}  // namespace chn

using namespace chn;

extern "C" int chn_device_count(int *count) {
    if (!count) return set_err(nullptr, CHN_E_INVALID, "count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) { *count = 0; return CHN_OK; }
    if (e != hipSuccess) return hip_fail(nullptr, e, "hipGetDeviceCount");
    *count = n;
    return CHN_OK;
}

extern "C" int chn_init(int device, chn_ctx **out) {
    if (!out) return set_err(nullptr, CHN_E_INVALID, "out is NULL");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || (e == hipSuccess && n == 0))
        return set_err(nullptr, CHN_E_NO_DEVICE, "no HIP device visible");
    if (e != hipSuccess) return hip_fail(nullptr, e, "hipGetDeviceCount");
    if (device < 0 || device >= n)
        return set_err(nullptr, CHN_E_NO_DEVICE, "device %d out of range (%d visible)", device, n);
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(nullptr, e, "hipSetDevice");
    chn_ctx *ctx = new chn_ctx();
    ctx->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
        // some runtimes leave the marketing name empty: the gfx target stands alone then
        ctx->name = prop.name;
        if (prop.gcnArchName[0]) ctx->name += ctx->name.empty() ? std::string(prop.gcnArchName)
                                                                : " (" + std::string(prop.gcnArchName) + ")";
    }
    if (ctx->name.empty()) ctx->name = "HIP device " + std::to_string(device);
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&ctx->t0);
    if (e == hipSuccess) e = hipEventCreate(&ctx->t1);
    if (e != hipSuccess) {
        int rc = hip_fail(nullptr, e, "stream/event create");
        if (ctx->t0) (void)hipEventDestroy(ctx->t0);
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return rc;
    }
    if (noalloc_scratch_init(ctx) != CHN_OK) {
        const int rc = set_err(nullptr, CHN_E_HIP, "%s", ctx->err.c_str());
        chn_destroy(ctx);
        return rc;
    }
    *out = ctx;
    return CHN_OK;
}

// a recording (chn_record_end): the instantiated graph and the workspace
// generation it was made at
struct chn_recording {
    chn_ctx *ctx;
    hipGraphExec_t exec;
    uint64_t ws_gen;
};

static void release_recording(chn_recording *rec) {
    (void)hipGraphExecDestroy(rec->exec);
    delete rec;
}

extern "C" void chn_destroy(chn_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->recording) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(ctx->stream, &g);
        if (g) (void)hipGraphDestroy(g);
    }
    (void)hipStreamSynchronize(ctx->stream);
    for (chn_recording *r : ctx->recs) release_recording(r);
    ctx->recs.clear();
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    (void)hipEventDestroy(ctx->t0);
    (void)hipEventDestroy(ctx->t1);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

extern "C" const char *chn_device_name(const chn_ctx *ctx) { return ctx ? ctx->name.c_str() : ""; }

extern "C" const char *chn_last_error(const chn_ctx *ctx) {
    return ctx ? ctx->err.c_str() : g_init_err.c_str();
}

extern "C" int chn_alloc(chn_ctx *ctx, size_t bytes, void **dptr) {
    if (!ctx || !dptr) return set_err(ctx, CHN_E_INVALID, "NULL argument");
    *dptr = nullptr;
    if (bytes == 0) bytes = 256;
    CHN_HIP(ctx, hipSetDevice(ctx->device));
    CHN_HIP(ctx, hipMalloc(dptr, bytes));
    return CHN_OK;
}

extern "C" int chn_free(chn_ctx *ctx, void *dptr) {
    if (!ctx) return set_err(ctx, CHN_E_INVALID, "NULL ctx");
    if (!dptr) return CHN_OK;
    CHN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    CHN_HIP(ctx, hipFree(dptr));
    return CHN_OK;
}

extern "C" int chn_upload(chn_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return set_err(ctx, CHN_E_INVALID, "NULL argument");
    if (!bytes) return CHN_OK;
    CHN_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    // The source is pageable host memory owned by the caller: wait so that
    // it may be reused as soon as this returns.
    CHN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return CHN_OK;
}

extern "C" int chn_download(chn_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return set_err(ctx, CHN_E_INVALID, "NULL argument");
    if (!bytes) return CHN_OK;
    CHN_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    CHN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return CHN_OK;
}

extern "C" int chn_copy(chn_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return set_err(ctx, CHN_E_INVALID, "NULL argument");
    if (!bytes) return CHN_OK;
    CHN_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return CHN_OK;
}

extern "C" int chn_fill_u32(chn_ctx *ctx, void *dst, uint32_t value, size_t count) {
    if (!ctx || (!dst && count)) return set_err(ctx, CHN_E_INVALID, "NULL argument");
    if (!count) return CHN_OK;
    size_t blocks = (count + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    k_fill_u32<<<dim3((unsigned)blocks), dim3(256), 0, ctx->stream>>>((uint32_t *)dst, value, count);
    CHN_LAUNCHED(ctx, "k_fill_u32");
    return CHN_OK;
}

// ---- recordings (the reference's pre-recorded command buffers) ----------


extern "C" int chn_record_begin(chn_ctx *ctx) {
    if (!ctx) return set_err(ctx, CHN_E_INVALID, "NULL ctx");
    CHN_REQUIRE(ctx, !ctx->recording, "already recording");
    CHN_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->recording = true;
    return CHN_OK;
}

extern "C" int chn_record_end(chn_ctx *ctx, chn_recording **out) {
    if (!ctx || !out) return set_err(ctx, CHN_E_INVALID, "NULL argument");
    *out = nullptr;
    CHN_REQUIRE(ctx, ctx->recording, "not recording");
    ctx->recording = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e != hipSuccess || !g) {
        if (g) (void)hipGraphDestroy(g);
        // a call that failed while recording invalidates the capture
        return hip_fail(ctx, e != hipSuccess ? e : hipErrorStreamCaptureInvalidated, "hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphInstantiate");
    *out = new chn_recording{ctx, exec, ctx->ws_gen};
    ctx->recs.push_back(*out);
    return CHN_OK;
}

extern "C" int chn_submit(chn_ctx *ctx, const chn_recording *rec) {
    if (!ctx || !rec) return set_err(ctx, CHN_E_INVALID, "NULL argument");
    CHN_REQUIRE(ctx, rec->ctx == ctx, "the recording belongs to another context");
    CHN_REQUIRE(ctx, !ctx->recording, "cannot submit while recording");
    CHN_REQUIRE(ctx, rec->ws_gen == ctx->ws_gen,
                "the context workspace was reallocated after this recording was made: record it again");
    CHN_HIP(ctx, hipGraphLaunch(rec->exec, ctx->stream));
    return CHN_OK;
}

extern "C" void chn_recording_free(chn_recording *rec) {
    if (!rec) return;
    chn_ctx *ctx = rec->ctx;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (size_t i = 0; i < ctx->recs.size(); ++i)
        if (ctx->recs[i] == rec) {
            ctx->recs.erase(ctx->recs.begin() + i);
            break;
        }
    release_recording(rec);
}

extern "C" int chn_sync(chn_ctx *ctx) {
    if (!ctx) return set_err(ctx, CHN_E_INVALID, "NULL ctx");
    CHN_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return CHN_OK;
}

extern "C" int chn_timer_start(chn_ctx *ctx) {
    if (!ctx) return set_err(ctx, CHN_E_INVALID, "NULL ctx");
    CHN_HIP(ctx, hipEventRecord(ctx->t0, ctx->stream));
    return CHN_OK;
}

extern "C" int chn_timer_stop(chn_ctx *ctx, float *ms) {
    if (!ctx || !ms) return set_err(ctx, CHN_E_INVALID, "NULL argument");
    CHN_HIP(ctx, hipEventRecord(ctx->t1, ctx->stream));
    CHN_HIP(ctx, hipEventSynchronize(ctx->t1));
    CHN_HIP(ctx, hipEventElapsedTime(ms, ctx->t0, ctx->t1));
    return CHN_OK;
}
