// Context, device memory helpers and the per-thread error message.
// The error convention mirrors needle_last_error (crates/needle-c/src/lib.rs:27-39):
// a failing call records a message on the calling thread and returns non-zero.
#include "nd_internal.h"

#include <cstdio>
#include <new>

namespace {
thread_local std::string g_last_error;
thread_local bool g_has_error = false;
}  // namespace

namespace nd {

int fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    g_has_error = true;
    return code;
}

void clear_error()
{
    g_has_error = false;
    g_last_error.clear();
}

int hip_fail(hipError_t e, const char *what)
{
    return fail(e == hipErrorOutOfMemory ? ND_ERR_NOMEM : ND_ERR_HIP, "%s: %s", what,
                hipGetErrorString(e));
}

int claim(Owner &o, const char *what)
{
    return owner_claim(o) ? ND_OK : fail(ND_ERR_BUSY, "%s is in use by another thread", what);
}

Entry::Entry(nd_ctx *ctx)
{
    if (!ctx) {
        rc = fail(ND_ERR_ARG, "null context");
        return;
    }
    clear_error();
    if ((rc = claim(ctx->owner, "the context")) != ND_OK) return;
    ctx_ = ctx;
    const hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) rc = hip_fail(e, "hipSetDevice(ctx->device)");
}

Entry::~Entry()
{
    if (ctx_) release(ctx_->owner);
}

int workspace(nd_ctx *ctx, size_t bytes, void **out)
{
    if (bytes > ctx->work_bytes) {
        if (ctx->work) {
            ND_HIP(hipStreamSynchronize(ctx->stream));
            ND_HIP(hipFree(ctx->work));
            ctx->work = nullptr;
            ctx->work_bytes = 0;
        }
        size_t want = align_up(bytes, size_t(1) << 20);
        ND_HIP(hipMalloc(&ctx->work, want));
        ctx->work_bytes = want;
    }
    *out = ctx->work;
    return ND_OK;
}

int check_launch(const char *kernel)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ND_ERR_HIP, "launch of %s: %s", kernel, hipGetErrorString(e));
    return ND_OK;
}

}  // namespace nd

extern "C" {

const char *nd_last_error(void) { return g_has_error ? g_last_error.c_str() : nullptr; }

static int ctx_create(int device, bool own, void *stream, nd_ctx **out)
{
    nd::clear_error();
    if (!out) return nd::fail(ND_ERR_ARG, "null output pointer");
    *out = nullptr;
    int n = 0;
    ND_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return nd::fail(ND_ERR_ARG, "device %d out of range (%d devices)", device, n);
    ND_HIP(hipSetDevice(device));
    nd_ctx *c = new (std::nothrow) nd_ctx;
    if (!c) return nd::fail(ND_ERR_NOMEM, "host allocation of the context failed");
    c->device = device;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        delete c;
        return nd::hip_fail(e, "hipGetDeviceProperties");
    }
    c->num_cus = prop.multiProcessorCount;
    // The no-allocation entry point's scratch address: optional, so a
    // failure here leaves it unset (that entry point then reports it) and
    // the context is created all the same.
    if (nd::noalloc_setup(device) != ND_OK) {
        (void)hipGetLastError();
        nd::clear_error();
    }
    if (!own) {
        c->stream = static_cast<hipStream_t>(stream);
    } else {
        e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete c;
            return nd::hip_fail(e, "hipStreamCreateWithFlags");
        }
        c->owns_stream = true;
    }
    *out = c;
    return ND_OK;
}

int nd_ctx_create(int device, nd_ctx **out) { return ctx_create(device, true, nullptr, out); }

int nd_ctx_create_on_stream(int device, void *stream, nd_ctx **out)
{
    return ctx_create(device, false, stream, out);
}

void nd_ctx_destroy(nd_ctx *ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->work) (void)hipFree(ctx->work);
    if (ctx->owns_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int nd_ctx_synchronize(nd_ctx *ctx)
{
    ND_ENTER(ctx);
    ND_HIP(hipStreamSynchronize(ctx->stream));
    return ND_OK;
}

int nd_malloc(nd_ctx *ctx, size_t bytes, void **out)
{
    ND_ENTER(ctx);
    ND_REQUIRE(out, "null output pointer");
    *out = nullptr;
    ND_HIP(hipMalloc(out, bytes ? bytes : 1));
    return ND_OK;
}

int nd_free(nd_ctx *ctx, void *ptr)
{
    ND_ENTER(ctx);
    if (!ptr) return ND_OK;
    ND_HIP(hipStreamSynchronize(ctx->stream));
    ND_HIP(hipFree(ptr));
    return ND_OK;
}

int nd_memcpy_htod(nd_ctx *ctx, void *dst, const void *src, size_t bytes)
{
    ND_ENTER(ctx);
    if (!bytes) return ND_OK;
    ND_REQUIRE(dst && src, "null pointer");
    ND_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    ND_HIP(hipStreamSynchronize(ctx->stream));
    return ND_OK;
}

int nd_memcpy_dtoh(nd_ctx *ctx, void *dst, const void *src, size_t bytes)
{
    ND_ENTER(ctx);
    if (!bytes) return ND_OK;
    ND_REQUIRE(dst && src, "null pointer");
    ND_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    ND_HIP(hipStreamSynchronize(ctx->stream));
    return ND_OK;
}

}  // extern "C"
