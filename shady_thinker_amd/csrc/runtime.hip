// Context, memory and stream entry points of the C ABI. These replace the
// wgpu GpuContext of the reference (src/gpu.rs:7-297): one device, one
// stream (the reference's one queue), device buffers handed out as plain
// pointers.
#include "common.hpp"

#include <cstdlib>
#include <cstring>
#include <mutex>

namespace st {

static thread_local std::string g_last_error;

void set_error(const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

}  // namespace st

static constexpr size_t kDefaultWorkspace = size_t(64) << 20;

// Scratch of st_gptq_i4_matvec_noalloc: one fixed array per GPU, held from
// load until the process ends. Host code never passes the array's name (a
// host-side stand-in, not a device address): each GPU's copy is looked up
// once, with that device current, and its address kept per device.
static __device__ __align__(256) unsigned char scratch[ST_NOALLOC_SCRATCH_BYTES];
static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch[kMaxDevices] = {};

// The scratch address on `device` (which must be current).
static int scratch_for(int device, void **out) {
    if (device >= kMaxDevices) return st::fail(ST_ERR_UNSUPPORTED, "scratch: device %d >= %d", device, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[device]) {
        void *ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return st::hip_fail(e, "hipGetSymbolAddress(scratch)");
        g_scratch[device] = ptr;
    }
    *out = g_scratch[device];
    return ST_OK;
}

extern "C" {

const char *st_last_error(void) { return st::g_last_error.c_str(); }

const char *st_version(void) { return "shady_hip 0.1 gfx950 abi-1"; }

int st_context_create(int device, st_context **out) {
    if (!out) return st::fail(ST_ERR_INVALID, "st_context_create: out is NULL");
    *out = nullptr;
    int count = 0;
    ST_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
        return st::fail(ST_ERR_INVALID, "st_context_create: device %d of %d", device, count);
    ST_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    ST_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return st::fail(ST_ERR_UNSUPPORTED, "st_context_create: device is %s, this library is built for gfx950",
                        prop.gcnArchName);
    void *scr = nullptr;
    if (int rc = scratch_for(device, &scr)) return rc;
    st_context *ctx = new st_context();
    ctx->device = device;
    ctx->scratch = scr;
    ctx->num_cus = prop.multiProcessorCount;
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return st::hip_fail(e, "hipStreamCreateWithFlags");
    }
    ctx->own_stream = true;
    e = hipMalloc(&ctx->ws, kDefaultWorkspace);
    if (e != hipSuccess) {
        if (ctx->ws) (void)hipFree(ctx->ws);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return st::hip_fail(e, "st_context_create: workspace");
    }
    ctx->ws_bytes = kDefaultWorkspace;
    e = hipMalloc(&ctx->split_counters, st::kSplitCounters * sizeof(unsigned));
    if (e == hipSuccess) e = hipMemset(ctx->split_counters, 0, st::kSplitCounters * sizeof(unsigned));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (ctx->split_counters) (void)hipFree(ctx->split_counters);
        (void)hipFree(ctx->ws);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return st::hip_fail(e, "st_context_create: split-K counters");
    }
    *out = ctx;
    st::clear_error();
    return ST_OK;
}

int st_context_set_stream(st_context *ctx, void *hip_stream) {
    if (!ctx) return st::fail(ST_ERR_INVALID, "st_context_set_stream: ctx is NULL");
    hipStream_t ns = static_cast<hipStream_t>(hip_stream);
    if (ns == ctx->stream) return ST_OK;
    // No synchronisation here (it would be illegal under stream capture):
    // ordering between the old and the new stream is the caller's, as for
    // any library handle's set-stream call.
    if (ctx->own_stream) {
        ST_HIP(hipSetDevice(ctx->device));
        ST_HIP(hipStreamSynchronize(ctx->stream));  // our private stream: drain it before destroying
        ST_HIP(hipStreamDestroy(ctx->stream));
        ctx->own_stream = false;
    }
    ctx->stream = ns;  // NULL selects the device's null stream
    return ST_OK;
}

void *st_context_stream(st_context *ctx) { return ctx ? ctx->stream : nullptr; }

int st_context_reserve_workspace(st_context *ctx, size_t bytes) {
    if (!ctx) return st::fail(ST_ERR_INVALID, "st_context_reserve_workspace: ctx is NULL");
    if (bytes <= ctx->ws_bytes) return ST_OK;
    if (ctx->ws_pins > 0)
        return st::fail(ST_ERR_INVALID,
                        "st_context_reserve_workspace: %d captured graph(s) point into the workspace; reserve "
                        "before capturing",
                        ctx->ws_pins);
    ST_HIP(hipSetDevice(ctx->device));
    ST_HIP(hipStreamSynchronize(ctx->stream));
    float *nws = nullptr;
    ST_HIP(hipMalloc(&nws, bytes));
    (void)hipFree(ctx->ws);
    ctx->ws = nws;
    ctx->ws_bytes = bytes;
    return ST_OK;
}

int st_context_set_tune(st_context *ctx, int knob, int value) {
    if (!ctx) return st::fail(ST_ERR_INVALID, "st_context_set_tune: ctx is NULL");
    if (knob < 0 || knob >= ST_TUNE_COUNT) return st::fail(ST_ERR_INVALID, "st_context_set_tune: knob %d", knob);
    ctx->tune[knob] = value < 0 ? -1 : value;
    return ST_OK;
}

int st_context_get_tune(st_context *ctx, int knob, int *value) {
    if (!ctx || !value) return st::fail(ST_ERR_INVALID, "st_context_get_tune: NULL argument");
    if (knob < 0 || knob >= ST_TUNE_COUNT) return st::fail(ST_ERR_INVALID, "st_context_get_tune: knob %d", knob);
    *value = ctx->tune[knob];
    return ST_OK;
}

int st_context_set_timing_events(st_context *ctx, void *start, void *stop) {
    if (!ctx) return st::fail(ST_ERR_INVALID, "st_context_set_timing_events: ctx is NULL");
    ctx->t_start = static_cast<hipEvent_t>(start);
    ctx->t_stop = static_cast<hipEvent_t>(stop);
    return ST_OK;
}

int st_context_pin_workspace(st_context *ctx, int delta) {
    if (!ctx) return st::fail(ST_ERR_INVALID, "st_context_pin_workspace: ctx is NULL");
    if ((delta != 1 && delta != -1) || ctx->ws_pins + delta < 0)
        return st::fail(ST_ERR_INVALID, "st_context_pin_workspace: delta %d with %d pins held", delta, ctx->ws_pins);
    ctx->ws_pins += delta;
    return ST_OK;
}

int st_context_destroy(st_context *ctx) {
    if (!ctx) return ST_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->split_counters) (void)hipFree(ctx->split_counters);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return ST_OK;
}

int st_alloc(st_context *ctx, size_t bytes, void **out) {
    if (!ctx || !out) return st::fail(ST_ERR_INVALID, "st_alloc: NULL argument");
    ST_HIP(hipSetDevice(ctx->device));
    size_t aligned = (bytes + 3) & ~size_t(3);  // src/gpu.rs:86
    if (aligned == 0) aligned = 4;
    hipError_t e = hipMalloc(out, aligned);
    if (e == hipErrorOutOfMemory) return st::fail(ST_ERR_OOM, "st_alloc: %zu bytes: out of memory", bytes);
    if (e != hipSuccess) return st::hip_fail(e, "hipMalloc");
    return ST_OK;
}

int st_free(st_context *ctx, void *ptr) {
    if (!ctx) return st::fail(ST_ERR_INVALID, "st_free: ctx is NULL");
    if (!ptr) return ST_OK;
    ST_HIP(hipSetDevice(ctx->device));
    ST_HIP(hipStreamSynchronize(ctx->stream));
    ST_HIP(hipFree(ptr));
    return ST_OK;
}

int st_upload(st_context *ctx, void *dst, const void *host_src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!host_src && bytes)) return st::fail(ST_ERR_INVALID, "st_upload: NULL argument");
    if (!bytes) return ST_OK;
    ST_HIP(hipMemcpyAsync(dst, host_src, bytes, hipMemcpyHostToDevice, ctx->stream));
    ST_HIP(hipStreamSynchronize(ctx->stream));
    return ST_OK;
}

int st_write(st_context *ctx, void *dst, size_t offset, const void *host_src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!host_src && bytes)) return st::fail(ST_ERR_INVALID, "st_write: NULL argument");
    if (!bytes) return ST_OK;
    // Pageable host memory: hipMemcpyAsync stages it before returning, so the
    // caller may reuse host_src immediately (queue.write_buffer semantics).
    ST_HIP(hipMemcpyAsync(static_cast<char *>(dst) + offset, host_src, bytes, hipMemcpyHostToDevice, ctx->stream));
    return ST_OK;
}

int st_read(st_context *ctx, const void *src, void *host_dst, size_t bytes) {
    if (!ctx || (!src && bytes) || (!host_dst && bytes)) return st::fail(ST_ERR_INVALID, "st_read: NULL argument");
    if (!bytes) return ST_OK;
    ST_HIP(hipMemcpyAsync(host_dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    ST_HIP(hipStreamSynchronize(ctx->stream));
    return ST_OK;
}

int st_copy(st_context *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return st::fail(ST_ERR_INVALID, "st_copy: NULL argument");
    if (!bytes) return ST_OK;
    ST_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return ST_OK;
}

int st_flush(st_context *ctx) {
    if (!ctx) return st::fail(ST_ERR_INVALID, "st_flush: ctx is NULL");
    ST_HIP(hipStreamSynchronize(ctx->stream));
    return ST_OK;
}

}  // extern "C"
