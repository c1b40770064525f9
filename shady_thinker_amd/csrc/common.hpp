// Shared runtime pieces of libshady_hip: the context, error reporting and
// argument checks. gfx950 (CDNA4) only.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "shady_hip.h"

struct st_context {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    int num_cus = 256;
    // Workspace: the prefill GEMM's pre-processed A and split-K partials,
    // and the multi-token decode's split-K partials (each call overwrites
    // what it uses; calls on one context are ordered by its stream).
    float *ws = nullptr;
    size_t ws_bytes = 0;
    int ws_pins = 0;  // captured graphs that point into ws (st_context_pin_workspace)
    // split-K counters of the decode kernels (kSplitCounters words, zero
    // between calls: the last slice of each tile group clears its own)
    unsigned *split_counters = nullptr;
    // the no-allocation entry point's scratch on this context's GPU (the
    // device address of runtime.hip's static array)
    void *scratch = nullptr;
    // kernel-path overrides (st_tune); -1 = automatic
    int tune[ST_TUNE_COUNT];
    // timing events (st_context_set_timing_events): the next launch records
    // t_start at its kernel's start, every launch records t_stop at its end
    hipEvent_t t_start = nullptr, t_stop = nullptr;
    st_context() {
        for (int &t : tune) t = -1;
    }
};

namespace st {

constexpr int kSplitCounters = 4096;

// A kernel-path setting of the context, or `dflt` when it is automatic.
inline int tune(const st_context *ctx, int knob, int dflt) {
    const int v = ctx->tune[knob];
    return v < 0 ? dflt : v;
}

void set_error(const char *fmt, ...);
void clear_error();

inline int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_error("%s", buf);
    return code;
}

inline int hip_fail(hipError_t e, const char *what) {
    return fail(ST_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define ST_HIP(call)                                                       \
    do {                                                                   \
        hipError_t _e = (call);                                            \
        if (_e != hipSuccess) return ::st::hip_fail(_e, #call);            \
    } while (0)

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launch-error check after a kernel launch (launch failures only; faults
// surface at the next synchronising call).
inline int launch_check(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    return ST_OK;
}

// Every kernel launch of the library. With timing events armed on the
// context, the launch goes through hipExtLaunchKernel, which stamps the events
// with the kernel's own start and end (the dispatch's timestamps, as a
// profiler sees them, without the gap between launches): t_start on the first
// launch after arming, t_stop on every launch, so that over a call of several
// launches the pair spans all of them. A stream under capture gets plain
// launches (the events are left alone).
template <typename F, typename... Args>
inline void launch(st_context *ctx, F kernel, dim3 grid, dim3 block, size_t lds, Args... args) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if ((ctx->t_start || ctx->t_stop) && hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess &&
        cs == hipStreamCaptureStatusNone) {
        hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)lds, ctx->stream, ctx->t_start, ctx->t_stop, 0u,
                              args...);
        ctx->t_start = nullptr;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, ctx->stream, args...);
    }
}

// Multi-token INT8 matvec with f16 x on f16 MFMA (i8mm.hip); the caller
// (st_int8_matvec) has checked the arguments.
int int8_mm_f16(st_context *ctx, const void *x, const int8_t *w, const float *scale, float *y, int M, int K, int N);
// Multi-token GPTQ int4 matvec / gate-up on f16 MFMA (i4mm.hip), tiled
// weights (act-order through perm, or NULL), M <= 16; checked by the caller.
// -1: not taken (a K split whose partials do not fit the workspace).
// On at most one 16-column tile per CU it takes groups of kI4mmSplitTiles
// tiles with K split across workgroups (0: the integer-limb kernels).
constexpr int kI4mmSplitTiles = 8;
int int4_mm_f16(st_context *ctx, const void *x, bool x_f32, const int32_t *perm, const uint32_t *const qw[2],
                const uint16_t *const sc[2], const uint32_t *const qz[2], int zoff, float *y, int M, int K, int N,
                int gs, int nsrc);

}  // namespace st
