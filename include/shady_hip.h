/*
 * shady_hip.h: C ABI of the MI355X (gfx950) quantized-linear backend.
 *
 * Drop-in for the GPTQ linear path of tmzt/shady-thinker: the Rust host keeps
 * `Model::gptq_matvec` / `Model::fused_silu_gptq_down` and its call sites
 * (src/model.rs:357-408, called from Model::forward src/model.rs:669-969 and
 * InferenceSession::generate_tokens src/inference.rs:72-131); inside, those
 * helpers call these functions instead of GpuContext::dispatch
 * (src/gpu.rs:188-234) with a WGSL shader.
 *
 * Conventions
 *  - Plain pointers and sizes only. Every tensor argument is a device pointer
 *    (from st_alloc or any hipMalloc allocation) unless the name says `host`.
 *  - Layouts are the reference's, unmodified (src/weights.rs:398 uploads the
 *    GPTQ safetensors bytes verbatim):
 *      qweight u32[K/8, N]  eight 4-bit values per word along K, low nibble =
 *                           lowest k (src/shaders/gptq_matvec.wgsl:51-59)
 *      scales  f16[K/gs, N] (read as u32 pairs by the WGSL, :41-45)
 *      qzeros  u32[K/gs, N/8] eight zero points per word along N (AutoGPTQ;
 *                           dropped by the reference, src/weights.rs:372-374)
 *      x       [M, K] row-major, y [M, N] row-major (M = 1 for decode)
 *    INT8 weights (no reference counterpart) are int8[N, K] row-major with
 *    f32 per-output-channel scales[N].
 *  - Every call is asynchronous and ordered on the context's stream, like the
 *    reference's single queue (src/gpu.rs:176-242). st_flush() waits.
 *  - Return value: ST_OK (0) or an st_status code; st_last_error() gives the
 *    message for the calling thread. The Rust side `expect`s on non-zero to
 *    keep the reference's panic semantics.
 *  - A context is not thread-safe (the reference serialises through
 *    `&mut GpuContext`).
 *  - No call allocates. The context's workspace (st_context_reserve_workspace)
 *    holds the prefill GEMM's pre-processed A and split-K partials, the
 *    split-K partials of multi-token (M > 1) decode calls on linears with few
 *    16-column tiles, and the split f32 x of multi-token GPTQ calls with
 *    act-order; one-token decode calls use none. Calls on one context
 *    are ordered by its stream, so they never overlap on it.
 */
#ifndef SHADY_HIP_H
#define SHADY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct st_context st_context;

typedef enum {
    ST_OK = 0,
    ST_ERR_INVALID = 1,     /* null pointer / bad enum */
    ST_ERR_SHAPE = 2,       /* K, N, M or group size not supported */
    ST_ERR_ALIGN = 3,       /* pointer not 16-byte aligned */
    ST_ERR_UNSUPPORTED = 4, /* valid request this build does not implement */
    ST_ERR_HIP = 5,         /* HIP runtime error */
    ST_ERR_WORKSPACE = 6,   /* context workspace too small */
    ST_ERR_OOM = 7
} st_status;

typedef enum { ST_F32 = 0, ST_F16 = 1, ST_BF16 = 2 } st_dtype;

/* flags */
#define ST_FLAG_ZEROS_PLUS_ONE 0x1u /* qzeros hold z - 1 (AutoGPTQ v1 files) */
#define ST_FLAG_TILED 0x2u          /* weights in the tiled layout of st_gptq_i4_repack / st_int8_repack */

/* ------------------------------------------------------------ runtime */

/* Message of the last failed call on this thread ("" if none). */
const char *st_last_error(void);

/* Version string of the built library (kernels + ABI revision). */
const char *st_version(void);

/* Replaces GpuContext::new (src/gpu.rs:17-78): binds `device`, creates one
 * stream and the split-K workspace (default 64 MiB). */
int st_context_create(int device, st_context **out);

/* Replaces GpuContext::from_device_queue (src/gpu.rs:24-33): run on a caller
 * stream (hipStream_t passed as void*; NULL = the device's null stream)
 * instead of the context's own. Does not synchronise (ordering between the
 * old and the new stream is the caller's); legal during stream capture. */
int st_context_set_stream(st_context *ctx, void *hip_stream);
void *st_context_stream(st_context *ctx);

/* Grow the split-K workspace to at least `bytes` (call at init, never on the
 * hot path; kernels never allocate). */
int st_context_reserve_workspace(st_context *ctx, size_t bytes);

int st_context_destroy(st_context *ctx);

/* Kernel-path overrides of one context. No counterpart in the reference (its
 * WGSL path has one shader per op); for tests that force each path and for
 * tuning. Every setting starts at -1 (automatic: the library's shape rules
 * choose); a call made after a change uses the new value. Nothing is read
 * from the environment. */
typedef enum {
    ST_TUNE_DECODE_KERNEL = 0, /* 1-4 tokens on tiled weights: 0 register-ring, 1 streaming */
    ST_TUNE_STAGE_MODE,        /* register-ring, one token block: 1 staging waves, 2 per-wave staging */
    ST_TUNE_STAGE_ROUNDS,      /* register-ring staging waves: 64-item rounds each (1..4) */
    ST_TUNE_WAVES,             /* register-ring, one tile per workgroup: waves (4..16) */
    ST_TUNE_NO_COOP,           /* 1: register-ring per-wave fallback only */
    ST_TUNE_ONE_TILE,          /* 1: one 16-column tile per workgroup */
    ST_TUNE_NO_CHUNK,          /* 1: no K-chunked cooperative staging (several tokens) */
    ST_TUNE_NO_KSPLIT,         /* 1: no split-K of several-token decode on few tiles */
    ST_TUNE_SPLIT_TILES_CU,    /* several-token decode: split K up to this many tiles per CU */
    ST_TUNE_TOKEN_BLOCK,       /* decode: tokens per launch (1..16) */
    ST_TUNE_I4MM_MIN_M,        /* GPTQ decode: fewest tokens for the f16-MFMA kernel (default 5 on more tiles than CUs, 9 on fewer) */
    ST_TUNE_I4MM_MIN_TILES,    /* GPTQ decode: fewest 16-column tiles for the f16-MFMA kernel */
    ST_TUNE_I8MM_MIN_M,        /* INT8 decode: fewest tokens for the f16-MFMA kernel */
    ST_TUNE_GEMM_CB,           /* prefill GEMM: 32-column blocks per wave (1 or 2) */
    ST_TUNE_GEMM_NO_SPLIT,     /* 1: prefill GEMM without split-K */
    ST_TUNE_STREAM_WAVES,      /* streaming decode kernel: waves per workgroup (8 or 16) */
    ST_TUNE_STREAM_TILES_WG,   /* streaming decode kernel: 16-column tiles per workgroup (0: a workgroup per CU) */
    ST_TUNE_STREAM_SYNC,       /* streaming decode kernel: ring blocks between workgroup barriers (0: none) */
    ST_TUNE_SPLIT_REDUCE_KERNEL, /* several-token split-K decode: 1 reduce kernel, 0 fused (default: fused up to 8 tokens) */
    ST_TUNE_I4MM_WAVES,        /* f16-MFMA GPTQ decode: 16 forces 16-wave workgroups (default: 12 when the tiles use at most 12) */
    ST_TUNE_I4MM_PAIR,         /* f16-MFMA gate/up: 0 gives each wave one source (default 1: both sources of a tile per wave) */
    ST_TUNE_I4MM_PREPASS,      /* f16-MFMA GPTQ decode, f32 x: 1 splits x in a pre-pass launch (default: in the kernel, unless act-order) */
    ST_TUNE_I4MM_SPLIT_TILES,  /* f16-MFMA GPTQ decode on at most one 16-column tile per CU: tiles per workgroup, K split across workgroups (0: limb kernels) */
    ST_TUNE_COUNT
} st_tune;
int st_context_set_tune(st_context *ctx, int knob, int value);
int st_context_get_tune(st_context *ctx, int knob, int *value);

/* Kernel timing, in place of the reference's wgpu timestamp-less submits
 * (src/gpu.rs:188-242 has no timing): arms two hipEvent_t (created by the
 * caller, passed as void*) on the context. The next kernel launch records
 * `start` at its kernel's start; every launch records `stop` at its kernel's
 * end (hipExtLaunchKernel's dispatch timestamps, the duration a profiler
 * reports, without the gap between launches), so over one entry-point call
 * the pair spans its kernels. Stays armed until called again; NULL, NULL
 * disarms. Not for stream capture. */
int st_context_set_timing_events(st_context *ctx, void *start, void *stop);

/* Pins the context's workspace (delta +1) or releases a pin (-1): a captured
 * HIP graph holds kernels that point into the workspace, so while any pin is
 * held st_context_reserve_workspace refuses to reallocate it. DecoderStack's
 * capture (the host mirror of src/model.rs:669-969) takes one for the life
 * of its graph; no reference counterpart (wgpu has no graphs). */
int st_context_pin_workspace(st_context *ctx, int delta);

/* Replaces GpuContext::create_buffer / create_storage_buffer (src/gpu.rs:80-103): device
 * allocation, size rounded up to 4 bytes, 256-byte aligned. */
int st_alloc(st_context *ctx, size_t bytes, void **out);
int st_free(st_context *ctx, void *ptr);

/* Replaces GpuContext::upload_buffer (src/gpu.rs:105-117): host -> device,
 * returns when the data is on the device. */
int st_upload(st_context *ctx, void *dst, const void *host_src, size_t bytes);

/* Replaces GpuContext::write_buffer (src/gpu.rs:278-282): stream-ordered
 * host -> device write at a byte offset. */
int st_write(st_context *ctx, void *dst, size_t offset, const void *host_src, size_t bytes);

/* Replaces GpuContext::read_buffer (src/gpu.rs:252-276): waits for all queued
 * work, then copies device -> host. */
int st_read(st_context *ctx, const void *src, void *host_dst, size_t bytes);

/* Replaces GpuContext::copy_buffer (src/gpu.rs:245-250), stream-ordered. */
int st_copy(st_context *ctx, void *dst, const void *src, size_t bytes);

/* Replaces GpuContext::flush (src/gpu.rs:237-242): wait for the stream. */
int st_flush(st_context *ctx);

/* -------------------------------------------------------- GPTQ int4 */

/* y = x . dequant(W), W[k, n] = (q[k, n] - z[g(k), n]) * scales[g(k), n].
 * Replaces Model::gptq_matvec (src/model.rs:357-381) dispatching
 * gptq_matvec(_4t).wgsl (src/shaders/gptq_matvec_4t.wgsl:20-86).
 *   x        [M, K] in x_dtype (ST_F32 or ST_F16)
 *   qzeros   NULL = symmetric z = 8, the reference's only mode
 *   perm     NULL, or int32[K] from st_gptq_i4_act_order (then qweight is the
 *            act-order-sorted copy): x is read as x[:, perm[k]]
 *   y        f32 [M, N]
 *   flags    ST_FLAG_ZEROS_PLUS_ONE, ST_FLAG_TILED (qweight from st_gptq_i4_repack)
 * Requires K % group_size == 0, group_size in {64, 128, 256}, N % 8 == 0,
 * 1 <= M <= 32, 16-byte aligned qweight and x. Accumulation: exact integer
 * products of the nibbles with a 3 x 8-bit split of x scaled by a power of
 * two per group, f32 across groups (rel-L2 vs f64 ~1e-7). For 5-32 tokens
 * on tiled weights when N has more 16-column tiles than the GPU has CUs, and
 * 9-32 when it has fewer (then with K split across workgroups and partial
 * sums in the context workspace), with or without perm: f16 MFMA on exact
 * (q - z) and x (f16 x as is; f32 x split into two f16 parts per 128 k while
 * it is staged, or with perm by a pre-pass into the context workspace), f32
 * sums, rel-L2 vs f64 ~1e-7, the weights read once for up to 32 tokens. The
 * same rule applies to st_gptq_i4_gate_up_silu. */
int st_gptq_i4_matvec(st_context *ctx, const void *x, int x_dtype,
                      const uint32_t *qweight, const uint16_t *scales,
                      const uint32_t *qzeros, const int32_t *perm, float *y,
                      int M, int K, int N, int group_size, uint32_t flags);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). st_gptq_i4_matvec with everything its kernels keep
 * beyond the inputs and outputs (the f16-MFMA kernel's split of f32 x into
 * f16 rows, split-K partial sums) in a fixed array of
 * ST_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs on,
 * from the context's creation until the process ends, instead of the
 * context workspace. Allocates nothing. A call whose scratch would exceed
 * the array fails with ST_ERR_WORKSPACE and launches nothing. The check is
 * conservative: for f32 x (and for f16 x under act-order) it counts the
 * f16-MFMA kernel's split rows of one launch, 4 M K + M K / 32 bytes
 * (f16 x with perm: 2 M K), with M capped at 32, whichever kernel the call
 * then takes; split-K partials are not counted (they shrink or go unsplit
 * to fit the array). Every call on
 * one GPU shares that GPU's array (nothing in it needs to start at zero;
 * each call overwrites what it reads): calls that overlap on one GPU (other
 * streams or contexts) race. */
#define ST_NOALLOC_SCRATCH_BYTES (8u << 20)
int st_gptq_i4_matvec_noalloc(st_context *ctx, const void *x, int x_dtype, const uint32_t *qweight,
                              const uint16_t *scales, const uint32_t *qzeros, const int32_t *perm, float *y, int M,
                              int K, int N, int group_size, uint32_t flags);

/* y = (silu(a) * b) . dequant(W), silu(v) = v / (1 + exp(-v)).
 * Replaces Model::fused_silu_gptq_down (src/model.rs:383-408) dispatching
 * fused_silu_gptq(_4t).wgsl (src/shaders/fused_silu_gptq_4t.wgsl:26-81).
 * a, b: f32 [M, K]. Other arguments as st_gptq_i4_matvec. */
int st_gptq_i4_silu_matvec(st_context *ctx, const float *a, const float *b,
                           const uint32_t *qweight, const uint16_t *scales,
                           const uint32_t *qzeros, const int32_t *perm, float *y,
                           int M, int K, int N, int group_size, uint32_t flags);

/* y = silu(x . dequant(Wg)) * (x . dequant(Wu)), both [K, N].
 * Replaces fused_gate_up_silu(_4t).wgsl (src/shaders/fused_gate_up_silu_4t.wgsl:28-91,
 * declared at src/model.rs:8; the reference's forward runs gate and up as two
 * gptq_matvec calls at src/model.rs:803-808). Both weights share perm.
 * 1 <= M <= 32; other arguments as st_gptq_i4_matvec. */
int st_gptq_i4_gate_up_silu(st_context *ctx, const void *x, int x_dtype,
                            const uint32_t *qweight_gate, const uint16_t *scales_gate,
                            const uint32_t *qzeros_gate, const uint32_t *qweight_up,
                            const uint16_t *scales_up, const uint32_t *qzeros_up,
                            const int32_t *perm, float *y, int M, int K, int N,
                            int group_size, uint32_t flags);

/* Materialise dequant(W) as out[K, N] in out_dtype (ST_F32 exact; ST_BF16
 * round-to-nearest-even, which is src/weights.rs:257-313
 * dequant_gptq_to_bf16). g_idx NULL = k / group_size (no act-order);
 * otherwise the original int32 g_idx[K] of the checkpoint. */
int st_gptq_i4_dequant(st_context *ctx, const uint32_t *qweight, const uint16_t *scales,
                       const uint32_t *qzeros, const int32_t *g_idx, void *out, int out_dtype,
                       int K, int N, int group_size, uint32_t flags);

/* Upload-time repack into the decode kernels' tiled layout (no reference
 * counterpart; an optional step of the weight upload, src/weights.rs:398):
 * per 16-column tile and group, the 64 lanes' words are contiguous, so the
 * kernel reads 1 KiB contiguous per group with 128-bit loads. Dequantized
 * values are unchanged (a permutation of whole words). qweight_tiled must hold
 * st_gptq_i4_tiled_words(K, N, group_size) words; pass ST_FLAG_TILED to the
 * matvec entry points with it. */
size_t st_gptq_i4_tiled_words(int K, int N, int group_size);
int st_gptq_i4_repack(st_context *ctx, const uint32_t *qweight, uint32_t *qweight_tiled, int K, int N,
                      int group_size);

/* Upload-time act-order preparation (the reference drops .g_idx,
 * src/weights.rs:372-374). Sorts K by group: perm_out[j] = the original row
 * placed at position j (stable, ascending g_idx), and qweight_out = qweight
 * with its rows permuted the same way (re-packed nibbles; dequantized values
 * unchanged). Each group must hold exactly group_size rows. Scales and
 * qzeros are unchanged. g_idx is a device pointer; blocks until done. */
int st_gptq_i4_act_order(st_context *ctx, const uint32_t *qweight, const int32_t *g_idx,
                         uint32_t *qweight_out, int32_t *perm_out, int K, int N,
                         int group_size);

/* bf16 matvec: y[M, N] = x[M, K] . W^T, W bf16 row-major [N, K] (two bf16 per
 * u32, low half first), x f32 or f16 (x_dtype), y f32, 1 <= M <= 8,
 * K % 8 == 0, K <= 10240 (M <= 4) or 5120 (M <= 8). Replaces src/shaders/bf16_matvec.wgsl:21-72 (the
 * lm_head / tied-embedding projection, dispatched at src/model.rs:455-468
 * and :824-831); f32 accumulation, results within 1e-4 rel-L2 of f64. */
int st_bf16_matvec(st_context *ctx, const void *x, int x_dtype, const uint16_t *w, float *y, int M, int K,
                   int N);

/* Prefill GEMM: C[M, N] = A[M, K] . dequant(W), A f16, C in c_dtype (ST_F32
 * or ST_F16). No reference counterpart (the reference prefills token by
 * token, src/inference.rs:93-95). MFMA f16 with integer-valued (q - z)
 * operands, f32 accumulation, per-group scale applied after each group.
 * perm as st_gptq_i4_matvec. */
int st_gptq_i4_gemm(st_context *ctx, const uint16_t *a, const uint32_t *qweight,
                    const uint16_t *scales, const uint32_t *qzeros, const int32_t *perm,
                    void *c, int c_dtype, int M, int K, int N, int group_size,
                    uint32_t flags);

/* Gate and up projections of one MLP for M tokens in one call:
 * c_gate = a . dequant(W_gate) and c_up = a . dequant(W_up), both [M, N],
 * from one pre-processed A and (when no split-K is needed) one launch whose
 * grid holds the tiles of both weights. The M-token form of the gate/up
 * half of the reference's MLP (src/model.rs:803-811, the separate gate and
 * up matvecs it runs one token at a time); st_gptq_i4_silu_gemm then takes
 * c_gate and c_up for the down projection. Both weights share K, N,
 * group_size, flags and perm; either may have qzeros or not. Each output is
 * bit for bit what st_gptq_i4_gemm gives for that weight. */
int st_gptq_i4_gate_up_gemm(st_context *ctx, const uint16_t *a, const uint32_t *gate_qweight,
                            const uint16_t *gate_scales, const uint32_t *gate_qzeros,
                            const uint32_t *up_qweight, const uint16_t *up_scales,
                            const uint32_t *up_qzeros, const int32_t *perm, void *c_gate, void *c_up,
                            int c_dtype, int M, int K, int N, int group_size, uint32_t flags);

/* Prefill GEMM on silu(gate) * up: C[M, N] = (silu(gate) * up)[M, K] .
 * dequant(W), gate and up f16 [M, K], silu(v) = v / (1 + exp(-v)) in f32,
 * the product rounded once to f16. The M-token form of
 * Model::fused_silu_gptq_down (src/model.rs:383-408, fused_silu_gptq(_4t).wgsl),
 * which the reference runs one token at a time (src/model.rs:803-811). Other
 * arguments as st_gptq_i4_gemm. */
int st_gptq_i4_silu_gemm(st_context *ctx, const uint16_t *gate, const uint16_t *up,
                         const uint32_t *qweight, const uint16_t *scales, const uint32_t *qzeros,
                         const int32_t *perm, void *c, int c_dtype, int M, int K, int N,
                         int group_size, uint32_t flags);

/* ------------------------------------------------------------- INT8 */

/* y[M, N] = x[M, K] . (w[N, K]^T * scale[N]), int8 symmetric per output
 * channel. No reference counterpart. x in x_dtype (ST_F16 or ST_F32),
 * 1 <= M <= 32, K % 128 == 0, N % 4 == 0. flags: ST_FLAG_TILED when w is in
 * the layout of st_int8_repack (else row-major int8[N, K]). Two or more
 * tokens with f16 x on tiled weights run on f16 MFMA (every product exact,
 * f32 sums; the weights are read once for all tokens); otherwise exact
 * integer products with a split of x as for st_gptq_i4_matvec. */
int st_int8_matvec(st_context *ctx, const void *x, int x_dtype, const int8_t *w,
                   const float *scale, float *y, int M, int K, int N, uint32_t flags);

/* INT8 prefill GEMM (W8A16): C[M, N] = A[M, K] . (w[N, K]^T * scale[N]),
 * A f16 row-major, C f32 or f16 (c_dtype). No reference counterpart: the
 * north star's INT8 GEMM for prefill, the M-token form of st_int8_matvec
 * for M above its 32 (the reference prefills token by token through the
 * matvec, src/inference.rs:93-95). Every product is exact in f32 (int8 and
 * f16 are exact in f16), the sums are f32, the channel scale is applied once
 * per output. K % 128 == 0, N % 4 == 0; a and w 16-byte aligned; flags:
 * ST_FLAG_TILED for st_int8_repack's layout. Small grids split K across
 * workgroups (f32 partials in the context workspace, added in a fixed order). */
int st_int8_gemm(st_context *ctx, const uint16_t *a, const int8_t *w, const float *scale, void *c,
                 int c_dtype, int M, int K, int N, uint32_t flags);

/* Upload-time INT8 repack (no reference counterpart): row-major w[N, K] ->
 * tiles of 16 rows in which, per 128-k group, each of a wave's 64 lanes
 * holds 32 contiguous bytes, so the kernel reads 2 KiB contiguous per group.
 * Values are unchanged (a permutation of 16-byte pieces). w_tiled must hold
 * st_int8_tiled_bytes(K, N) bytes; pass ST_FLAG_TILED to st_int8_matvec. */
size_t st_int8_tiled_bytes(int K, int N);
int st_int8_repack(st_context *ctx, const int8_t *w, int8_t *w_tiled, int K, int N);

#ifdef __cplusplus
}
#endif

#endif /* SHADY_HIP_H */
