// C entry points of the decode kernels (GPTQ int4 and INT8 matvec / skinny
// GEMM) and the upload-time GPTQ repack. The kernel itself is in
// qmv_kernel.hpp; see there for the design.
#include "qmv_kernel.hpp"

namespace st {
namespace qmv {
// defined in qmv_i4_p{0,1}.hip, qmv_i4t_p{0,1}.hip, qmv_i8.hip
template <>
int dispatch<FMT_I4, false>(st_context *, Params &, int, int);
template <>
int dispatch<FMT_I4, true>(st_context *, Params &, int, int);
template <>
int dispatch<FMT_I4T, false>(st_context *, Params &, int, int);
template <>
int dispatch<FMT_I4T, true>(st_context *, Params &, int, int);
template <>
int dispatch<FMT_I8, false>(st_context *, Params &, int, int);
template <>
int dispatch<FMT_I8T, false>(st_context *, Params &, int, int);
}  // namespace qmv
}  // namespace st

namespace {

using namespace st::qmv;
using QmvParams = st::qmv::Params;

// Re-tile GPTQ qweight [K/8, N]: tile T (16 columns), group g becomes 64
// lanes x (gs/32) words, lane (q, c) holding, for each 64-k step st and h in
// {0, 1}, word [g*gs/8 + 8 st + 2q + h][16T + c]. Values are unchanged.
__global__ __launch_bounds__(256) void repack_kernel(const uint32_t *__restrict__ qw, uint32_t *__restrict__ out, int K,
                                                     int N, int gs, int ntiles) {
    const int wpl = gs / 32;  // words per lane per group
    const long long total = (long long)ntiles * (K / gs) * 64 * wpl;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int j = (int)(idx % wpl);
    const int lane = (int)((idx / wpl) % 64);
    const long long tg = idx / ((long long)wpl * 64);
    const int g = (int)(tg % (K / gs));
    const int T = (int)(tg / (K / gs));
    const int q = lane >> 4, c = lane & 15;
    const int st = j >> 1, h = j & 1;
    const int n = min(16 * T + c, N - 1);
    const size_t pr = (size_t)g * (gs / 8) + st * 8 + 2 * q + h;
    out[idx] = qw[pr * N + n];
}

// Re-tile INT8 w [N, K]: tile T (16 rows), group u (128 k), lane (q, c)
// gets 32 contiguous bytes, k = 128 u + 16 q + 64 st + j (st < 2, j < 16) of
// row 16 T + c (rows past N repeat row N - 1). One thread per 16 bytes.
__global__ __launch_bounds__(256) void repack8_kernel(const int8_t *__restrict__ w, int8_t *__restrict__ out, int K,
                                                      int N, int ntiles) {
    const int units = K / 128;
    const long long total = (long long)ntiles * units * 64 * 2;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int st = (int)(idx & 1);
    const int lane = (int)((idx >> 1) & 63);
    const long long tu = idx >> 7;
    const int u = (int)(tu % units);
    const int T = (int)(tu / units);
    const int n = min(16 * T + (lane & 15), N - 1);
    const size_t k0 = (size_t)u * 128 + 16 * (lane >> 4) + 64 * st;
    reinterpret_cast<uint4 *>(out)[idx] = *reinterpret_cast<const uint4 *>(w + (size_t)n * K + k0);
}

// The GPTQ entry points take the f16-MFMA kernel (tiled weights, with or
// without act-order, f32 or f16 x) from kI4mmMinM tokens on when N has more
// 16-column tiles than the GPU has CUs, and from kI4mmSplitMinM tokens on
// (groups of tiles, K split across workgroups) when it has fewer. Measured
// against the integer-limb kernels (kernel durations, MI355X): at 5 tokens
// configs[4] q|k|v 9.45 -> 7.61 us, gate/up 12.44 -> 9.58, the lm_head
// 77.3 -> 51.3, Llama-7B gate/up 14.95 -> 11.86; at 4 tokens the lm_head
// stays on the streaming kernel (39.3 against 50.9 us). On few tiles the
// limb kernels' fused split-K reduction keeps 5-8 tokens (configs[4] o at 8
// tokens 9.24 against 10.27 us); at 9-16 tokens the split kernel wins
// (o 11.8 -> 10.5, down 16.4 -> 12.3, Llama-7B down 21.8 -> 13.7 us).
constexpr int kI4mmMinM = 5;
constexpr int kI4mmSplitMinM = 9;

// mmax: 16, or 32 for one source (17-32 tokens in one launch, the weights
// read once; the integer-limb kernels take 16-token blocks)
bool use_i4mm(const st_context *ctx, const QmvParams &p, bool tiled, int xm, int mmax = 16) {
    const int ntiles = (p.N + kTileN - 1) / kTileN;
    const bool few = ntiles <= ctx->num_cus;
    const int min_m = std::max(2, st::tune(ctx, ST_TUNE_I4MM_MIN_M, few ? kI4mmSplitMinM : kI4mmMinM));
    const int min_tiles = st::tune(ctx, ST_TUNE_I4MM_MIN_TILES, ctx->num_cus + 1);
    const bool split = few && st::tune(ctx, ST_TUNE_I4MM_SPLIT_TILES, st::kI4mmSplitTiles) > 0;
    return tiled && (xm == XM_F32 || xm == XM_F16) && p.M <= mmax && p.M >= min_m && (ntiles >= min_tiles || split) &&
           p.K % 128 == 0 && (size_t)ntiles * kTileN * p.K / 2 < (size_t(1) << 31);
}

int launch_i4(st_context *ctx, QmvParams &p, bool tiled, int nsrc, int xm) {
    if (use_i4mm(ctx, p, tiled, xm)) {
        const int rc = st::int4_mm_f16(ctx, p.x, xm == XM_F32, p.perm, p.qw, p.sc, p.qz, p.zoff, p.y, p.M, p.K, p.N,
                                       p.gs, nsrc);
        if (rc != -1) return rc;  // (-1: the K split's partials do not fit the workspace)
    }
    p.units = p.K / p.gs;
    p.ntiles = (p.N + kTileN - 1) / kTileN;
    // the tiled kernels address the weights with 32-bit buffer offsets
    if (tiled && (size_t)p.ntiles * kTileN * p.K / 2 >= (size_t(1) << 31))
        return st::fail(ST_ERR_SHAPE, "qmv: tiled weight of %d x %d exceeds 2 GiB", p.K, p.N);
    if (tiled) return p.perm ? dispatch<FMT_I4T, true>(ctx, p, nsrc, xm) : dispatch<FMT_I4T, false>(ctx, p, nsrc, xm);
    return p.perm ? dispatch<FMT_I4, true>(ctx, p, nsrc, xm) : dispatch<FMT_I4, false>(ctx, p, nsrc, xm);
}

// Calls with more than kTokenBlock tokens run as blocks of kTokenBlock: the
// per-wave staging of the multi-token kernels grows with M * K per wave, and
// at 32 tokens two blocks of 16 (or eight of 4) measured several times
// faster than one launch, even though every block streams the weights again.
// (A skinny-GEMM kernel that reuses the weights across blocks is the better
// design for M > 4.)
constexpr int kTokenBlock = 16;

// Fewest tokens for which st_int8_matvec takes the f16-MFMA kernel (f16 x, tiled weights).
constexpr int kI8mmMinM = 2;

template <typename F>
int by_token_blocks(const st_context *ctx, QmvParams &p, int xm, F &&launch) {
    const int blk = std::max(1, std::min(kTokenBlock, st::tune(ctx, ST_TUNE_TOKEN_BLOCK, kTokenBlock)));
    if (p.M <= blk) return launch(p);
    const size_t xe = xm == XM_F16 ? 2 : 4;
    for (int m0 = 0; m0 < p.M; m0 += blk) {
        QmvParams q = p;
        q.M = std::min(blk, p.M - m0);
        q.x = static_cast<const char *>(p.x) + (size_t)m0 * p.K * xe;
        if (p.xb) q.xb = p.xb + (size_t)m0 * p.K;
        q.y = p.y + (size_t)m0 * p.N;
        if (int rc = launch(q)) return rc;
    }
    return ST_OK;
}

int check_i4(const char *fn, int M, int K, int N, int gs, int mmax) {
    if (gs != 64 && gs != 128 && gs != 256)
        return st::fail(ST_ERR_SHAPE, "%s: group_size %d not in {64,128,256}", fn, gs);
    if (M < 1 || M > mmax) return st::fail(ST_ERR_SHAPE, "%s: M=%d not in [1,%d]", fn, M, mmax);
    if (K <= 0 || K % gs) return st::fail(ST_ERR_SHAPE, "%s: K=%d not a positive multiple of group_size %d", fn, K, gs);
    if (N <= 0 || N % 8) return st::fail(ST_ERR_SHAPE, "%s: N=%d not a positive multiple of 8", fn, N);
    return ST_OK;
}

bool sc_ok(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 1) == 0; }

}  // namespace

extern "C" {

int st_gptq_i4_matvec(st_context *ctx, const void *x, int x_dtype, const uint32_t *qweight, const uint16_t *scales,
                      const uint32_t *qzeros, const int32_t *perm, float *y, int M, int K, int N, int group_size,
                      uint32_t flags) {
    if (!ctx || !x || !qweight || !scales || !y) return st::fail(ST_ERR_INVALID, "st_gptq_i4_matvec: NULL argument");
    if (int rc = check_i4("st_gptq_i4_matvec", M, K, N, group_size, 32)) return rc;
    if (!st::aligned16(qweight) || !st::aligned16(x) || !st::aligned16(perm) || !sc_ok(scales))
        return st::fail(ST_ERR_ALIGN, "st_gptq_i4_matvec: x/qweight/perm must be 16-byte aligned");
    if (x_dtype != ST_F32 && x_dtype != ST_F16) return st::fail(ST_ERR_INVALID, "st_gptq_i4_matvec: x_dtype %d", x_dtype);
    QmvParams p{};
    p.x = x;
    p.perm = perm;
    p.qw[0] = p.qw[1] = qweight;
    p.sc[0] = p.sc[1] = scales;
    p.qz[0] = p.qz[1] = qzeros;
    p.y = y;
    p.M = M;
    p.K = K;
    p.N = N;
    p.gs = group_size;
    p.zoff = (flags & ST_FLAG_ZEROS_PLUS_ONE) ? 1 : 0;
    const bool tiled = flags & ST_FLAG_TILED;
    const int xm = x_dtype == ST_F32 ? XM_F32 : XM_F16;
    // 17-32 tokens in one f16-MFMA launch when it takes the call (not group
    // 64 with f32 x: its four 16-row blocks would spill)
    if (M > kTokenBlock && !(group_size == 64 && xm == XM_F32) && use_i4mm(ctx, p, tiled, xm, 2 * kTokenBlock)) {
        const int rc = st::int4_mm_f16(ctx, p.x, xm == XM_F32, p.perm, p.qw, p.sc, p.qz, p.zoff, p.y, p.M, p.K, p.N,
                                       p.gs, 1);
        if (rc != -1) return rc;  // (-1: the K split's partials do not fit the workspace)
    }
    return by_token_blocks(ctx, p, xm, [&](QmvParams &q) { return launch_i4(ctx, q, tiled, 1, xm); });
}

int st_gptq_i4_matvec_noalloc(st_context *ctx, const void *x, int x_dtype, const uint32_t *qweight,
                              const uint16_t *scales, const uint32_t *qzeros, const int32_t *perm, float *y, int M,
                              int K, int N, int group_size, uint32_t flags) {
    if (!ctx) return st::fail(ST_ERR_INVALID, "st_gptq_i4_matvec_noalloc: ctx is NULL");
    if (!ctx->scratch) return st::fail(ST_ERR_WORKSPACE, "st_gptq_i4_matvec_noalloc: no scratch on this device");
    // The most any path of the call keeps: the f16-MFMA kernel's split of up
    // to 32 tokens of f32 x (one launch; 2 f16 rows per token and a factor per 128 k)
    // or, for f16 x under act-order, its gathered rows; split-K partials
    // shrink (or go unsplit) to fit what is there.
    if (M > 0 && K > 0 && (x_dtype == ST_F32 || perm)) {
        // (f16 x under act-order: the gathered rows, mb K halves)
        const size_t mb = (size_t)std::min(M, 2 * kTokenBlock);
        const size_t need = x_dtype == ST_F32 ? 2 * mb * K * 2 + mb * (size_t)(K / 128) * 4 : mb * K * 2;
        if (need > ST_NOALLOC_SCRATCH_BYTES)
            return st::fail(ST_ERR_WORKSPACE, "st_gptq_i4_matvec_noalloc: %zu bytes of scratch needed, %u held", need,
                            (unsigned)ST_NOALLOC_SCRATCH_BYTES);
    }
    st_context view = *ctx;  // the same stream and settings, the scratch as workspace
    view.ws = static_cast<float *>(ctx->scratch);
    view.ws_bytes = ST_NOALLOC_SCRATCH_BYTES;
    view.own_stream = false;
    return st_gptq_i4_matvec(&view, x, x_dtype, qweight, scales, qzeros, perm, y, M, K, N, group_size, flags);
}

int st_gptq_i4_silu_matvec(st_context *ctx, const float *a, const float *b, const uint32_t *qweight,
                           const uint16_t *scales, const uint32_t *qzeros, const int32_t *perm, float *y, int M, int K,
                           int N, int group_size, uint32_t flags) {
    if (!ctx || !a || !b || !qweight || !scales || !y)
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_silu_matvec: NULL argument");
    if (int rc = check_i4("st_gptq_i4_silu_matvec", M, K, N, group_size, 32)) return rc;
    if (!st::aligned16(qweight) || !st::aligned16(a) || !st::aligned16(b) || !st::aligned16(perm) || !sc_ok(scales))
        return st::fail(ST_ERR_ALIGN, "st_gptq_i4_silu_matvec: a/b/qweight/perm must be 16-byte aligned");
    QmvParams p{};
    p.x = a;
    p.xb = b;
    p.perm = perm;
    p.qw[0] = p.qw[1] = qweight;
    p.sc[0] = p.sc[1] = scales;
    p.qz[0] = p.qz[1] = qzeros;
    p.y = y;
    p.M = M;
    p.K = K;
    p.N = N;
    p.gs = group_size;
    p.zoff = (flags & ST_FLAG_ZEROS_PLUS_ONE) ? 1 : 0;
    const bool tiled = flags & ST_FLAG_TILED;
    return by_token_blocks(ctx, p, XM_SILU, [&](QmvParams &q) { return launch_i4(ctx, q, tiled, 1, XM_SILU); });
}

int st_gptq_i4_gate_up_silu(st_context *ctx, const void *x, int x_dtype, const uint32_t *qweight_gate,
                            const uint16_t *scales_gate, const uint32_t *qzeros_gate, const uint32_t *qweight_up,
                            const uint16_t *scales_up, const uint32_t *qzeros_up, const int32_t *perm, float *y, int M,
                            int K, int N, int group_size, uint32_t flags) {
    if (!ctx || !x || !qweight_gate || !scales_gate || !qweight_up || !scales_up || !y)
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_gate_up_silu: NULL argument");
    if (int rc = check_i4("st_gptq_i4_gate_up_silu", M, K, N, group_size, 32)) return rc;
    if ((qzeros_gate == nullptr) != (qzeros_up == nullptr))
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_gate_up_silu: give qzeros for both or neither");
    if (!st::aligned16(qweight_gate) || !st::aligned16(qweight_up) || !st::aligned16(x) || !st::aligned16(perm) ||
        !sc_ok(scales_gate) || !sc_ok(scales_up))
        return st::fail(ST_ERR_ALIGN, "st_gptq_i4_gate_up_silu: x/qweight/perm must be 16-byte aligned");
    if (x_dtype != ST_F32 && x_dtype != ST_F16)
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_gate_up_silu: x_dtype %d", x_dtype);
    QmvParams p{};
    p.x = x;
    p.perm = perm;
    p.qw[0] = qweight_gate;
    p.qw[1] = qweight_up;
    p.sc[0] = scales_gate;
    p.sc[1] = scales_up;
    p.qz[0] = qzeros_gate;
    p.qz[1] = qzeros_up;
    p.y = y;
    p.M = M;
    p.K = K;
    p.N = N;
    p.gs = group_size;
    p.zoff = (flags & ST_FLAG_ZEROS_PLUS_ONE) ? 1 : 0;
    const bool tiled = flags & ST_FLAG_TILED;
    const int xm = x_dtype == ST_F32 ? XM_F32 : XM_F16;
    if (M > kTokenBlock && !(group_size == 64 && xm == XM_F32) && use_i4mm(ctx, p, tiled, xm, 2 * kTokenBlock)) {
        const int rc = st::int4_mm_f16(ctx, p.x, xm == XM_F32, p.perm, p.qw, p.sc, p.qz, p.zoff, p.y, p.M, p.K, p.N,
                                       p.gs, 2);
        if (rc != -1) return rc;
    }
    return by_token_blocks(ctx, p, xm, [&](QmvParams &q) { return launch_i4(ctx, q, tiled, 2, xm); });
}

size_t st_gptq_i4_tiled_words(int K, int N, int group_size) {
    if (K <= 0 || N <= 0 || group_size <= 0 || K % group_size) return 0;
    return (size_t)((N + kTileN - 1) / kTileN) * kTileN * (size_t)(K / 8);
}

int st_gptq_i4_repack(st_context *ctx, const uint32_t *qweight, uint32_t *qweight_tiled, int K, int N,
                      int group_size) {
    if (!ctx || !qweight || !qweight_tiled) return st::fail(ST_ERR_INVALID, "st_gptq_i4_repack: NULL argument");
    if (int rc = check_i4("st_gptq_i4_repack", 1, K, N, group_size, 1)) return rc;
    if (!st::aligned16(qweight_tiled))
        return st::fail(ST_ERR_ALIGN, "st_gptq_i4_repack: output must be 16-byte aligned");
    const int ntiles = (N + kTileN - 1) / kTileN;
    const long long total = (long long)ntiles * (K / group_size) * 64 * (group_size / 32);
    st::launch(ctx, repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, qweight,
                       qweight_tiled, K, N, group_size, ntiles);
    return st::launch_check("repack_kernel");
}

size_t st_int8_tiled_bytes(int K, int N) {
    if (K <= 0 || N <= 0) return 0;
    return (size_t)((N + kTileN - 1) / kTileN) * kTileN * (size_t)K;
}

int st_int8_repack(st_context *ctx, const int8_t *w, int8_t *w_tiled, int K, int N) {
    if (!ctx || !w || !w_tiled) return st::fail(ST_ERR_INVALID, "st_int8_repack: NULL argument");
    if (K <= 0 || K % 128 || N <= 0) return st::fail(ST_ERR_SHAPE, "st_int8_repack: K=%d (multiple of 128), N=%d", K, N);
    if (!st::aligned16(w) || !st::aligned16(w_tiled))
        return st::fail(ST_ERR_ALIGN, "st_int8_repack: w and w_tiled must be 16-byte aligned");
    const int ntiles = (N + kTileN - 1) / kTileN;
    const long long total = (long long)ntiles * (K / 128) * 128;
    st::launch(ctx, repack8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, w, w_tiled, K,
                       N, ntiles);
    return st::launch_check("repack8_kernel");
}

int st_int8_matvec(st_context *ctx, const void *x, int x_dtype, const int8_t *w, const float *scale, float *y, int M,
                   int K, int N, uint32_t flags) {
    if (!ctx || !x || !w || !scale || !y) return st::fail(ST_ERR_INVALID, "st_int8_matvec: NULL argument");
    if (M < 1 || M > 32) return st::fail(ST_ERR_SHAPE, "st_int8_matvec: M=%d not in [1,32]", M);
    if (K <= 0 || K % 128) return st::fail(ST_ERR_SHAPE, "st_int8_matvec: K=%d not a positive multiple of 128", K);
    if (N <= 0 || N % 4) return st::fail(ST_ERR_SHAPE, "st_int8_matvec: N=%d not a positive multiple of 4", N);
    const bool tiled = (flags & ST_FLAG_TILED) != 0;
    if ((long long)((N + kTileN - 1) / kTileN) * kTileN * K >= (1ll << 31))  // 32-bit buffer offsets
        return st::fail(ST_ERR_SHAPE, "st_int8_matvec: weight of %d x %d exceeds 2 GiB", N, K);
    if (!st::aligned16(w) || !st::aligned16(x))
        return st::fail(ST_ERR_ALIGN, "st_int8_matvec: w and x must be 16-byte aligned");
    if (x_dtype != ST_F32 && x_dtype != ST_F16) return st::fail(ST_ERR_INVALID, "st_int8_matvec: x_dtype %d", x_dtype);
    // Several tokens with f16 x on tiled weights: the f16-MFMA skinny GEMM,
    // which reads the weights once for all tokens.
    if (tiled && x_dtype == ST_F16 && M >= st::tune(ctx, ST_TUNE_I8MM_MIN_M, kI8mmMinM))
        return st::int8_mm_f16(ctx, x, w, scale, y, M, K, N);
    QmvParams p{};
    p.x = x;
    p.w8 = w;
    p.scale8 = scale;
    p.y = y;
    p.M = M;
    p.K = K;
    p.N = N;
    p.gs = 128;
    p.units = K / 128;
    p.ntiles = (N + kTileN - 1) / kTileN;
    const int xm = x_dtype == ST_F32 ? XM_F32 : XM_F16;
    return by_token_blocks(ctx, p, xm, [&](QmvParams &q) {
        return tiled ? dispatch<FMT_I8T, false>(ctx, q, 1, xm) : dispatch<FMT_I8, false>(ctx, q, 1, xm);
    });
}

}  // extern "C"
