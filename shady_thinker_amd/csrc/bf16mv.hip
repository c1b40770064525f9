// bf16 matvec for the lm_head / tied embeddings: y[m, n] = sum_k bf16(W[n, k])
// * x[m, k], W row-major [N, K] (two bf16 per u32, low half first), x f32 or
// f16 [M, K], y f32 [M, N], M <= 8. Replaces src/shaders/bf16_matvec.wgsl:21-72
// (dispatched at src/model.rs:455-468, 824-831).
//
// A pure HBM stream (151936 x 2560 bf16 = 778 MB for one token of configs[4]);
// the arithmetic is one shift or mask and one f32 FMA per weight, far below
// the VALU rate, so no matrix cores:
//  * 8 lanes share a row: one 16-byte load per lane covers 128 contiguous
//    bytes of each of 8 rows per instruction (full cache lines), and a row's
//    8 partial sums meet in 3 cross-lane steps.
//  * x is staged once per workgroup in LDS as f32; the 8 lanes of a row read
//    different 32-byte pieces, which every row group shares (broadcast).
//  * Waves loop over row groups (8 rows) with UNR loads in flight per lane.
#include "common.hpp"

#include <algorithm>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 8;  // 16-byte weight loads in flight per lane

template <int MT, bool F16X>
__global__ __launch_bounds__(kThreads) void bf16mv_kernel(const void *__restrict__ xp, const uint16_t *__restrict__ w,
                                                          float *__restrict__ y, int M, int K, int N, int groups_per_wave) {
    extern __shared__ __align__(16) float xs[];  // [MT][K]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane >> 3;  // row within the group of 8
    const int c = lane & 7;   // 16-byte piece within a 128-byte row segment

    // x -> LDS (f32), rows beyond M zero
    for (int i = tid * 4; i < MT * K; i += kThreads * 4) {
        const int m = i / K, k = i - m * K;  // K % 8 == 0, so 4 elements never cross a row
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (m < M) {
            if constexpr (F16X) {
                const _Float16 *s = static_cast<const _Float16 *>(xp) + (size_t)m * K + k;
                v = f32x4{(float)s[0], (float)s[1], (float)s[2], (float)s[3]};
            } else {
                v = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(xp) + (size_t)m * K + k);
            }
        }
        *reinterpret_cast<f32x4 *>(&xs[i]) = v;
    }
    __syncthreads();

    const int nseg = K / 64;           // full 128-byte segments per row
    const int tail = (K % 64) / 8;     // 16-byte pieces in the last partial segment
    const int nsteps = nseg + (tail > 0 ? 1 : 0);
    const int ngroups = (N + 7) / 8;
    const int gw = blockIdx.x * (kThreads / 64) + wave;  // first group of this wave
    const int gstride = gridDim.x * (kThreads / 64);

    for (int gi = 0; gi < groups_per_wave; ++gi) {
        const int g = gw + gi * gstride;
        if (g >= ngroups) break;  // uniform per wave
        const int row = min(g * 8 + r, N - 1);
        const u32x4 *wr = reinterpret_cast<const u32x4 *>(w + (size_t)row * K);
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        for (int s0 = 0; s0 < nsteps; s0 += kUnroll) {
            u32x4 wv[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                // piece c of segment s; past the row's end: a clamped valid
                // address, masked below
                const int piece = min((s0 + u) * 8 + c, K / 8 - 1);
                wv[u] = __builtin_nontemporal_load(wr + piece);
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int s = s0 + u;
                const bool ok = s < nseg || (s == nseg && c < tail);
                if (!ok) continue;
                const int k = (s * 8 + c) * 8;
                // bf16 -> f32 is the upper half of an f32: low half << 16,
                // high half masked (copied out of the vector first: a bit
                // cast straight from a vector element miscompiles)
                const unsigned w4[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
                float wf[8];
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const unsigned lo = w4[h] << 16, hi = w4[h] & 0xFFFF0000u;
                    wf[2 * h] = __builtin_bit_cast(float, lo);
                    wf[2 * h + 1] = __builtin_bit_cast(float, hi);
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(&xs[m * K + k]);
                    const f32x4 b = *reinterpret_cast<const f32x4 *>(&xs[m * K + k + 4]);
                    float t = acc[m];
                    t = fmaf(wf[0], a.x, t);
                    t = fmaf(wf[1], a.y, t);
                    t = fmaf(wf[2], a.z, t);
                    t = fmaf(wf[3], a.w, t);
                    t = fmaf(wf[4], b.x, t);
                    t = fmaf(wf[5], b.y, t);
                    t = fmaf(wf[6], b.z, t);
                    t = fmaf(wf[7], b.w, t);
                    acc[m] = t;
                }
            }
        }
        // the row's 8 partial sums (lanes 8r .. 8r+7)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = acc[m];
            v += __shfl_xor(v, 1);
            v += __shfl_xor(v, 2);
            v += __shfl_xor(v, 4);
            acc[m] = v;
        }
        const int n = g * 8 + r;
        if (c == 0 && n < N) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (m < M) y[(size_t)m * N + n] = acc[m];
        }
    }
}

template <int MT, bool F16X>
int launch(st_context *ctx, const void *x, const uint16_t *w, float *y, int M, int K, int N) {
    const int ngroups = (N + 7) / 8;
    const int waves_per_wg = kThreads / 64;
    // about 8 workgroups (32 waves) per CU, each wave a few row groups
    const int target_wgs = std::max(1, ctx->num_cus * 8);
    const int gpw = std::max(1, (ngroups + target_wgs * waves_per_wg - 1) / (target_wgs * waves_per_wg));
    const int wgs = (ngroups + gpw * waves_per_wg - 1) / (gpw * waves_per_wg);
    const size_t lds = (size_t)MT * K * sizeof(float);
    auto kern = bf16mv_kernel<MT, F16X>;
    if (lds > 64 * 1024)
        ST_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    st::launch(ctx, kern, dim3(wgs), dim3(kThreads), lds, x, w, y, M, K, N, gpw);
    return st::launch_check("bf16mv_kernel");
}

template <bool F16X>
int by_m(st_context *ctx, const void *x, const uint16_t *w, float *y, int M, int K, int N) {
    if (M == 1) return launch<1, F16X>(ctx, x, w, y, M, K, N);
    if (M <= 4) return launch<4, F16X>(ctx, x, w, y, M, K, N);
    return launch<8, F16X>(ctx, x, w, y, M, K, N);
}

}  // namespace

extern "C" int st_bf16_matvec(st_context *ctx, const void *x, int x_dtype, const uint16_t *w, float *y, int M, int K,
                              int N) {
    if (!ctx || !x || !w || !y) return st::fail(ST_ERR_INVALID, "st_bf16_matvec: NULL argument");
    if (M < 1 || M > 8) return st::fail(ST_ERR_SHAPE, "st_bf16_matvec: M=%d not in [1,8]", M);
    if (K <= 0 || K % 8 || N <= 0) return st::fail(ST_ERR_SHAPE, "st_bf16_matvec: K=%d (multiple of 8), N=%d", K, N);
    const int mt = M == 1 ? 1 : (M <= 4 ? 4 : 8);  // token rows of the LDS x copy
    if ((size_t)mt * K * sizeof(float) > 160 * 1024)
        return st::fail(ST_ERR_SHAPE, "st_bf16_matvec: M=%d K=%d too large for the LDS x copy", M, K);
    if (x_dtype != ST_F32 && x_dtype != ST_F16) return st::fail(ST_ERR_INVALID, "st_bf16_matvec: x_dtype %d", x_dtype);
    if (!st::aligned16(w) || !st::aligned16(x))
        return st::fail(ST_ERR_ALIGN, "st_bf16_matvec: x and w must be 16-byte aligned");
    return x_dtype == ST_F16 ? by_m<true>(ctx, x, w, y, M, K, N) : by_m<false>(ctx, x, w, y, M, K, N);
}
