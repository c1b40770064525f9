// Multi-token INT8 decode with f16 activations on f16 MFMA (a skinny GEMM):
// y[m, n] = scale[n] * sum_k W[n, k] * x[m, k], W in the tiled INT8 layout
// (st_int8_repack), x f16 [M, K], M <= 32, y f32 [M, N]. No reference
// counterpart: the reference has no INT8 path.
//
//  * Exact arithmetic up to the f32 sum: an int8 weight and an f16 x are
//    both exact in f16 and their product (at most 19 significant bits) is
//    exact in f32, so v_mfma_f32_16x16x32_f16 with f32 accumulation
//    computes the dot product with only f32 summation error, and the
//    per-channel scale is applied once at the end.
//  * Weight reuse across tokens: every weight is read from HBM once for all
//    M tokens (the integer-limb matvec kernels stream the weights once per
//    16-token block, and their per-token VALU work grows with M).
//  * Work split: one workgroup per CU owns a contiguous run of 16-column
//    tiles; S waves share a tile and split each K chunk by groups of 128.
//    x is staged chunk by chunk (1024 k) into LDS, double buffered, by all
//    waves, and every wave keeps the next chunk's weights in flight in
//    registers while it computes the current one. The S partial sums of a
//    tile meet in LDS at the end, in a fixed order.
//  * int8 -> f16: v_perm puts each byte (xor 0x80) under the f16 exponent of
//    1024, and one packed f16 add of -1152 gives the signed value exactly.
#include "common.hpp"

#include <algorithm>
#include <cstdlib>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileN = 16;
constexpr int kKC = 1024;                // k per staged chunk
constexpr int kCG = kKC / 128;           // groups of 128 k per chunk
constexpr int kPitch = kKC + 8;          // halves per LDS row: a 16-byte pad keeps the 16 rows of a fragment read on distinct banks
constexpr int kRsrcWord3 = 0x00020000;   // raw 32-bit buffer data (gfx9-class)
constexpr unsigned kNoLoad = 0x80000000u;  // buffer offset past every resource: reads 0, touches no memory
constexpr int kMaxTilesPerWg = 8;

__device__ __forceinline__ half8 i8x8_to_h8(unsigned d0, unsigned d1) {
    const half2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    d0 ^= 0x80808080u;
    d1 ^= 0x80808080u;
    const half2_t h0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, d0, 0x04010400u)) + off;
    const half2_t h1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, d0, 0x04030402u)) + off;
    const half2_t h2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, d1, 0x04010400u)) + off;
    const half2_t h3 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, d1, 0x04030402u)) + off;
    const u32x4 r = {__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1), __builtin_bit_cast(unsigned, h2),
                     __builtin_bit_cast(unsigned, h3)};
    return __builtin_bit_cast(half8, r);
}

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// MB = 16-row MFMA blocks (tokens 16 MB), GW = groups per wave per chunk
// (kCG / S, S = waves per tile).
template <int MB, int GW>
__global__ __launch_bounds__(kThreads) void i8mm_kernel(const _Float16 *__restrict__ x, const int8_t *__restrict__ w,
                                                        const float *__restrict__ scale, float *__restrict__ y, int M,
                                                        int K, int N, int ntiles) {
    constexpr int S = kCG / GW;
    constexpr int ROWS = 16 * MB;
    constexpr int XL = ROWS * kKC / 8 / kThreads;  // 16-byte x loads per thread per chunk
    __shared__ __align__(16) _Float16 xs0[ROWS * kPitch];
    __shared__ __align__(16) _Float16 xs1[ROWS * kPitch];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = (int)((long long)blockIdx.x * ntiles / gridDim.x);
    const int t1 = (int)((long long)(blockIdx.x + 1) * ntiles / gridDim.x);
    const int tb = wave / S, slice = wave % S;
    const bool active = t0 + tb < t1;
    const int T = min(t0 + tb, ntiles - 1);  // inactive waves load nothing (see load_w)
    const int units = K / 128;
    const int nch = (units + kCG - 1) / kCG;

    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)x, (short)0, 0x7FFFFFFF, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)w, (short)0, 0x7FFFFFFF, kRsrcWord3);

    // x chunk c: thread item i = j * kThreads + tid is row i / (kKC / 8),
    // 8 halves at column 8 (i % (kKC / 8)). Rows >= M and k >= K read 0.
    // x is loaded XS chunks ahead (register set c % XS holds chunk c): two
    // where the registers allow it, so that a chunk's staging does not wait
    // for a load issued in the same chunk (32 tokens with 4 groups per wave:
    // one, two spilled)
    constexpr int XS = (MB == 2 && GW == 4) ? 1 : 2;
    u32x4 xr2[XS][XL];
    auto load_x = [&](u32x4 (&xr)[XL], int c) {
#pragma unroll
        for (int j = 0; j < XL; ++j) {
            const int i = j * kThreads + tid;
            const int row = i / (kKC / 8), k = c * kKC + 8 * (i % (kKC / 8));
            const unsigned off = (row < M && k < K) ? (unsigned)(row * K + k) * 2u : kNoLoad;
            xr[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
        }
    };
    auto store_x = [&](const u32x4 (&xr)[XL], _Float16 *xs) {
#pragma unroll
        for (int j = 0; j < XL; ++j) {
            const int i = j * kThreads + tid;
            *reinterpret_cast<u32x4 *>(&xs[(i / (kKC / 8)) * kPitch + 8 * (i % (kKC / 8))]) = xr[j];
        }
    };
    // Weights of group u of tile T: lane l's 32 bytes at ((T units + u) 64 + l) 32,
    // bytes 16 st + j holding k = 128 u + 16 (l / 16) + 64 st + j of column 16 T + l % 16.
    u32x4 wr[2][GW][2];
    auto load_w = [&](u32x4 (&dst)[GW][2], int c) {
#pragma unroll
        for (int g = 0; g < GW; ++g) {
            const int u = c * kCG + slice * GW + g;
            const unsigned off = (active && u < units) ? (unsigned)(((T * units + u) * 64 + lane) * 32) : kNoLoad;
            dst[g][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0);
            dst[g][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 16, 0);
        }
    };

    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int q = lane >> 4, r16 = lane & 15;
    auto compute = [&](const _Float16 *xs, const u32x4 (&src)[GW][2]) {
#pragma unroll
        for (int g = 0; g < GW; ++g)
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const half8 b = i8x8_to_h8(src[g][st][2 * h], src[g][st][2 * h + 1]);
                    const int kk = (slice * GW + g) * 128 + 64 * st + 16 * q + 8 * h;
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        const half8 a = *reinterpret_cast<const half8 *>(&xs[(16 * mb + r16) * kPitch + kk]);
                        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[mb], 0, 0, 0);
                    }
                }
    };

    load_x(xr2[0], 0);
    if constexpr (XS == 2) load_x(xr2[XS - 1], 1);
    load_w(wr[0], 0);
    store_x(xr2[0], xs0);
    lds_barrier();
    // Two chunks per trip so that buffer indices are compile-time. The loads
    // of the next chunk are unconditional (past the last chunk they read
    // nothing), so the compiler's wait counts are the same on every path.
    for (int c = 0; c < nch; c += 2) {
        load_x(xr2[0], c + XS);  // (set 0 was stored for chunk c at the end of chunk c - 1)
        load_w(wr[1], c + 1);
        if (active) compute(xs0, wr[0]);  // a wave without a tile skips the work (and its LDS reads)
        store_x(xr2[XS - 1], xs1);  // chunk c + 1
        lds_barrier();
        if (c + 1 >= nch) break;
        load_x(xr2[XS - 1], c + 1 + XS);
        load_w(wr[0], c + 2);
        if (active) compute(xs1, wr[1]);
        store_x(xr2[0], xs0);  // chunk c + 2
        lds_barrier();
    }

    // Partial sums of the S waves of a tile, added in slice order.
    float *red = reinterpret_cast<float *>(xs1);
    static_assert(kWaves * MB * 4 * 64 * 4 <= (int)sizeof(xs1), "reduction buffer");
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[((wave * MB + mb) * 4 + i) * 64 + lane] = acc[mb][i];
    lds_barrier();
    if (!active || slice != 0) return;
    const int n = kTileN * T + r16;
    if (n >= N) return;
    const float s = scale[n];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = 0.f;
            for (int sl = 0; sl < S; ++sl) v += red[(((tb * S + sl) * MB + mb) * 4 + i) * 64 + lane];
            const int m = 16 * mb + 4 * q + i;
            if (m < M) y[(size_t)m * N + n] = s * v;
        }
}

template <int MB>
int launch_mb(st_context *ctx, const _Float16 *x, const int8_t *w, const float *scale, float *y, int M, int K, int N,
              int ntiles, int G, int gw) {
    const dim3 grid(G), block(kThreads);
    switch (gw) {
        case 1: st::launch(ctx, (i8mm_kernel<MB, 1>), grid, block, 0, x, w, scale, y, M, K, N, ntiles); break;
        case 2: st::launch(ctx, (i8mm_kernel<MB, 2>), grid, block, 0, x, w, scale, y, M, K, N, ntiles); break;
        default: st::launch(ctx, (i8mm_kernel<MB, 4>), grid, block, 0, x, w, scale, y, M, K, N, ntiles); break;
    }
    return st::launch_check("i8mm_kernel");
}

}  // namespace

namespace st {

// Arguments are checked by st_int8_matvec (tiled weights, f16 x, M <= 32,
// K % 128 == 0, 16-byte alignment, 32-bit weight offsets).
int int8_mm_f16(st_context *ctx, const void *x, const int8_t *w, const float *scale, float *y, int M, int K, int N) {
    const int ntiles = (N + kTileN - 1) / kTileN;
    // one workgroup per CU, at most kMaxTilesPerWg tiles each
    const int G = std::max(std::min(ctx->num_cus, ntiles), (ntiles + kMaxTilesPerWg - 1) / kMaxTilesPerWg);
    const int tbmax = (ntiles + G - 1) / G;
    int s = 1;  // waves per tile: the largest power of two with s * tbmax <= 16, at most kCG
    while (2 * s * tbmax <= kWaves && 2 * s <= kCG) s *= 2;
    const int gw = kCG / s;  // 1, 2 or 4
    const _Float16 *xh = static_cast<const _Float16 *>(x);
    return M <= 16 ? launch_mb<1>(ctx, xh, w, scale, y, M, K, N, ntiles, G, gw)
                   : launch_mb<2>(ctx, xh, w, scale, y, M, K, N, ntiles, G, gw);
}

}  // namespace st
