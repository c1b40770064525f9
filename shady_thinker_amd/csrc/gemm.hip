// Prefill GEMM on gfx950: C[M, N] = A[M, K] (f16) . dequant(W), W GPTQ int4.
// No reference counterpart: the reference prefills token by token through
// the matvec (src/inference.rs:93-95). Dequant semantics are the reference's
// ((q - z) * s, src/shaders/gptq_matvec.wgsl:51-58) and stay exact:
//
//  * B operand = (q - z) as integer-valued f16 (exact: |q - z| <= 15). A
//    GPTQ word holds 8 consecutive k of one column, which is exactly one
//    lane's B fragment of v_mfma_f32_32x32x16_f16, so weights go straight
//    from HBM to registers (no LDS): word -> 4 f16 pairs with one shift,
//    one and-or with the f16 1024 bias, one packed subtract each.
//  * Each group (128 k) accumulates in f32 from zero; its partial is then
//    multiplied by the column's f16 scale and added to the running total.
//    So the only roundings are the MFMA's f32 accumulation and one f32
//    multiply-add per group, as in an f32 dequant-then-GEMM.
//  * A (activations, f16) is staged through LDS, double buffered, with a
//    padded row stride; each lane's 8 halves are stored in the order of the
//    B register halves (k = 0,4,1,5,2,6,3,7 within the 8), so A and B
//    fragments pair element for element.
//  * Workgroup tile 128 (M) x 128 (N), 4 waves as 2 x 2, each wave 64 x 64 =
//    2 x 2 MFMA blocks of 32 x 32 (group partials + totals: 128 registers,
//    so two waves fit per SIMD). Tiles are ordered XCD-major: the workgroups of
//    one XCD share A rows, which then stay in that XCD's L2.
//  * Act-order: K is sorted by group at upload (st_gptq_i4_act_order); the
//    matching column gather of A runs first (permute_cols_kernel) into the
//    context workspace.
#include "common.hpp"

#include <algorithm>
#include <type_traits>

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128;              // rows of A per workgroup
constexpr int BN = 128;              // columns per workgroup
constexpr int WN = 2;                // waves along N (and 2 along M)
constexpr int RB = 2, CB = 2;        // 32 x 32 MFMA blocks per wave (rows, columns)
constexpr int KT = 128;              // k per LDS tile
constexpr int ALD = KT + 8;          // LDS row stride in halves (padding against bank conflicts)
constexpr int kThreads = 256;
// Buffer resource word 3 for gfx9-class GPUs: raw (untyped) 32-bit data.
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kChunks = BM * KT / 8 / kThreads;  // 16-byte A chunks per thread per tile (8)

// 8 halves k..k+7 (4 dwords a0..a3 = (k0,k1),(k2,k3),(k4,k5),(k6,k7)) ->
// register order of the B conversion: (k0,k4),(k1,k5),(k2,k6),(k3,k7).
__device__ __forceinline__ u32x4 to_b_order(u32x4 a) {
    u32x4 r;
    r.x = __builtin_amdgcn_perm(a.z, a.x, 0x05040100u);  // lo(a.x), lo(a.z)
    r.y = __builtin_amdgcn_perm(a.z, a.x, 0x07060302u);  // hi(a.x), hi(a.z)
    r.z = __builtin_amdgcn_perm(a.w, a.y, 0x05040100u);  // lo(a.y), lo(a.w)
    r.w = __builtin_amdgcn_perm(a.w, a.y, 0x07060302u);  // hi(a.y), hi(a.w)
    return r;
}

// GPTQ word (nibbles n0..n7 = k0..k7) -> B fragment halves
// (n0,n4),(n1,n5),(n2,n6),(n3,n7) minus the zero point, exact.
__device__ __forceinline__ half8 word_to_b(unsigned w, half2_t zb) {
    half8 b;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned t = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;  // f16 1024 + n
        const half2_t h = __builtin_bit_cast(half2_t, t) - zb;            // (n - z), exact
        b[2 * j] = h.x;
        b[2 * j + 1] = h.y;
    }
    return b;
}

template <int GS, bool TILED, bool F16OUT>
__global__ __launch_bounds__(kThreads, (GS == 64 ? 1 : 2)) void gemm_kernel(const _Float16 *__restrict__ A, const uint32_t *__restrict__ qw,
                                                           const uint16_t *__restrict__ sc, const uint32_t *__restrict__ qz,
                                                           int zoff, void *__restrict__ C, int M, int K, int N) {
    __shared__ __align__(16) _Float16 As[2][BM * ALD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // XCD-major tile order: consecutive ids run on the same XCD.
    const int MT = (M + BM - 1) / BM, NT = (N + BN - 1) / BN;
    const int T = MT * NT;
    const int b = blockIdx.x;
    const int id = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    const int mt = id / NT, nt = id % NT;
    const int m0 = mt * BM, n0 = nt * BN;
    const int nw = n0 + 32 * CB * (wave % WN);  // this wave's columns
    const int mw = 32 * RB * (wave / WN);       // and its rows within the tile

    int col[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) col[cb] = min(nw + 32 * cb + l32, N - 1);

    const int ntiles = K / KT;

    // ---------------------------------------------------------------- loads
    // Buffer loads: one scalar resource per operand, a 32-bit per-lane
    // offset fixed for the whole K loop and a uniform offset per tile, so
    // the 24 loads per tile need no 64-bit address registers.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, 0x7FFFFFFF, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb_ = __builtin_amdgcn_make_buffer_rsrc((void *)qw, (short)0, 0x7FFFFFFF, kRsrcWord3);
    int aoff[kChunks];  // bytes: row (clamped to M - 1) and 16-byte chunk of this thread's A loads
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
        const int c = tid + kThreads * j;
        aoff[j] = (min(m0 + (c >> 4), M - 1) * K + 8 * (c & 15)) * 2;
    }
    // B words: bw[buffer][t][cb] is the word of k-step t (16 k) for this
    // lane's column block cb; koff(t) is where its 8 k sit in the A tile.
    //  * [K/8, N] layout: k-step t, lane half hi -> packed row 2t + hi.
    //  * tiled layout (st_gptq_i4_repack): a lane (q, c) of tile T holds the
    //    words of packed rows 8 st + 2q + h of each group contiguously. Lane
    //    half hi takes q = 2 hi + ql (ql in {0, 1}): two loads of 4 words per
    //    tile and column block. Word j of load ql is packed row
    //    8 (j / 2) + 2q + j % 2 of the tile and is used at k-step
    //    t = 4 (j / 2) + 2 ql + j % 2, so the tile's first 64 k are steps 0..3
    //    (the group boundary rule is the same for both layouts).
    constexpr int WPL = GS / 32;  // tiled: words per lane per group
    int boff[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        if constexpr (TILED) {
            const int G = K / GS;
            boff[cb] = (((col[cb] >> 4) * G * 64 + 32 * hi + (col[cb] & 15)) * WPL) * 4;
        } else {
            boff[cb] = (hi * N + col[cb]) * 4;
        }
    }
    auto koff = [&](int t) { return TILED ? 64 * (t >> 2) + 32 * hi + 16 * ((t >> 1) & 1) + 8 * (t & 1) : 16 * t + 8 * hi; };

    u32x4 apre[kChunks];
    auto load_a = [&](int kt) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) apre[j] = __builtin_amdgcn_raw_buffer_load_b128(ra, aoff[j], kt * KT * 2, 0);
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            const int c = tid + kThreads * j;
            *reinterpret_cast<u32x4 *>(&As[buf][(c >> 4) * ALD + 8 * (c & 15)]) = to_b_order(apre[j]);
        }
    };
    unsigned bw[2][KT / 16][CB];
    auto load_b = [&](unsigned (&dst)[KT / 16][CB], int kt) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            if constexpr (TILED) {
#pragma unroll
                for (int ql = 0; ql < 2; ++ql) {
                    u32x4 w;
                    if constexpr (GS == 64) {  // two groups per tile, 2 words each
                        const int so = kt * 2 * 64 * WPL * 4;
                        const u32x2 w0 = __builtin_amdgcn_raw_buffer_load_b64(rb_, boff[cb] + ql * 16 * WPL * 4, so, 0);
                        const u32x2 w1 = __builtin_amdgcn_raw_buffer_load_b64(rb_, boff[cb] + ql * 16 * WPL * 4,
                                                                              so + 64 * WPL * 4, 0);
                        w = u32x4{w0.x, w0.y, w1.x, w1.y};
                    } else {  // 128: the whole group; 256: half (st pair) kt % 2
                        const int so = (kt * KT / GS) * 64 * WPL * 4 + ((kt * KT) % GS) / 64 * 2 * 4;
                        w = __builtin_amdgcn_raw_buffer_load_b128(rb_, boff[cb] + ql * 16 * WPL * 4, so, 0);
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) dst[4 * (j >> 1) + 2 * ql + (j & 1)][cb] = w[j];
                }
            } else {
#pragma unroll
                for (int t = 0; t < KT / 16; ++t)
                    dst[t][cb] = __builtin_amdgcn_raw_buffer_load_b32(rb_, boff[cb], (kt * (KT / 8) + 2 * t) * N * 4, 0);
            }
        }
    };

    f32x16 acc[RB][CB], tot[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            acc[rb][cb] = f32x16{};
            tot[rb][cb] = f32x16{};
        }

    half2_t zb[CB];
    float s[CB];
    // zero point (as f16 1024 + z in both halves) and scale of group g
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)sc, (short)0, 0x7FFFFFFF, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rz =
        __builtin_amdgcn_make_buffer_rsrc((void *)(qz ? qz : qw), (short)0, 0x7FFFFFFF, kRsrcWord3);
    auto group_consts = [&](int g) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            int z = 8;
            if (qz)
                z = (int)((__builtin_amdgcn_raw_buffer_load_b32(rz, (col[cb] >> 3) * 4, g * (N >> 3) * 4, 0) >>
                           (4 * (col[cb] & 7))) &
                          0xF) +
                    zoff;
            const _Float16 zz = (_Float16)(1024 + z);
            zb[cb] = half2_t{zz, zz};
            const unsigned sw = __builtin_amdgcn_raw_buffer_load_b32(rs, (col[cb] >> 1) * 4, g * N * 2, 0);
            s[cb] = (float)__builtin_bit_cast(_Float16, (uint16_t)(sw >> (16 * (col[cb] & 1))));
        }
    };

    load_a(0);
    load_b(bw[0], 0);
    store_a(0);
    __syncthreads();

    // One K tile from LDS buffer BUF = kt & 1. The tile loop is unrolled by
    // two so that the register buffer index and the group boundaries are
    // compile-time (kt * KT mod GS depends only on BUF for GS <= 2 KT).
    auto tile = [&](auto BUFC, int kt) {
        constexpr int BUF = decltype(BUFC)::value;
        const bool more = kt + 1 < ntiles;
        if (more) {
            load_a(kt + 1);
            load_b(bw[BUF ^ 1], kt + 1);
        }
#pragma unroll
        for (int s16 = 0; s16 < KT / 16; ++s16) {
            const int kin = BUF * KT + 16 * s16;  // == k mod GS (mod 2 KT)
            if (kin % GS == 0) group_consts((kt * KT + 16 * s16) / GS);
            half8 bf[CB];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) bf[cb] = word_to_b(bw[BUF][s16][cb], zb[cb]);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const half8 af =
                    *reinterpret_cast<const half8 *>(&As[BUF][(mw + rb * 32 + l32) * ALD + koff(s16)]);
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[cb], acc[rb][cb], 0, 0, 0);
            }
            if ((kin + 16) % GS == 0) {  // group complete: scale into the total
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
                        for (int i = 0; i < 16; ++i) tot[rb][cb][i] = fmaf(acc[rb][cb][i], s[cb], tot[rb][cb][i]);
                        acc[rb][cb] = f32x16{};
                    }
            }
        }
        if (more) {
            store_a(BUF ^ 1);
            __syncthreads();
        }
    };
    // K % 256 == 0 when GS == 256, so its groups never end on an odd last tile.
    for (int kt = 0; kt < ntiles; kt += 2) {
        tile(std::integral_constant<int, 0>{}, kt);
        if (kt + 1 < ntiles) tile(std::integral_constant<int, 1>{}, kt + 1);
    }

    // ------------------------------------------------------------ output
    // 32 x 32 block: lane l holds column l % 32, rows 8 (i / 4) + 4 (l / 32) + i % 4.
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const int n = nw + 32 * cb + l32;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int m = m0 + mw + rb * 32 + 8 * (i >> 2) + 4 * hi + (i & 3);
                if (m >= M) continue;
                if constexpr (F16OUT)
                    static_cast<_Float16 *>(C)[(size_t)m * N + n] = (_Float16)tot[rb][cb][i];
                else
                    static_cast<float *>(C)[(size_t)m * N + n] = tot[rb][cb][i];
            }
        }
}

// A'[m][j] = A[m][perm[j]]: one workgroup per row, the row staged in LDS.
__global__ __launch_bounds__(256) void permute_cols_kernel(const _Float16 *__restrict__ A, const int32_t *__restrict__ perm,
                                                           _Float16 *__restrict__ out, int K) {
    extern __shared__ _Float16 row[];
    const size_t base = (size_t)blockIdx.x * K;
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8)
        *reinterpret_cast<u32x4 *>(&row[k]) = *reinterpret_cast<const u32x4 *>(A + base + k);
    __syncthreads();
    for (int j = threadIdx.x; j < K; j += 256) out[base + j] = row[perm[j]];
}

template <int GS, bool TILED>
int launch_gs(st_context *ctx, const _Float16 *A, const uint32_t *qw, const uint16_t *sc, const uint32_t *qz, int zoff,
              void *C, bool f16out, int M, int K, int N) {
    const int T = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (f16out)
        hipLaunchKernelGGL((gemm_kernel<GS, TILED, true>), dim3(T), dim3(kThreads), 0, ctx->stream, A, qw, sc, qz, zoff, C,
                           M, K, N);
    else
        hipLaunchKernelGGL((gemm_kernel<GS, TILED, false>), dim3(T), dim3(kThreads), 0, ctx->stream, A, qw, sc, qz, zoff,
                           C, M, K, N);
    return st::launch_check("gemm_kernel");
}

template <bool TILED>
int launch_tiled(st_context *ctx, const _Float16 *A, const uint32_t *qw, const uint16_t *sc, const uint32_t *qz, int zoff,
                 void *C, bool f16out, int M, int K, int N, int gs) {
    switch (gs) {
        case 64: return launch_gs<64, TILED>(ctx, A, qw, sc, qz, zoff, C, f16out, M, K, N);
        case 128: return launch_gs<128, TILED>(ctx, A, qw, sc, qz, zoff, C, f16out, M, K, N);
        default: return launch_gs<256, TILED>(ctx, A, qw, sc, qz, zoff, C, f16out, M, K, N);
    }
}

}  // namespace

extern "C" int st_gptq_i4_gemm(st_context *ctx, const uint16_t *a, const uint32_t *qweight, const uint16_t *scales,
                               const uint32_t *qzeros, const int32_t *perm, void *c, int c_dtype, int M, int K, int N,
                               int group_size, uint32_t flags) {
    if (!ctx || !a || !qweight || !scales || !c) return st::fail(ST_ERR_INVALID, "st_gptq_i4_gemm: NULL argument");
    if (group_size != 64 && group_size != 128 && group_size != 256)
        return st::fail(ST_ERR_SHAPE, "st_gptq_i4_gemm: group_size %d not in {64,128,256}", group_size);
    if (M < 1 || K <= 0 || K % KT || K % group_size || N <= 0 || N % 8)
        return st::fail(ST_ERR_SHAPE, "st_gptq_i4_gemm: M=%d K=%d N=%d (K %% 128, K %% group_size, N %% 8)", M, K, N);
    if (c_dtype != ST_F32 && c_dtype != ST_F16) return st::fail(ST_ERR_INVALID, "st_gptq_i4_gemm: c_dtype %d", c_dtype);
    if (!st::aligned16(a) || !st::aligned16(qweight))
        return st::fail(ST_ERR_ALIGN, "st_gptq_i4_gemm: a and qweight must be 16-byte aligned");
    if ((size_t)M * K * 2 > 0x7FFFFFFFu || (size_t)K / 8 * ((N + 15) / 16 * 16) * 4 > 0x7FFFFFFFu)
        return st::fail(ST_ERR_SHAPE, "st_gptq_i4_gemm: A or qweight above 2 GiB (M=%d K=%d N=%d); split M or N", M, K,
                        N);
    const _Float16 *A = reinterpret_cast<const _Float16 *>(a);
    if (perm) {
        if (K > 32768) return st::fail(ST_ERR_SHAPE, "st_gptq_i4_gemm: act-order K=%d above 32768", K);
        const size_t need = (size_t)M * K * sizeof(_Float16);
        if (need > ctx->ws_bytes)
            return st::fail(ST_ERR_WORKSPACE,
                            "st_gptq_i4_gemm: act-order needs %zu B of workspace (st_context_reserve_workspace)", need);
        _Float16 *Ap = reinterpret_cast<_Float16 *>(ctx->ws);
        hipLaunchKernelGGL(permute_cols_kernel, dim3(M), dim3(256), (size_t)K * sizeof(_Float16), ctx->stream, A, perm, Ap,
                           K);
        if (int rc = st::launch_check("permute_cols_kernel")) return rc;
        A = Ap;
    }
    const int zoff = (flags & ST_FLAG_ZEROS_PLUS_ONE) ? 1 : 0;
    const bool f16out = c_dtype == ST_F16;
    if (flags & ST_FLAG_TILED) return launch_tiled<true>(ctx, A, qweight, scales, qzeros, zoff, c, f16out, M, K, N, group_size);
    return launch_tiled<false>(ctx, A, qweight, scales, qzeros, zoff, c, f16out, M, K, N, group_size);
}
