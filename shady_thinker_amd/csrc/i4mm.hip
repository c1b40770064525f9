// Multi-token GPTQ int4 decode on f16 MFMA (a skinny GEMM), for 2..32
// tokens on tiled weights (st_gptq_i4_repack; act-order x
// through a pre-pass):
//   y[m, n]  = sum_g s[g, n] * sum_{k in g} (q[k, n] - z[g, n]) * x[m, k]
//   (st_gptq_i4_matvec), or silu(gate) * up of two such sums
//   (st_gptq_i4_gate_up_silu). Semantics of gptq_matvec.wgsl:51-58 and
//   fused_gate_up_silu_4t.wgsl:24-90; the reference runs one token at a time.
//
//  * Exact products: (q - z) is an integer in [-15, 15], exact in f16 (the
//    f16 1024 bias: 1024 + q, minus 1024 + z). f16 x is used as is. f32 x is
//    split per token and per 128 k: x 2^-e (2^e just above the block's
//    largest |x|) = hi + lo, two f16 rows of the MFMA A operand (about 21
//    significant bits: hi its top 11 bits, lo the rest rounded toward
//    zero), as each chunk of x is staged into LDS (with
//    act-order, by a pre-pass into the context workspace). Every
//    product is exact in f32; each 64 (or 128) k block sums into a fresh
//    accumulator that is then scaled by s 2^e in f32.
//  * Every weight is read from HBM once for all tokens (the integer-limb
//    matvec kernels grow their per-token staging and epilogue work with M).
//  * Work split as in i8mm.hip: one workgroup per CU owns a run of 16-column
//    tiles (gate/up: the gate and up tiles of each); S waves per tile each
//    take one 128-k unit of every S-unit chunk (gate/up in PAIR mode: of
//    both the gate and the up tile). 16 waves per workgroup, or 12 when its
//    tiles use at most 12. x is copied per chunk into
//    LDS (double buffered, one chunk ahead); each wave keeps a ring of three
//    chunks of weights, scales and zeros, two in flight while it computes
//    one. Partial sums meet in LDS in a fixed order.
//  * On at most one tile per CU (narrow linears): groups of tiles with K
//    split across workgroups, whole chunks per slice; each slice's sums go
//    to the workspace and i4mm_reduce_kernel adds them in slice order.
#include "common.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileN = 16;
constexpr int kRsrcWord3 = 0x00020000;     // raw 32-bit buffer data (gfx9-class)
constexpr unsigned kNoLoad = 0x80000000u;  // buffer offset past every resource: reads 0, touches no memory
constexpr int kMaxTilesPerWg = 8;
constexpr int kMaxSplit = 16;  // K slices of a split launch

// v_and_or_b32 with both constants in registers (a VOP3 takes no literal).
__device__ __forceinline__ unsigned and_or(unsigned a, unsigned m, unsigned c) {
    unsigned r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c));
    return r;
}

// GPTQ word (nibbles n0..n7 = k0..k7) -> (n0 - z, n4 - z), (n1 - z, n5 - z),
// (n2 - z, n6 - z), (n3 - z, n7 - z) in f16, exactly: 1024 + n - (1024 + z),
// or (1024 + 16 n) / 16 - (64 + z) for the odd nibbles.
__device__ __forceinline__ half8 word_to_b(unsigned w, half2_t zlo, half2_t zhi) {
    const unsigned m_lo = 0x000F000Fu, m_hi = 0x00F000F0u, bias = 0x64006400u;
    const half2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
    const unsigned w8 = w >> 8;
    const half2_t h0 = __builtin_bit_cast(half2_t, and_or(w, m_lo, bias)) - zlo;
    const half2_t h1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, and_or(w, m_hi, bias)), sixteenth, zhi);
    const half2_t h2 = __builtin_bit_cast(half2_t, and_or(w8, m_lo, bias)) - zlo;
    const half2_t h3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, and_or(w8, m_hi, bias)), sixteenth, zhi);
    const u32x4 r = {__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1), __builtin_bit_cast(unsigned, h2),
                     __builtin_bit_cast(unsigned, h3)};
    return __builtin_bit_cast(half8, r);
}

// 8 halves (k0..k7, as 4 dwords) -> the order of word_to_b: k0,k4,k1,k5,k2,k6,k3,k7.
__device__ __forceinline__ u32x4 to_b_order(u32x4 a) {
    u32x4 r;
    r.x = __builtin_amdgcn_perm(a.z, a.x, 0x05040100u);
    r.y = __builtin_amdgcn_perm(a.z, a.x, 0x07060302u);
    r.z = __builtin_amdgcn_perm(a.w, a.y, 0x05040100u);
    r.w = __builtin_amdgcn_perm(a.w, a.y, 0x07060302u);
    return r;
}

// 8 f32 x (k0..k7) times 2^-e (|x 2^-e| < 1) -> hi and lo f16 in the
// order of word_to_b, |x 2^-e - hi - lo| < 2^-20 |x 2^-e| + 2^-24:
// hi keeps the top 11 significant bits of x 2^-e (a mask, so hi - x 2^-e is
// exact in f32 and hi is exact in f16), lo is the rest rounded toward zero
// to f16. v_cvt_pkrtz packs two of them per instruction, paired as the B
// fragment wants them (k0 k4, k1 k5, k2 k6, k3 k7).
__device__ __forceinline__ void split_hi_lo(const float (&v)[8], float down, u32x4 &H, u32x4 &L) {
    float hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float xs = v[e] * down;
        hi[e] = __uint_as_float(__float_as_uint(xs) & 0xFFFFE000u);
        lo[e] = xs - hi[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        H[e] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_pkrtz(hi[e], hi[e + 4]));
        L[e] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_pkrtz(lo[e], lo[e + 4]));
    }
}

template <int CTRL>
__device__ __forceinline__ unsigned dpp_u(unsigned v) {
    return (unsigned)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
// 2^e just above the largest |x| of a 128-k unit (its 16 lanes hold 8 k
// each): e = 0 for an all-zero unit. The maximum is taken on the bit
// patterns of |x| (ordered like the values), so no canonicalizing float max.
__device__ __forceinline__ int unit_exponent(const float (&v)[8]) {
    unsigned m = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) m = max(m, __float_as_uint(v[e]) & 0x7FFFFFFFu);
    m = max(m, dpp_u<0xB1>(m));   // quad_perm [1,0,3,2]
    m = max(m, dpp_u<0x4E>(m));   // quad_perm [2,3,0,1]
    m = max(m, dpp_u<0x141>(m));  // row_half_mirror
    m = max(m, dpp_u<0x140>(m));  // row_mirror
    return m ? __builtin_amdgcn_frexp_expf(__uint_as_float(m)) : 0;  // |x| < 2^e
}

// silu(v) = v / (1 + exp(-v)) (fused_gate_up_silu_4t.wgsl)
__device__ __forceinline__ float silu_f(float v) { return __fdividef(v, 1.0f + __expf(-v)); }

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int GS>
struct Unit {  // what a wave loads for one 128-k unit of its tile and source
    static constexpr int NG = GS == 64 ? 2 : 1;  // groups in the unit
    u32x4 w;                                      // words (st, h) = (0,0), (0,1), (1,0), (1,1)
    unsigned s[NG];                               // raw f16 scale (low half)
    unsigned z[NG];                               // raw qzeros word
};

// f32 x -> rows 2t (hi) and 2t + 1 (lo) of xp [2M, K] f16 and the factor
// 2^e of each (token, 128-k unit) in pe [M, K / 128]: x 2^-e = hi + lo with
// |x 2^-e| < 1 over the unit. Every 8 k are stored in the B order of
// word_to_b. One 16-lane DPP row per (token, unit), 8 k per lane.
__global__ __launch_bounds__(256) void i4mm_prep_kernel(const float *__restrict__ x, const int32_t *__restrict__ perm,
                                                        _Float16 *__restrict__ xp, float *__restrict__ pe, int M, int K) {
    const int units = K / 128;
    const int gid = blockIdx.x * 16 + (threadIdx.x >> 4), l = threadIdx.x & 15;
    const bool ok = gid < M * units;  // every lane runs the DPP max below
    const int t = ok ? gid / units : 0, u = ok ? gid % units : 0;
    const size_t k = (size_t)u * 128 + 8 * l;
    f32x4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
    if (ok && perm) {  // act-order: k of the sorted weight rows reads x[perm[k]]
        const int4 p0 = *reinterpret_cast<const int4 *>(perm + k), p1 = *reinterpret_cast<const int4 *>(perm + k + 4);
        const float *xr = x + (size_t)t * K;
        a = f32x4{xr[p0.x], xr[p0.y], xr[p0.z], xr[p0.w]};
        b = f32x4{xr[p1.x], xr[p1.y], xr[p1.z], xr[p1.w]};
    } else if (ok) {
        a = *reinterpret_cast<const f32x4 *>(x + (size_t)t * K + k);
        b = *reinterpret_cast<const f32x4 *>(x + (size_t)t * K + k + 4);
    }
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const int ex = unit_exponent(v);
    u32x4 H, L;
    split_hi_lo(v, __builtin_amdgcn_ldexpf(1.0f, -ex), H, L);
    if (!ok) return;
    *reinterpret_cast<u32x4 *>(xp + (size_t)(2 * t) * K + k) = H;
    *reinterpret_cast<u32x4 *>(xp + (size_t)(2 * t + 1) * K + k) = L;
    if (l == 0) pe[(size_t)t * units + u] = __builtin_amdgcn_ldexpf(1.0f, ex);
}

// XM: f16 x (0), the pre-pass output (1: xp, pe, two f16 rows per token) or
// f32 x split at staging (2);
// NSRC: 1 (matvec) or 2 (gate/up); MB: 16-row MFMA blocks; KCU: 128-k units
// per staged chunk; GW: units per wave per chunk (S = KCU / GW waves per tile
// and source).
// NW waves per workgroup: 16, or 12 when the workgroup's tiles use at most 12
// (a wave without a tile still issues every VALU instruction of the loop).
// PAIR (two sources): a wave takes its units of both the gate and the up
// weight of a tile, so every x fragment read from LDS and every load
// address serves two MFMA chains.
// HZ: some source has zero points (without, no zero words are loaded: z = 8).
template <int XM, int NSRC, int MB, int GS, int KCU, int GW, int NW, bool PAIR, bool HZ>
__global__ __launch_bounds__(64 * NW) void i4mm_kernel(const void *__restrict__ x, const float *__restrict__ pe,
                                                        const uint32_t *__restrict__ qw0,
                                                        const uint16_t *__restrict__ sc0, const uint32_t *__restrict__ qz0,
                                                        const uint32_t *__restrict__ qw1, const uint16_t *__restrict__ sc1,
                                                        const uint32_t *__restrict__ qz1, int zoff, float *__restrict__ y,
                                                        int M, int K, int N, int ntiles, float *__restrict__ part, int ks) {
    // XM: 0 f16 x; 1 f32 x split by i4mm_prep_kernel (hi / lo rows and
    // factors in the workspace); 2 f32 x split here, at staging, with the
    // same arithmetic (no pre-pass launch)
    constexpr bool F32X = XM != 0;
    constexpr bool RAW = XM == 2;
    constexpr int kKC = 128 * KCU;        // k per staged chunk
    constexpr int kPitch = kKC + 8;       // halves per LDS row (16-byte pad: fragment rows on distinct banks)
    constexpr int S = KCU / GW;
    constexpr int R = F32X ? 2 : 1;       // MFMA rows per token
    constexpr int ROWS = 16 * MB;
    constexpr int TPB = 16 / R;           // tokens per 16-row block
    // f32 x: 2^e factors per (unit, token) of a chunk, PT tokens per unit
    constexpr int PT = ROWS / 2 > 16 ? ROWS / 2 : 16;
    constexpr int NG = Unit<GS>::NG;
    constexpr int EK = GS == 64 ? 2 : 4;  // MFMA steps (32 k) per scaled block
    // x items of 8 k: rows (tokens, or hi/lo rows of f32 tokens) x kKC / 8
    // per chunk, one 16-byte load each
    constexpr int XITEMS = ROWS * (kKC / 8);
    constexpr int kThr = 64 * NW;
    constexpr int XL = (XITEMS + kThr - 1) / kThr;
    // RAW: items of 8 k of one token (32 bytes of f32 x, two loads), each
    // giving the 8 k of its hi and lo rows; 16 consecutive items (lanes of
    // one DPP row) are one 128-k unit of one token
    constexpr int RITEMS = (ROWS / 2) * (kKC / 8);
    constexpr int XLR = (RITEMS + kThr - 1) / kThr;
    // two x buffers; at the end, the partial sums of every wave
    constexpr int PS = PAIR ? 2 : 1;  // sources per wave
    static_assert(!PAIR || NSRC == 2, "PAIR needs two sources");
    constexpr int kRedBytes = NW * PS * MB * (F32X ? 2 : 4) * 64 * 4;
    constexpr int kXsHalves = 2 * ROWS * kPitch > kRedBytes / 2 ? 2 * ROWS * kPitch : kRedBytes / 2;
    __shared__ __align__(16) _Float16 xs[kXsHalves];
    _Float16 *const xs0 = xs, *const xs1 = xs + ROWS * kPitch;
    __shared__ float ps0[F32X ? KCU * PT : 1];  // 2^e per (unit, token) of the chunk in xs0 / xs1
    __shared__ float ps1[F32X ? KCU * PT : 1];

    // The wave index through readfirstlane: the compiler takes tid >> 6 as
    // divergent, and the source chosen from it (gate or up) then put the
    // weight, scale and zero resources in VGPRs, every load of them in a
    // waterfall loop.
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // K split (ks > 1): workgroup b takes K slice b % ks of tile group b / ks
    const int kslice = blockIdx.x % ks, ngrp = gridDim.x / ks, grp = blockIdx.x / ks;
    const int t0 = (int)((long long)grp * ntiles / ngrp);
    const int t1 = (int)((long long)(grp + 1) * ntiles / ngrp);
    const int tb = PAIR ? wave / S : wave / (NSRC * S), src = PAIR ? 0 : (wave / S) % NSRC, slice = wave % S;
    const bool active = t0 + tb < t1;
    const int T = min(t0 + tb, ntiles - 1);
    const int G = K / GS;
    const int units = K / 128;
    // this slice's chunks [cb, ce), its units below uend, its k below kend
    const int nch_all = (units + KCU - 1) / KCU;
    const int cb = kslice * nch_all / ks, ce = (kslice + 1) * nch_all / ks;
    const int uend = min(units, ce * KCU), kend = min(K, ce * kKC);
    const int q = lane >> 4, r16 = lane & 15;
    const int n = min(kTileN * T + r16, N - 1);  // this lane's column (the last tile's padding repeats N - 1)

    // per source the wave reads (PAIR: gate, up; otherwise its own source)
    __amdgpu_buffer_rsrc_t rw[PS], rs[PS], rz[PS];
    bool has_z[PS];
#pragma unroll
    for (int ps = 0; ps < PS; ++ps) {
        const int sr = PAIR ? ps : src;
        const uint32_t *qw = (NSRC == 2 && sr) ? qw1 : qw0;
        const uint16_t *sc = (NSRC == 2 && sr) ? sc1 : sc0;
        const uint32_t *qz = (NSRC == 2 && sr) ? qz1 : qz0;
        has_z[ps] = qz != nullptr;
        rw[ps] = __builtin_amdgcn_make_buffer_rsrc((void *)qw, (short)0, 0x7FFFFFFF, kRsrcWord3);
        rs[ps] = __builtin_amdgcn_make_buffer_rsrc((void *)sc, (short)0, 0x7FFFFFFF, kRsrcWord3);
        // without qzeros the zero loads read nothing (z = 8)
        rz[ps] = __builtin_amdgcn_make_buffer_rsrc((void *)(has_z[ps] ? (const void *)qz : (const void *)sc), (short)0,
                                                   0x7FFFFFFF, kRsrcWord3);
    }
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)x, (short)0, 0x7FFFFFFF, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc((void *)pe, (short)0, 0x7FFFFFFF, kRsrcWord3);

    // ------------------------------------------------------------- x staging
    // Rows already in B order: the chunk is copied. With f32 x, threads
    // tid < KCU 16 also copy the chunk's 2^e factors (unit tid / 16, token tid % 16).
    const int nrows = F32X ? 2 * M : M;
    // x is loaded XS chunks ahead (register set c % XS holds chunk c): two
    // where the registers allow it (12-wave workgroups, or 2-unit chunks),
    // else one, which leaves each chunk's staging waiting for its x
    constexpr int XS = (NW <= 12 || KCU <= 2) ? 2 : 1;
    u32x4 xr2[XS][RAW ? 2 * XLR : XL];
    unsigned pr2[XS];
    auto load_x = [&](u32x4 (&xr)[RAW ? 2 * XLR : XL], unsigned &pr, int c) {
        if constexpr (RAW) {
#pragma unroll
            for (int j = 0; j < XLR; ++j) {
                const int i = j * kThr + tid;
                const int t = i / (kKC / 8), k = c * kKC + 8 * (i % (kKC / 8));
                const bool ok = i < RITEMS && t < M && k < kend;
                const unsigned o = ok ? (unsigned)(t * K + k) * 4u : kNoLoad;
                xr[2 * j] = __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0);
                xr[2 * j + 1] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? o + 16u : kNoLoad, 0, 0);
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < XL; ++j) {
            const int i = j * kThr + tid;
            const int row = i / (kKC / 8), k = c * kKC + 8 * (i % (kKC / 8));
            const bool ok = i < XITEMS && row < nrows && k < kend;
            xr[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? (unsigned)(row * K + k) * 2u : kNoLoad, 0, 0);
        }
        if constexpr (F32X) {
            const int t = tid % PT, u = c * KCU + tid / PT;
            const bool ok = tid < KCU * PT && t < M && u < uend;
            pr = __builtin_amdgcn_raw_buffer_load_b32(rp, ok ? (unsigned)(t * units + u) * 4u : kNoLoad, 0, 0);
        }
    };
    auto store_x = [&](const u32x4 (&xr)[RAW ? 2 * XLR : XL], unsigned pr, _Float16 *xs, float *ps) {
        if constexpr (RAW) {
            // the split of i4mm_prep_kernel: x 2^-e (2^e just above the
            // unit's largest |x|) = hi + lo, 8 k per item in B order
#pragma unroll
            for (int j = 0; j < XLR; ++j) {
                const int i = j * kThr + tid;
                // A wave whose items all belong to tokens >= M (or lie past
                // the chunk's items) skips them: only output rows that are
                // never written read those rows of xs (a uniform branch)
                if ((j * kThr + wave * 64) / (kKC / 8) >= M) continue;
                // (each word through a scalar first: hipcc's __builtin_bit_cast
                // of an ext_vector component reads component 0)
                const u32x4 a = xr[2 * j], b = xr[2 * j + 1];
                const unsigned wv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = __uint_as_float(wv[e]);
                // (every lane of the wave takes part: items past the end read zeros)
                const int ex = unit_exponent(v);
                u32x4 H, L;
                split_hi_lo(v, __builtin_amdgcn_ldexpf(1.0f, -ex), H, L);
                if (RITEMS % kThr == 0 || i < RITEMS) {
                    const int t = i / (kKC / 8), kq = i % (kKC / 8);
                    *reinterpret_cast<u32x4 *>(&xs[(2 * t) * kPitch + 8 * kq]) = H;
                    *reinterpret_cast<u32x4 *>(&xs[(2 * t + 1) * kPitch + 8 * kq]) = L;
                    if ((kq & 15) == 0) ps[(kq >> 4) * PT + t] = __builtin_amdgcn_ldexpf(1.0f, ex);
                }
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < XL; ++j) {
            const int i = j * kThr + tid;
            if (XITEMS % kThr == 0 || i < XITEMS)
                *reinterpret_cast<u32x4 *>(&xs[(i / (kKC / 8)) * kPitch + 8 * (i % (kKC / 8))]) =
                    F32X ? xr[j] : to_b_order(xr[j]);
        }
        if constexpr (F32X) {
            if (tid < KCU * PT) ps[tid] = __builtin_bit_cast(float, pr);
        }
    };

    // ------------------------------------------------------ weights, scales
    // Tiled words of group g: lane l's GS / 32 words at ((T G + g) 64 + l) GS / 32,
    // word 2 st + h = packed row GS / 8 g + 8 st + 2 (l / 16) + h.
    Unit<GS> ur[3][GW][PS];  // a ring of three chunks: loaded two chunks ahead
    auto load_u = [&](Unit<GS> (&dsts)[GW][PS], int c) {
#pragma unroll
        for (int ps = 0; ps < PS; ++ps)
#pragma unroll
        for (int gi = 0; gi < GW; ++gi) {
            Unit<GS> &du = dsts[gi][ps];
            const int u = c * KCU + slice * GW + gi;
            const bool ok = active && u < uend;
            if constexpr (GS == 64) {
                unsigned o0 = ok ? (unsigned)(((T * G + 2 * u) * 64 + lane) * 8) : kNoLoad;
                asm volatile("" : "+v"(o0));
                const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rw[ps], o0, 0, 0);
                const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(rw[ps], o0, 64 * 8, 0);
                du.w = u32x4{a.x, a.y, b.x, b.y};
            } else {
                // (offsets pinned in VGPRs: see the scale loads below)
                unsigned ow = ok ? (GS == 128 ? (unsigned)(((T * G + u) * 64 + lane) * 16)
                                              : (unsigned)(((T * G + u / 2) * 64 + lane) * 32 + 16 * (u & 1)))
                                 : kNoLoad;
                asm volatile("" : "+v"(ow));
                du.w = __builtin_amdgcn_raw_buffer_load_b128(rw[ps], ow, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                const int g = GS == 64 ? 2 * u + j : (u * 128) / GS;
                // offsets pinned in VGPRs: left as selects on a uniform
                // condition, the compiler turned each load into two loads on
                // two branches, and its load waits after those joins drained
                // the loads of the chunks in flight
                // (with zero words in the stream the compiler's waits before
                // a chunk's compute still drain the previous chunk's loads:
                // symmetric weights, the common case, load none)
                unsigned os = ok ? (unsigned)(g * N + n) * 2u : kNoLoad;
                asm volatile("" : "+v"(os));
                du.s[j] = __builtin_amdgcn_raw_buffer_load_b16(rs[ps], os, 0, 0);
                if constexpr (HZ) {
                    unsigned oz = (ok && has_z[ps]) ? (unsigned)(g * (N / 8) + n / 8) * 4u : kNoLoad;
                    asm volatile("" : "+v"(oz));
                    du.z[j] = __builtin_amdgcn_raw_buffer_load_b32(rz[ps], oz, 0, 0);
                } else {
                    du.z[j] = 0;
                }
            }
        }
    };

    // Running sums: F32X: tokens TPB mb + 2 q + t2 (t2 < 2); f16: rows 16 mb + 4 q + i.
    constexpr int YV = F32X ? 2 : 4;
    float ys[PS][MB][YV];
#pragma unroll
    for (int ps = 0; ps < PS; ++ps)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < YV; ++i) ys[ps][mb][i] = 0.f;

    // A wave without a tile (its workgroup owns fewer tiles than it has wave
    // groups) computes on: its sums are never used, a branch around the work
    // made the compiler's load waits drain everything in flight, and with its
    // x reads all on one address (a broadcast) they take one LDS access
    // instead of eight from the other waves.
    const int amask = active ? -1 : 0;
    auto compute = [&](const _Float16 *xs, const float *pf, const Unit<GS> (&src_u)[GW][PS]) {
#pragma unroll
        for (int gi = 0; gi < GW; ++gi) {
            const int ul = slice * GW + gi;  // unit within the chunk
            f32x2 pw[MB];                     // 2^e of this lane's two tokens per block
            if constexpr (F32X) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) pw[mb] = *reinterpret_cast<const f32x2 *>(&pf[ul * PT + TPB * mb + 2 * q]);
            }
#pragma unroll
            for (int blk = 0; blk < 4 / EK; ++blk) {  // scaled blocks of EK steps
                const int j = GS == 64 ? blk : 0;      // group of the block within the unit
                half2_t zlo[PS], zhi[PS];
                float s[PS];
                f32x4 acc[PS][MB];
#pragma unroll
                for (int ps = 0; ps < PS; ++ps) {
                    const int z = (HZ && has_z[ps]) ? (int)((src_u[gi][ps].z[j] >> (4 * (n & 7))) & 0xF) + zoff : 8;
                    const _Float16 zl = (_Float16)(1024 + z), zh = (_Float16)(-(64 + z));
                    zlo[ps] = half2_t{zl, zl};
                    zhi[ps] = half2_t{zh, zh};
                    s[ps] = (float)__builtin_bit_cast(_Float16, (uint16_t)src_u[gi][ps].s[j]);
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) acc[ps][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int e = 0; e < EK; ++e) {
                    const int step = blk * EK + e;  // word 2 st + h
                    const int st = step >> 1, h = step & 1;
                    half8 b[PS];
#pragma unroll
                    for (int ps = 0; ps < PS; ++ps) b[ps] = word_to_b(src_u[gi][ps].w[step], zlo[ps], zhi[ps]);
                    const int kk = ul * 128 + 64 * st + 16 * q + 8 * h;
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        const half8 a = *reinterpret_cast<const half8 *>(&xs[((16 * mb + r16) * kPitch + kk) & amask]);
#pragma unroll
                        for (int ps = 0; ps < PS; ++ps)
                            acc[ps][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[ps], acc[ps][mb], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int ps = 0; ps < PS; ++ps)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    if constexpr (F32X) {
                        ys[ps][mb][0] = __builtin_fmaf(s[ps] * pw[mb].x, acc[ps][mb][0] + acc[ps][mb][1], ys[ps][mb][0]);
                        ys[ps][mb][1] = __builtin_fmaf(s[ps] * pw[mb].y, acc[ps][mb][2] + acc[ps][mb][3], ys[ps][mb][1]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) ys[ps][mb][i] = __builtin_fmaf(s[ps], acc[ps][mb][i], ys[ps][mb][i]);
                    }
                }
            }
        }
    };

    // Chunk c: its x was loaded during chunk c - XS and staged into LDS buffer
    // c % 2 at the end of chunk c - 1; its weights were loaded during chunk
    // c - 2 into ring slot c % 3. Six chunks per trip so that every buffer
    // index is compile-time; loads are unconditional (past the end they read
    // nothing), so the compiler's wait counts are the same on every path.
    load_x(xr2[0], pr2[0], cb);
    if constexpr (XS == 2) load_x(xr2[1], pr2[1], cb + 1);
    load_u(ur[0], cb);
    load_u(ur[1], cb + 1);
    store_x(xr2[0], pr2[0], xs0, ps0);
    lds_barrier();
    auto chunk = [&](auto P, int c) {
        constexpr int p = decltype(P)::value;
        load_x(xr2[p % XS], pr2[p % XS], c + XS);
        load_u(ur[(p + 2) % 3], c + 2);
        // the chunk's loads stay at its top (left alone, the scheduler sank
        // some into the compute below, where their issue then waited)
        __builtin_amdgcn_sched_barrier(0);
        compute(p % 2 ? xs1 : xs0, p % 2 ? ps1 : ps0, ur[p % 3]);
        store_x(xr2[(p + 1) % XS], pr2[(p + 1) % XS], p % 2 ? xs0 : xs1, p % 2 ? ps0 : ps1);  // chunk c + 1
        lds_barrier();
    };
    for (int c = cb; c < ce; c += 6) {
        chunk(std::integral_constant<int, 0>{}, c);
        if (c + 1 >= ce) break;
        chunk(std::integral_constant<int, 1>{}, c + 1);
        if (c + 2 >= ce) break;
        chunk(std::integral_constant<int, 2>{}, c + 2);
        if (c + 3 >= ce) break;
        chunk(std::integral_constant<int, 3>{}, c + 3);
        if (c + 4 >= ce) break;
        chunk(std::integral_constant<int, 4>{}, c + 4);
        if (c + 5 >= ce) break;
        chunk(std::integral_constant<int, 5>{}, c + 5);
    }

    // Partial sums of the S waves of a tile (and source), added in slice order.
    float *red = reinterpret_cast<float *>(xs);
    static_assert(NW * PS * MB * YV * 64 * 4 == kRedBytes, "reduction buffer");
    // slot of (tile tb, source, slice): the wave index of the one-source layout
#pragma unroll
    for (int ps = 0; ps < PS; ++ps) {
        const int vw = (tb * NSRC + (PAIR ? ps : src)) * S + slice;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < YV; ++i) red[((vw * MB + mb) * YV + i) * 64 + lane] = ys[ps][mb][i];
    }
    lds_barrier();
    if (!active || slice != 0 || src != 0) return;
    const int nc = kTileN * T + r16;
    if (nc >= N) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < YV; ++i) {
            float v[NSRC];
#pragma unroll
            for (int sr = 0; sr < NSRC; ++sr) {
                v[sr] = 0.f;
                for (int sl = 0; sl < S; ++sl)
                    v[sr] += red[((((tb * NSRC + sr) * S + sl) * MB + mb) * YV + i) * 64 + lane];
            }
            const int m = F32X ? TPB * mb + 2 * q + i : 16 * mb + 4 * q + i;
            if (m >= M) continue;
            if (ks > 1) {  // the slice's sums, to i4mm_reduce_kernel
#pragma unroll
                for (int sr = 0; sr < NSRC; ++sr) part[((size_t)(kslice * NSRC + sr) * M + m) * N + nc] = v[sr];
            } else if constexpr (NSRC == 2) {
                y[(size_t)m * N + nc] = silu_f(v[0]) * v[1];
            } else {
                y[(size_t)m * N + nc] = v[0];
            }
        }
}

// K split: y = epilogue(sum over slices s < ks of part[s][src]), the slices
// added in order (deterministic), the epilogue silu(gate) * up for two sources.
template <int NSRC>
__global__ __launch_bounds__(256) void i4mm_reduce_kernel(const float *__restrict__ part, float *__restrict__ y, int MN,
                                                          int ks) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= MN) return;
    float t[kMaxSplit][NSRC];  // every slice's load issued before the first add
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s)
#pragma unroll
        for (int sr = 0; sr < NSRC; ++sr) t[s][sr] = s < ks ? part[(size_t)(s * NSRC + sr) * MN + idx] : 0.f;
    float v[NSRC];
#pragma unroll
    for (int sr = 0; sr < NSRC; ++sr) {
        v[sr] = 0.f;
#pragma unroll
        for (int s = 0; s < kMaxSplit; ++s)
            if (s < ks) v[sr] += t[s][sr];
    }
    y[idx] = NSRC == 2 ? silu_f(v[0]) * v[1] : v[0];
}

template <int XM, int NSRC, int MB, int GS>
int launch_gs(st_context *ctx, const void *x, const float *pe, const uint32_t *const *qw, const uint16_t *const *sc,
              const uint32_t *const *qz, int zoff, float *y, int M, int K, int N, int ntiles, int G, int wpt, int nw,
              bool pair, float *part, int ks) {
    const dim3 grid(G * ks);
    const bool hz = qz[0] || (NSRC == 2 && qz[1]);
#define ST_I4MM_P(KCU_, GW_, NW_, PAIR_)                                                                           \
    do {                                                                                                           \
        if (hz)                                                                                                    \
            st::launch(ctx, (i4mm_kernel<XM, NSRC, MB, GS, KCU_, GW_, NW_, PAIR_, true>), grid, dim3(64 * NW_), 0,  \
                       x, pe, qw[0], sc[0], qz[0], qw[1], sc[1], qz[1], zoff, y, M, K, N, ntiles, part, ks);    \
        else                                                                                                       \
            st::launch(ctx, (i4mm_kernel<XM, NSRC, MB, GS, KCU_, GW_, NW_, PAIR_, false>), grid, dim3(64 * NW_), 0, \
                       x, pe, qw[0], sc[0], qz[0], qw[1], sc[1], qz[1], zoff, y, M, K, N, ntiles, part, ks);    \
    } while (0)
#define ST_I4MM(KCU_, GW_, NW_) ST_I4MM_P(KCU_, GW_, NW_, false)
    // 17-32 tokens of f32 x (64 MFMA rows): 2-unit chunks (the two x buffers
    // of 4-unit chunks would not fit the LDS)
    if constexpr (MB == 4) {
        if (nw == 12)
            ST_I4MM(2, 1, 12);
        else
            ST_I4MM(2, 1, 16);
        return st::launch_check("i4mm_kernel");
    } else {
        // gate/up with both sources in a wave: wpt is then waves per tile pair
        if constexpr (NSRC == 2 && GS != 64) {  // (group 64 with two sources per wave spills)
            if (pair) {
                if (wpt >= 4)
                    ST_I4MM_P(4, 1, 12, true);
                else
                    ST_I4MM_P(2, 1, 12, true);
                return st::launch_check("i4mm_kernel");
            }
        }
        // waves per tile and source = 128-k units per chunk (one unit per wave):
        // 8 (1024-k chunks), 4 or 2. Group size 64 stops at 4: its 8-unit chunk
        // spilled 30 VGPRs inside the loop (one source, 16 tokens, 2560 x 6144:
        // 15.5 -> 13.7 us with 4; gate/up unchanged).
        if constexpr (GS != 64) {
            if (wpt >= 8) {
                ST_I4MM(8, 1, 16);
                return st::launch_check("i4mm_kernel");
            }
        }
        if (wpt >= 4) {
            if (nw == 12)
                ST_I4MM(4, 1, 12);
            else
                ST_I4MM(4, 1, 16);
        } else {
            if (nw == 12)
                ST_I4MM(2, 1, 12);
            else
                ST_I4MM(2, 1, 16);
        }
        return st::launch_check("i4mm_kernel");
    }
#undef ST_I4MM
#undef ST_I4MM_P
}

// Act-order with f16 x: xg[t, k] = x[t, perm[k]] (the sorted weight rows'
// order), 8 k per thread, into the workspace.
__global__ __launch_bounds__(256) void i4mm_gather_kernel(const uint16_t *__restrict__ x, const int32_t *__restrict__ perm,
                                                          uint16_t *__restrict__ xg, int M, int K) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i >= (size_t)M * K) return;
    const size_t t = i / K, k = i % K;
    const int4 p0 = *reinterpret_cast<const int4 *>(perm + k), p1 = *reinterpret_cast<const int4 *>(perm + k + 4);
    const uint16_t *xr = x + t * K;
    const u32x4 v = {xr[p0.x] | ((unsigned)xr[p0.y] << 16), xr[p0.z] | ((unsigned)xr[p0.w] << 16),
                     xr[p1.x] | ((unsigned)xr[p1.y] << 16), xr[p1.z] | ((unsigned)xr[p1.w] << 16)};
    *reinterpret_cast<u32x4 *>(xg + i) = v;
}

template <int XM, int NSRC, int MB>
int launch_mb(st_context *ctx, const void *x, const float *pe, const uint32_t *const *qw, const uint16_t *const *sc,
              const uint32_t *const *qz, int zoff, float *y, int M, int K, int N, int gs, int ntiles, int G, int wpt,
              int nw, bool pair, float *part, int ks) {
    switch (gs) {
        case 64:  // (four 16-row blocks with group 64 spill: the entry point takes 16-token blocks)
            if constexpr (MB == 4)
                return st::fail(ST_ERR_UNSUPPORTED, "int4_mm_f16: group 64 with %d tokens of f32 x", M);
            else
                return launch_gs<XM, NSRC, MB, 64>(ctx, x, pe, qw, sc, qz, zoff, y, M, K, N, ntiles, G, wpt, nw, pair, part,
                                                   ks);
        case 128:
            return launch_gs<XM, NSRC, MB, 128>(ctx, x, pe, qw, sc, qz, zoff, y, M, K, N, ntiles, G, wpt, nw, pair, part, ks);
        default:
            return launch_gs<XM, NSRC, MB, 256>(ctx, x, pe, qw, sc, qz, zoff, y, M, K, N, ntiles, G, wpt, nw, pair, part, ks);
    }
}

template <int XM, int NSRC>
int launch_src(st_context *ctx, const void *x, const float *pe, const uint32_t *const *qw, const uint16_t *const *sc,
               const uint32_t *const *qz, int zoff, float *y, int M, int K, int N, int gs, int ntiles, int G, int wpt,
               int nw, bool pair, float *part, int ks) {
    // tokens per 16-row block: 8 (f32 x: hi and lo rows) or 16; four blocks
    // only with f32 x (17-32 tokens)
    const int mb = (M * (XM ? 2 : 1) + 15) / 16;
    int rc;
    if (mb <= 1)
        rc = launch_mb<XM, NSRC, 1>(ctx, x, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks);
    else if (mb <= 2)
        rc = launch_mb<XM, NSRC, 2>(ctx, x, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks);
    else if constexpr (XM != 0)
        rc = launch_mb<XM, NSRC, 4>(ctx, x, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks);
    else
        return st::fail(ST_ERR_SHAPE, "int4_mm_f16: %d tokens", M);
    if (rc || ks == 1) return rc;
    const int mn = M * N;
    st::launch(ctx, (i4mm_reduce_kernel<NSRC>), dim3((mn + 255) / 256), dim3(256), 0, part, y, mn, ks);
    return st::launch_check("i4mm_reduce_kernel");
}

}  // namespace

namespace st {

// Arguments are checked by the entry points (tiled weights, M <= 16, K %
// 128 == 0, K % group_size == 0, N % 8 == 0, alignment, 32-bit offsets).
// Returns -1, having launched nothing, when the shape would split K and the
// slices' partial sums do not fit the workspace (the caller then takes the
// integer-limb kernels).
// perm (act-order, may be NULL): x is read as x[:, perm[k]], by the f32
// pre-pass or, for f16 x, by a gather pass into the workspace.
int int4_mm_f16(st_context *ctx, const void *x, bool x_f32, const int32_t *perm, const uint32_t *const qw[2],
                const uint16_t *const sc[2], const uint32_t *const qz[2], int zoff, float *y, int M, int K, int N,
                int gs, int nsrc) {
    const int ntiles = (N + kTileN - 1) / kTileN;
    const int maxt = kMaxTilesPerWg / nsrc;  // tiles per workgroup: each tile (and source) keeps >= 2 waves
    // At most one tile per CU: groups of split_tiles tiles, K split across
    // workgroups so that the grid fills the CUs (0: one workgroup per tile)
    const int split_tiles =
        ntiles <= ctx->num_cus ? std::min(tune(ctx, ST_TUNE_I4MM_SPLIT_TILES, kI4mmSplitTiles), maxt) : 0;
    int G = std::max(std::min(ctx->num_cus, ntiles), (ntiles + maxt - 1) / maxt);
    if (split_tiles > 0) G = (ntiles + split_tiles - 1) / split_tiles;
    const int tbmax = (ntiles + G - 1) / G;
    int wpt = 2;  // waves per tile and source: a power of two, wpt * nsrc * tbmax <= 16
    while (wpt < 8 && 2 * wpt * nsrc * tbmax <= kWaves) wpt *= 2;
    if (x_f32 && M > 16) wpt = 2;  // 17-32 tokens of f32 x: 2-unit chunks only
    if (wpt * nsrc * tbmax > kWaves) return fail(ST_ERR_SHAPE, "int4_mm_f16: %d tiles per workgroup", tbmax);
    // 12-wave workgroups when the tiles use at most 12 waves (gate/up with 3
    // tile pairs per workgroup): idle waves would still issue the loop's VALU
    int nw = (wpt <= 4 && wpt * nsrc * tbmax <= 12 && tune(ctx, ST_TUNE_I4MM_WAVES, 0) != 16) ? 12 : 16;
    // gate/up: both sources in one wave when the tile pairs then use 10-12
    // of 12 waves (wpt becomes waves per tile pair: 3 pairs of 4 waves, or
    // 5-6 pairs of 2)
    bool pair = false;
    if (nsrc == 2 && gs != 64 && !(x_f32 && M > 16) && tune(ctx, ST_TUNE_I4MM_PAIR, 1) != 0 &&
        tune(ctx, ST_TUNE_I4MM_WAVES, 0) != 16) {  // (not four 16-row blocks: both sources' sums would spill)
        int wpp = 2;
        while (wpp < 4 && 2 * wpp * tbmax <= 12) wpp *= 2;
        if (wpp * tbmax >= 10 && wpp * tbmax <= 12) {
            pair = true;
            wpt = wpp;
            nw = 12;
        }
    }
    const void *xa = x;
    const float *pe = nullptr;
    // f32 x without act-order: split inside the kernel (XM 2); with
    // act-order, or when the setting asks for it, by the pre-pass (XM 1)
    const bool split_in = x_f32 && !perm && tune(ctx, ST_TUNE_I4MM_PREPASS, 0) != 1;
    // K slices (whole chunks each) and their f32 partials in the workspace,
    // after what the pre-pass or the gather writes there
    int ks = 1;
    float *part = nullptr;
    if (split_tiles > 0) {
        const int kcu = pair ? (wpt >= 4 ? 4 : 2) : (wpt >= 8 && gs != 64 ? 8 : (wpt >= 4 ? 4 : 2));
        const int nch = (K / 128 + kcu - 1) / kcu;
        ks = std::max(1, std::min({ctx->num_cus / G, kMaxSplit, nch}));
        if (ks > 1) {
            const size_t pre = x_f32 && !split_in ? (((size_t)2 * M * K * 2 + 255) & ~size_t(255)) + (size_t)M * (K / 128) * 4
                                                  : (perm ? (size_t)M * K * 2 : 0);
            const size_t off = (pre + 255) & ~size_t(255);
            if (!ctx->ws || off + (size_t)ks * nsrc * M * N * sizeof(float) > ctx->ws_bytes) return -1;  // not taken
            part = reinterpret_cast<float *>(reinterpret_cast<char *>(ctx->ws) + off);
        }
    }
    if (x_f32 && !split_in) {  // the pre-pass writes [2M, K] f16 rows and [M, K / 128] factors into the workspace
        const size_t xbytes = ((size_t)2 * M * K * 2 + 255) & ~size_t(255);
        if (!ctx->ws || xbytes + (size_t)M * (K / 128) * 4 > ctx->ws_bytes)
            return fail(ST_ERR_WORKSPACE, "int4_mm_f16: workspace below %zu B", xbytes + (size_t)M * (K / 128) * 4);
        _Float16 *xp = reinterpret_cast<_Float16 *>(ctx->ws);
        pe = reinterpret_cast<const float *>(reinterpret_cast<const char *>(ctx->ws) + xbytes);
        const int groups = M * (K / 128);
        st::launch(ctx, i4mm_prep_kernel, dim3((groups + 15) / 16), dim3(256), 0,
                           static_cast<const float *>(x), perm, xp, const_cast<float *>(pe), M, K);
        if (int rc = launch_check("i4mm_prep_kernel")) return rc;
        xa = xp;
    } else if (perm) {
        const size_t xbytes = (size_t)M * K * 2;
        if (!ctx->ws || xbytes > ctx->ws_bytes) return fail(ST_ERR_WORKSPACE, "int4_mm_f16: workspace below %zu B", xbytes);
        uint16_t *xg = reinterpret_cast<uint16_t *>(ctx->ws);
        st::launch(ctx, i4mm_gather_kernel, dim3((unsigned)(((size_t)M * K / 8 + 255) / 256)), dim3(256), 0, static_cast<const uint16_t *>(x), perm, xg, M, K);
        if (int rc = launch_check("i4mm_gather_kernel")) return rc;
        xa = xg;
    }
    if (split_in)
        return nsrc == 2 ? launch_src<2, 2>(ctx, xa, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks)
                         : launch_src<2, 1>(ctx, xa, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks);
    if (nsrc == 2)
        return x_f32 ? launch_src<1, 2>(ctx, xa, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks)
                     : launch_src<0, 2>(ctx, xa, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks);
    return x_f32 ? launch_src<1, 1>(ctx, xa, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks)
                 : launch_src<0, 1>(ctx, xa, pe, qw, sc, qz, zoff, y, M, K, N, gs, ntiles, G, wpt, nw, pair, part, ks);
}

}  // namespace st
