// Quantized matvec / skinny GEMM for decode (M = 1..32 rows) on gfx950:
// the kernel template and its launcher. Instantiated per weight format and
// act-order in qmv_i4_p{0,1}.hip (GPTQ, reference layout), qmv_i4t_p{0,1}.hip
// (GPTQ, tiled layout) and qmv_i8.hip (INT8); the C entry points are in
// qmv.hip.
//
// Replaces the reference's GPTQ WGSL kernels (src/shaders/gptq_matvec_4t.wgsl,
// fused_silu_gptq_4t.wgsl, fused_gate_up_silu_4t.wgsl) and adds the INT8
// per-channel path. The math is the reference's: y[n] = sum_k (q - z) * s * x[k]
// with z = 8 in the reference (gptq_matvec.wgsl:51-58).
//
// Design (CDNA4, wave64), 16-column tiles:
//  * A workgroup owns whole 16-column tiles for the whole of K, so no
//    workgroup ever talks to another (cross-workgroup release fences and
//    atomics cost several microseconds per launch on MI355X). Its waves split
//    K by groups and meet once, at the end, in LDS. When N has more tiles
//    than the GPU has CUs, one workgroup per CU owns 2..4 tiles (x is staged
//    once per CU instead of once per tile).
//  * The dot products run on the int8 matrix cores (v_mfma_i32_16x16x64_i8,
//    16 rows x 16 columns x 64 k). B = weights: lane (q, c) supplies column c,
//    k-chunk q. A GPTQ word (8 nibbles of one column) becomes two int8
//    operand registers with one AND and one shift+AND; the values 0..15 are
//    exact. INT8 weights are operands as loaded.
//  * A = activations as exact integers. For every 128-k group (the GPTQ group
//    for int4) and token, x is scaled by 2^e so that max|x| 2^e lies in
//    [2^21, 2^22) and rounded to an integer X = L2*65536 + L1*256 + L0 with
//    signed 8-bit limbs; rows 4t..4t+2 of the MFMA hold token t's three limbs,
//    so one MFMA serves 4 tokens. Inside a group everything is exact int32,
//    including the zero point as -z * sum(X); each group result is rounded to
//    f32 once and scaled by s * 2^-e. Error ~2^-22 relative, far below the
//    reference's f32 FMA chain.
//  * Each wave keeps a ring of D groups of weight loads in flight (registers).
//  * Staging x (the decode case, one token block): either a few staging
//    waves that load no weights stage all of K into shared LDS, one or two
//    64-item rounds each, while the other waves start streaming weights and
//    wait at one bare barrier that leaves their loads in flight; or, for long
//    K, every wave stages its own groups (no barrier). Group max and sum use
//    DPP row moves; the integer conversion is one FMA. Several tokens and
//    long K: each wave stages its own chunks (fallback).
//  * vmcnt discipline: global loads complete in issue order and the compiler
//    counts them per path. Every load the wave issues while the ring is in
//    flight is unconditional (absent items read a clamped valid address, or,
//    with buffer loads, an out-of-range offset that accesses nothing) and
//    act-order is a template parameter, so no uniform branch changes the
//    number of loads in flight; otherwise the compiler's waits can be too
//    loose across the merge and registers are read before their loads land.
//    Zero points are read once into LDS before anything else is in flight.
//  * Weights are read in the reference layout (dword loads, 64 contiguous
//    bytes per 16 lanes) or, after st_gptq_i4_repack, in a tiled layout in
//    which each wave reads 1 KiB contiguous per group with 128-bit loads.
#pragma once

#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace st {
namespace qmv {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTileN = 16;     // output columns per workgroup (per source)
// Buffer resource word 3 for gfx9-class GPUs: raw (untyped) 32-bit data.
constexpr int kBufWord3 = 0x00020000;
// Tiled weights are read with buffer loads over a 2 GiB range; a ring slot
// with nothing left to load uses this offset, which is out of range: the
// load returns zeros without a memory access, and still counts as a load.
constexpr unsigned kNoLoad = 0x80000000u;
// Buffer-load cache policy of the weight ring: non-temporal for the
// two-source gate/up kernel (11.3 against 12.8-13.0 us with the default),
// the default for the others (down 7.7 against 8.0 us, INT8 16.7 against
// 17.9 us non-temporal).
constexpr int kNt = 2;
template <int NSRC>
constexpr int ring_cache_policy = NSRC == 2 ? kNt : 0;
constexpr int kMaxZeroUnits = 64;  // groups per wave whose zero points fit the LDS table

enum Fmt { FMT_I4 = 0, FMT_I4T = 1, FMT_I8 = 2, FMT_I8T = 3 };
// INT8 weights, row-major [N, K] (FMT_I8) or tiled (FMT_I8T, st_int8_repack)
constexpr bool is_i8(int fmt) { return fmt == FMT_I8 || fmt == FMT_I8T; }
enum XMode { XM_F32 = 0, XM_F16 = 1, XM_SILU = 2 };

struct Params {
    const void *x;          // [M, K] f32 / f16; `a` for XM_SILU
    const float *xb;        // `b` for XM_SILU
    const int32_t *perm;    // act-order gather (PERM kernels only)
    const uint32_t *qw[2];  // GPTQ qweight per source (reference or tiled layout)
    const uint16_t *sc[2];  // GPTQ scales  [K/gs, N]
    const uint32_t *qz[2];  // GPTQ qzeros  [K/gs, N/8] or null
    const int8_t *w8;       // INT8 weights [N, K]
    const float *scale8;    // INT8 scales [N]
    float *y;               // [M, N]
    int M, K, N;
    int gs;        // group length in k (GPTQ group size; 128 for INT8)
    int zoff;      // added to stored zero points
    int units;     // K / gs
    int ntiles;    // ceil(N / 16)
    int rb;        // A rows kept per (step, block, chunk): 4M when M < 4, else 16
    int chunk;     // groups staged per round trip
    int wave_lds;  // bytes of LDS per wave
    int nwaves;    // waves per workgroup (K is split among them)
    int tpw;       // COOP: most tiles one workgroup owns (LDS zero table rows)
    int grid;      // workgroups
    int nstage;    // COOP: staging waves (they load no weights)
    int ksplit;    // CHK: K slices (1 = none); > 1 writes f32 partials to part
    int ssync;     // streaming kernel: ring blocks between workgroup barriers (0: none)
    float *part;   // CHK split: [ksplit][NSRC][M][N] partial sums (before the epilogue)
    unsigned *cnt; // CHK split: per tile group, slices done (zero between calls); NULL: a reduce kernel follows
};

// silu(v) = v / (1 + exp(-v)) (fused_silu_gptq.wgsl:19-21), with the hardware
// exp and reciprocal (a few ulp; WGSL's exp and division are not correctly
// rounded either).
__device__ __forceinline__ float silu_f(float v) { return __fdividef(v, 1.0f + __expf(-v)); }

// k offset, within a lane's 16-k chunk, of int8 operand byte J for GPTQ:
// register r = J/4 holds nibbles 2(J%4) (+1 for odd r) of word r/2.
__device__ __forceinline__ constexpr int i4_koff(int J) { return ((J >> 3) << 3) + ((J & 3) << 1) + ((J >> 2) & 1); }

// One staging item: x[m, k .. k+15] (through perm under act-order), loaded
// with no arithmetic on the values, so that the loads stay in flight while
// the wave issues its other loads (arithmetic right after a load makes the
// wave wait for it): f32 as is; f16 as raw bits (two halves per dword, or
// one half per dword under act-order); silu(a) * b as a in v and b in vb.
// x_finish converts, at staging.
template <int XM, bool PERM>
__device__ __forceinline__ void load_x16(const Params &p, int m, int k, float v[16], float vb[16]) {
    const size_t row = (size_t)m * p.K;
    if constexpr (PERM) {
        int idx[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int4 t = *reinterpret_cast<const int4 *>(p.perm + k + 4 * j);
            idx[4 * j] = t.x;
            idx[4 * j + 1] = t.y;
            idx[4 * j + 2] = t.z;
            idx[4 * j + 3] = t.w;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if constexpr (XM == XM_F16) {
                const unsigned short h = static_cast<const unsigned short *>(p.x)[row + idx[j]];
                v[j] = __builtin_bit_cast(float, (unsigned)h);
            } else {
                v[j] = static_cast<const float *>(p.x)[row + idx[j]];
                if constexpr (XM == XM_SILU) vb[j] = p.xb[row + idx[j]];
            }
        }
    } else {
        // f32 / silu: 16 values; f16: 8 dwords of raw halves
        constexpr int NV = XM == XM_F16 ? 2 : 4;
        const float4 *src = XM == XM_F16
                                ? reinterpret_cast<const float4 *>(static_cast<const _Float16 *>(p.x) + row + k)
                                : reinterpret_cast<const float4 *>(static_cast<const float *>(p.x) + row + k);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const float4 t = src[j];
            v[4 * j] = t.x;
            v[4 * j + 1] = t.y;
            v[4 * j + 2] = t.z;
            v[4 * j + 3] = t.w;
        }
        if constexpr (XM == XM_SILU) {
            const float4 *bsrc = reinterpret_cast<const float4 *>(p.xb + row + k);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 u = bsrc[j];
                vb[4 * j] = u.x;
                vb[4 * j + 1] = u.y;
                vb[4 * j + 2] = u.z;
                vb[4 * j + 3] = u.w;
            }
        }
    }
}

// The 16 f32 values of a staging item from what load_x16 left.
template <int XM, bool PERM>
__device__ __forceinline__ void x_finish(float v[16], const float vb[16]) {
    if constexpr (XM == XM_F16) {
        float t[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const unsigned d = __builtin_bit_cast(unsigned, v[PERM ? j : j / 2]);
            const unsigned short h = (unsigned short)(PERM ? d : ((j & 1) ? d >> 16 : d & 0xFFFFu));
            t[j] = (float)__builtin_bit_cast(_Float16, h);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = t[j];
    } else if constexpr (XM == XM_SILU) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = silu_f(v[j]) * vb[j];
    }
}

// Cross-lane max / sum over aligned groups of G lanes (G = 4, 8, 16) with
// DPP row moves: quad_perm [1,0,3,2] and [2,3,0,1] combine a quad,
// row_half_mirror pairs the two quads of 8 lanes, row_mirror the two halves
// of 16.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
    static_assert(G == 4 || G == 8 || G == 16, "group of 4, 8 or 16 lanes");
    v = fmaxf(v, __builtin_bit_cast(float, dpp_mov<0xB1>(__builtin_bit_cast(int, v))));
    v = fmaxf(v, __builtin_bit_cast(float, dpp_mov<0x4E>(__builtin_bit_cast(int, v))));
    if constexpr (G >= 8) v = fmaxf(v, __builtin_bit_cast(float, dpp_mov<0x141>(__builtin_bit_cast(int, v))));
    if constexpr (G >= 16) v = fmaxf(v, __builtin_bit_cast(float, dpp_mov<0x140>(__builtin_bit_cast(int, v))));
    return v;
}
template <int G>
__device__ __forceinline__ int group_sum(int v) {
    static_assert(G == 4 || G == 8 || G == 16, "group of 4, 8 or 16 lanes");
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    if constexpr (G >= 8) v += dpp_mov<0x141>(v);
    if constexpr (G >= 16) v += dpp_mov<0x140>(v);
    return v;
}

// dword of byte `bp` of a, b, c, d (in that order, low byte first).
__device__ __forceinline__ unsigned pack4(unsigned a, unsigned b, unsigned c, unsigned d, int bp) {
    const unsigned sel = 0x0C0C0000u | ((4u + bp) << 8) | (unsigned)bp;
    const unsigned lo = __builtin_amdgcn_perm(b, a, sel);
    const unsigned hi = __builtin_amdgcn_perm(d, c, sel);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// One staging item: 16 values of x (token m, k0 .. k0+15 of a group,
// already converted to f32) become three signed 8-bit limbs per value,
// written as the A-operand rows dst[0..2] (dst[3], the token's fourth row, is
// zero), with the group's scale 2^-e and the split of sum(X) into es_dst
// when the item is the group's first (es_dst non-null). The IPU lanes of a
// group are consecutive and aligned; every lane calls (the cross-lane max and
// sum need them all), `ok` = the item exists. NAT: operand byte J holds value
// J (INT8), else value i4_koff(J) (GPTQ nibble order).
template <int IPU, bool NAT>
__device__ __forceinline__ void quantize_item(float (&v)[16], bool ok, u32x4 *dst, u32x4 *es_dst) {
    float amax = 0.0f, nf = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        amax = fmaxf(amax, fabsf(v[j]));
        nf = fmaf(v[j], 0.0f, nf);  // NaN iff some x is NaN or inf
    }
    // a non-finite x poisons its group: amax = inf -> 2^-e = NaN -> y = NaN
    amax = (nf == nf) ? amax : INFINITY;
    if (!ok) amax = 0.0f;
    amax = group_max<IPU>(amax);
    int e = 0;
    float em = 1.0f;
    if (amax == INFINITY) {
        em = __builtin_nanf("");
    } else if (amax > 0.0f) {
        // amax = f 2^fe, f in [0.5, 1): floor(log2 amax) = fe - 1
        e = 22 - __builtin_amdgcn_frexp_expf(amax);
        e = e > 100 ? 100 : (e < -100 ? -100 : e);
        em = __builtin_amdgcn_ldexpf(1.0f, -e);
    }
    const float sc2 = __builtin_amdgcn_ldexpf(1.0f, e);
    // X = round(x 2^e) in one FMA: |x 2^e| < 2^22 when amax is finite
    // (otherwise the group is NaN anyway), so v = x 2^e + 1.5 * 2^23 lies in
    // [2^23, 2^24), where the floats are the integers: the FMA rounds x 2^e
    // to the nearest integer (ties to even) and bits(v) = 0x4B400000 + X.
    unsigned Z[16];
    unsigned ysum = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const unsigned y = __builtin_bit_cast(unsigned, fmaf(v[j], sc2, 12582912.0f));
        ysum += y;
        // Z = Y + 0xC08080 = X + 0x8080 (mod 2^24): byte 2 of Z is the limb
        // L2 = byte 2 of X + 32896, bytes 1 and 0 of Z are L1 = byte 1 of X +
        // 128 and L0 = byte 0 of X, each plus 128 (mod 256)
        Z[j] = y + 0xC08080u;
    }
    const int sum = group_sum<IPU>((int)(ysum - 16u * 0x4B400000u));
    if (!ok) return;
    u32x4 L2v, L1v, L0v;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const unsigned a = Z[NAT ? 4 * rr : i4_koff(4 * rr)];
        const unsigned bb = Z[NAT ? 4 * rr + 1 : i4_koff(4 * rr + 1)];
        const unsigned cc = Z[NAT ? 4 * rr + 2 : i4_koff(4 * rr + 2)];
        const unsigned dd = Z[NAT ? 4 * rr + 3 : i4_koff(4 * rr + 3)];
        // [a0 b0 a1 b1], [c0 d0 c1 d1], [a2 b2 -- --], [c2 d2 -- --]
        const unsigned ab01 = __builtin_amdgcn_perm(bb, a, 0x05010400u);
        const unsigned cd01 = __builtin_amdgcn_perm(dd, cc, 0x05010400u);
        const unsigned ab2 = __builtin_amdgcn_perm(bb, a, 0x0C0C0602u);
        const unsigned cd2 = __builtin_amdgcn_perm(dd, cc, 0x0C0C0602u);
        L2v[rr] = __builtin_amdgcn_perm(cd2, ab2, 0x05040100u);
        L1v[rr] = __builtin_amdgcn_perm(cd01, ab01, 0x07060302u) ^ 0x80808080u;
        L0v[rr] = __builtin_amdgcn_perm(cd01, ab01, 0x05040100u) ^ 0x80808080u;
    }
    dst[0] = L2v;
    dst[1] = L1v;
    dst[2] = L0v;
    dst[3] = u32x4{0, 0, 0, 0};  // row 4t+3
    if (es_dst) {
        const int h = (sum + 32768) >> 16;
        *es_dst = u32x4{__builtin_bit_cast(unsigned, em), (unsigned)(-h), (unsigned)(-(sum - (h << 16))), 0u};
    }
}

constexpr int kMaxKSplit = 16;  // CHK split-K: most K slices

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup shapes. COOP kernels stage the whole K slice of x once per
// workgroup into shared LDS with every lane of every wave, behind one
// barrier (single-block tokens, when the slice fits); up to 16 waves for one
// source (128 VGPRs each) or 8 for two. The fallback stages per wave, in
// chunks, with 4 waves (256 VGPRs).
template <int NSRC, bool COOP>
constexpr int kMaxWavesFor = COOP ? (NSRC == 1 ? 16 : 12) : 4;
constexpr int kMaxTilesPerWg = 4;  // COOP: tiles one workgroup may own
// COOP: ring slots issued before the staging barrier (or, per-wave staging,
// before the staging): more would keep the barrier waiting for waves stalled
// at a full memory queue; fewer delay the weight stream
constexpr int kRingBeforeBarrier = 2;

constexpr int kCoopRounds = 4;  // x staging rounds per staging wave in COOP kernels
// (silu(a) * b holds a and b until staging: two rounds, within the registers)
template <int XM>
constexpr int coop_rounds = XM == XM_SILU ? 2 : kCoopRounds;
// CHK kernels: consecutive groups per wave per K chunk (the ring depth); 3
// and 4 measured slower (32 INT8 tokens: 84 and 119 against 65 us)
constexpr int kChunkSlots = 2;
// CHK kernels: x staging rounds per wave per chunk. One for one source (16
// waves cover a chunk of 16 tokens in one round): the next chunk's x is held
// in registers across the compute, and a second round made the 16-token
// kernels spill (each spill reload is a scratch load, whose wait drains
// every load in flight).
template <int NSRC>
constexpr int kChunkRounds = NSRC == 1 ? 1 : 2;
// CHK kernels: waves per workgroup. Four token blocks (16 tokens) take
// fewer than the other cooperative kernels so that they fit the registers
// without spills (at most 170 VGPRs with 12 waves, 256 with 8); fewer
// blocks keep 16 / 12.
template <int NSRC, int MB>
constexpr int kChunkWaves = MB >= 4 ? (NSRC == 1 ? 12 : 8) : (NSRC == 1 ? 16 : 12);
constexpr int kScaleUnits = 16;  // groups per wave covered by the COOP scale block (two loads per source)

// Prefetch ring depth: the registers of weights in flight per lane, about 24
// under a 128-VGPR budget (16-wave workgroups) and 40 for the dual kernel
// (3 waves per SIMD, so every gate/up tile of a 7B layer is resident at once).
template <int FMT, int NSRC, int SPU, bool COOP>
constexpr int ring_depth() {
    constexpr int WPU = (is_i8(FMT)) ? 4 * SPU : 2 * SPU;
    // (COOP keeps the depth it had with the scale in the ring: rings of 6
    // and 8 measured slower, more registers and more loads queued at issue)
    constexpr int RPU = NSRC * (WPU + (is_i8(FMT) ? 0 : 1));
    constexpr int budget = (COOP && NSRC == 2) ? 40 : 24;
    return (budget / RPU) < 2 ? 2 : ((budget / RPU) > 6 ? 6 : (budget / RPU));
}

// CM (staging mode): 0 = per-wave chunks (fallback), 1 = cooperative with
// staging waves, 2 = cooperative, each wave staging its own groups, 3 =
// cooperative in K chunks (several token blocks: all waves stage each chunk,
// each wave computes kChunkSlots consecutive groups of every chunk).
template <int FMT, int NSRC, int XM, int MB, int SPU, bool PERM, int CM>
__global__ __launch_bounds__((64 * (CM == 3 ? kChunkWaves<NSRC, MB> : kMaxWavesFor<NSRC, (CM != 0)>))) void qmv_kernel(Params p) {
    constexpr bool COOP = CM != 0;
    constexpr bool CHK = CM == 3;
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int D = CHK ? kChunkSlots : ring_depth<FMT, NSRC, SPU, COOP>();
    constexpr int DPRE = kRingBeforeBarrier < D ? kRingBeforeBarrier : D;  // COOP: slots before the barrier
    constexpr int IPU = 4 * SPU;                              // 16-k items per group and token
    constexpr int WPU = (is_i8(FMT)) ? 4 * SPU : 2 * SPU;  // weight dwords per lane per group
    // staging rounds per lane: per-wave chunk (fallback) or whole slice (COOP)
    constexpr int RMAX = CHK ? kChunkRounds<NSRC> : (COOP ? coop_rounds<XM> : (4 * MB * IPU + 63) / 64);

    constexpr bool SCB = (CM == 1 || CM == 2) && !is_i8(FMT);  // per-wave scale block (see below)
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int q = lane >> 4;  // k-chunk of the operands; token within a 4-token block
    const int c = lane & 15;  // A row / B column
    const int M = p.M, K = p.K, N = p.N, RB = p.rb;
    const int NW = p.nwaves;

    // Workgroups are dealt to the 8 XCDs round-robin; give each XCD a
    // contiguous run of tiles so neighbouring tiles share L2 lines.
    // COOP: workgroup r owns tiles [t0, t0 + TB) (TB >= 1; more than one when
    // N has more tiles than the grid has workgroups, so x is staged once for
    // them all); compute wave cw serves tile t0 + cw % TB, K slice cw / TB.
    // Fallback: one tile per workgroup.
    // CHK split-K: workgroup blockIdx.x = ksp * G + b takes K slice ksp of
    // tile group b
    const int KS = CHK ? p.ksplit : 1;
    const int G = gridDim.x / KS;
    const int b = blockIdx.x % G;
    const int ksp = blockIdx.x / G;
    const int r_wg = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
    // (32-bit divisions: the host keeps ntiles * G below 2^31 when G < ntiles)
    const bool multi = COOP && G != p.ntiles;
    const int t0 = multi ? (int)((unsigned)(r_wg * p.ntiles) / (unsigned)G) : r_wg;
    const int TB = multi ? (int)((unsigned)((r_wg + 1) * p.ntiles) / (unsigned)G) - t0 : 1;
    // COOP: waves [0, NS) only stage x (at most RMAX rounds of 64 items
    // each); the others split the tiles' K. Fallback: every wave stages its
    // own chunk.
    constexpr bool PW = CM == 2;  // per-wave staging of the wave's own groups, no staging waves
    const int CH = (COOP && !CHK) ? p.units : p.chunk;  // units the A region holds
    const int NS = (CM == 1) ? p.nstage : 0;  // host: ceil(items / 64 RMAX) <= NS <= NW - TB
    const int cw = wave - NS;             // compute-wave index (< 0: a staging wave)
    // compute waves per tile; the rest idle (CHK: fixed by the chunk, CH =
    // WPT * D, for every workgroup; waves beyond TB * WPT only stage)
    const int WPT = CHK ? p.chunk / D : (NW - NS) / TB;
    const int tj = cw >= 0 ? cw % TB : 0;  // tile slot of this wave
    const int ks = cw >= 0 ? cw / TB : WPT;  // K slice of this wave (WPT: none)
    const int tile = t0 + tj;
    const int n0 = tile * kTileN;
    const int ncol = min(n0 + c, N - 1);  // clamped column this lane loads

    // CHK: this workgroup's K slice of groups [ku0, ku1)
    const int ku0 = CHK ? (int)((unsigned)(ksp * p.units) / (unsigned)KS) : 0;
    const int ku1 = CHK ? (int)((unsigned)((ksp + 1) * p.units) / (unsigned)KS) : p.units;
    // contiguous K slice [u0, u1) (CHK: none; see its loop)
    const int u0 = (ks < WPT && !CHK) ? (int)((unsigned)(ks * p.units) / (unsigned)WPT) : 0;
    const int u1 = (ks < WPT && !CHK) ? (int)((unsigned)((ks + 1) * p.units) / (unsigned)WPT) : 0;
    int SW = PW ? u1 - u0 : CH;  // units staged by the staging rounds (CHK: per chunk)
    int items = M * SW * IPU;

    // LDS: A operands [unit][step][mb][q][row] (16 B each), per (unit, token)
    // 2^-e, -H, -L (sum(X) = H*65536 + L), zero points [unit][src][column].
    // COOP: one region for the workgroup, units = all groups; fallback: one
    // region per wave, units = one chunk (zero table: the wave's groups).
    const int ZU = COOP ? p.units : (u1 - u0);
    unsigned char *region = smem + (COOP ? 0 : (size_t)wave * p.wave_lds);
    u32x4 *abuf = reinterpret_cast<u32x4 *>(region);
    const int afrags = CH * SPU * MB * 4 * RB;
    // per (unit, token): {2^-e bits, -H, -L, 0}, one 16-byte read in the epilogue
    u32x4 *s_es = abuf + afrags;
    unsigned char *s_z = reinterpret_cast<unsigned char *>(s_es + CH * M);
    const int zbase = COOP ? 0 : u0;  // unit index of s_z row 0
    // COOP scale table: [wave][src][group - u0 (< kScaleUnits = 16)][16 columns], after the reduction area
    uint16_t *s_sc = reinterpret_cast<uint16_t *>(smem + (size_t)p.wave_lds + (size_t)NW * NSRC * MB * 64 * sizeof(float));

    // ------------------------------------------- zero points (before all loads)
    bool have_z[NSRC];
#pragma unroll
    for (int src = 0; src < NSRC; ++src) have_z[src] = !is_i8(FMT) && p.qz[src] != nullptr;
    if constexpr (!is_i8(FMT)) {
        if (have_z[0]) {
            // [tile slot][unit][src][column]; PW: each wave its own tile and
            // groups; CHK: the workgroup's K slice [ku0, ku1) of every tile
            const int zs = CHK ? ku1 - ku0 : ZU;  // units filled per tile
            const int nz = PW ? (u1 - u0) * NSRC * 16 : TB * zs * NSRC * 16;
            const int first = (COOP && !PW) ? tid : lane, stride = (COOP && !PW) ? 64 * NW : 64;
            for (int i0 = first; i0 < nz; i0 += stride) {
                const int i = PW ? (tj * ZU + u0) * NSRC * 16 + i0
                                 : (CHK ? ((i0 / (zs * NSRC * 16)) * ZU + ku0) * NSRC * 16 + i0 % (zs * NSRC * 16) : i0);
                const int col = i & 15, src = (i >> 4) % NSRC, uz = (i / (16 * NSRC)) % ZU, tz = i / (16 * NSRC * ZU);
                const int zc = min((t0 + tz) * kTileN + col, N - 1);
                const unsigned w = p.qz[src][(size_t)(zbase + uz) * (N >> 3) + (zc >> 3)];
                s_z[i] = (unsigned char)(((w >> (4 * (zc & 7))) & 0xF) + p.zoff);
            }
            wait_vm_all();  // nothing may be in flight across this branch
        }
    }

    // ------------------------------------------------------- weight loads
    struct Unit {
        unsigned w[NSRC][WPU];
        unsigned short s[NSRC];
    };
    // tiled layout: one buffer resource per source (separate variables: an
    // array of resources loses the kernel's host stub)
    const __amdgpu_buffer_rsrc_t rq0 = __builtin_amdgcn_make_buffer_rsrc((void *)p.qw[0], (short)0, 0x7FFFFFFF, kBufWord3);
    const __amdgpu_buffer_rsrc_t rq1 =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.qw[NSRC - 1], (short)0, 0x7FFFFFFF, kBufWord3);
    const __amdgpu_buffer_rsrc_t rw8 = __builtin_amdgcn_make_buffer_rsrc((void *)p.w8, (short)0, 0x7FFFFFFF, kBufWord3);
    // !live: an empty ring slot (u is then a clamped valid group; the tiled
    // layout skips the memory access, the others read that group again)
    auto load_unit = [&](Unit &U, int u, bool live) {
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
            if constexpr (FMT == FMT_I4) {
#pragma unroll
                for (int st = 0; st < SPU; ++st)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const size_t pr = (size_t)u * (p.gs >> 3) + st * 8 + 2 * q + h;
                        U.w[src][2 * st + h] = __builtin_nontemporal_load(p.qw[src] + pr * N + ncol);
                    }
            } else if constexpr (FMT == FMT_I4T) {
                const unsigned off = live ? (unsigned)(((tile * p.units + u) * 64 + lane) * WPU * 4) : kNoLoad;
                const __amdgpu_buffer_rsrc_t rq = src == 0 ? rq0 : rq1;
                if constexpr (WPU == 2) {
                    const u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(rq, off, 0, ring_cache_policy<NSRC>);
                    U.w[src][0] = t.x;
                    U.w[src][1] = t.y;
                } else {
#pragma unroll
                    for (int j = 0; j < WPU; j += 4) {
                        const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rq, off + j * 4, 0, ring_cache_policy<NSRC>);
                        U.w[src][j] = t.x;
                        U.w[src][j + 1] = t.y;
                        U.w[src][j + 2] = t.z;
                        U.w[src][j + 3] = t.w;
                    }
                }
            } else if constexpr (FMT == FMT_I8T) {
                // tile T, group u, lane (q, c): 32 contiguous bytes, k = 128 u
                // + 16 q + 64 st + j (st_int8_repack); a wave reads 2 KiB
                const unsigned off = live ? (unsigned)(((tile * p.units + u) * 64 + lane) * 32) : kNoLoad;
#pragma unroll
                for (int st = 0; st < SPU; ++st) {
                    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rw8, off + 16 * st, 0, ring_cache_policy<NSRC>);
                    U.w[src][4 * st] = t.x;
                    U.w[src][4 * st + 1] = t.y;
                    U.w[src][4 * st + 2] = t.z;
                    U.w[src][4 * st + 3] = t.w;
                }
            } else {
                const unsigned off = live ? (unsigned)(ncol * K + u * 128 + 16 * q) : kNoLoad;
#pragma unroll
                for (int st = 0; st < SPU; ++st) {
                    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rw8, off + 64 * st, 0, ring_cache_policy<NSRC>);
                    U.w[src][4 * st] = t.x;
                    U.w[src][4 * st + 1] = t.y;
                    U.w[src][4 * st + 2] = t.z;
                    U.w[src][4 * st + 3] = t.w;
                }
            }
            if constexpr (!is_i8(FMT) && !SCB) U.s[src] = p.sc[src][(size_t)u * N + ncol];
        }
    };

    Unit ring[D];

    // ------------------------------------------------------ x staging
    // Round r of wave w covers the 64 items of row w + NS r in COOP kernels
    // (waves [0, NS) stage everything, the others only stream weights), of
    // row r in the fallback (each wave its own chunk); item i = row * 64 +
    // lane is token m = i / (CH*IPU), group cs + (i % (CH*IPU)) / IPU, 16 k of
    // it. Every lane of a wave with items in a round loads (absent items read
    // a clamped valid address).
    const int span = COOP ? 64 * NW : 64;
    const int tt = COOP ? tid : lane;
    const int rstep = CHK ? NW : ((COOP && !PW) ? NS : 1);  // row stride between rounds
    const int wave0 = (COOP && !PW) ? wave : 0;  // row of round 0
    int uend = (COOP && !PW) ? p.units : u1;  // staged groups end here (CHK: per chunk)
    float xv[RMAX][16];
    float xb[XM == XM_SILU ? RMAX : 1][16];  // silu(a) * b: b
    // A wave with no item in a round skips it (loads and work): the branch
    // is uniform per wave and the same condition guards the loads and their
    // only consumer, stage().
    auto xload = [&](int cs) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            const int row = wave0 + r * rstep;
            if (row * 64 >= items) continue;
            const int i = min(row * 64 + lane, items - 1);
            int m = 0, w = i;
            if (M > 1) {
                m = i / (SW * IPU);
                w = i - m * (SW * IPU);
            }
            const int u = min(cs + w / IPU, uend - 1);
            load_x16<XM, PERM>(p, m, u * p.gs + 16 * (w % IPU), xv[r], xb[XM == XM_SILU ? r : 0]);
        }
    };
    auto stage = [&](int cs) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            const int row = wave0 + r * rstep;
            if (row * 64 >= items) continue;  // uniform per wave
            const int i = row * 64 + lane;
            int m = 0, w = i;
            if (M > 1) {
                m = i / (SW * IPU);
                w = i - m * (SW * IPU);
            }
            const int ui = w / IPU, ii = w % IPU;
            const int ua = (COOP && !CHK) ? cs + ui : ui;  // A-region unit (COOP: the group itself)
            const bool ok = i < items && cs + ui < uend;
            x_finish<XM, PERM>(xv[r], xb[XM == XM_SILU ? r : 0]);
            const int st = ii >> 2, qq = ii & 3;
            quantize_item<IPU, is_i8(FMT)>(xv[r], ok,
                                           abuf + (((size_t)(ua * SPU + st) * MB + (m >> 2)) * 4 + qq) * RB + 4 * (m & 3),
                                           ii == 0 ? &s_es[ua * M + m] : nullptr);
        }
    };

    // Rows of absent tokens must read as zero. COOP kernels (one token block)
    // have none, and every other row is written by exactly one staging item
    // (row 4t+3 included), so they need no fill: a fill by one wave would race
    // with the staging writes of the others, there being no barrier between.
    // The per-wave fallback zeroes its private region first (the same wave
    // writes both, in order).
    if constexpr (!COOP)
        for (int i = tt; i < afrags; i += span) abuf[i] = u32x4{0, 0, 0, 0};
    // CHK: rows of absent tokens (M not a multiple of 4) are zeroed once; no
    // staging item ever writes them, so this races with nothing.
    if constexpr (CHK)
        if (M < 4 * MB)
            for (int i = tid; i < afrags; i += 64 * NW)
                if ((i / (RB * 4)) % MB * 4 + (i % RB) / 4 >= M) abuf[i] = u32x4{0, 0, 0, 0};

    // --------------------------------------------------------- main loop
    float tot[NSRC][MB];
#pragma unroll
    for (int src = 0; src < NSRC; ++src)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) tot[src][mb] = 0.0f;

    const u32x4 *alane = abuf + q * RB + c;  // this lane's A operand of (unit 0, step 0, block 0)
    auto compute = [&](const Unit &U, int u, int ui) {
        v4i acc[NSRC][MB];
#pragma unroll
        for (int src = 0; src < NSRC; ++src)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[src][mb] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int st = 0; st < SPU; ++st) {
            v4i A[MB];
            // (several token blocks: RB = 16, every lane reads; its address
            // is the lane's base plus a constant per (st, mb))
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                A[mb] = (MB > 1 || c < RB) ? __builtin_bit_cast(v4i, alane[((ui * SPU + st) * MB + mb) * 4 * RB])
                                           : v4i{0, 0, 0, 0};
#pragma unroll
            for (int src = 0; src < NSRC; ++src) {
                v4i Bf;
                if constexpr (is_i8(FMT)) {
                    Bf = v4i{(int)U.w[src][4 * st], (int)U.w[src][4 * st + 1], (int)U.w[src][4 * st + 2],
                             (int)U.w[src][4 * st + 3]};
                } else {
                    const unsigned w0 = U.w[src][2 * st], w1 = U.w[src][2 * st + 1];
                    Bf = v4i{(int)(w0 & 0x0F0F0F0Fu), (int)((w0 >> 4) & 0x0F0F0F0Fu), (int)(w1 & 0x0F0F0F0Fu),
                             (int)((w1 >> 4) & 0x0F0F0F0Fu)};
                }
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[src][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mb], Bf, acc[src][mb], 0, 0, 0);
            }
        }
        // group epilogue: exact sum(q*X) - z*sum(X) as hi*65536 + lo, one
        // rounding to f32, then * s * 2^-e
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int m = min(mb * 4 + q, M - 1);
            const u32x4 es = s_es[ui * M + m];
            const float em = __builtin_bit_cast(float, (unsigned)es.x);  // (a prvalue: bit_cast of a vector element lvalue reads element 0)
            const int nh = (int)es.y, nl = (int)es.z;
#pragma unroll
            for (int src = 0; src < NSRC; ++src) {
                const v4i S = acc[src][mb];
                float f;
                int z = 0;
                if constexpr (is_i8(FMT)) {
                    f = em;
                } else {
                    const uint16_t sh = SCB ? s_sc[(wave * NSRC + src) * 256 + (u - u0) * 16 + c] : U.s[src];
                    f = (float)__builtin_bit_cast(_Float16, sh) * em;
                    z = have_z[src] ? (int)s_z[((tj * ZU + u - zbase) * NSRC + src) * 16 + c] : 8;
                }
                const int hi = S.x + __mul24(z, nh);
                const int lo = (S.y << 8) + S.z + __mul24(z, nl);
                tot[src][mb] = fmaf(fmaf((float)hi, 65536.0f, (float)lo), f, tot[src][mb]);
            }
        }
    };

    // Fallback only: at a chunk change (a wave's range exceeds one chunk:
    // several tokens and a long K) the chunk's x is loaded, waited for and
    // staged at once, so no load count differs across the branch and x is
    // not held in registers across the main loop.
    auto next_chunk = [&](int u) {
        xload(u);
        wait_vm_all();
        stage(u);
    };

    if constexpr (CHK) {
        // K in chunks of CH = WPT * D groups; in chunk cc, compute wave
        // (tile tj, slice ks) owns groups cc*CH + ks*D + d, d < D, which are
        // its ring slots. Per chunk: x of the next chunk is loaded (into
        // registers) before this chunk's groups are computed and the ring
        // is refilled with the next chunk's groups; then all waves stage the
        // next chunk between two bare barriers (the ring stays in flight).
        // Every load is unconditional (the last chunk's x is loaded again
        // at the end; groups past K are empty slots).
        const int nch = (ku1 - ku0 + CH - 1) / CH;
        int cs = ku0;
        auto set_chunk = [&](int cc) {
            cs = ku0 + cc * CH;
            uend = min(cs + CH, ku1);
            SW = uend - cs;
            items = M * SW * IPU;
        };
        const bool comp = ks < WPT;  // a compute wave (others only stage)
        set_chunk(0);
        xload(cs);
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int u = ku0 + ks * D + d;
            load_unit(ring[d], min(u, ku1 - 1), comp && u < ku1);
        }
        stage(cs);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        for (int cc = 0; cc < nch; ++cc) {
            set_chunk(min(cc + 1, nch - 1));
            xload(cs);
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int u = ku0 + cc * CH + ks * D + d;
                if (comp && u < ku1) compute(ring[d], u, u - ku0 - cc * CH);
                const int un = u + CH;
                load_unit(ring[d], min(un, ku1 - 1), comp && cc + 1 < nch && un < ku1);
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // chunk cc's A operands are free
            if (cc + 1 < nch) stage(cs);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // chunk cc + 1 is staged
        }
    } else {
    // COOP: the staging waves load x, wait for it and stage it; they issue no
    // weight load, so neither x nor the staging queues behind the weight
    // stream at the CU's memory port, and the other waves start streaming at
    // once. Nothing is in flight across the branch. Fallback: x first (loads complete in issue order),
    // then the ring, then the staging.
    const int cs0 = (COOP && !PW) ? 0 : u0;
    if (COOP && !PW && wave < NS) {
        xload(cs0);
        wait_vm_all();
        stage(cs0);
    }
    if (PW) xload(cs0);  // (a wave without groups has no items: uniform skip inside)
    // per-wave staging: every wave's x loads enter the CU's memory queue
    // before any weight load (the waves of a workgroup start up to ~0.6 us
    // apart, and a late wave's x would otherwise wait behind the early
    // waves' weights: configs[4] down 7.2 -> 6.8 us); a bare barrier (no
    // wait for loads), met by every wave
    if constexpr (PW) asm volatile("s_barrier" ::: "memory");
    if (!COOP && u0 < u1) xload(cs0);
    // COOP GPTQ: the scales of the wave's (at most kScaleUnits) groups for
    // the tile's 16 columns in two 4-byte loads per lane and source (lane l,
    // load h: group u0 + 8h + l / 8, columns 2 (l % 8) and +1; lanes past the
    // wave's groups load nothing), instead of one 2-byte load per group in
    // the ring. Issued before the ring, so waiting for them never waits for
    // the ring; parked in LDS before the barrier.
    unsigned scw[NSRC][2];
    if constexpr (SCB) {
        const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc((void *)p.sc[0], (short)0, 0x7FFFFFFF, kBufWord3);
        const __amdgpu_buffer_rsrc_t rs1 =
            __builtin_amdgcn_make_buffer_rsrc((void *)p.sc[NSRC - 1], (short)0, 0x7FFFFFFF, kBufWord3);
        const int cl = min(n0 + 2 * (lane & 7), N - 2);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int ug = u0 + 8 * h + (lane >> 3);
            const unsigned off = ug < u1 ? (unsigned)(((size_t)ug * N + cl) * 2) : kNoLoad;
#pragma unroll
            for (int src = 0; src < NSRC; ++src)
                scw[src][h] = __builtin_amdgcn_raw_buffer_load_b32(src == 0 ? rs0 : rs1, off, 0, 0);
        }
    }
    // COOP: issued by every wave (waves without groups issue only empty
    // slots, which access no memory): a branch here would make the compiler
    // wait for the whole ring wherever it waits for the scales.
    if (COOP || u0 < u1) {
#pragma unroll
        for (int d = 0; d < (COOP ? DPRE : D); ++d)
            load_unit(ring[d], min(u0 + d, max(u1 - 1, 0)), u0 + d < u1);
    }
    if (!COOP && u0 < u1) stage(cs0);
    if constexpr (PW) {
        stage(cs0);
#pragma unroll
        for (int d = DPRE; d < D; ++d) load_unit(ring[d], min(u0 + d, max(u1 - 1, 0)), u0 + d < u1);
    } else if constexpr (COOP) {
        // The staged x (and the zero table) are complete: this wave's LDS
        // writes have landed (lgkmcnt(0)) and every wave has arrived. Not
        // __syncthreads(): its release fence also waits for every load in
        // flight (vmcnt(0)), i.e. for the ring. The asm's memory clobber
        // keeps the compiler from moving LDS accesses across it.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // the rest of the ring, after the barrier: issuing it can stall while
        // the CU's memory queue is full, and that must not hold up the barrier
#pragma unroll
        for (int d = DPRE; d < D; ++d) load_unit(ring[d], min(u0 + d, max(u1 - 1, 0)), u0 + d < u1);
    }
    if constexpr (SCB) {  // the wave's own scale table: no barrier needed
#pragma unroll
        for (int src = 0; src < NSRC; ++src)
#pragma unroll
            for (int h = 0; h < 2; ++h) reinterpret_cast<unsigned *>(s_sc)[(wave * NSRC + src) * 128 + h * 64 + lane] = scw[src][h];
    }
    if (u0 < u1) {
        int ui = COOP ? u0 : 0;  // A-buffer index of the current group
        int base = u0;
        for (; base + D <= u1; base += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int u = base + d;
                if (!COOP && ui == CH) {
                    ui = 0;
                    next_chunk(u);
                }
                compute(ring[d], u, ui);
                ++ui;
                load_unit(ring[d], min(u + D, u1 - 1), u + D < u1);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {  // tail: fewer than D groups left, all in the ring
            const int u = base + d;
            if (u < u1) {
                if (!COOP && ui == CH) {
                    ui = 0;
                    next_chunk(u);
                }
                compute(ring[d], u, ui);
                ++ui;
            }
        }
    }

    }

    // ------------------------------------------- reduce the waves, write y
    float *red = reinterpret_cast<float *>(smem + (COOP ? (size_t)p.wave_lds : (size_t)NW * p.wave_lds));
#pragma unroll
    for (int src = 0; src < NSRC; ++src)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) red[((wave * NSRC + src) * MB + mb) * 64 + lane] = tot[src][mb];
    __syncthreads();
    // split K with the reduction fused (p.cnt): every slice writes its
    // partial through to memory (sc0 sc1 stores, completed before the
    // counter), the last of the tile group's slices to count in adds them in
    // slice order and writes y. Nobody waits for anybody.
    const bool fused = CHK && KS > 1 && p.cnt != nullptr;
    if (!fused && wave >= TB) {
        return;
    }  // wave j (< TB) sums the K slices of tile t0 + j, in slice order
    const int n = (t0 + wave) * kTileN + c;  // column of tile t0 + wave
    const __amdgpu_buffer_rsrc_t rpart =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.part, (short)0, 0x7FFFFFFF, kBufWord3);
    constexpr int kCoherent = 1 | 16;  // sc0 sc1: write through / read past this XCD's L2
#pragma unroll
    for (int mb = 0; mb < MB && wave < TB; ++mb) {
        const int m = mb * 4 + q;
        float v[NSRC];
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
            // the WPT slices of the tile, in slice order: every read issued
            // before the first add (a loop of dependent LDS reads costs ~0.05
            // us a slice), slots past the last slice masked to +0
            constexpr int SMAX = CM == 3 ? kChunkWaves<NSRC, MB> : kMaxWavesFor<NSRC, (CM != 0)>;
            float r[SMAX];
#pragma unroll
            for (int k = 0; k < SMAX; ++k) {
                const int w = min(wave + k * TB, TB * WPT - 1);
                r[k] = red[(((NS + w) * NSRC + src) * MB + mb) * 64 + lane];
            }
            float a = 0.0f;
#pragma unroll
            for (int k = 0; k < SMAX; ++k)
                a += __builtin_bit_cast(float, __builtin_bit_cast(unsigned, r[k]) & (k < WPT ? ~0u : 0u));
            v[src] = a;
        }
        if (m >= M || n >= N) continue;
        if (KS > 1) {  // split-K partial: the reduce (fused below, or a kernel) applies the epilogue
#pragma unroll
            for (int src = 0; src < NSRC; ++src) {
                const unsigned off = (unsigned)(((((size_t)ksp * NSRC + src) * M + m) * N + n) * 4);
                if (fused)
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v[src]), rpart, off, 0, kCoherent);
                else
                    p.part[(((size_t)ksp * NSRC + src) * M + m) * N + n] = v[src];
            }
            continue;
        }
        float out = v[0];
        if constexpr (NSRC == 2) out = silu_f(v[0]) * v[1];
        if constexpr (is_i8(FMT)) out *= p.scale8[n];
        p.y[(size_t)m * N + n] = out;
    }
    // Why the slices' partials are visible to the last one without a
    // release/acquire pair in the source: the partials are stored with sc0
    // sc1 (system coherence: written through this XCD's L2 to memory, no dirty
    // line left behind) and read back with sc0 sc1 (past the L2, from the
    // point of coherence); gfx9 counts stores in vmcnt and returns a
    // write-through store's count only when the write is acknowledged there,
    // so vmcnt(0) then the workgroup barrier put every wave's partials in
    // memory before thread 0's counter add, and the adds themselves are
    // performed at the point of coherence (system scope), so the slice that
    // reads KS - 1 comes after every other slice's partials. This is the
    // sequence the compiler emits for a system-scope release of such stores,
    // less its L2 write-back (buffer_wbl2), which has nothing to write here,
    // and its acquire's L2 invalidate, which the sc0 sc1 loads do not need;
    // both cost microseconds per launch on MI355X. The asm statements carry
    // memory clobbers, so the compiler keeps every access on its side.
    if (fused) {
        __shared__ unsigned s_last;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partials are in memory
        __syncthreads();
        if (tid == 0) {
            const unsigned done = __hip_atomic_fetch_add(&p.cnt[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            s_last = done == (unsigned)KS - 1;
            if (s_last)  // every slice has counted in: clear for the next call
                __hip_atomic_store(&p.cnt[b], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        __syncthreads();
        if (s_last && wave < TB) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int m = mb * 4 + q;
                if (m >= M || n >= N) continue;
                float v[NSRC];
#pragma unroll
                for (int src = 0; src < NSRC; ++src) {
                    // every slice's load in flight at once (slots past KS read
                    // nothing: an offset past the buffer), then the adds in order
                    unsigned r[kMaxKSplit];
#pragma unroll
                    for (int k = 0; k < kMaxKSplit; ++k)
                        r[k] = __builtin_amdgcn_raw_buffer_load_b32(
                            rpart, k < KS ? (unsigned)(((((size_t)k * NSRC + src) * M + m) * N + n) * 4) : kNoLoad, 0,
                            kCoherent);
                    float a = 0.0f;
#pragma unroll
                    for (int k = 0; k < kMaxKSplit; ++k) a += __builtin_bit_cast(float, r[k] & (k < KS ? ~0u : 0u));
                    v[src] = a;
                }
                float out = v[0];
                if constexpr (NSRC == 2) out = silu_f(v[0]) * v[1];
                if constexpr (is_i8(FMT)) out *= p.scale8[n];
                p.y[(size_t)m * N + n] = out;
            }
        }
    }
}

// CHK split-K: y[m, n] = epilogue(sum over s < S of part[s][src][m][n]), the
// slices added in a fixed order (deterministic); the epilogue is the main
// kernel's (silu(g) * u for two sources, the INT8 scale).
template <int NSRC, bool I8>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *__restrict__ part,
                                                           const float *__restrict__ scale8, float *__restrict__ y,
                                                           int M, int N, int S) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    const int MN = M * N;
    if (idx >= MN) return;
    // Every slice's load is issued before the first add (a loop of load,
    // wait, add paid one memory latency per slice); the adds keep slice order.
    float t[kMaxKSplit][NSRC];
#pragma unroll
    for (int s = 0; s < kMaxKSplit; ++s)
#pragma unroll
        for (int src = 0; src < NSRC; ++src) t[s][src] = s < S ? part[(size_t)(s * NSRC + src) * MN + idx] : 0.0f;
    float v[NSRC];
#pragma unroll
    for (int src = 0; src < NSRC; ++src) v[src] = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxKSplit; ++s)
        if (s < S)
#pragma unroll
            for (int src = 0; src < NSRC; ++src) v[src] += t[s][src];
    float out = v[0];
    if constexpr (NSRC == 2) out = silu_f(v[0]) * v[1];
    if constexpr (I8) out *= scale8[idx % N];
    y[idx] = out;
}

// ----------------------------------------------------------------- host side

// MFMA token blocks of 4 per launch (calls run in blocks of at most 16 tokens)
inline int mb_for(int M) { return M <= 4 ? 1 : (M <= 8 ? 2 : 4); }

// Bytes of one staged group (A operands, scalars, zero table row).
template <int FMT, int NSRC, int MB, int SPU>
inline size_t unit_bytes(const Params &p) {
    return (size_t)SPU * MB * 4 * p.rb * 16 + (size_t)p.M * 16 + (is_i8(FMT) ? 0 : (size_t)NSRC * 16);
}

template <int FMT, int NSRC, int XM, int MB, int SPU, bool PERM, int CM>
int launch_kernel(st_context *ctx, Params &p, size_t lds) {
    auto kern = qmv_kernel<FMT, NSRC, XM, MB, SPU, PERM, CM>;
    if (lds > 64 * 1024)
        ST_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    st::launch(ctx, kern, dim3(p.grid), dim3(64 * p.nwaves), lds, p);
    return launch_check("qmv_kernel");
}

// COOP kernels run one workgroup per CU (one tile each when there are no more
// tiles than CUs, else a CU's run of tiles), so they may take nearly all of
// its 160 KiB: two tokens on Llama-7B's down (86 groups, ~100 KiB of staged x)
// fit only above the former 96 KiB.
constexpr size_t kCoopLdsBudget = 152 * 1024;
constexpr size_t kChunkLdsBudget = 150 * 1024;  // one workgroup per CU
constexpr int kSplitTiles = 4;  // CHK split-K: tiles per workgroup
constexpr int kSplitTilesPerCu = 1;  // CHK: split K when the grid has at most this many tiles per CU
constexpr int kSplitMinUnits1 = 48;  // CHK, one token block: split only K of at least this many groups
constexpr int kLongK12Waves = 8192;  // one-tile GPTQ decode: K from which 12 waves per workgroup beat 16

// The K-chunked cooperative kernel (CM 3) for several tokens: a workgroup
// per CU owning 2..kMaxTilesPerWg tiles, or (split) groups of kSplitTiles
// tiles with K split across workgroups. Returns -1 when the shape does not
// fit it (nothing launched, p unchanged).
template <int FMT, int NSRC, int XM, int MB, int SPU, bool PERM>
int launch_chk(st_context *ctx, Params &p, bool split, int ncu, int tiles_cu) {
    constexpr int IPU = 4 * SPU;
    int grid, tpw, ks = 1;
    if (!split) {
        grid = tiles_cu <= kMaxTilesPerWg ? ncu : (p.ntiles + kMaxTilesPerWg - 1) / kMaxTilesPerWg;
        tpw = (p.ntiles + grid - 1) / grid;
    } else {
        // Fewer tiles than CUs: groups of kSplitTiles tiles share
        // their x, and K is split into slices so that the grid fills
        // the CUs (each slice stages only its part of x); f32
        // partials in the workspace, then split_reduce_kernel.
        tpw = std::min(kSplitTiles, p.ntiles);
        grid = (p.ntiles + tpw - 1) / tpw;
        ks = std::max(1, std::min({ncu / grid, kMaxKSplit, p.units / 2}));
        if (tune(ctx, ST_TUNE_NO_KSPLIT, 0)) ks = 1;
        const size_t need = (size_t)ks * NSRC * p.M * p.N * sizeof(float);
        if (ks > 1 && (need > ctx->ws_bytes || !ctx->ws)) ks = 1;
    }
    // compute waves per tile: as many as the waves allow, and no more
    // than one chunk's staging (kChunkRounds rounds of all waves) covers
    const int nw = kChunkWaves<NSRC, MB>;
    const int cap = (int)(64ll * kChunkRounds<NSRC> * nw / ((long long)p.M * IPU * kChunkSlots));
    const int wpt = std::min(nw / tpw, cap);
    const int ch = wpt * kChunkSlots;
    const size_t a_bytes = (size_t)ch * ((size_t)SPU * MB * 4 * p.rb * 16 + (size_t)p.M * 16);
    const size_t region =
        (a_bytes + (!is_i8(FMT) ? (size_t)tpw * p.units * NSRC * 16 : 0) + 15) & ~size_t(15);
    const size_t lds = region + (size_t)nw * NSRC * MB * 64 * sizeof(float);
    if ((long long)p.ntiles * grid < (1ll << 31) && wpt >= 1 &&
        (long long)p.M * ch * IPU <= 64ll * kChunkRounds<NSRC> * nw && lds <= kChunkLdsBudget) {
        p.nwaves = nw;
        p.tpw = tpw;
        p.grid = grid * ks;
        p.chunk = ch;
        p.nstage = 0;
        p.wave_lds = (int)region;
        p.ksplit = ks;
        p.part = ks > 1 ? ctx->ws : nullptr;
        // the reduction fused into the kernel (one counter per tile
        // group) for up to 8 tokens: graph replay, configs[4] down at 4
        // tokens 9.8 -> 8.9 us, Llama-7B down 11.9 -> 10.9, o and down at
        // 8 tokens 0.3-0.8 us faster; at 16 tokens the last slice's
        // reads (4 token blocks) cost more than the reduce launch
        // (0.2-0.6 us slower per call; the configs[4] stack at 16 tokens
        // 1950 us per step with the reduce launch, 2048 fused). Not when
        // the context has no counters or the setting asks for the reduce
        // kernel.
        const int fuse_dflt = MB <= 2 ? 0 : 1;
        p.cnt = (ks > 1 && ctx->split_counters && grid <= kSplitCounters &&
                 !tune(ctx, ST_TUNE_SPLIT_REDUCE_KERNEL, fuse_dflt))
                    ? ctx->split_counters
                    : nullptr;
        if (int rc = launch_kernel<FMT, NSRC, XM, MB, SPU, PERM, 3>(ctx, p, lds)) {
            // the counters must be zero for the next call; a launch that did
            // not go through may not have left them so (an error path, never
            // inside a capture that is to be replayed)
            if (p.cnt) (void)hipMemsetAsync(ctx->split_counters, 0, kSplitCounters * sizeof(unsigned), ctx->stream);
            return rc;
        }
        if (ks == 1 || p.cnt) return ST_OK;
        const int mn = p.M * p.N;
        st::launch(ctx, (split_reduce_kernel<NSRC, is_i8(FMT)>), dim3((mn + 255) / 256), dim3(256), 0, p.part, p.scale8, p.y, p.M, p.N, ks);
        return launch_check("split_reduce_kernel");
    }
    return -1;
}

template <int FMT, int NSRC, int XM, int MB, int SPU, bool PERM>
int launch_t(st_context *ctx, Params &p) {
    constexpr int IPU = 4 * SPU;
    p.rb = p.M >= 4 ? 16 : 4 * p.M;
    p.chunk = std::max(1, 64 / (p.M * IPU));
    // Waves per workgroup: aim at ~4 waves per SIMD over the whole grid
    // (each workgroup is one 16-column tile).
    // Several tokens: K-chunked cooperative staging (CM 3). Many tiles (and
    // several token blocks): a workgroup per CU owning 2..kMaxTilesPerWg
    // tiles; few tiles (at most kSplitTilesPerCu per CU): groups of
    // kSplitTiles tiles and K split across workgroups. One token block with
    // many tiles goes to the single-block kernels below.
    // (up to 16 tokens: calls with more run as 16-token blocks, and 8 token
    // blocks would not fit the registers)
    bool chk_last = false, split = false;  // the CHK kernel after the COOP one; its K split
    const int ncu = std::max(1, ctx->num_cus);
    const int tiles_cu = (p.ntiles + ncu - 1) / ncu;
    if constexpr (MB <= 4 && FMT != FMT_I4) {
        // (measured, configs[4] shapes: one token block splits only a long K,
        // down 17 -> 9.8 us at 4 tokens while o_proj, K = 4096, lost; four
        // blocks split up to 2 tiles per CU, qkv 18.4 -> 16.7 us at 16)
        const int split_max = tune(ctx, ST_TUNE_SPLIT_TILES_CU, MB >= 4 ? 2 : kSplitTilesPerCu);
        split = tiles_cu <= split_max && (MB > 1 || p.units >= kSplitMinUnits1);
        // (one token: the split costs more than it saves, configs[4] down
        // 7.2 -> 9.2 us with the reduce launch, 6.75 -> 8.8 us with the
        // reduction fused)
        if (p.M > 1 && (MB > 1 || split) && !tune(ctx, ST_TUNE_NO_CHUNK, 0)) {
            // Two tokens in one block: the one-tile COOP kernel below first
            // (Llama-7B down 9.8 -> 8.5 us, configs[4] down 8.3 -> 8.1; at 3
            // tokens they tie), this one when that does not fit
            if (MB == 1 && p.M == 2) {
                chk_last = true;
            } else if (const int rc = launch_chk<FMT, NSRC, XM, MB, SPU, PERM>(ctx, p, split, ncu, tiles_cu); rc != -1) {
                return rc;
            }
        }
    }
    const int want = (ctx->num_cus * 16) / std::max(1, p.ntiles);
    if constexpr (MB == 1 && FMT != FMT_I4) {
        constexpr int NWX = kMaxWavesFor<NSRC, true>;
        const long long items = (long long)p.M * p.units * IPU;
        // launches the COOP kernel with this shape if it fits; -1 = it does not.
        // Staging waves: as many as one round each needs (staging latency),
        // fewer (up to coop_rounds rounds each) when K needs the waves.
        auto try_coop = [&](int nw, int tpw, int grid) -> int {
            const size_t ub = unit_bytes<FMT, NSRC, MB, SPU>(p);
            const size_t region =
                (ub * p.units + (!is_i8(FMT) ? (size_t)(tpw - 1) * p.units * NSRC * 16 : 0) + 15) & ~size_t(15);
            const size_t lds = region + (size_t)nw * NSRC * MB * 64 * sizeof(float) +
                               (!is_i8(FMT) ? (size_t)nw * NSRC * 128 * sizeof(unsigned) : 0);
            if (lds > kCoopLdsBudget) return -1;
            p.nwaves = nw;
            p.tpw = tpw;
            p.grid = grid;
            p.wave_lds = (int)region;
            // Staging waves (mode 1): one round each, two when the workgroup
            // owns several tiles (more waves left for K). When they would
            // take 6 or more waves (long K) or stage the costly silu(a)*b,
            // each wave stages its own groups instead (mode 2): all waves
            // stream weights. ST_TUNE_STAGE_MODE / _ROUNDS override (tests, tuning).
            const int mode = tune(ctx, ST_TUNE_STAGE_MODE, 0);
            const int env_r = tune(ctx, ST_TUNE_STAGE_ROUNDS, 0);
            constexpr int CR = coop_rounds<XM>;
            const int r0 = env_r > 0 ? std::min(env_r, CR) : std::min(CR, tpw > 1 ? 2 : 1);
            const long long ns0 = (items + 64 * r0 - 1) / (64 * r0);
            const bool per_wave = mode == 2 || (mode == 0 && (ns0 >= 6 || XM == XM_SILU));
            if (!per_wave) {
                for (int rounds = r0; rounds <= CR; ++rounds) {
                    const long long ns = (items + 64 * rounds - 1) / (64 * rounds);
                    const long long wpt = (nw - ns) / tpw;  // compute waves per tile in the fullest workgroup
                    if (wpt < 1) continue;
                    if (!is_i8(FMT) && (p.units + wpt - 1) / wpt > kScaleUnits) continue;  // the scale block
                    p.nstage = (int)ns;
                    return launch_kernel<FMT, NSRC, XM, MB, SPU, PERM, 1>(ctx, p, lds);
                }
                if (mode == 1) return -1;
            }
            const int wpt = nw / tpw;
            if (wpt < 1) return -1;
            const int upw = (p.units + wpt - 1) / wpt;  // groups per wave
            if (!is_i8(FMT) && upw > kScaleUnits) return -1;
            if ((long long)p.M * upw * IPU > 64ll * CR) return -1;  // its staging rounds
            p.nstage = 0;
            return launch_kernel<FMT, NSRC, XM, MB, SPU, PERM, 2>(ctx, p, lds);
        };
        if (!tune(ctx, ST_TUNE_NO_COOP, 0)) {
            if (tiles_cu >= 2 && !tune(ctx, ST_TUNE_ONE_TILE, 0)) {
                // more tiles than CUs: a workgroup per CU (all the waves a CU
                // holds) owns 2..kMaxTilesPerWg tiles and stages x once for them
                // (every CU: a grid of ceil(ntiles / 3) even workgroups for
                // gate/up measured 11.9 against 11.2 us)
                const int grid = tiles_cu <= kMaxTilesPerWg ? ncu : (p.ntiles + kMaxTilesPerWg - 1) / kMaxTilesPerWg;
                if ((long long)p.ntiles * grid < (1ll << 31)) {
                    const int rc = try_coop(NWX, (p.ntiles + grid - 1) / grid, grid);
                    if (rc != -1) return rc;
                }
            }
            int nw = want >= 16 ? 16 : (want >= 8 ? 8 : 4);
            // GPTQ with a long K (per-wave staging): 12 waves, not 16, keep
            // more of each wave's weight stream in flight per SIMD (measured:
            // K = 11008 down 7.6 -> 7.4 us, K = 9728 6.6 -> 6.1 us, their silu
            // forms 0.8 us faster; K = 4096 is 0.4 us slower at 12)
            if (!is_i8(FMT) && nw == 16 && p.K >= kLongK12Waves) nw = 12;
            nw = std::max(4, std::min({nw, NWX, std::max(4, p.units)}));
            nw = std::max(4, std::min(NWX, tune(ctx, ST_TUNE_WAVES, nw)));
            // more waves when the staging waves leave too few for K (GPTQ:
            // at most kScaleUnits groups per wave, the scale block)
            for (;; nw = std::min(2 * nw, NWX)) {
                const int rc = try_coop(nw, 1, p.ntiles);
                if (rc != -1 || nw == NWX) {
                    if (rc != -1) return rc;
                    break;
                }
            }
        }
    }
    if constexpr (MB <= 4 && FMT != FMT_I4)
        if (chk_last)
            if (const int rc = launch_chk<FMT, NSRC, XM, MB, SPU, PERM>(ctx, p, split, ncu, tiles_cu); rc != -1) return rc;
    // fallback: per-wave chunked staging, 4 waves, one tile per workgroup
    const int nw = 4;
    p.nwaves = nw;
    p.tpw = 1;
    p.grid = p.ntiles;
    const int max_units = (p.units + nw - 1) / nw;
    if (!is_i8(FMT) && max_units > kMaxZeroUnits && (p.qz[0] || p.qz[1]))
        return fail(ST_ERR_SHAPE, "qmv: %d groups per wave exceed the zero-point table", max_units);
    const int afr = p.chunk * SPU * MB * 4 * p.rb;
    const int ztab = (is_i8(FMT)) ? 0 : std::min(max_units, kMaxZeroUnits) * NSRC * 16;
    p.wave_lds = (afr * 16 + p.chunk * p.M * 16 + ztab + 15) & ~15;
    const size_t lds = (size_t)nw * p.wave_lds + (size_t)nw * NSRC * MB * 64 * sizeof(float);
    return launch_kernel<FMT, NSRC, XM, MB, SPU, PERM, 0>(ctx, p, lds);
}

template <int FMT, int NSRC, int XM, int SPU, bool PERM>
int launch_mb(st_context *ctx, Params &p) {
    switch (mb_for(p.M)) {
        case 1: return launch_t<FMT, NSRC, XM, 1, SPU, PERM>(ctx, p);
        case 2: return launch_t<FMT, NSRC, XM, 2, SPU, PERM>(ctx, p);
        case 4:
            if (p.M <= 16) return launch_t<FMT, NSRC, XM, 4, SPU, PERM>(ctx, p);
            [[fallthrough]];
        default:
            return fail(ST_ERR_SHAPE, "qmv: %d tokens in one launch (at most 16)", p.M);
    }
}

template <int FMT, int NSRC, int XM, bool PERM>
int launch_gs(st_context *ctx, Params &p) {
    if constexpr (is_i8(FMT)) {
        return launch_mb<FMT, NSRC, XM, 2, PERM>(ctx, p);
    } else {
        switch (p.gs) {
            case 64: return launch_mb<FMT, NSRC, XM, 1, PERM>(ctx, p);
            case 128: return launch_mb<FMT, NSRC, XM, 2, PERM>(ctx, p);
            case 256: return launch_mb<FMT, NSRC, XM, 4, PERM>(ctx, p);
        }
        return fail(ST_ERR_SHAPE, "qmv: group size %d", p.gs);
    }
}

// Entry used by qmv.hip; specialised per (format, act-order) in
// qmv_i4_p{0,1}.hip, qmv_i4t_p{0,1}.hip, qmv_i8.hip and qmv_i8t.hip so the
// variants compile in parallel.
template <int FMT, bool PERM>
int dispatch(st_context *ctx, Params &p, int nsrc, int xm);

}  // namespace qmv
}  // namespace st

#include "qmv_stream.hpp"

namespace st {
namespace qmv {

// 1-4 tokens on tiled weights: the streaming kernel (qmv_stream.hpp) for
//  * gate/up (two sources) from 2 tiles per CU on, with 8-wave workgroups
//    (graph replay, one token: Llama-7B 4096 x 2 x 11008 12.2 -> 10.4-11.1
//    us; configs[4] 2560 x 2 x 9728 9.1-9.3 -> 7.7-8.2 us; at 4 tokens 16.8
//    -> 13.0 us);
//  * one source from kStreamMinTilesCu tiles per CU on, with 16-wave
//    workgroups (the int4 lm_head 2560 x 151936, 37 tiles per CU: 51 ->
//    39-42 us, 65 -> 43 us at 4 tokens; 8 waves are 1.5-2 us slower);
//  * one source with 2-4 tokens from 2 tiles per CU on, with 8-wave
//    workgroups (4096 x 11008: 9.0 / 11.5 / 14.6-15.1 -> 8.7 / 8.8 / 10.0 us
//    at 2 / 3 / 4 tokens);
//  * one GPTQ source with one token from 2.5 tiles per CU on when K >=
//    kStreamLongK, with 8-wave workgroups (4096 x 12288, 3 tiles per CU:
//    7.5 -> 7.25 us; 4096 x 16384: 9.3 -> 8.6 us; 4096 x 10240, 2.5 tiles
//    per CU, within noise), and with a shorter K only above 4 tiles per CU,
//    where the register-ring kernel's workgroups run out of tiles (2560 x
//    10240, configs[4]'s gated q|k|v: 6.08 against 6.40 us on the ring;
//    2560 x 16384 6.81 against 6.89; 2560 x 20480 10.7 against 7.8). INT8
//    with one token keeps the register-ring kernel below 8 tiles per CU
//    (configs[2], 3.4 tiles per CU: 16.2 against 16.4-16.5 us).
// With fewer tiles the register-ring kernel is 0.2-1 us faster (q_proj
// 4.7 against 5.6, down 7.9 against 8.8, configs[4] o 4.4 against 5.6 and
// q|k|v, 1.5 tiles per CU, 5.9-6.3 against 6.0-6.5).
constexpr int kStreamMinTilesCu = 8;
constexpr int kStreamMinTilesCu2 = 2;  // two sources; one source with 2+ tokens
constexpr int kStreamLongK = 4096;     // one GPTQ source, one token: from 2.5 tiles per CU at this K

// The streaming kernel when it is chosen and the call fits it, else the
// register-ring kernels.
template <int FMT, int NSRC, int XM, bool PERM>
int launch_fmt(st_context *ctx, Params &p) {
    if constexpr (FMT == FMT_I4T || FMT == FMT_I8T) {
        const int ncu = std::max(1, ctx->num_cus);
        const int pick = tune(ctx, ST_TUNE_DECODE_KERNEL, -1);
        const int tiles_cu = (p.ntiles + ncu - 1) / ncu;
        const bool many = NSRC == 1 && tiles_cu >= kStreamMinTilesCu;  // 16-wave workgroups
        // one GPTQ source: 2.5+ tiles per CU with a long K, else 4+
        const bool gptq_mid = !is_i8(FMT) && 2 * p.ntiles >= 5 * ncu && (p.K >= kStreamLongK || p.ntiles > 4 * ncu);
        const bool auto_stream = NSRC == 2 ? tiles_cu >= kStreamMinTilesCu2
                                           : (many || gptq_mid || (p.M >= 2 && p.ntiles >= kStreamMinTilesCu2 * ncu));
        const int waves = many ? 16 : 8;
        if (p.M <= 4 && (pick == 1 || (pick < 0 && auto_stream))) {
            int rc = -1;
            if constexpr (is_i8(FMT)) {
                rc = launch_stream<FMT, NSRC, XM, 2, PERM>(ctx, p, waves);
            } else {
                switch (p.gs) {
                    case 64: rc = launch_stream<FMT, NSRC, XM, 1, PERM>(ctx, p, waves); break;
                    case 128: rc = launch_stream<FMT, NSRC, XM, 2, PERM>(ctx, p, waves); break;
                    case 256: rc = launch_stream<FMT, NSRC, XM, 4, PERM>(ctx, p, waves); break;
                }
            }
            if (rc != -1) return rc;
        }
    }
    return launch_gs<FMT, NSRC, XM, PERM>(ctx, p);
}

template <int FMT, bool PERM>
int dispatch_impl(st_context *ctx, Params &p, int nsrc, int xm) {
    if constexpr (is_i8(FMT)) {
        if (xm == XM_F32) return launch_fmt<FMT, 1, XM_F32, false>(ctx, p);
        return launch_fmt<FMT, 1, XM_F16, false>(ctx, p);
    } else {
        if (nsrc == 2) {
            if (xm == XM_F32) return launch_fmt<FMT, 2, XM_F32, PERM>(ctx, p);
            return launch_fmt<FMT, 2, XM_F16, PERM>(ctx, p);
        }
        if (xm == XM_F32) return launch_fmt<FMT, 1, XM_F32, PERM>(ctx, p);
        if (xm == XM_F16) return launch_fmt<FMT, 1, XM_F16, PERM>(ctx, p);
        return launch_fmt<FMT, 1, XM_SILU, PERM>(ctx, p);
    }
}

}  // namespace qmv
}  // namespace st
