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
// Design (CDNA4, wave64), one workgroup per 16 output columns:
//  * A workgroup owns a 16-column tile for the whole of K, so no workgroup
//    ever talks to another (cross-workgroup release fences and atomics cost
//    several microseconds per launch on MI355X). Its waves (4..16) split K
//    by groups and meet once, at the end, in LDS.
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
//  * Each wave keeps a ring of D groups of weight loads in flight (registers)
//    and stages its own slice of x into a private LDS buffer, with
//    cross-lane shuffles for the per-group max and sum: no barrier until the
//    final reduction.
//  * vmcnt discipline: global loads complete in issue order and the compiler
//    counts them per path. Every load the wave issues while the ring is in
//    flight is unconditional (absent items read a clamped valid address) and
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
constexpr int kMaxZeroUnits = 64;  // groups per wave whose zero points fit the LDS table

enum Fmt { FMT_I4 = 0, FMT_I4T = 1, FMT_I8 = 2 };
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
};

// silu(v) = v / (1 + exp(-v)) (fused_silu_gptq.wgsl:19-21), with the hardware
// exp and reciprocal (a few ulp; WGSL's exp and division are not correctly
// rounded either).
__device__ __forceinline__ float silu_f(float v) { return __fdividef(v, 1.0f + __expf(-v)); }

// k offset, within a lane's 16-k chunk, of int8 operand byte J for GPTQ:
// register r = J/4 holds nibbles 2(J%4) (+1 for odd r) of word r/2.
__device__ __forceinline__ constexpr int i4_koff(int J) { return ((J >> 3) << 3) + ((J & 3) << 1) + ((J >> 2) & 1); }

template <int XM>
__device__ __forceinline__ float x_elem(const Params &p, size_t idx) {
    if constexpr (XM == XM_F32) {
        return static_cast<const float *>(p.x)[idx];
    } else if constexpr (XM == XM_F16) {
        return (float)static_cast<const _Float16 *>(p.x)[idx];
    } else {
        return silu_f(static_cast<const float *>(p.x)[idx]) * p.xb[idx];
    }
}

// x[m, k .. k+15] (through perm under act-order) with 128-bit loads.
template <int XM, bool PERM>
__device__ __forceinline__ void load_x16(const Params &p, int m, int k, float v[16]) {
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
        for (int j = 0; j < 16; ++j) v[j] = x_elem<XM>(p, row + idx[j]);
    } else if constexpr (XM == XM_F16) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        const h8 *src = reinterpret_cast<const h8 *>(static_cast<const _Float16 *>(p.x) + row + k);
        const h8 a = src[0], b = src[1];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = (float)a[j];
            v[8 + j] = (float)b[j];
        }
    } else {
        const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(p.x) + row + k);
        float4 t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = src[j];
        if constexpr (XM == XM_SILU) {
            const float4 *bsrc = reinterpret_cast<const float4 *>(p.xb + row + k);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 u = bsrc[j];
                v[4 * j] = silu_f(t[j].x) * u.x;
                v[4 * j + 1] = silu_f(t[j].y) * u.y;
                v[4 * j + 2] = silu_f(t[j].z) * u.z;
                v[4 * j + 3] = silu_f(t[j].w) * u.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[4 * j] = t[j].x;
                v[4 * j + 1] = t[j].y;
                v[4 * j + 2] = t[j].z;
                v[4 * j + 3] = t[j].w;
            }
        }
    }
}

// dword of byte `bp` of a, b, c, d (in that order, low byte first).
__device__ __forceinline__ unsigned pack4(unsigned a, unsigned b, unsigned c, unsigned d, int bp) {
    const unsigned sel = 0x0C0C0000u | ((4u + bp) << 8) | (unsigned)bp;
    const unsigned lo = __builtin_amdgcn_perm(b, a, sel);
    const unsigned hi = __builtin_amdgcn_perm(d, c, sel);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup shapes. COOP kernels stage the whole K slice of x once per
// workgroup into shared LDS with every lane of every wave, behind one
// barrier (single-block tokens, when the slice fits); up to 16 waves for one
// source (128 VGPRs each) or 8 for two. The fallback stages per wave, in
// chunks, with 4 waves (256 VGPRs).
template <int NSRC, bool COOP>
constexpr int kMaxWavesFor = COOP ? (NSRC == 1 ? 16 : 8) : 4;

constexpr int kCoopRounds = 2;  // x staging rounds per lane in COOP kernels (bounds M * K)
constexpr int kScaleUnits = 8;  // groups per wave covered by the COOP scale block (one load per source)

// Prefetch ring depth: the registers of weights in flight per lane, about 24
// under a 128-VGPR budget (16-wave workgroups) and 40 for the dual kernel
// (3 waves per SIMD, so every gate/up tile of a 7B layer is resident at once).
template <int FMT, int NSRC, int SPU, bool COOP>
constexpr int ring_depth() {
    constexpr int WPU = (FMT == FMT_I8) ? 4 * SPU : 2 * SPU;
    // (COOP keeps the depth it had with the scale in the ring: deeper rings
    // measured slower, more registers and more loads queued at issue)
    constexpr int RPU = NSRC * (WPU + (FMT == FMT_I8 ? 0 : 1));
    constexpr int budget = (COOP && NSRC == 2) ? 40 : 24;
    return (budget / RPU) < 2 ? 2 : ((budget / RPU) > 6 ? 6 : (budget / RPU));
}

template <int FMT, int NSRC, int XM, int MB, int SPU, bool PERM, bool COOP>
__global__ __launch_bounds__((64 * kMaxWavesFor<NSRC, COOP>)) void qmv_kernel(Params p) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int D = ring_depth<FMT, NSRC, SPU, COOP>();
    constexpr int IPU = 4 * SPU;                              // 16-k items per group and token
    constexpr int WPU = (FMT == FMT_I8) ? 4 * SPU : 2 * SPU;  // weight dwords per lane per group
    // staging rounds per lane: per-wave chunk (fallback) or whole slice (COOP)
    constexpr int RMAX = COOP ? kCoopRounds : (4 * MB * IPU + 63) / 64;

    constexpr bool SCB = COOP && FMT != FMT_I8;  // per-wave scale block (see below)
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int q = lane >> 4;  // k-chunk of the operands; token within a 4-token block
    const int c = lane & 15;  // A row / B column
    const int M = p.M, K = p.K, N = p.N, RB = p.rb;
    const int NW = p.nwaves;

    // Workgroups are dealt to the 8 XCDs round-robin; give each XCD a
    // contiguous run of tiles so neighbouring tiles share L2 lines.
    const int b = blockIdx.x;
    const int tile = (p.ntiles % 8 == 0) ? (b % 8) * (p.ntiles / 8) + b / 8 : b;
    const int n0 = tile * kTileN;
    const int ncol = min(n0 + c, N - 1);  // clamped column this lane loads

    const int u0 = (int)((long long)wave * p.units / NW);
    const int u1 = (int)((long long)(wave + 1) * p.units / NW);

    // LDS: A operands [unit][step][mb][q][row] (16 B each), per (unit, token)
    // 2^-e, -H, -L (sum(X) = H*65536 + L), zero points [unit][src][column].
    // COOP: one region for the workgroup, units = all groups; fallback: one
    // region per wave, units = one chunk (zero table: the wave's groups).
    const int CH = COOP ? p.units : p.chunk;  // units staged at once
    const int ZU = COOP ? p.units : (u1 - u0);
    unsigned char *region = smem + (COOP ? 0 : (size_t)wave * p.wave_lds);
    u32x4 *abuf = reinterpret_cast<u32x4 *>(region);
    const int afrags = CH * SPU * MB * 4 * RB;
    float *s_em = reinterpret_cast<float *>(abuf + afrags);
    int *s_nh = reinterpret_cast<int *>(s_em + CH * M);
    int *s_nl = s_nh + CH * M;
    unsigned char *s_z = reinterpret_cast<unsigned char *>(s_nl + CH * M);
    const int zbase = COOP ? 0 : u0;  // unit index of s_z row 0
    // COOP scale table: [wave][src][group - u0 (< kScaleUnits)][16 columns], after the reduction area
    uint16_t *s_sc = reinterpret_cast<uint16_t *>(smem + (size_t)p.wave_lds + (size_t)NW * NSRC * MB * 64 * sizeof(float));

    // ------------------------------------------- zero points (before all loads)
    bool have_z[NSRC];
#pragma unroll
    for (int src = 0; src < NSRC; ++src) have_z[src] = FMT != FMT_I8 && p.qz[src] != nullptr;
    if constexpr (FMT != FMT_I8) {
        if (have_z[0]) {
            const int nz = ZU * NSRC * 16;
            const int first = COOP ? tid : lane, stride = COOP ? 64 * NW : 64;
            for (int i = first; i < nz; i += stride) {
                const int col = i & 15, src = (i >> 4) % NSRC, uz = i / (16 * NSRC);
                const int zc = min(n0 + col, N - 1);
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
    auto load_unit = [&](Unit &U, int u) {
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
                const uint32_t *base = p.qw[src] + (((size_t)tile * p.units + u) * 64 + lane) * WPU;
                if constexpr (WPU == 2) {
                    const u32x2 t = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(base));
                    U.w[src][0] = t.x;
                    U.w[src][1] = t.y;
                } else {
#pragma unroll
                    for (int j = 0; j < WPU; j += 4) {
                        const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + j));
                        U.w[src][j] = t.x;
                        U.w[src][j + 1] = t.y;
                        U.w[src][j + 2] = t.z;
                        U.w[src][j + 3] = t.w;
                    }
                }
            } else {
                const int8_t *row = p.w8 + (size_t)ncol * K + (size_t)u * 128 + 16 * q;
#pragma unroll
                for (int st = 0; st < SPU; ++st) {
                    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(row + 64 * st));
                    U.w[src][4 * st] = t.x;
                    U.w[src][4 * st + 1] = t.y;
                    U.w[src][4 * st + 2] = t.z;
                    U.w[src][4 * st + 3] = t.w;
                }
            }
            if constexpr (FMT != FMT_I8 && !COOP) U.s[src] = p.sc[src][(size_t)u * N + ncol];
        }
    };

    Unit ring[D];

    // ------------------------------------------------------ x staging
    // Round r covers items i = r * span + t (t = thread index in the staging
    // group: the workgroup for COOP, the wave otherwise). Item i is token
    // m = i / (CH*IPU), group cs + (i % (CH*IPU)) / IPU, 16 k of it. Every
    // thread loads in every round (absent items read a clamped valid address).
    const int span = COOP ? 64 * NW : 64;
    const int tt = COOP ? tid : lane;
    const int uend = COOP ? p.units : u1;  // staged groups end here
    float xv[RMAX][16];
    const int items = M * CH * IPU;
    // A wave with no item in a round skips it (loads and work): the branch
    // is uniform per wave and the same condition guards the loads and their
    // only consumer, stage().
    const int wfirst = COOP ? wave * 64 : 0;
    auto xload = [&](int cs) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            if (r * span + wfirst >= items) continue;
            const int i = min(r * span + tt, items - 1);
            const int m = i / (CH * IPU), w = i - m * (CH * IPU);
            const int u = min(cs + w / IPU, uend - 1);
            load_x16<XM, PERM>(p, m, u * p.gs + 16 * (w % IPU), xv[r]);
        }
    };
    auto stage = [&](int cs) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            if (r * span + wfirst >= items) continue;  // uniform per wave
            const int i = r * span + tt;
            const int m = i / (CH * IPU), w = i - m * (CH * IPU);
            const int ui = w / IPU, ii = w % IPU;
            const bool ok = i < items && cs + ui < uend;
            float amax = 0.0f, nf = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                amax = fmaxf(amax, fabsf(xv[r][j]));
                nf = fmaf(xv[r][j], 0.0f, nf);  // NaN iff some x is NaN or inf
            }
            // a non-finite x poisons its group: amax = inf -> 2^-e = NaN -> y = NaN
            amax = (nf == nf) ? amax : INFINITY;
            if (!ok) amax = 0.0f;
#pragma unroll
            for (int o = 1; o < IPU; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
            int e = 0;
            float em = 1.0f;
            if (amax == INFINITY) {
                em = __builtin_nanf("");
            } else if (amax > 0.0f) {
                e = 21 - ilogbf(amax);
                e = e > 100 ? 100 : (e < -100 ? -100 : e);
                em = ldexpf(1.0f, -e);
            }
            const float sc2 = ldexpf(1.0f, e);
            int X[16];
            int sum = 0;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                // |x| 2^e < 2^22 when amax is finite; otherwise the group is NaN anyway
                X[j] = __float2int_rn(xv[r][j] * sc2);
                sum += X[j];
            }
#pragma unroll
            for (int o = 1; o < IPU; o <<= 1) sum += __shfl_xor(sum, o);
            if (ok) {
                // Operand byte J holds element koff(J) (GPTQ nibble order) or J.
                // Limb bytes: L0 = byte 0 of X, L1 = byte 1 of X + 128,
                // L2 = byte 2 of X + 32896 (balanced base-256 digits).
                u32x4 L2v, L1v, L0v;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    constexpr bool nat = FMT == FMT_I8;
                    const unsigned a = (unsigned)X[nat ? 4 * rr : i4_koff(4 * rr)];
                    const unsigned bb = (unsigned)X[nat ? 4 * rr + 1 : i4_koff(4 * rr + 1)];
                    const unsigned cc = (unsigned)X[nat ? 4 * rr + 2 : i4_koff(4 * rr + 2)];
                    const unsigned dd = (unsigned)X[nat ? 4 * rr + 3 : i4_koff(4 * rr + 3)];
                    L2v[rr] = pack4(a + 32896u, bb + 32896u, cc + 32896u, dd + 32896u, 2);
                    L1v[rr] = pack4(a + 128u, bb + 128u, cc + 128u, dd + 128u, 1);
                    L0v[rr] = pack4(a, bb, cc, dd, 0);
                }
                const int st = ii >> 2, qq = ii & 3;
                u32x4 *dst = abuf + (((size_t)(ui * SPU + st) * MB + (m >> 2)) * 4 + qq) * RB + 4 * (m & 3);
                dst[0] = L2v;
                dst[1] = L1v;
                dst[2] = L0v;
                dst[3] = u32x4{0, 0, 0, 0};  // row 4t+3 (see the zero fill below)
                if (ii == 0) {
                    const int h = (sum + 32768) >> 16;
                    s_em[ui * M + m] = em;
                    s_nh[ui * M + m] = -h;
                    s_nl[ui * M + m] = -(sum - (h << 16));
                }
            }
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

    // --------------------------------------------------------- main loop
    float tot[NSRC][MB];
#pragma unroll
    for (int src = 0; src < NSRC; ++src)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) tot[src][mb] = 0.0f;

    auto compute = [&](const Unit &U, int u, int ui) {
        v4i acc[NSRC][MB];
#pragma unroll
        for (int src = 0; src < NSRC; ++src)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[src][mb] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int st = 0; st < SPU; ++st) {
            v4i A[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                A[mb] = (c < RB) ? __builtin_bit_cast(v4i, abuf[(((size_t)(ui * SPU + st) * MB + mb) * 4 + q) * RB + c])
                                 : v4i{0, 0, 0, 0};
#pragma unroll
            for (int src = 0; src < NSRC; ++src) {
                v4i Bf;
                if constexpr (FMT == FMT_I8) {
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
            const float em = s_em[ui * M + m];
            const int nh = s_nh[ui * M + m], nl = s_nl[ui * M + m];
#pragma unroll
            for (int src = 0; src < NSRC; ++src) {
                const v4i S = acc[src][mb];
                float f;
                int z = 0;
                if constexpr (FMT == FMT_I8) {
                    f = em;
                } else {
                    const uint16_t sh = COOP ? s_sc[(wave * NSRC + src) * 128 + (u - u0) * 16 + c] : U.s[src];
                    f = (float)__builtin_bit_cast(_Float16, sh) * em;
                    z = have_z[src] ? (int)s_z[((u - zbase) * NSRC + src) * 16 + c] : 8;
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

    // x first (loads complete in issue order, so the x slice must not queue
    // behind the weight ring), then the ring, all unconditionally.
    const int cs0 = COOP ? 0 : u0;
    if (COOP || u0 < u1) xload(cs0);
    // COOP GPTQ: the scales of the wave's (at most kScaleUnits) groups for
    // the tile's 16 columns in one 4-byte load per lane and source (lane l:
    // group u0 + l / 8, columns 2 (l % 8) and +1), instead of one 2-byte
    // load per group in the ring: half the ring's load instructions. Issued
    // after x and before the ring, so waiting for them never waits for the
    // ring; parked in LDS after the staging.
    unsigned scw[NSRC];
    if constexpr (SCB) {
        const int ul = min(u0 + (lane >> 3), max(u1, 1) - 1);
        const int cl = min(n0 + 2 * (lane & 7), N - 2);
#pragma unroll
        for (int src = 0; src < NSRC; ++src)
            scw[src] = *reinterpret_cast<const unsigned *>(p.sc[src] + (size_t)ul * N + cl);
    }
    if (u0 < u1) {
#pragma unroll
        for (int d = 0; d < D; ++d) load_unit(ring[d], min(u0 + d, u1 - 1));
    }
    if (COOP || u0 < u1) stage(cs0);
    if constexpr (SCB) {
#pragma unroll
        for (int src = 0; src < NSRC; ++src) reinterpret_cast<unsigned *>(s_sc)[(wave * NSRC + src) * 64 + lane] = scw[src];
    }
    if constexpr (COOP) __syncthreads();
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
                load_unit(ring[d], min(u + D, u1 - 1));
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

    // ------------------------------------------- reduce the waves, write y
    float *red = reinterpret_cast<float *>(smem + (COOP ? (size_t)p.wave_lds : (size_t)NW * p.wave_lds));
#pragma unroll
    for (int src = 0; src < NSRC; ++src)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) red[((wave * NSRC + src) * MB + mb) * 64 + lane] = tot[src][mb];
    __syncthreads();
    if (wave != 0) return;
    const int n = n0 + c;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = mb * 4 + q;
        float v[NSRC];
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
            float a = 0.0f;
            for (int w = 0; w < NW; ++w) a += red[((w * NSRC + src) * MB + mb) * 64 + lane];
            v[src] = a;
        }
        if (m >= M || n >= N) continue;
        float out = v[0];
        if constexpr (NSRC == 2) out = silu_f(v[0]) * v[1];
        if constexpr (FMT == FMT_I8) out *= p.scale8[n];
        p.y[(size_t)m * N + n] = out;
    }
}

// ----------------------------------------------------------------- host side

inline int env_int(const char *name, int dflt) {
    const char *v = std::getenv(name);
    return (v && *v) ? std::atoi(v) : dflt;
}

inline int mb_for(int M) { return M <= 4 ? 1 : (M <= 8 ? 2 : (M <= 16 ? 4 : 8)); }

// Bytes of one staged group (A operands, scalars, zero table row).
template <int FMT, int NSRC, int MB, int SPU>
inline size_t unit_bytes(const Params &p) {
    return (size_t)SPU * MB * 4 * p.rb * 16 + (size_t)p.M * 12 + (FMT == FMT_I8 ? 0 : (size_t)NSRC * 16);
}

template <int FMT, int NSRC, int XM, int MB, int SPU, bool PERM, bool COOP>
int launch_kernel(st_context *ctx, Params &p, size_t lds) {
    auto kern = qmv_kernel<FMT, NSRC, XM, MB, SPU, PERM, COOP>;
    if (lds > 64 * 1024)
        ST_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(kern, dim3(p.ntiles), dim3(64 * p.nwaves), lds, ctx->stream, p);
    return launch_check("qmv_kernel");
}

constexpr size_t kCoopLdsBudget = 96 * 1024;

template <int FMT, int NSRC, int XM, int MB, int SPU, bool PERM>
int launch_t(st_context *ctx, Params &p) {
    constexpr int IPU = 4 * SPU;
    p.rb = p.M >= 4 ? 16 : 4 * p.M;
    p.chunk = std::max(1, 64 / (p.M * IPU));
    // Waves per workgroup: aim at ~4 waves per SIMD over the whole grid
    // (each workgroup is one 16-column tile).
    const int want = (ctx->num_cus * 16) / std::max(1, p.ntiles);
    if constexpr (MB == 1 && FMT != FMT_I4) {
        constexpr int NWX = kMaxWavesFor<NSRC, true>;
        int nw = want >= 16 ? 16 : (want >= 8 ? 8 : 4);
        nw = std::max(4, std::min({nw, NWX, std::max(4, p.units)}));
        nw = std::max(4, std::min(NWX, env_int("ST_QMV_WAVES", nw)));
        // GPTQ: at most kScaleUnits groups per wave (the scale block)
        if (FMT != FMT_I8)
            while ((p.units + nw - 1) / nw > kScaleUnits && nw < NWX) nw *= 2;
        const bool scb_ok = FMT == FMT_I8 || (p.units + nw - 1) / nw <= kScaleUnits;
        const size_t ub = unit_bytes<FMT, NSRC, MB, SPU>(p);
        const size_t lds = ((ub * p.units + 15) & ~size_t(15)) + (size_t)nw * NSRC * MB * 64 * sizeof(float) +
                           (FMT != FMT_I8 ? (size_t)nw * NSRC * 64 * sizeof(unsigned) : 0);
        const long long items = (long long)p.M * p.units * IPU;
        if (scb_ok && lds <= kCoopLdsBudget && items <= (long long)kCoopRounds * 64 * nw &&
            !env_int("ST_QMV_NO_COOP", 0)) {
            p.nwaves = nw;
            p.wave_lds = (int)((ub * p.units + 15) & ~size_t(15));
            return launch_kernel<FMT, NSRC, XM, MB, SPU, PERM, true>(ctx, p, lds);
        }
    }
    // fallback: per-wave chunked staging, 4 waves
    const int nw = 4;
    p.nwaves = nw;
    const int max_units = (p.units + nw - 1) / nw;
    if (FMT != FMT_I8 && max_units > kMaxZeroUnits && (p.qz[0] || p.qz[1]))
        return fail(ST_ERR_SHAPE, "qmv: %d groups per wave exceed the zero-point table", max_units);
    const int afr = p.chunk * SPU * MB * 4 * p.rb;
    const int ztab = (FMT == FMT_I8) ? 0 : std::min(max_units, kMaxZeroUnits) * NSRC * 16;
    p.wave_lds = (afr * 16 + p.chunk * p.M * 12 + ztab + 15) & ~15;
    const size_t lds = (size_t)nw * p.wave_lds + (size_t)nw * NSRC * MB * 64 * sizeof(float);
    return launch_kernel<FMT, NSRC, XM, MB, SPU, PERM, false>(ctx, p, lds);
}

template <int FMT, int NSRC, int XM, int SPU, bool PERM>
int launch_mb(st_context *ctx, Params &p) {
    switch (mb_for(p.M)) {
        case 1: return launch_t<FMT, NSRC, XM, 1, SPU, PERM>(ctx, p);
        case 2: return launch_t<FMT, NSRC, XM, 2, SPU, PERM>(ctx, p);
        case 4: return launch_t<FMT, NSRC, XM, 4, SPU, PERM>(ctx, p);
        default:
            if constexpr (NSRC == 1) return launch_t<FMT, NSRC, XM, 8, SPU, PERM>(ctx, p);
            return fail(ST_ERR_SHAPE, "qmv: M too large for the dual kernel");
    }
}

template <int FMT, int NSRC, int XM, bool PERM>
int launch_gs(st_context *ctx, Params &p) {
    if constexpr (FMT == FMT_I8) {
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
// qmv_i4_p{0,1}.hip, qmv_i4t_p{0,1}.hip and qmv_i8.hip so the variants
// compile in parallel.
template <int FMT, bool PERM>
int dispatch(st_context *ctx, Params &p, int nsrc, int xm);

template <int FMT, bool PERM>
int dispatch_impl(st_context *ctx, Params &p, int nsrc, int xm) {
    if constexpr (FMT == FMT_I8) {
        if (xm == XM_F32) return launch_gs<FMT, 1, XM_F32, false>(ctx, p);
        return launch_gs<FMT, 1, XM_F16, false>(ctx, p);
    } else {
        if (nsrc == 2) {
            if (xm == XM_F32) return launch_gs<FMT, 2, XM_F32, PERM>(ctx, p);
            return launch_gs<FMT, 2, XM_F16, PERM>(ctx, p);
        }
        if (xm == XM_F32) return launch_gs<FMT, 1, XM_F32, PERM>(ctx, p);
        if (xm == XM_F16) return launch_gs<FMT, 1, XM_F16, PERM>(ctx, p);
        return launch_gs<FMT, 1, XM_SILU, PERM>(ctx, p);
    }
}

}  // namespace qmv
}  // namespace st
