// Prefill GEMM on gfx950: C[M, N] = A[M, K] (f16) . dequant(W), W GPTQ int4
// or INT8 (per-output-channel scale). No reference counterpart: the reference prefills token by token through
// the matvec (src/inference.rs:93-95). Dequant semantics are the reference's
// ((q - z) * s, src/shaders/gptq_matvec.wgsl:51-58):
//
//  * B operand = (q - z) * s rounded once to f16 per weight (the dequant of
//    the usual f16 GPTQ GEMMs; rel-L2 ~2e-4 against the f64 oracle, bar
//    2e-3). A GPTQ word holds 8 consecutive k of one column, which is exactly
//    one lane's B fragment of v_mfma_f32_32x32x16_f16, so weights go straight
//    from HBM to registers (no LDS). Word -> 4 f16 pairs: and-or of the even
//    nibble pairs into the f16 1024 bias (1024 + q) and of the odd pairs in
//    place (1024 + 16 q), one shift by 8 for the upper half, then one packed
//    subtract (- (1024 + z)) or packed fma (* 1/16 - (64 + z)) per pair,
//    which forms (q - z) exactly, and one packed multiply by the scale.
//  * A (activations, f16) first goes through a pre-pass (prep_a_kernel)
//    into the context workspace: act-order column gather if any, and each
//    8-k chunk reordered to the B register order (k = 0,4,1,5,2,6,3,7), so A
//    and B fragments pair element for element. The GEMM then moves A tiles
//    HBM -> LDS with the buffer-to-LDS DMA (no registers, no VALU), double
//    buffered one tile ahead. A DMA instruction fills 1 KiB of LDS lane by
//    lane, so rows are not padded: row r's 16-byte chunk c sits at chunk
//    c ^ (r % 16), which makes the MFMA fragment reads conflict-free.
//  * Workgroup tile 128 (M) x 256 (N), 4 waves side by side along N, each
//    wave 128 x 64 = 4 x 2 MFMA blocks of 32 x 32: every converted B
//    fragment feeds 4 MFMAs, every A fragment read from LDS feeds 2, and no
//    B column is converted twice in a workgroup. 128 accumulator registers,
//    two waves per SIMD; B words and the next k-step's A fragments are read
//    one step ahead. Tiles are ordered XCD-major: the workgroups of one XCD
//    share A rows, which then stay in that XCD's L2.
//  * Small grids split K (f32 partials in the workspace, a fixed-order
//    reduce kernel).
//  * Act-order: K is sorted by group at upload (st_gptq_i4_act_order); the
//    matching column gather of A is part of the pre-pass.
//  * INT8 (st_int8_gemm, W8A16): a lane's B fragment is 8 consecutive k of
//    one weight row, so A needs no reordering and the tiles are DMA'd from
//    the caller's buffer (no pre-pass). Bytes -> f16: xor 0x80, v_perm each
//    byte under the f16 exponent of 1024 (1024 + b + 128), one packed add of
//    -1152: exact. Every product int8 x f16 is exact in f32, so only the f32
//    sums round; the channel scale multiplies C once in the epilogue.
#include "common.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128;              // rows of A per workgroup
constexpr int BN = 256;              // columns per workgroup
constexpr int WN = 4;                // waves along N (1 along M)
constexpr int RB = 4, CB = 2;        // 32 x 32 MFMA blocks per wave (rows, columns)
constexpr int KT = 128;              // k per LDS tile
constexpr int kThreads = 256;
#ifndef ST_GEMM_VPM
#define ST_GEMM_VPM 3  // VALU instructions scheduled after each MFMA
#endif
#ifndef ST_GEMM_WAVES
#define ST_GEMM_WAVES 2
#endif
constexpr int kWavesPerSimd = ST_GEMM_WAVES;
// Buffer resource word 3 for gfx9-class GPUs: raw (untyped) 32-bit data.
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kDmaPerWave = BM * KT * 2 / 1024 / (kThreads / 64);  // 1 KiB A DMAs per wave per tile (8)

// v_and_or_b32 with both constants in VGPRs (a VOP3 on gfx9 takes no
// literal, and at most one SGPR), so the compiler cannot split it in two.
__device__ __forceinline__ unsigned and_or(unsigned a, unsigned m, unsigned c) {
    unsigned r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c));
    return r;
}

struct BConv {
    unsigned m_lo, m_hi, bias;  // 0x000F000F, 0x00F000F0, f16 1024 in both halves
    half2_t zlo;                // 1024 + z
    half2_t zhi;                // -(64 + z)
    half2_t sh;                 // the group's scale
};

// GPTQ word (nibbles n0..n7 = k0..k7) -> B fragment halves
// (n0,n4),(n1,n5),(n2,n6),(n3,n7), each (q - z) * s: (q - z) is formed
// exactly (1024 + q - (1024 + z), or (1024 + 16 q) / 16 - (64 + z)), then
// one f16 multiply by the group scale rounds it once.
__device__ __forceinline__ half8 word_to_b(unsigned w, const BConv &c) {
    const half2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
    const unsigned w8 = w >> 8;
    const half2_t h0 = (__builtin_bit_cast(half2_t, and_or(w, c.m_lo, c.bias)) - c.zlo) * c.sh;
    const half2_t h1 =
        __builtin_elementwise_fma(__builtin_bit_cast(half2_t, and_or(w, c.m_hi, c.bias)), sixteenth, c.zhi) * c.sh;
    const half2_t h2 = (__builtin_bit_cast(half2_t, and_or(w8, c.m_lo, c.bias)) - c.zlo) * c.sh;
    const half2_t h3 =
        __builtin_elementwise_fma(__builtin_bit_cast(half2_t, and_or(w8, c.m_hi, c.bias)), sixteenth, c.zhi) * c.sh;
    const u32x4 r = {__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1), __builtin_bit_cast(unsigned, h2),
                     __builtin_bit_cast(unsigned, h3)};
    return __builtin_bit_cast(half8, r);
}

// 8 int8 weights (two words, k0..k7) -> the f16 B fragment in k order:
// (b ^ 0x80) under the exponent byte 0x64 is 1024 + 128 + b, minus 1152.
__device__ __forceinline__ half8 bytes_to_b(unsigned w0, unsigned w1) {
    const unsigned e = 0x64646464u;
    const half2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    w0 ^= 0x80808080u;
    w1 ^= 0x80808080u;
    const half2_t h0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(e, w0, 0x04010400u)) + off;
    const half2_t h1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(e, w0, 0x04030402u)) + off;
    const half2_t h2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(e, w1, 0x04010400u)) + off;
    const half2_t h3 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(e, w1, 0x04030402u)) + off;
    const u32x4 r = {__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1), __builtin_bit_cast(unsigned, h2),
                     __builtin_bit_cast(unsigned, h3)};
    return __builtin_bit_cast(half8, r);
}

// CB_ = 32-column MFMA blocks per wave: 2 (workgroup tile 128 x 256) or 1
// (128 x 128, for grids whose 128 x 256 tiles would leave CUs idle).
// I8: qw is INT8 w (row-major [N, K] or st_int8_repack's tiles), sc / qz /
// zoff unused, chs the f32 channel scales.
template <int GS, bool TILED, bool F16OUT, int CB_, bool I8>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void gemm_kernel(const _Float16 *__restrict__ A, const uint32_t *__restrict__ qw,
                                                           const uint16_t *__restrict__ sc, const uint32_t *__restrict__ qz,
                                                           int zoff, const float *__restrict__ rsc, const float *__restrict__ chs,
                                                           void *__restrict__ C, int M, int K, int N, int kps,
                                                           float *__restrict__ part, int vec, const uint32_t *qw1,
                                                           const uint16_t *sc1, const uint32_t *qz1, void *C1) {
    constexpr int CB = CB_;            // (hides the namespace-scope defaults)
    constexpr int BN = 32 * CB * WN;
    // Two separate arrays (not one [2][...]) so that alias analysis can tell
    // the stage being read from the stage the DMA is filling; otherwise every
    // LDS read waits for the in-flight DMA.
    __shared__ __align__(16) _Float16 As0[BM * KT];
    __shared__ __align__(16) _Float16 As1[BM * KT];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // XCD-major tile order: consecutive ids run on the same XCD. With a
    // second weight (C1 != NULL: the same A times two [K, N] weights, as the
    // gate and up projections of an MLP) the N tiles of both form one grid.
    const int MT = (M + BM - 1) / BM, NT1 = (N + BN - 1) / BN, NT = C1 ? 2 * NT1 : NT1;
    const int T = MT * NT;
    // split-K: workgroup b takes K tiles [kt0, kt1) of tile b % T (kps is
    // even whenever it is not all of K, so a split starts on a group of 256)
    const int split = blockIdx.x / T;
    const int b = blockIdx.x % T;
    const int id = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    // INT8 (B twice GPTQ's bytes): M first within an XCD's run of tiles, so a
    // few weight strips serve every M tile while they sit in that XCD's L2
    // (configs[2]: 2-3.5% faster; GPTQ: no change).
    const int mt = I8 ? id % MT : id / NT;
    int nt = I8 ? id / MT : id % NT;
    if (C1 && nt >= NT1) {  // uniform per workgroup: the second weight's tile
        nt -= NT1;
        qw = qw1;
        sc = sc1;
        qz = qz1;
        C = C1;
    }
    const int m0 = mt * BM, n0 = nt * BN;
    const int nw = n0 + 32 * CB * (wave % WN);  // this wave's columns
    const int mw = 32 * RB * (wave / WN);       // and its rows within the tile

    int col[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) col[cb] = min(nw + 32 * cb + l32, N - 1);

    const int ntiles = K / KT;
    const int kt0 = split * kps, kt1 = min(kt0 + kps, ntiles);

    // ---------------------------------------------------------------- loads
    // Buffer loads: one scalar resource per operand, a 32-bit per-lane
    // offset fixed for the whole K loop and a uniform offset per tile, so
    // the 24 loads per tile need no 64-bit address registers.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)A, (short)0, 0x7FFFFFFF, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb_ = __builtin_amdgcn_make_buffer_rsrc((void *)qw, (short)0, 0x7FFFFFFF, kRsrcWord3);
    // A DMA j of this wave fills tile rows 4 (8 wave + j) .. +3; lane i
    // writes LDS chunk i % 16 of row + i / 16, i.e. logical chunk
    // (i % 16) ^ (row % 16). Rows past M - 1 repeat row M - 1.
    auto a_dma = [&](auto STAGE, int kt) {
        _Float16 *as = decltype(STAGE)::value ? As1 : As0;
#pragma unroll
        for (int j = 0; j < kDmaPerWave; ++j) {
            const int r = 4 * (kDmaPerWave * wave + j) + (lane >> 4);
            const int c = (lane & 15) ^ (r & 15);
            const int voff = (min(m0 + r, M - 1) * K + 8 * c) * 2;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)&as[(4 * (kDmaPerWave * wave + j)) * KT], 16, voff,
                kt * KT * 2, 0, 0);
        }
    };
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
    //  * INT8: a lane's bytes of a K tile are four 16-byte pieces p, each
    //    two k-steps (8 k each). Row-major: 64 contiguous bytes of row col
    //    at k = 64 hi + 16 p. Tiled (one 128-k group per K tile): lane
    //    block q = 2 hi + p / 2 (32 bytes), half st = p % 2, k = 16 q + 64 st.
    constexpr int WPL = GS / 32;  // tiled: words per lane per group
    int boff[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        if constexpr (I8) {
            if constexpr (TILED)
                boff[cb] = (((col[cb] >> 4) * (K / KT) * 64 + 32 * hi + (col[cb] & 15)) * 32);
            else
                boff[cb] = col[cb] * K + 64 * hi;
        } else if constexpr (TILED) {
            const int G = K / GS;
            boff[cb] = (((col[cb] >> 4) * G * 64 + 32 * hi + (col[cb] & 15)) * WPL) * 4;
        } else {
            boff[cb] = (hi * N + col[cb]) * 4;
        }
    }
    // logical 16-byte chunk (8 k) of the A tile that k-step t uses in this lane
    auto kchunk = [&](int t) {
        if constexpr (I8) return TILED ? 8 * ((t >> 1) & 1) + 4 * hi + 2 * (t >> 2) + (t & 1) : 8 * hi + t;
        return TILED ? 8 * (t >> 2) + 4 * hi + 2 * ((t >> 1) & 1) + (t & 1) : 2 * t + hi;
    };

    // INT8 keeps one B buffer: piece p of the next K tile is loaded into
    // the registers of this tile's piece p once both of its k-steps are
    // converted, at step 2p + 1 (GPTQ: the next tile's words go to the other
    // buffer at the start of the tile).
    constexpr int BWN = I8 ? KT / 8 : KT / 16;  // B words per lane per K tile and column block
    unsigned bw[I8 ? 1 : 2][BWN][CB];
    auto load_piece = [&](unsigned (&dst)[BWN][CB], int kt, int p) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const int po = TILED ? (p >> 1) * 16 * 32 + (p & 1) * 16 : 16 * p;
            const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rb_, boff[cb] + po, TILED ? kt * 64 * 32 : kt * KT, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[4 * p + j][cb] = w[j];
        }
    };
    auto load_b = [&](unsigned (&dst)[BWN][CB], int kt) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            if constexpr (I8) {
                if (cb == 0)
#pragma unroll
                    for (int p = 0; p < 4; ++p) load_piece(dst, kt, p);
            } else if constexpr (TILED) {
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

    f32x16 acc[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = f32x16{};

    BConv bc[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        bc[cb].m_lo = 0x000F000Fu;
        bc[cb].m_hi = 0x00F000F0u;
        bc[cb].bias = 0x64006400u;
    }
    // Group constants: the raw scale / zero words of a tile's groups are
    // loaded one tile ahead, before that tile's A and B loads. Loads complete
    // in issue order, so a scale load issued after the prefetch would make
    // its wait drain the whole prefetch.
    constexpr int GPT = KT / GS > 0 ? KT / GS : 1;  // groups starting per tile (GS = 256: one, every other tile)
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)sc, (short)0, 0x7FFFFFFF, kRsrcWord3);
    // Without qzeros the zero words are read from the scales (always in
    // bounds: G * N/8 words < G * N halves) and ignored, so the load needs no
    // branch.
    const bool has_z = qz != nullptr;
    const __amdgpu_buffer_rsrc_t rz =
        __builtin_amdgcn_make_buffer_rsrc((void *)(has_z ? (const void *)qz : (const void *)sc), (short)0, 0x7FFFFFFF,
                                          kRsrcWord3);
    unsigned sraw[2][GPT][CB], zraw[2][GPT][CB];
    auto load_groups = [&](int slot, int kt) {
        if constexpr (I8) return;
#pragma unroll
        for (int gi = 0; gi < GPT; ++gi) {
            const int g = (kt * KT) / GS + gi;
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                sraw[slot][gi][cb] = __builtin_amdgcn_raw_buffer_load_b32(rs, (col[cb] >> 1) * 4, g * N * 2, 0);
                zraw[slot][gi][cb] = __builtin_amdgcn_raw_buffer_load_b32(rz, (col[cb] >> 3) * 4, g * (N >> 3) * 4, 0);
            }
        }
    };
    auto group_consts = [&](int slot, int gi) {
        if constexpr (I8) return;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const int z = has_z ? (int)((zraw[slot][gi][cb] >> (4 * (col[cb] & 7))) & 0xF) + zoff : 8;
            const _Float16 zl = (_Float16)(1024 + z), zh = (_Float16)(-(64 + z));
            bc[cb].zlo = half2_t{zl, zl};
            bc[cb].zhi = half2_t{zh, zh};
            const _Float16 sf = __builtin_bit_cast(_Float16, (uint16_t)(sraw[slot][gi][cb] >> (16 * (col[cb] & 1))));
            bc[cb].sh = half2_t{sf, sf};
        }
    };

    load_groups(0, kt0);
    a_dma(std::integral_constant<int, 0>{}, kt0);
    load_b(bw[0], kt0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's DMAs are in LDS
    __syncthreads();

    // One K tile from LDS buffer BUF = (kt - kt0) & 1. The tile loop is
    // unrolled by two so that the register buffer index and the group
    // boundaries are compile-time (kt * KT mod GS depends only on BUF for
    // GS <= 2 KT, kt0 being even).
    // Software pipeline over the 8 k-steps: the A fragments (LDS) and the
    // converted B of step t + 1 are produced while step t's MFMAs run.
    auto tile = [&](auto BUFC, int kt) {
        constexpr int BUF = decltype(BUFC)::value;
        // The prefetch, its wait and the barrier are unconditional (the last
        // tile reloads itself into the idle stage): with no branch around
        // them, the compiler's wait counting never sees a path on which a
        // previous tile's loads are still in flight.
        const int kn = min(kt + 1, kt1 - 1);
        load_groups(BUF ^ 1, kn);
        a_dma(std::integral_constant<int, BUF ^ 1>{}, kn);  // stage BUF ^ 1 was last read before the previous barrier
        constexpr int RBUF = I8 ? 0 : BUF;                  // the B buffer this tile reads
        if constexpr (!I8) load_b(bw[BUF ^ 1], kn);
        // Keep the prefetch here: left alone, the scheduler sinks these loads
        // to the end of the tile (shorter live ranges), where the barrier
        // then waits for their whole latency.
        __builtin_amdgcn_sched_barrier(0);
        half8 af[RB];
        auto read_a1 = [&](int t, int rb) {
            const int row = mw + rb * 32 + l32;
            const _Float16 *as = BUF ? As1 : As0;
            af[rb] = *reinterpret_cast<const half8 *>(&as[row * KT + 8 * (kchunk(t) ^ (row & 15))]);
        };
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) read_a1(0, rb);
        // One A fragment per row block: it is reloaded for step t + 1 right
        // after its last MFMA of step t. B of step t + 1 is converted while
        // step t's MFMAs run. The scheduling groups interleave them (one
        // MFMA, then a share of the VALU and LDS reads), so that one wave
        // keeps the matrix and vector units busy together.
        half8 bf[2][CB];
        if ((BUF * KT) % GS == 0) group_consts(BUF, 0);
        auto to_b = [&](int t, int cb) {
            if constexpr (I8) return bytes_to_b(bw[RBUF][2 * t][cb], bw[RBUF][2 * t + 1][cb]);
            return word_to_b(bw[RBUF][t][cb], bc[cb]);
        };
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) bf[0][cb] = to_b(0, cb);
#pragma unroll
        for (int t = 0; t < KT / 16; ++t) {
            const int cur = t & 1;
            // INT8: piece (t - 1) / 2 of the next K tile, into the registers
            // its k-steps used here (both converted by step t - 1), pinned at
            // the top of the step: left alone, the scheduler sank these loads
            // to the end of the tile, where the next tile's first conversions
            // then waited for their whole latency.
            if constexpr (I8)
                if (t & 1) {
                    load_piece(bw[0], kn, t >> 1);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[rb], bf[cur][cb], acc[rb][cb], 0, 0, 0);
                if (t + 1 < KT / 16) read_a1(t + 1, rb);
            }
            if (t + 1 < KT / 16) {
                if ((BUF * KT + 16 * (t + 1)) % GS == 0) group_consts(BUF, (16 * (t + 1)) / GS);
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) bf[cur ^ 1][cb] = to_b(t + 1, cb);
#pragma unroll
                for (int i = 0; i < RB * CB; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                   // one MFMA
                    if (i % CB == CB - 1) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // its row block's next A
                    __builtin_amdgcn_sched_group_barrier(0x002, ST_GEMM_VPM, 0);         // VALU
                }
            }
        }
        // vmcnt(0): the next tile's A DMAs (and GPTQ B words) landed. INT8:
        // the 4 CB piece loads issued after the DMAs may stay in flight.
        __builtin_amdgcn_s_waitcnt(I8 ? 0x0F70 + 4 * CB : 0x0F70);
        __syncthreads();
    };
    // K % 256 == 0 when GS == 256 and kps is even, so a group never ends on
    // an odd last tile.
    for (int kt = kt0; kt < kt1; kt += 2) {
        tile(std::integral_constant<int, 0>{}, kt);
        if (kt + 1 < kt1) tile(std::integral_constant<int, 1>{}, kt + 1);
    }

    // ------------------------------------------------------------ output
    // Rows the pre-pass scaled down by 2^-e get 2^e back (exact); INT8 applies
    // its channel scale here. 32 x 32 block: lane l holds column l % 32, rows
    // 8 (i / 4) + 4 (l / 32) + i % 4.
    if (vec) {
        // Staged through LDS, 32 rows at a time: each wave writes its 32 x 32 CB
        // block into a region of its own (rows padded by 16 bytes) and reads it
        // back as 16-byte row chunks, so C is written in whole lines (16 stores
        // per lane for f16 C instead of 128 2-byte ones). The A tiles are free:
        // the last K tile ended with a barrier after every wave's last read.
        // vec: C (or the partials) 16-byte aligned and N a multiple of a chunk.
        auto staged = [&](auto tag) {
            using T = decltype(tag);
            constexpr int WC = 32 * CB;                      // columns of the wave
            constexpr int PITCH = WC * (int)sizeof(T) + 16;  // bytes per staged row
            constexpr int EPC = 16 / (int)sizeof(T);         // elements per chunk
            constexpr int CPR = WC / EPC;                    // chunks per row
            static_assert(2 * 32 * PITCH <= (int)sizeof(As0), "staging region");
            char *stg = reinterpret_cast<char *>((wave & 2) ? As1 : As0) + (wave & 1) * 32 * PITCH;
            T *dst = part ? reinterpret_cast<T *>(part + (size_t)split * M * N) : static_cast<T *>(C);
            float cs[CB];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) cs[cb] = I8 ? chs[min(nw + 32 * cb + l32, N - 1)] : 1.0f;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int r = 8 * (i >> 2) + 4 * hi + (i & 3);
                        float v = rsc ? acc[rb][cb][i] * rsc[min(m0 + mw + rb * 32 + r, M - 1)] : acc[rb][cb][i];
                        if constexpr (I8) v *= cs[cb];
                        *reinterpret_cast<T *>(stg + r * PITCH + (32 * cb + l32) * (int)sizeof(T)) = (T)v;
                    }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's block is in LDS
#pragma unroll
                for (int q = 0; q < 32 * CPR / 64; ++q) {
                    const int ch = q * 64 + lane, row = ch / CPR, cc = ch % CPR;
                    const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + row * PITCH + 16 * cc);
                    const int m = m0 + mw + rb * 32 + row, n = nw + EPC * cc;
                    if (m >= M) continue;
                    if (n + EPC <= N) {
                        *reinterpret_cast<u32x4 *>(dst + (size_t)m * N + n) = v;
                    } else {
                        T e[EPC];
                        __builtin_memcpy(e, &v, 16);
                        for (int j = 0; j < EPC && n + j < N; ++j) dst[(size_t)m * N + n + j] = e[j];
                    }
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next block's writes
            }
        };
        if (part || !F16OUT)
            staged(0.0f);
        else
            staged((_Float16)0);
        return;
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const int n = nw + 32 * cb + l32;
            if (n >= N) continue;
            const float cs = I8 ? chs[n] : 1.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int m = m0 + mw + rb * 32 + 8 * (i >> 2) + 4 * hi + (i & 3);
                if (m >= M) continue;
                float v = rsc ? acc[rb][cb][i] * rsc[m] : acc[rb][cb][i];
                if constexpr (I8) v *= cs;
                if (part)  // split-K: this split's f32 partial
                    part[((size_t)split * M + m) * N + n] = v;
                else if constexpr (F16OUT)
                    static_cast<_Float16 *>(C)[(size_t)m * N + n] = (_Float16)v;
                else
                    static_cast<float *>(C)[(size_t)m * N + n] = v;
            }
        }
}

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

// GEMM A operand: A'[m][8c + i] = A[m][perm[8c + o(i)]] (perm = identity
// when NULL), o = (0,4,1,5,2,6,3,7): the act-order gather and the B
// register order of each 8-k chunk in one pass. One workgroup per row, the
// row staged in LDS. With U non-NULL the row is first h = silu(A) * U,
// silu(v) = v / (1 + exp(-v)) (fused_silu_gptq.wgsl:19-21) in f32, rounded
// once to f16: the fused silu.down of the reference's MLP
// (src/model.rs:803-811) for a block of tokens.
__global__ __launch_bounds__(256) void prep_a_kernel(const _Float16 *__restrict__ A, const _Float16 *__restrict__ U,
                                                     const int32_t *__restrict__ perm, _Float16 *__restrict__ out,
                                                     float *__restrict__ rsc, int K) {
    extern __shared__ _Float16 row[];
    __shared__ unsigned s_hmax;
    const size_t base = (size_t)blockIdx.x * K;
    auto silu_mul = [&](int k) {
        const half8 g = *reinterpret_cast<const half8 *>(A + base + k);
        const half8 u = *reinterpret_cast<const half8 *>(U + base + k);
        float h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float gv = (float)g[e];
            h[e] = __fdividef(gv, 1.0f + __expf(-gv)) * (float)u[e];
        }
        return *reinterpret_cast<const f32x8 *>(h);
    };
    // silu(g) * u can exceed the f16 range (65504) although g and u are f16:
    // a row whose largest |h| is 2^15 or more is stored as h * 2^-e (e so
    // that it lies in [2^14, 2^15)) and the GEMM multiplies its row of C by
    // 2^e (rsc); other rows keep e = 0. Non-finite h is left as it is.
    float inv = 1.0f;
    if (U) {
        if (threadIdx.x == 0) s_hmax = 0;
        __syncthreads();
        float hm = 0.0f;
        for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
            const f32x8 h = silu_mul(k);
#pragma unroll
            for (int e = 0; e < 8; ++e) hm = fmaxf(hm, fabsf(h[e]));
        }
        atomicMax(&s_hmax, __float_as_uint(hm));  // non-negative floats order as their bits
        __syncthreads();
        const float hmax = __uint_as_float(s_hmax);
        int e = 0;
        if (hmax >= 32768.0f && hmax <= 3.4e38f) e = __builtin_amdgcn_frexp_expf(hmax) - 15;
        inv = __builtin_amdgcn_ldexpf(1.0f, -e);
        if (threadIdx.x == 0) rsc[blockIdx.x] = __builtin_amdgcn_ldexpf(1.0f, e);
    }
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
        if (U) {
            const f32x8 hv = silu_mul(k);
            half8 h;
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (_Float16)(hv[e] * inv);
            *reinterpret_cast<half8 *>(&row[k]) = h;
        } else {
            *reinterpret_cast<u32x4 *>(&row[k]) = *reinterpret_cast<const u32x4 *>(A + base + k);
        }
    }
    __syncthreads();
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
        u32x4 v;
        if (perm) {
            const u32x4 p0 = *reinterpret_cast<const u32x4 *>(perm + k);
            const u32x4 p1 = *reinterpret_cast<const u32x4 *>(perm + k + 4);
            const unsigned short *rs = reinterpret_cast<const unsigned short *>(row);
            v.x = rs[p0.x] | ((unsigned)rs[p1.x] << 16);
            v.y = rs[p0.y] | ((unsigned)rs[p1.y] << 16);
            v.z = rs[p0.z] | ((unsigned)rs[p1.z] << 16);
            v.w = rs[p0.w] | ((unsigned)rs[p1.w] << 16);
        } else {
            v = to_b_order(*reinterpret_cast<const u32x4 *>(&row[k]));
        }
        *reinterpret_cast<u32x4 *>(out + base + k) = v;
    }
}

constexpr int kMaxSplit = 8;  // K splits of a small GEMM grid (plan_split)

// C[m, n] = sum over s < S of part[s, m, n] (fixed order: deterministic).
template <bool F16OUT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ part, void *__restrict__ C,
                                                            size_t MN, int S) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= MN) return;  // MN % 4 == 0 (N % 8 == 0)
    // All slices' loads first (S <= kMaxSplit), then the adds in slice order:
    // a loop of load, wait, add paid one memory latency per slice.
    float4 t[kMaxSplit];
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s)
        t[s] = s < S ? *reinterpret_cast<const float4 *>(part + (size_t)s * MN + i) : float4{};
    float4 a = t[0];
#pragma unroll
    for (int s = 1; s < kMaxSplit; ++s)
        if (s < S) {
            a.x += t[s].x;
            a.y += t[s].y;
            a.z += t[s].z;
            a.w += t[s].w;
        }
    if constexpr (F16OUT) {
        _Float16 *c = static_cast<_Float16 *>(C) + i;
        c[0] = (_Float16)a.x;
        c[1] = (_Float16)a.y;
        c[2] = (_Float16)a.z;
        c[3] = (_Float16)a.w;
    } else {
        *reinterpret_cast<float4 *>(static_cast<float *>(C) + i) = a;
    }
}

struct Split {
    int S, kps;
    float *part;  // nullptr when S == 1
};

// The GEMM's operands. I8: qw is the INT8 weight, chs its channel scales
// (sc, qz, zoff unused).
struct GemmArgs {
    const _Float16 *A;
    const uint32_t *qw;
    const uint16_t *sc;
    const uint32_t *qz;
    int zoff;
    const float *rsc, *chs;
    void *C;
    bool f16out;
    int M, K, N;
    // optional second weight on the same A (C1 != NULL; no split-K)
    const uint32_t *qw1 = nullptr;
    const uint16_t *sc1 = nullptr;
    const uint32_t *qz1 = nullptr;
    void *C1 = nullptr;
};

// The staged epilogue needs 16-byte aligned rows: C (or the workspace
// partials) 16-byte aligned and N a multiple of the elements per 16 bytes.
int vec_ok(const GemmArgs &g, const Split &sp) {
    if (sp.part) return g.N % 4 == 0;
    return st::aligned16(g.C) && (!g.C1 || st::aligned16(g.C1)) && g.N % (g.f16out ? 8 : 4) == 0;
}

template <int GS, bool TILED, int CBL, bool I8>
int launch_cb(st_context *ctx, const GemmArgs &g, const Split &sp) {
    const int T = ((g.M + BM - 1) / BM) * ((g.N + 32 * CBL * WN - 1) / (32 * CBL * WN)) * (g.C1 ? 2 : 1);
    const dim3 grid(T * sp.S);
    if (g.f16out)
        st::launch(ctx, (gemm_kernel<GS, TILED, true, CBL, I8>), grid, dim3(kThreads), 0, g.A, g.qw, g.sc,
                           g.qz, g.zoff, g.rsc, g.chs, g.C, g.M, g.K, g.N, sp.kps, sp.part, vec_ok(g, sp), g.qw1, g.sc1,
                           g.qz1, g.C1);
    else
        st::launch(ctx, (gemm_kernel<GS, TILED, false, CBL, I8>), grid, dim3(kThreads), 0, g.A, g.qw, g.sc,
                           g.qz, g.zoff, g.rsc, g.chs, g.C, g.M, g.K, g.N, sp.kps, sp.part, vec_ok(g, sp), g.qw1, g.sc1,
                           g.qz1, g.C1);
    return st::launch_check("gemm_kernel");
}

template <int GS, bool TILED, bool I8 = false>
int launch_gs(st_context *ctx, const GemmArgs &g, int cb, const Split &sp) {
    const int rc = cb == 1 ? launch_cb<GS, TILED, 1, I8>(ctx, g, sp) : launch_cb<GS, TILED, 2, I8>(ctx, g, sp);
    if (rc) return rc;
    const int M = g.M, N = g.N;
    const bool f16out = g.f16out;
    void *C = g.C;
    if (sp.S > 1) {
        const size_t MN = (size_t)M * N;
        const dim3 rg((unsigned)((MN / 4 + 255) / 256));
        if (f16out)
            st::launch(ctx, splitk_reduce_kernel<true>, rg, dim3(256), 0, sp.part, C, MN, sp.S);
        else
            st::launch(ctx, splitk_reduce_kernel<false>, rg, dim3(256), 0, sp.part, C, MN, sp.S);
        return st::launch_check("splitk_reduce_kernel");
    }
    return ST_OK;
}

template <bool TILED>
int launch_tiled(st_context *ctx, const GemmArgs &g, int gs, int cb, const Split &sp) {
    switch (gs) {
        case 64: return launch_gs<64, TILED>(ctx, g, cb, sp);
        case 128: return launch_gs<128, TILED>(ctx, g, cb, sp);
        default: return launch_gs<256, TILED>(ctx, g, cb, sp);
    }
}

// 32-column blocks per wave: 1 (128 x 128 tiles) when 128 x 256 tiles would
// give at most one workgroup per CU (then two waves per SIMD instead of
// one); ST_TUNE_GEMM_CB forces 1 or 2. INT8 keeps the wide tiles down to
// half a workgroup per CU (configs[2]'s weight: M = 512, 216 wide tiles,
// 85 -> 76-78 us; M = 384, 162 tiles, 72-74 -> 69 us; at M = 256, 108
// tiles, the narrow ones win).
int pick_cb(st_context *ctx, int M, int N, bool i8) {
    const int f = st::tune(ctx, ST_TUNE_GEMM_CB, 0);
    if (f == 1 || f == 2) return f;
    const int T2 = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (i8) return 2 * T2 >= ctx->num_cus ? 2 : 1;
    return T2 <= ctx->num_cus ? 1 : 2;
}

// Split K when the tiles alone fill at most half the CUs (the f32 partials
// cost S * M * N * 8 bytes of extra traffic, which measured a loss at
// configs[3] M = 512, 224 tiles): S splits of an even number of K tiles
// each, as many as fill the workgroup slots (two per CU), at most 8, each at
// least 4 K tiles, within the workspace left after A'.
Split plan_split(st_context *ctx, int M, int K, int N, int cb, size_t ws_used) {
    Split sp{1, K / KT, nullptr};
    const int T = ((M + BM - 1) / BM) * ((N + 32 * cb * WN - 1) / (32 * cb * WN));
    const int slots = 2 * ctx->num_cus;
    const int ntiles = K / KT;
    if (2 * T > ctx->num_cus || ntiles < 8 || st::tune(ctx, ST_TUNE_GEMM_NO_SPLIT, 0)) return sp;
    int S = std::min({kMaxSplit, (slots + T - 1) / T, ntiles / 4});
    const size_t off = (ws_used + 255) & ~size_t(255);
    while (S > 1 && off + (size_t)S * M * N * sizeof(float) > ctx->ws_bytes) --S;
    if (S <= 1) return sp;
    int kps = (ntiles + S - 1) / S;
    kps += kps & 1;
    sp.S = (ntiles + kps - 1) / kps;
    sp.kps = kps;
    sp.part = sp.S > 1 ? reinterpret_cast<float *>(reinterpret_cast<char *>(ctx->ws) + off) : nullptr;
    if (sp.S == 1) sp.kps = ntiles;
    return sp;
}

}  // namespace

namespace {

// One weight set of a GEMM call.
struct GptqOperand {
    const uint32_t *qweight;
    const uint16_t *scales;
    const uint32_t *qzeros;
    void *c;
};

// The prefill GEMM behind the entry points: u == NULL for a . dequant(W),
// else silu(a) * u . dequant(W); with w1 (u == NULL) also C1 = a . dequant(W1)
// from the same pre-processed A.
int gemm_impl(const char *fn, st_context *ctx, const uint16_t *a, const uint16_t *u, const uint32_t *qweight,
              const uint16_t *scales, const uint32_t *qzeros, const int32_t *perm, void *c, int c_dtype, int M, int K,
              int N, int group_size, uint32_t flags, const GptqOperand *w1 = nullptr) {
    if (!ctx || !a || !qweight || !scales || !c) return st::fail(ST_ERR_INVALID, "%s: NULL argument", fn);
    if (w1 && (!w1->qweight || !w1->scales || !w1->c)) return st::fail(ST_ERR_INVALID, "%s: NULL argument", fn);
    if (w1 && !st::aligned16(w1->qweight)) return st::fail(ST_ERR_ALIGN, "%s: qweight must be 16-byte aligned", fn);
    if (group_size != 64 && group_size != 128 && group_size != 256)
        return st::fail(ST_ERR_SHAPE, "%s: group_size %d not in {64,128,256}", fn, group_size);
    if (M < 1 || K <= 0 || K % KT || K % group_size || N <= 0 || N % 8)
        return st::fail(ST_ERR_SHAPE, "%s: M=%d K=%d N=%d (K %% 128, K %% group_size, N %% 8)", fn, M, K, N);
    if (c_dtype != ST_F32 && c_dtype != ST_F16) return st::fail(ST_ERR_INVALID, "%s: c_dtype %d", fn, c_dtype);
    if (!st::aligned16(a) || !st::aligned16(u) || !st::aligned16(qweight))
        return st::fail(ST_ERR_ALIGN, "%s: activations and qweight must be 16-byte aligned", fn);
    if ((size_t)M * K * 2 > 0x7FFFFFFFu || (size_t)K / 8 * ((N + 15) / 16 * 16) * 4 > 0x7FFFFFFFu)
        return st::fail(ST_ERR_SHAPE, "%s: A or qweight above 2 GiB (M=%d K=%d N=%d); split M or N", fn, M,
                        K, N);
    if (K > 32768) return st::fail(ST_ERR_SHAPE, "%s: K=%d above 32768", fn, K);
    // workspace: A' (M K halves), then (silu only) one f32 row scale per row
    const size_t a_bytes = (size_t)M * K * sizeof(_Float16);
    const size_t rsc_off = (a_bytes + 255) & ~size_t(255);
    const size_t need = u ? rsc_off + (size_t)M * sizeof(float) : a_bytes;
    if (need > ctx->ws_bytes)
        return st::fail(ST_ERR_WORKSPACE, "%s: needs %zu B of workspace for A (st_context_reserve_workspace)", fn,
                        need);
    if (perm && !st::aligned16(perm)) return st::fail(ST_ERR_ALIGN, "%s: perm must be 16-byte aligned", fn);
    _Float16 *A = reinterpret_cast<_Float16 *>(ctx->ws);
    float *rsc = u ? reinterpret_cast<float *>(reinterpret_cast<char *>(ctx->ws) + rsc_off) : nullptr;
    st::launch(ctx, prep_a_kernel, dim3(M), dim3(256), (size_t)K * sizeof(_Float16),
                       reinterpret_cast<const _Float16 *>(a), reinterpret_cast<const _Float16 *>(u), perm, A, rsc, K);
    if (int rc = st::launch_check("prep_a_kernel")) return rc;
    GemmArgs g{A, qweight, scales, qzeros, (flags & ST_FLAG_ZEROS_PLUS_ONE) ? 1 : 0, rsc, nullptr, c,
               c_dtype == ST_F16, M, K, N};
    auto run = [&](const GemmArgs &ga, int cb, const Split &sp) {
        return (flags & ST_FLAG_TILED) ? launch_tiled<true>(ctx, ga, group_size, cb, sp)
                                       : launch_tiled<false>(ctx, ga, group_size, cb, sp);
    };
    const int cb = pick_cb(ctx, M, N, false);
    const Split sp = plan_split(ctx, M, K, N, cb, need);
    if (w1) {
        // Both weights' tiles in one grid when neither that grid nor one
        // weight's alone splits K (the partials are laid out for one C, and
        // a split changes the order of the f32 sums, so the results would no
        // longer be those of st_gptq_i4_gemm); otherwise two launches on A.
        const int cb2 = pick_cb(ctx, M, 2 * N, false);
        const Split sp2 = plan_split(ctx, M, K, 2 * N, cb2, need);
        if (sp2.S == 1 && sp.S == 1) {
            GemmArgs g2 = g;
            g2.qw1 = w1->qweight;
            g2.sc1 = w1->scales;
            g2.qz1 = w1->qzeros;
            g2.C1 = w1->c;
            return run(g2, cb2, sp2);
        }
    }
    if (int rc = run(g, cb, sp)) return rc;
    if (!w1) return ST_OK;
    GemmArgs g1 = g;
    g1.qw = w1->qweight;
    g1.sc = w1->scales;
    g1.qz = w1->qzeros;
    g1.C = w1->c;
    return run(g1, cb, sp);
}

}  // namespace

extern "C" int st_gptq_i4_gemm(st_context *ctx, const uint16_t *a, const uint32_t *qweight, const uint16_t *scales,
                               const uint32_t *qzeros, const int32_t *perm, void *c, int c_dtype, int M, int K, int N,
                               int group_size, uint32_t flags) {
    return gemm_impl("st_gptq_i4_gemm", ctx, a, nullptr, qweight, scales, qzeros, perm, c, c_dtype, M, K, N, group_size,
                     flags);
}

extern "C" int st_gptq_i4_gate_up_gemm(st_context *ctx, const uint16_t *a, const uint32_t *gate_qweight,
                                       const uint16_t *gate_scales, const uint32_t *gate_qzeros,
                                       const uint32_t *up_qweight, const uint16_t *up_scales, const uint32_t *up_qzeros,
                                       const int32_t *perm, void *c_gate, void *c_up, int c_dtype, int M, int K, int N,
                                       int group_size, uint32_t flags) {
    const GptqOperand up{up_qweight, up_scales, up_qzeros, c_up};
    return gemm_impl("st_gptq_i4_gate_up_gemm", ctx, a, nullptr, gate_qweight, gate_scales, gate_qzeros, perm, c_gate,
                     c_dtype, M, K, N, group_size, flags, &up);
}

extern "C" int st_gptq_i4_silu_gemm(st_context *ctx, const uint16_t *gate, const uint16_t *up, const uint32_t *qweight,
                                    const uint16_t *scales, const uint32_t *qzeros, const int32_t *perm, void *c,
                                    int c_dtype, int M, int K, int N, int group_size, uint32_t flags) {
    if (!up) return st::fail(ST_ERR_INVALID, "st_gptq_i4_silu_gemm: NULL argument");
    return gemm_impl("st_gptq_i4_silu_gemm", ctx, gate, up, qweight, scales, qzeros, perm, c, c_dtype, M, K, N,
                     group_size, flags);
}

extern "C" int st_int8_gemm(st_context *ctx, const uint16_t *a, const int8_t *w, const float *scale, void *c,
                            int c_dtype, int M, int K, int N, uint32_t flags) {
    const char *fn = "st_int8_gemm";
    if (!ctx || !a || !w || !scale || !c) return st::fail(ST_ERR_INVALID, "%s: NULL argument", fn);
    if (M < 1 || K <= 0 || K % KT || N <= 0 || N % 4)
        return st::fail(ST_ERR_SHAPE, "%s: M=%d K=%d N=%d (K %% 128, N %% 4)", fn, M, K, N);
    if (c_dtype != ST_F32 && c_dtype != ST_F16) return st::fail(ST_ERR_INVALID, "%s: c_dtype %d", fn, c_dtype);
    if (!st::aligned16(a) || !st::aligned16(w)) return st::fail(ST_ERR_ALIGN, "%s: a and w must be 16-byte aligned", fn);
    const bool tiled = (flags & ST_FLAG_TILED) != 0;
    const size_t wbytes = tiled ? st_int8_tiled_bytes(K, N) : (size_t)K * N;
    if ((size_t)M * K * 2 > 0x7FFFFFFFu || wbytes > 0x7FFFFFFFu)
        return st::fail(ST_ERR_SHAPE, "%s: a or w above 2 GiB (M=%d K=%d N=%d); split M or N", fn, M, K, N);
    const GemmArgs g{reinterpret_cast<const _Float16 *>(a), reinterpret_cast<const uint32_t *>(w), nullptr, nullptr, 0,
                     nullptr, scale, c, c_dtype == ST_F16, M, K, N};
    const int cb = pick_cb(ctx, M, N, true);
    const Split sp = plan_split(ctx, M, K, N, cb, 0);
    return tiled ? launch_gs<128, true, true>(ctx, g, cb, sp) : launch_gs<128, false, true>(ctx, g, cb, sp);
}
