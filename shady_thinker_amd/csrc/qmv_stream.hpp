// One-token-block decode (M <= 4) on tiled weights with the weight stream
// decoupled from x: the kernel the decode entry points take for 1-4 tokens
// on GPTQ (st_gptq_i4_repack layout) and INT8 (st_int8_repack layout)
// weights whose N is a multiple of 16 and spans many 16-column tiles per CU
// (an lm_head; launch_fmt in qmv_kernel.hpp decides). Included by
// qmv_kernel.hpp; the
// arithmetic (exact int8-limb x on v_mfma_i32_16x16x64_i8, one f32 rounding
// per group) is the one described there.
//
// Why a second kernel. In the register-ring kernel a wave can hold only a
// few groups of weights before x is staged, and x arrives about a
// microsecond after the wave starts (behind the weight stream), so every
// launch pays the x -> staging -> first compute chain on top of the stream.
// Here the weights never pass through registers on their way in:
//  * Each wave owns a ring of D unit slots in LDS (a unit = one group of one
//    16-column tile, 64 lanes x 16 B for g128) and fills it with the
//    buffer-to-LDS DMA (buffer_load_dwordx4 ... lds). The DMAs do not depend
//    on x, so ~96 KiB per CU are requested from the first cycles on, while x
//    is loaded and staged.
//  * The workgroup (16 or 8 waves) owns a contiguous run of tiles;
//    their units, flattened tile-major, are one contiguous byte range of the
//    tiled layout. Wave w takes the w-th sixteenth of that range, so every
//    wave streams the same number of units (no 3-versus-2-tile imbalance)
//    whatever the tile count: a wave's range may start or end inside a tile
//    (partial sums meet in LDS at the end, in wave order), or cover many
//    tiles (written out as each finishes).
//  * A ring slot is waited for with an explicit s_waitcnt vmcnt(N): every
//    wave issues the same LPU loads per unit (absent units use an
//    out-of-range buffer offset, which accesses nothing but still counts),
//    and loads complete in order, so N = (D - 1) * LPU is a constant. The
//    ring is read with inline-asm ds_read (the compiler would otherwise wait
//    for every DMA in flight before any read of the ring).
//  * Scales (and zero words) ride in a register ring next to the LDS one:
//    one 2-byte (4-byte) buffer load per lane, unit and source.
//  * x: the first waves load x (their first loads, so x is at the head of
//    their queue), issue their own rings, wait for x alone and stage it into
//    int8 limbs in LDS (quantize_item); one bare s_barrier (not
//    __syncthreads, which would wait for every DMA) publishes x.
#pragma once

namespace st {
namespace qmv {

constexpr int kStreamRingPerWave = 6144;  // LDS ring bytes per wave (D is derived from it)
// x staging: at most this many 64-item rows per wave (8-wave workgroups have
// the registers for three: up to 256 VGPRs a wave)
template <int NW>
constexpr int kStreamRows = NW == 8 ? 3 : 2;
constexpr size_t kLdsBytes = 160 * 1024;
constexpr bool kStreamPrio = true;

template <int FMT, int SPU>
constexpr int stream_wpu() { return is_i8(FMT) ? 8 : 2 * SPU; }  // weight dwords per lane per unit
template <int FMT, int SPU>
constexpr int stream_wd() {  // DMA instructions per unit and source
    return stream_wpu<FMT, SPU>() >= 4 ? stream_wpu<FMT, SPU>() / 4 : 2;
}
template <int FMT, int NSRC, int SPU>
constexpr int stream_depth() {
    constexpr int wb = 256 * stream_wpu<FMT, SPU>();
    constexpr int d = kStreamRingPerWave / (NSRC * wb);
    constexpr int dmax = 63 / (NSRC * (stream_wd<FMT, SPU>() + 2));  // D loads per unit stay below vmcnt's 64
    constexpr int dc = d > dmax ? dmax : d;
    return dc < 2 ? 2 : (dc > 12 ? 12 : dc);
}
template <int FMT, int NSRC, int SPU, bool HZ>
constexpr int stream_lpu() {  // loads per unit: weight DMAs + scale (+ zero word); INT8: + its column scale
    return NSRC * (stream_wd<FMT, SPU>() + 1 + (HZ ? 1 : 0));
}
template <int FMT, int NSRC, int SPU, int NW>
constexpr int stream_ring_bytes() {
    return NW * stream_depth<FMT, NSRC, SPU>() * NSRC * 256 * stream_wpu<FMT, SPU>();
}

// s_waitcnt vmcnt(n) for a constant n < 64 (expcnt, lgkmcnt left at their maxima)
// (inline asm with a memory clobber: no load may be scheduled across it, or
// the count of loads in flight behind the awaited one would change)
template <int n>
__device__ __forceinline__ void wait_vm() {
    static_assert(n >= 0 && n < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}

// 16-byte-per-lane buffer-to-LDS DMA (a helper of its own: with the 16-byte
// form written inside a kernel template the host pass drops the kernel's
// launch stub without a diagnostic)
template <int AUX>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, unsigned char *lds, unsigned off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, off, 0, 0, AUX);
}


template <int FMT, int NSRC, int XM, int SPU, bool PERM, bool HZ, int NW>
__global__ __launch_bounds__(64 * NW) void qmv_stream_kernel(Params p) {
    constexpr int IPU = 4 * SPU;  // 16-k staging items per group and token
    constexpr int WPU = stream_wpu<FMT, SPU>();
    constexpr int WB = 256 * WPU;  // LDS bytes of one unit of one source (= its HBM bytes)
    constexpr int WD = stream_wd<FMT, SPU>();
    constexpr int D = stream_depth<FMT, NSRC, SPU>();
    constexpr int LPU = stream_lpu<FMT, NSRC, SPU, HZ>();
    static_assert(D * LPU < 64, "ring wait exceeds vmcnt");
    constexpr int RMAX = kStreamRows<NW>;
    __shared__ __align__(16) unsigned char ring[stream_ring_bytes<FMT, NSRC, SPU, NW>()];
    extern __shared__ __align__(16) unsigned char smem[];  // A operands, es, a zero block, partial sums

    // Everything indexed by the wave is uniform: the wave index is read into
    // a scalar register, so the cursors below live in SGPRs and the per-unit
    // bookkeeping is scalar work.
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, c = lane & 15;
    const int M = p.M, N = p.N, G = p.units, RB = p.rb;

    // tiles [t0, t1) of this workgroup; XCD-contiguous runs of workgroups
    const int grid = gridDim.x, bid = blockIdx.x;
    const int r_wg = (grid % 8 == 0) ? (bid % 8) * (grid / 8) + bid / 8 : bid;
    const int t0 = (int)((long long)r_wg * p.ntiles / grid);
    const int t1 = (int)((long long)(r_wg + 1) * p.ntiles / grid);
    const int U = (t1 - t0) * G;  // units of the workgroup (per source)
    // wave w's units [range(w), range(w + 1)) (32-bit: the host keeps U * NW
    // below 2^31; NW is a power of two, so this is a multiply and a shift)
    const auto range = [&](int w) { return (int)((unsigned)w * (unsigned)U / (unsigned)NW); };
    const int ua = range(wave), ub = range(wave + 1);
    const int nu = ub - ua;

    const int ASTEP = 4 * RB;                // u32x4 per (group, step) of A
    const int AUNIT = SPU * ASTEP;           // u32x4 per group of A
    u32x4 *abuf = reinterpret_cast<u32x4 *>(smem);  // [group][step][q][row]
    u32x4 *s_es = abuf + (size_t)G * AUNIT;  // [group][token]
    u32x4 *zblk = s_es + (size_t)G * M;      // AUNIT zero records (the A operand of rows >= RB)
    float *red = reinterpret_cast<float *>(zblk + AUNIT);  // [wave][first, last][src][lane]

    // ------------------------------------------------------------ staging
    // The first nrows waves stage x, 64 items (16 k of one group and token)
    // per row: x loads first, then the wave's ring, then the wait for x only
    const int items = M * G * IPU;
    const int nrows = (items + 63) >> 6;
    const bool stager = wave < nrows;
    float xv[RMAX][16], xb[XM == XM_SILU ? RMAX : 1][16];
    if (stager) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            const int row = wave + r * NW;
            if (row >= nrows) continue;  // uniform per wave
            const int i = min(row * 64 + lane, items - 1);
            const int m = i / (G * IPU), w = i - m * (G * IPU);
            load_x16<XM, PERM>(p, m, (w / IPU) * p.gs + 16 * (w % IPU), xv[r], xb[XM == XM_SILU ? r : 0]);
        }
    }

    // --------------------------------------------------------------- ring
    // Weights: one buffer resource per wave and source covering exactly the
    // wave's units, so the ring's issues past the last unit are out of
    // range (no memory access, still one load each): every unit issues the
    // same LPU loads and the ring wait is a constant.
    constexpr unsigned UB = 64u * WPU * 4u;  // HBM bytes of one unit of one source
    const size_t wfirst = ((size_t)t0 * G + ua) * UB;
    const unsigned wrange = (unsigned)nu * UB;
    const char *wsrc0 = static_cast<const char *>(is_i8(FMT) ? (const void *)p.w8 : (const void *)p.qw[0]) + wfirst;
    const char *wsrc1 = reinterpret_cast<const char *>(p.qw[NSRC - 1]) + wfirst;
    const __amdgpu_buffer_rsrc_t rw0 = __builtin_amdgcn_make_buffer_rsrc((void *)wsrc0, (short)0, wrange, kBufWord3);
    const __amdgpu_buffer_rsrc_t rw1 = __builtin_amdgcn_make_buffer_rsrc((void *)wsrc1, (short)0, wrange, kBufWord3);
    const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(is_i8(FMT) ? (const void *)p.scale8 : (const void *)p.sc[0]), (short)0, 0x7FFFFFFF, kBufWord3);
    const __amdgpu_buffer_rsrc_t rs1 =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.sc[NSRC - 1], (short)0, 0x7FFFFFFF, kBufWord3);
    const __amdgpu_buffer_rsrc_t rz0 = __builtin_amdgcn_make_buffer_rsrc((void *)p.qz[0], (short)0, 0x7FFFFFFF, kBufWord3);
    const __amdgpu_buffer_rsrc_t rz1 =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.qz[NSRC - 1], (short)0, 0x7FFFFFFF, kBufWord3);

    unsigned char *wring = ring + (size_t)wave * D * NSRC * WB;
    const unsigned vlane_w = lane * (WPU >= 4 ? WPU * 4 : 8);  // per-lane part of a unit's weight offset
    const unsigned vlane_s = c * (is_i8(FMT) ? 4u : 2u);      // ... of its scale
    const unsigned vlane_z = (c >> 3) * 4u;                    // ... of its zero word
    unsigned meta[NSRC][D];  // scale bits (GPTQ: f16; INT8: the column's f32 scale)
    unsigned zw[NSRC][HZ ? D : 1];
    // issue cursor (scalar): the unit's tile t0 + it, group ig, and the
    // scalar byte offsets of its scales and zero words; past the wave's
    // last unit the cursor stays there (those scale loads read a valid,
    // cached address and are never used)
    int it = ua / max(G, 1), ig = ua - it * G;
    unsigned soff = is_i8(FMT) ? (unsigned)(t0 + it) * 64u : ((unsigned)ig * N + (unsigned)(t0 + it) * 16u) * 2u;
    unsigned zoff = ((unsigned)ig * (N >> 3) + (unsigned)(t0 + it) * 2u) * 4u;
    auto issue = [&](int i, int d) {  // unit i into ring slot d (d constant after unrolling)
        const unsigned vw = vlane_w + (unsigned)i * UB;
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
            const __amdgpu_buffer_rsrc_t rw = src == 0 ? rw0 : rw1;
            unsigned char *dst = wring + (d * NSRC + src) * WB;
#pragma unroll
            for (int j = 0; j < WD; ++j) {
                if constexpr (WPU >= 4)
                    dma16<ring_cache_policy<NSRC>>(rw, dst + 1024 * j, vw + 16 * j);
                else
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (__attribute__((address_space(3))) void *)(dst + 256 * j),
                                                             4, vw + 4 * j, 0, 0, ring_cache_policy<NSRC>);
            }
            if constexpr (is_i8(FMT)) {
                meta[src][d] = __builtin_amdgcn_raw_buffer_load_b32(rs0, vlane_s, soff, 0);
            } else {
                meta[src][d] = __builtin_amdgcn_raw_buffer_load_b16(src == 0 ? rs0 : rs1, vlane_s, soff, 0);
                if constexpr (HZ) zw[src][d] = __builtin_amdgcn_raw_buffer_load_b32(src == 0 ? rz0 : rz1, vlane_z, zoff, 0);
            }
        }
        if (i + 1 < nu) {
            if constexpr (!is_i8(FMT)) {
                soff += 2u * N;
                zoff += 4u * (N >> 3);
            }
            if (++ig == G) {
                ig = 0;
                ++it;
                soff = is_i8(FMT) ? (unsigned)(t0 + it) * 64u : (unsigned)(t0 + it) * 32u;
                zoff = (unsigned)(t0 + it) * 8u;
            }
        }
    };
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);
    if (stager) {
        wait_vm<D * LPU>();  // x has landed; the ring stays in flight
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            const int row = wave + r * NW;
            if (row >= nrows) continue;
            const int i = row * 64 + lane;
            const int ic = min(i, items - 1);
            const int m = ic / (G * IPU), w = ic - m * (G * IPU);
            const int u = w / IPU, ii = w % IPU;
            x_finish<XM, PERM>(xv[r], xb[XM == XM_SILU ? r : 0]);
            quantize_item<IPU, is_i8(FMT)>(xv[r], i < items,
                                           abuf + ((size_t)(u * SPU + (ii >> 2)) * 4 + (ii & 3)) * RB + 4 * m,
                                           ii == 0 ? &s_es[u * M + m] : nullptr);
        }
    }
    if (wave == 0)
        for (int i = lane; i < AUNIT; i += 64) zblk[i] = u32x4{0, 0, 0, 0};
    // x staged (and this wave's LDS writes landed) in every wave; the DMAs stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // -------------------------------------------------------------- compute
    float tot[NSRC];
#pragma unroll
    for (int src = 0; src < NSRC; ++src) tot[src] = 0.0f;
    const int zoff8 = p.zoff;
    // y of one tile from the full sums (lane: token q, column c)
    auto write_y = [&](int tile, const float (&v)[NSRC], float s8) {
        const int n = tile * kTileN + c;
        if (q >= M) return;
        float out = v[0];
        if constexpr (NSRC == 2) out = silu_f(v[0]) * v[1];
        if constexpr (is_i8(FMT)) out *= s8;
        p.y[(size_t)q * N + n] = out;
    };
    const auto lds_addr = [](const void *ptr) {
        return (unsigned)(size_t)((__attribute__((address_space(3))) const unsigned char *)ptr);
    };
    // per-lane LDS addresses of the A operand (rows >= RB read the zero
    // block, which does not advance) and of the group scalars, advanced by
    // one add per unit
    const bool arow = c < RB;
    const unsigned a_lane0 = arow ? lds_addr(abuf + q * RB + c) : lds_addr(zblk);
    const unsigned a_step = arow ? (unsigned)ASTEP * 16u : 0u;
    const unsigned a_unit = arow ? (unsigned)AUNIT * 16u : 0u;
    const unsigned e_lane0 = lds_addr(s_es + min(q, M - 1));
    int ct = ua / max(G, 1), cg = ua - ct * G;  // compute cursor (tile t0 + ct, group cg)
    unsigned aaddr = a_lane0 + (unsigned)cg * a_unit;
    unsigned eaddr = e_lane0 + (unsigned)(cg * M) * 16u;
    auto compute = [&](int i, int d) {  // unit i from ring slot d
        wait_vm<(D - 1) * LPU>();
        // every LDS read of the unit, issued together; one wait (tied to the
        // values, so nothing uses them before it)
        unsigned w[NSRC][WPU];
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
            const unsigned la = lds_addr(wring + (d * NSRC + src) * WB);
            if constexpr (WPU == 2) {
                // early-clobber outputs: the first read must not land in the
                // address register the second one still uses
                asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %2 offset:256"
                             : "=&v"(w[src][0]), "=&v"(w[src][1])
                             : "v"(la + lane * 4u)
                             : "memory");
            } else {
#pragma unroll
                for (int j = 0; j < WPU / 4; ++j) {
                    u32x4 t;
                    asm volatile("ds_read_b128 %0, %1" : "=v"(t) : "v"(la + lane * 16u + 1024u * j) : "memory");
                    w[src][4 * j] = t.x, w[src][4 * j + 1] = t.y, w[src][4 * j + 2] = t.z, w[src][4 * j + 3] = t.w;
                }
            }
        }
        u32x4 A[SPU], es;
#pragma unroll
        for (int st = 0; st < SPU; ++st)
            asm volatile("ds_read_b128 %0, %1" : "=v"(A[st]) : "v"(aaddr + (unsigned)st * a_step) : "memory");
        asm volatile("ds_read_b128 %0, %1" : "=v"(es) : "v"(eaddr) : "memory");
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int src = 0; src < NSRC; ++src)
#pragma unroll
            for (int j = 0; j < WPU; ++j) asm volatile("" : "+v"(w[src][j]));
#pragma unroll
        for (int st = 0; st < SPU; ++st) asm volatile("" : "+v"(A[st]));
        asm volatile("" : "+v"(es));
        v4i acc[NSRC];
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
            acc[src] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int st = 0; st < SPU; ++st) {
                v4i Bf;
                if constexpr (is_i8(FMT)) {
                    Bf = v4i{(int)w[src][4 * st], (int)w[src][4 * st + 1], (int)w[src][4 * st + 2], (int)w[src][4 * st + 3]};
                } else {
                    const unsigned w0 = w[src][2 * st], w1 = w[src][2 * st + 1];
                    Bf = v4i{(int)(w0 & 0x0F0F0F0Fu), (int)((w0 >> 4) & 0x0F0F0F0Fu), (int)(w1 & 0x0F0F0F0Fu),
                             (int)((w1 >> 4) & 0x0F0F0F0Fu)};
                }
                acc[src] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, A[st]), Bf, acc[src], 0, 0, 0);
            }
        }
        // group epilogue: exact sum(q X) - z sum(X) as hi 65536 + lo, one
        // rounding to f32, then * s * 2^-e
        const float em = __builtin_bit_cast(float, (unsigned)es.x);
        const int nh = (int)es.y, nl = (int)es.z;
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
            const v4i S = acc[src];
            float f = em;
            int z = is_i8(FMT) ? 0 : 8;  // INT8 is symmetric; GPTQ without zero points: z = 8
            if constexpr (!is_i8(FMT)) {
                f = (float)__builtin_bit_cast(_Float16, (unsigned short)meta[src][d]) * em;
                if constexpr (HZ) z = (int)((zw[src][d] >> (4 * (c & 7))) & 0xF) + zoff8;
            }
            const int hi = S.x + __mul24(z, nh);
            const int lo = (S.y << 8) + S.z + __mul24(z, nl);
            tot[src] = fmaf(fmaf((float)hi, 65536.0f, (float)lo), f, tot[src]);
        }
        // end of a tile, or of this wave's range (a scalar test): full tiles
        // go out, partial ones to LDS (slot 0: the tile began before this
        // range; slot 1: it began in it and runs on past it)
        const int f = ua + i;
        if (cg == G - 1 || f == ub - 1) {
            const int ts = ct * G;
            const bool began = ts >= ua, ends = ts + G <= ub;
            if (began && ends) {
                write_y(t0 + ct, tot, __builtin_bit_cast(float, meta[0][d]));
            } else {
                const int slot_ = began ? 1 : 0;
#pragma unroll
                for (int src = 0; src < NSRC; ++src) red[((wave * 2 + slot_) * NSRC + src) * 64 + lane] = tot[src];
            }
#pragma unroll
            for (int src = 0; src < NSRC; ++src) tot[src] = 0.0f;
        }
        aaddr += a_unit;
        eaddr += (unsigned)M * 16u;
        if (++cg == G) {
            cg = 0;
            ++ct;
            aaddr = a_lane0;
            eaddr = e_lane0;
        }
    };
    // Issue priority follows the work left: the CU's memory queue is always
    // full, and by default the oldest waves win every free slot, so they
    // finish first and the youngest run the last part alone with a quarter
    // of the loads in flight. A wave lowers its priority as its remaining
    // share shrinks (quarters of its range), which keeps the waves level.
    //
    // Every ssync ring blocks the workgroup meets at a bare s_barrier (the
    // DMAs stay in flight): the waves ahead wait there with full rings, so
    // the memory queue serves the waves behind. Every wave runs the same
    // number of blocks (the largest range's), so every wave meets every
    // barrier; blocks past a wave's own range compute nothing.
    int prio = 3;
    const int numax = (U + NW - 1) / NW;  // no wave's range is longer
    const int ssync = p.ssync;
    int scount = 0;
    __builtin_amdgcn_s_setprio(3);
    for (int i0 = 0; i0 < numax; i0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (i0 + d < nu) compute(i0 + d, d);
            issue(i0 + d + D, d);  // always: the count of loads per unit is fixed
        }
        if (ssync > 0 && ++scount == ssync) {
            scount = 0;
            asm volatile("s_barrier" ::: "memory");
        }
        const int rem = nu - (i0 + D);  // units left after this block
        const int tp = rem <= 0 ? 0 : min(3, rem * 4 / nu);
        if (kStreamPrio && tp < prio) {
            prio = tp;
            if (prio == 2) __builtin_amdgcn_s_setprio(2);
            else if (prio == 1) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        }
    }
    __builtin_amdgcn_s_setprio(0);
    // ------------------------------------------ tiles split across waves
    __syncthreads();
    if (nu > 0) {
        const int tl = (ub - 1) / G, ts = tl * G, te = ts + G;
        if (ts >= ua && te > ub) {  // began in this range, continues past it: this wave finishes it
            // the first-tile partials of the later waves whose ranges begin
            // inside this tile, added in wave order, without branches (after
            // the barrier the four waves of a SIMD run this part one after
            // another, oldest first, and a taken scalar branch costs tens of
            // cycles): range(w) < te <=> w U < te NW, so the last such wave
            // is (te NW - 1) / U; the reads are all issued before the adds,
            // and a partial left out is masked to +0 (its slot may hold
            // anything, so no multiply by 0)
            const int wl = min(NW - 1, (int)(((unsigned)te * NW - 1u) / (unsigned)U));
            float r[NW - 1][NSRC];
#pragma unroll
            for (int k = 1; k < NW; ++k) {
                const int w2 = min(wave + k, NW - 1);
#pragma unroll
                for (int src = 0; src < NSRC; ++src) r[k - 1][src] = red[((w2 * 2) * NSRC + src) * 64 + lane];
            }
            float v[NSRC];
#pragma unroll
            for (int src = 0; src < NSRC; ++src) v[src] = red[((wave * 2 + 1) * NSRC + src) * 64 + lane];
            // U >= NW: no range is empty; else a wave with an empty range wrote no partial
            const unsigned nonempty = U >= NW ? 0xFFFFu : [&] {
                unsigned m = 0;
                for (int w2 = 0; w2 < NW; ++w2) m |= (range(w2) < range(w2 + 1) ? 1u : 0u) << w2;
                return m;
            }();
#pragma unroll
            for (int k = 1; k < NW; ++k) {
                const int w2 = wave + k;
                const unsigned keep = (w2 <= wl && ((nonempty >> (w2 & 15)) & 1u)) ? ~0u : 0u;
#pragma unroll
                for (int src = 0; src < NSRC; ++src)
                    v[src] += __builtin_bit_cast(float, __builtin_bit_cast(unsigned, r[k - 1][src]) & keep);
            }
            write_y(t0 + tl, v, is_i8(FMT) ? p.scale8[(t0 + tl) * kTileN + c] : 0.0f);
        }
    }
}

// One launch shape of the streaming kernel; -1 (nothing launched) when the
// call does not fit it.
template <int FMT, int NSRC, int XM, int SPU, bool PERM, int NW>
int launch_stream_nw(st_context *ctx, Params &p, int grid) {
    const int items = p.M * p.units * 4 * SPU;
    if (items > 64 * kStreamRows<NW> * NW) return -1;
    const size_t dyn = (size_t)p.units * SPU * 4 * p.rb * 16 + (size_t)p.units * p.M * 16 + (size_t)SPU * 4 * p.rb * 16 +
                       (size_t)NW * 2 * NSRC * 64 * sizeof(float);
    if (dyn + stream_ring_bytes<FMT, NSRC, SPU, NW>() > kLdsBytes) return -1;
    p.grid = grid;
    p.nwaves = NW;
    const bool hz = !is_i8(FMT) && p.qz[0];
    if (!is_i8(FMT) && !p.qz[0] != !p.qz[NSRC - 1]) return -1;  // zero points on one source only
    auto go = [&](auto kern) -> int {
        ST_HIP(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn));
        st::launch(ctx, kern, dim3(p.grid), dim3(64 * NW), dyn, p);
        return launch_check("qmv_stream_kernel");
    };
    if constexpr (!is_i8(FMT)) {
        if (hz) return go(qmv_stream_kernel<FMT, NSRC, XM, SPU, PERM, true, NW>);
    }
    return go(qmv_stream_kernel<FMT, NSRC, XM, SPU, PERM, false, NW>);
}

// Launches the streaming kernel when the call fits it; returns -1 (nothing
// launched) when it does not: the caller then takes the register-ring kernel.
// Shape: one workgroup per CU of `waves` waves (the caller's choice, 8 or
// 16), unless the context settings STREAM_WAVES (8 or 16) / STREAM_TILES_WG
// (tiles per workgroup) say otherwise.
template <int FMT, int NSRC, int XM, int SPU, bool PERM>
int launch_stream(st_context *ctx, Params &p, int waves) {
    if (p.M > 4 || p.N % kTileN) return -1;
    // 32-bit buffer offsets (weights, scales, zero words)
    if ((size_t)p.ntiles * kTileN * p.K / 2 * (is_i8(FMT) ? 2 : 1) >= (size_t(1) << 31)) return -1;
    p.rb = 4 * p.M;
    p.ssync = std::max(0, tune(ctx, ST_TUNE_STREAM_SYNC, 0));
    const int ncu = std::max(1, ctx->num_cus);
    const int tpw = tune(ctx, ST_TUNE_STREAM_TILES_WG, 0);
    const int grid = std::min(p.ntiles, tpw > 0 ? (p.ntiles + tpw - 1) / tpw : ncu);
    // the kernel splits a workgroup's units over its waves in 32-bit arithmetic
    if ((long long)((p.ntiles + grid - 1) / grid) * p.units * 16 >= (1LL << 31)) return -1;
    if (tune(ctx, ST_TUNE_STREAM_WAVES, waves) == 8)
        return launch_stream_nw<FMT, NSRC, XM, SPU, PERM, 8>(ctx, p, grid);
    return launch_stream_nw<FMT, NSRC, XM, SPU, PERM, 16>(ctx, p, grid);
}

}  // namespace qmv
}  // namespace st
