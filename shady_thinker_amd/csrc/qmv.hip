// Quantized matvec / skinny GEMM for decode (M = 1..32 rows) on gfx950.
//
// Replaces the reference's GPTQ WGSL kernels (src/shaders/gptq_matvec_4t.wgsl,
// fused_silu_gptq_4t.wgsl, fused_gate_up_silu_4t.wgsl) and adds the INT8
// per-channel path. The math is the reference's: y[n] = sum_k (q - z) * s * x[k]
// with z = 8 in the reference (gptq_matvec.wgsl:51-58).
//
// Design (CDNA4, wave64):
//  * Weights are read once, straight from the reference layout, with 128-bit
//    loads: for GPTQ each lane loads 4 adjacent u32 words (4 columns x 8 k) of
//    one packed row, so 16 lanes read 256 contiguous bytes of a row.
//  * The dot products run on the int8 matrix cores
//    (v_mfma_i32_16x16x64_i8): a nibble word splits into two bytes-of-nibbles
//    registers with one AND and one shift+AND, which are exact int8 operands.
//    The activations become exact integers too: per block of k (one GPTQ group,
//    or the whole K-slice for INT8) x is scaled by a power of two so that
//    max|x| * 2^e lies in [2^21, 2^22), rounded to an integer X, and X is split
//    into three signed 8-bit limbs X = L2*65536 + L1*256 + L0. Each token uses
//    three MFMA rows (limbs), so one 16-row MFMA serves 4 tokens. Products and
//    the K-sum inside a group are exact int32; the zero point enters as
//    -z * sum(X) (exact integer); the group result is rounded to f32 once and
//    multiplied by s * 2^-e. Accuracy is bounded by the 2^-22 relative
//    rounding of X, far below the reference's f32 FMA chain.
//  * VALU work per 8 nibbles is 3 ops (and, shift, and), so the kernel stays
//    HBM-bound; there is no LDS traffic for weights and no cross-lane
//    reduction: each lane owns whole output columns.
//  * K is split across workgroups when there are too few column blocks to
//    fill 256 CUs. Partial sums go to the context workspace; the last
//    workgroup to arrive for a column block (device-scope atomic counter)
//    sums the splits in split order (deterministic) and applies the
//    epilogue (identity, or silu(gate) * up). The counter is reset by that
//    workgroup, so nothing needs clearing between calls.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves
constexpr int kColsPerWave = 64;
constexpr int kColsPerBlock = 256;

enum Fmt { FMT_I4 = 0, FMT_I8 = 1 };
enum XMode { XM_F32 = 0, XM_F16 = 1, XM_SILU = 2 };

struct QmvParams {
    const void *x;          // [M, K] f32 / f16; `a` for XM_SILU
    const float *xb;        // `b` for XM_SILU
    const int32_t *perm;    // act-order gather (I4), or null
    const uint32_t *qw[2];  // GPTQ qweight [K/8, N] per source
    const uint16_t *sc[2];  // GPTQ scales  [K/gs, N]
    const uint32_t *qz[2];  // GPTQ qzeros  [K/gs, N/8] or null
    const int8_t *w8;       // INT8 weights [N, K]
    const float *scale8;    // INT8 scales [N]
    float *y;               // [M, N]
    float *partial;         // [splits][nsrc][M][N]
    unsigned *counters;     // [cblocks]
    int M, K, N;
    int gs;       // GPTQ group size
    int zoff;     // added to stored zero points
    int units;    // I4: groups; I8: 64-wide k steps
    int splits;   // K splits
    int cblocks;  // 256-column blocks
    int max_steps;  // max 64-k steps in one split (LDS sizing)
    int max_nb;     // max exponent blocks in one split
};

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

// k offset (within a lane's 16-k chunk) of operand byte J for GPTQ: byte J of
// register r = J/4 comes from nibble 2*(J%4) (+1 for odd registers) of word
// r/2, i.e. k = 8*(J/8) + 2*(J%4) + ((J/4)%2).
__device__ __forceinline__ int i4_koff(int J) { return ((J >> 3) << 3) + ((J & 3) << 1) + ((J >> 2) & 1); }

template <int XM>
__device__ __forceinline__ float load_x(const QmvParams &p, int m, int k) {
    int kk = p.perm ? p.perm[k] : k;
    size_t idx = (size_t)m * p.K + kk;
    if constexpr (XM == XM_F32) {
        return static_cast<const float *>(p.x)[idx];
    } else if constexpr (XM == XM_F16) {
        return (float)static_cast<const _Float16 *>(p.x)[idx];
    } else {
        float a = static_cast<const float *>(p.x)[idx];
        return silu_f(a) * p.xb[idx];
    }
}

template <int FMT, int NSRC, int XM, int MB, int SPG>
__global__ __launch_bounds__(kThreads) void qmv_kernel(QmvParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int q = lane >> 4;   // k-chunk of the MFMA operands; token within a 4-token block
    const int c = lane & 15;   // operand row (A) / column (B) index
    const int M = p.M, K = p.K, N = p.N;

    // Block -> (column block, split). Workgroups are dealt to the 8 XCDs
    // round-robin; keep all splits of a column block on one XCD.
    const int total = p.cblocks * p.splits;
    const int b = blockIdx.x;
    const int id = (total % 8 == 0) ? (b % 8) * (total / 8) + b / 8 : b;
    const int cb = id / p.splits;
    const int sp = id % p.splits;
    const int u0 = (int)((long long)sp * p.units / p.splits);
    const int u1 = (int)((long long)(sp + 1) * p.units / p.splits);
    const int unit_k = (FMT == FMT_I4) ? p.gs : 64;
    const int k0 = u0 * unit_k;
    const int R = (u1 - u0) * unit_k;        // k extent of this split
    const int nsteps = R >> 6;                // 64-k MFMA steps
    const int NB = (FMT == FMT_I4) ? (u1 - u0) : 1;  // exponent blocks
    const int EB = (FMT == FMT_I4) ? p.gs : R;       // exponent block length

    // LDS: A operands [step][mb][q][row] (16 B each), then per (block, token)
    // exponent / 2^-e / -sum(X) split in high and low parts.
    u32x4 *afrag = reinterpret_cast<u32x4 *>(smem);
    unsigned *s_exp = reinterpret_cast<unsigned *>(afrag + (size_t)p.max_steps * MB * 64);
    const int nbm = p.max_nb * M;
    float *s_emul = reinterpret_cast<float *>(s_exp + nbm);
    int *s_negh = reinterpret_cast<int *>(s_emul + nbm);
    int *s_negl = s_negh + nbm;
    int *s_sum = s_negl + nbm;

    const int nbase = cb * kColsPerBlock + wave * kColsPerWave;

    // ---------------------------------------------------------------- loads
    // GPTQ: lane (q, c) owns columns nl..nl+3; per 64-k step it loads packed
    // rows pr and pr+1 (k = 16q .. 16q+15 of the step).
    const int nl = nbase + 4 * c;
    const bool col_ok = (FMT == FMT_I4) ? (nl < N) : true;
    const int nl_ld = col_ok ? nl : (N - 4);

    struct I4Buf {
        u32x4 w[NSRC][SPG][2];
        uint2 s[NSRC];
        unsigned z[NSRC];
    };
    auto load_i4 = [&](I4Buf &B, int g) {
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
#pragma unroll
            for (int st = 0; st < SPG; ++st) {
                const size_t pr = (size_t)g * (p.gs >> 3) + st * 8 + 2 * q;
                const uint32_t *base = p.qw[src] + pr * N + nl_ld;
                B.w[src][st][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base));
                B.w[src][st][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + N));
            }
            B.s[src] = *reinterpret_cast<const uint2 *>(p.sc[src] + (size_t)g * N + nl_ld);
            B.z[src] = p.qz[src] ? p.qz[src][(size_t)g * (N >> 3) + (nl_ld >> 3)] : 0u;
        }
    };

    // INT8: lane (q, c) reads row n = nbase + 16t + c, bytes 16q..16q+15 of
    // each 64-k step.
    struct I8Buf {
        u32x4 w[4];
    };
    auto load_i8 = [&](I8Buf &B, int step) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int n = nbase + 16 * t + c;
            n = n < N ? n : N - 1;
            const int8_t *ptr = p.w8 + (size_t)n * K + (size_t)step * 64 + 16 * q;
            B.w[t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(ptr));
        }
    };

    I4Buf ib0, ib1;
    I8Buf jb0, jb1;
    // Issue the first weight loads before staging x: they do not depend on it.
    if constexpr (FMT == FMT_I4) {
        if (u0 < u1) load_i4(ib0, u0);
    } else {
        if (u0 < u1) load_i8(jb0, u0);
    }

    // ------------------------------------------------------- stage x in LDS
    {
        const int nfrag = nsteps * MB * 64;
        for (int i = tid; i < nfrag; i += kThreads) afrag[i] = u32x4{0, 0, 0, 0};
        for (int i = tid; i < NB * M; i += kThreads) {
            s_exp[i] = 0;
            s_sum[i] = 0;
        }
        __syncthreads();
        const int nchunks = R >> 4;
        for (int i = tid; i < M * nchunks; i += kThreads) {
            const int m = i / nchunks, ch = i - m * nchunks;
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                float v = load_x<XM>(p, m, k0 + 16 * ch + j);
                float a = fabsf(v);
                // a non-finite x (NaN or inf) poisons its block: amax = inf -> y = NaN
                amax = (a == a && a < INFINITY) ? fmaxf(amax, a) : INFINITY;
            }
            atomicMax(&s_exp[((16 * ch) / EB) * M + m], __float_as_uint(amax));
        }
        __syncthreads();
        for (int i = tid; i < NB * M; i += kThreads) {
            const float a = __uint_as_float(s_exp[i]);
            int e = 0;
            float em = 1.0f;
            if (a == INFINITY) {
                em = __builtin_nanf("");
            } else if (a > 0.0f) {
                e = 21 - ilogbf(a);
                e = e > 100 ? 100 : (e < -100 ? -100 : e);
                em = ldexpf(1.0f, -e);
            }
            s_exp[i] = (unsigned)e;
            s_emul[i] = em;
        }
        __syncthreads();
        for (int i = tid; i < M * nchunks; i += kThreads) {
            const int m = i / nchunks, ch = i - m * nchunks;
            const int blk = (16 * ch) / EB;
            const int e = (int)s_exp[blk * M + m];
            int X[16];
            int sum = 0;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                float v = ldexpf(load_x<XM>(p, m, k0 + 16 * ch + j), e);
                int xi = (v == v && fabsf(v) < 8388608.0f) ? (int)rintf(v) : 0;
                X[j] = xi;
                sum += xi;
            }
            unsigned limb[3][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
            for (int J = 0; J < 16; ++J) {
                const int v = X[(FMT == FMT_I4) ? i4_koff(J) : J];
                const int l0 = (int)(signed char)(v & 0xFF);
                const int v1 = (v - l0) >> 8;
                const int l1 = (int)(signed char)(v1 & 0xFF);
                const int l2 = (v1 - l1) >> 8;
                limb[0][J >> 2] |= (unsigned)(l2 & 0xFF) << (8 * (J & 3));
                limb[1][J >> 2] |= (unsigned)(l1 & 0xFF) << (8 * (J & 3));
                limb[2][J >> 2] |= (unsigned)(l0 & 0xFF) << (8 * (J & 3));
            }
            const int step = ch >> 2, qq = ch & 3;
            u32x4 *dst = afrag + ((size_t)(step * MB + (m >> 2)) * 4 + qq) * 16 + 4 * (m & 3);
#pragma unroll
            for (int l = 0; l < 3; ++l) dst[l] = u32x4{limb[l][0], limb[l][1], limb[l][2], limb[l][3]};
            atomicAdd(&s_sum[blk * M + m], sum);
        }
        __syncthreads();
        for (int i = tid; i < NB * M; i += kThreads) {
            const int s = s_sum[i];
            const int h = (s + 32768) >> 16;
            s_negh[i] = -h;
            s_negl[i] = -(s - (h << 16));
        }
        __syncthreads();
    }

    // ------------------------------------------------------------ main loop
    float tot[NSRC][4][MB];
#pragma unroll
    for (int src = 0; src < NSRC; ++src)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) tot[src][t][mb] = 0.0f;

    if constexpr (FMT == FMT_I4) {
        auto compute = [&](const I4Buf &B, int g) {
            const int blk = g - u0;
            v4i acc[NSRC][4][MB];
#pragma unroll
            for (int src = 0; src < NSRC; ++src)
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) acc[src][t][mb] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int st = 0; st < SPG; ++st) {
                v4i A[MB];
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    A[mb] = __builtin_bit_cast(v4i, afrag[(size_t)((blk * SPG + st) * MB + mb) * 64 + lane]);
                }
#pragma unroll
                for (int src = 0; src < NSRC; ++src) {
                    const u32x4 a0 = B.w[src][st][0], a1 = B.w[src][st][1];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        v4i Bf = v4i{(int)(a0[t] & 0x0F0F0F0Fu), (int)((a0[t] >> 4) & 0x0F0F0F0Fu),
                                     (int)(a1[t] & 0x0F0F0F0Fu), (int)((a1[t] >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
                        for (int mb = 0; mb < MB; ++mb)
                            acc[src][t][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mb], Bf, acc[src][t][mb], 0, 0, 0);
                    }
                }
            }
            // Group epilogue: exact integer sum(q*X) - z*sum(X) in two int32
            // parts, one rounding to f32, then * scale * 2^-e.
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                int m = mb * 4 + q;
                m = m < M ? m : M - 1;
                const int bi = blk * M + m;
                const float em = s_emul[bi];
                const int nh = s_negh[bi], nlo = s_negl[bi];
#pragma unroll
                for (int src = 0; src < NSRC; ++src) {
                    const unsigned sw[2] = {B.s[src].x, B.s[src].y};
                    const int zsh = 4 * (nl_ld & 7);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const unsigned short hb = (unsigned short)(sw[t >> 1] >> (16 * (t & 1)));
                        const float s = (float)__builtin_bit_cast(_Float16, hb);
                        const int z = p.qz[src] ? (int)((B.z[src] >> (zsh + 4 * t)) & 0xF) + p.zoff : 8;
                        const v4i S = acc[src][t][mb];
                        const int hi = S.x + __mul24(z, nh);
                        const int lo = (S.y << 8) + S.z + __mul24(z, nlo);
                        const float v = fmaf((float)hi, 65536.0f, (float)lo);
                        tot[src][t][mb] = fmaf(v, s * em, tot[src][t][mb]);
                    }
                }
            }
        };
        for (int g = u0; g < u1; g += 2) {
            if (g + 1 < u1) load_i4(ib1, g + 1);
            compute(ib0, g);
            if (g + 2 < u1) load_i4(ib0, g + 2);
            if (g + 1 < u1) compute(ib1, g + 1);
        }
    } else {
        v4i acc[4][MB];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[t][mb] = v4i{0, 0, 0, 0};
        auto compute = [&](const I8Buf &B, int step) {
            const int ls = step - u0;
            v4i A[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                A[mb] = __builtin_bit_cast(v4i, afrag[(size_t)(ls * MB + mb) * 64 + lane]);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const v4i Bf = __builtin_bit_cast(v4i, B.w[t]);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[t][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mb], Bf, acc[t][mb], 0, 0, 0);
            }
        };
        for (int s = u0; s < u1; s += 2) {
            if (s + 1 < u1) load_i8(jb1, s + 1);
            compute(jb0, s);
            if (s + 2 < u1) load_i8(jb0, s + 2);
            if (s + 1 < u1) compute(jb1, s + 1);
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            int m = mb * 4 + q;
            m = m < M ? m : M - 1;
            const float em = s_emul[m];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                int n = nbase + 16 * t + c;
                n = n < N ? n : N - 1;
                const v4i S = acc[t][mb];
                const float v = fmaf((float)S.x, 65536.0f, fmaf((float)S.y, 256.0f, (float)S.z));
                tot[0][t][mb] = v * em * p.scale8[n];
            }
        }
    }

    // ------------------------------------------------------------- output
    auto finish = [&](float g, float u) -> float {
        if constexpr (NSRC == 2) return silu_f(g) * u;
        return g;
    };

    if (p.splits == 1) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int m = mb * 4 + q;
            if (m >= M) continue;
            if constexpr (FMT == FMT_I4) {
                if (!col_ok) continue;
                float4 o;
                o.x = finish(tot[0][0][mb], tot[NSRC - 1][0][mb]);
                o.y = finish(tot[0][1][mb], tot[NSRC - 1][1][mb]);
                o.z = finish(tot[0][2][mb], tot[NSRC - 1][2][mb]);
                o.w = finish(tot[0][3][mb], tot[NSRC - 1][3][mb]);
                *reinterpret_cast<float4 *>(p.y + (size_t)m * N + nl) = o;
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int n = nbase + 16 * t + c;
                    if (n < N) p.y[(size_t)m * N + n] = tot[0][t][mb];
                }
            }
        }
        return;
    }

    // Split-K: publish this split's partial sums.
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = mb * 4 + q;
        if (m >= M) continue;
#pragma unroll
        for (int src = 0; src < NSRC; ++src) {
            float *dst = p.partial + ((size_t)(sp * NSRC + src) * M + m) * N;
            if constexpr (FMT == FMT_I4) {
                if (col_ok)
                    *reinterpret_cast<float4 *>(dst + nl) =
                        make_float4(tot[src][0][mb], tot[src][1][mb], tot[src][2][mb], tot[src][3][mb]);
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int n = nbase + 16 * t + c;
                    if (n < N) dst[n] = tot[src][t][mb];
                }
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = __hip_atomic_fetch_add(&p.counters[cb], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (unsigned)(p.splits - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // Last arrival: reduce the splits in order and write y.
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = mb * 4 + q;
        if (m >= M) continue;
        if constexpr (FMT == FMT_I4) {
            if (!col_ok) continue;
            float4 acc[NSRC];
#pragma unroll
            for (int src = 0; src < NSRC; ++src) acc[src] = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int s = 0; s < p.splits; ++s) {
#pragma unroll
                for (int src = 0; src < NSRC; ++src) {
                    const float4 v = *reinterpret_cast<const float4 *>(
                        p.partial + ((size_t)(s * NSRC + src) * M + m) * N + nl);
                    acc[src].x += v.x;
                    acc[src].y += v.y;
                    acc[src].z += v.z;
                    acc[src].w += v.w;
                }
            }
            float4 o;
            o.x = finish(acc[0].x, acc[NSRC - 1].x);
            o.y = finish(acc[0].y, acc[NSRC - 1].y);
            o.z = finish(acc[0].z, acc[NSRC - 1].z);
            o.w = finish(acc[0].w, acc[NSRC - 1].w);
            *reinterpret_cast<float4 *>(p.y + (size_t)m * N + nl) = o;
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int n = nbase + 16 * t + c;
                if (n >= N) continue;
                float a = 0.0f;
                for (int s = 0; s < p.splits; ++s) a += p.partial[((size_t)s * M + m) * N + n];
                p.y[(size_t)m * N + n] = a;
            }
        }
    }
    if (tid == 0) __hip_atomic_store(&p.counters[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------------------------- host side

int env_int(const char *name, int dflt) {
    const char *v = std::getenv(name);
    return (v && *v) ? std::atoi(v) : dflt;
}

struct Plan {
    int splits, cblocks, max_steps, max_nb;
    size_t lds;
};

// Pick the K split so that ~wg_per_cu workgroups per CU exist, within the
// LDS budget and the workspace.
int plan(st_context *ctx, int fmt, int nsrc, int M, int N, int units, int steps_per_unit, int MB,
         Plan *out) {
    const int cblocks = (N + kColsPerBlock - 1) / kColsPerBlock;
    const int target = ctx->num_cus * env_int("ST_QMV_WG_PER_CU", 4);
    int splits = env_int("ST_QMV_SPLITS", 0);
    if (splits <= 0) {
        splits = std::max(1, target / cblocks);
        const int min_units = std::max(1, env_int("ST_QMV_MIN_UNITS", fmt == FMT_I4 ? 1 : 2));
        splits = std::min(splits, std::max(1, units / min_units));
    }
    splits = std::max(1, std::min(splits, units));
    const size_t lds_budget = (size_t)env_int("ST_QMV_LDS_KB", 48) << 10;
    auto lds_for = [&](int s, int *ms, int *mnb) {
        const int max_units = (units + s - 1) / s;
        *ms = max_units * steps_per_unit;
        *mnb = fmt == FMT_I4 ? max_units : 1;
        return (size_t)(*ms) * MB * 1024 + (size_t)(*mnb) * M * 20;
    };
    int ms, mnb;
    while (lds_for(splits, &ms, &mnb) > lds_budget && splits < units) ++splits;
    if (lds_for(splits, &ms, &mnb) > lds_budget)
        return st::fail(ST_ERR_SHAPE, "qmv: K slice does not fit LDS (M=%d)", M);
    if (splits > 1) {
        const size_t need = (size_t)splits * nsrc * M * N * sizeof(float);
        if (need > ctx->ws_bytes) {
            const int fit = (int)(ctx->ws_bytes / ((size_t)nsrc * M * N * sizeof(float)));
            if (fit < 1) return st::fail(ST_ERR_WORKSPACE, "qmv: workspace %zu B too small", ctx->ws_bytes);
            splits = fit;
            if (lds_for(splits, &ms, &mnb) > lds_budget)
                return st::fail(ST_ERR_WORKSPACE, "qmv: workspace too small for the LDS-limited split");
        }
        if (cblocks > ctx->n_counters) return st::fail(ST_ERR_SHAPE, "qmv: N=%d too large", N);
    }
    out->splits = splits;
    out->cblocks = cblocks;
    out->max_steps = ms;
    out->max_nb = mnb;
    out->lds = lds_for(splits, &ms, &mnb);
    return ST_OK;
}

template <int FMT, int NSRC, int XM, int MB, int SPG>
int launch_t(st_context *ctx, QmvParams &p, const Plan &pl) {
    dim3 grid(pl.cblocks * pl.splits), block(kThreads);
    hipLaunchKernelGGL((qmv_kernel<FMT, NSRC, XM, MB, SPG>), grid, block, pl.lds, ctx->stream, p);
    return st::launch_check("qmv_kernel");
}

template <int FMT, int NSRC, int XM, int SPG>
int launch_mb(st_context *ctx, QmvParams &p, const Plan &pl, int MB) {
    switch (MB) {
        case 1: return launch_t<FMT, NSRC, XM, 1, SPG>(ctx, p, pl);
        case 2: return launch_t<FMT, NSRC, XM, 2, SPG>(ctx, p, pl);
        case 4: return launch_t<FMT, NSRC, XM, 4, SPG>(ctx, p, pl);
        default:
            if constexpr (NSRC == 1) return launch_t<FMT, NSRC, XM, 8, SPG>(ctx, p, pl);
            return st::fail(ST_ERR_SHAPE, "qmv: M too large for the dual kernel");
    }
}

int mb_for(int M) { return M <= 4 ? 1 : (M <= 8 ? 2 : (M <= 16 ? 4 : 8)); }

template <int NSRC, int XM>
int launch_i4(st_context *ctx, QmvParams &p, int MB) {
    Plan pl;
    const int spu = p.gs / 64;
    int rc = plan(ctx, FMT_I4, NSRC, p.M, p.N, p.units, spu, MB, &pl);
    if (rc) return rc;
    p.splits = pl.splits;
    p.cblocks = pl.cblocks;
    p.max_steps = pl.max_steps;
    p.max_nb = pl.max_nb;
    p.partial = ctx->ws;
    p.counters = ctx->counters;
    switch (p.gs) {
        case 64: return launch_mb<FMT_I4, NSRC, XM, 1>(ctx, p, pl, MB);
        case 128: return launch_mb<FMT_I4, NSRC, XM, 2>(ctx, p, pl, MB);
        case 256: return launch_mb<FMT_I4, NSRC, XM, 4>(ctx, p, pl, MB);
    }
    return st::fail(ST_ERR_SHAPE, "qmv: group size %d", p.gs);
}

int check_i4(const char *fn, int M, int K, int N, int gs, int mmax) {
    if (gs != 64 && gs != 128 && gs != 256)
        return st::fail(ST_ERR_SHAPE, "%s: group_size %d not in {64,128,256}", fn, gs);
    if (M < 1 || M > mmax) return st::fail(ST_ERR_SHAPE, "%s: M=%d not in [1,%d]", fn, M, mmax);
    if (K <= 0 || K % gs) return st::fail(ST_ERR_SHAPE, "%s: K=%d not a positive multiple of group_size %d", fn, K, gs);
    if (N <= 0 || N % 8) return st::fail(ST_ERR_SHAPE, "%s: N=%d not a positive multiple of 8", fn, N);
    return ST_OK;
}

}  // namespace

extern "C" {

int st_gptq_i4_matvec(st_context *ctx, const void *x, int x_dtype, const uint32_t *qweight,
                      const uint16_t *scales, const uint32_t *qzeros, const int32_t *perm, float *y,
                      int M, int K, int N, int group_size, uint32_t flags) {
    if (!ctx || !x || !qweight || !scales || !y) return st::fail(ST_ERR_INVALID, "st_gptq_i4_matvec: NULL argument");
    if (int rc = check_i4("st_gptq_i4_matvec", M, K, N, group_size, 32)) return rc;
    if (!st::aligned16(qweight) || !st::aligned16(y) || (reinterpret_cast<uintptr_t>(scales) & 7))
        return st::fail(ST_ERR_ALIGN, "st_gptq_i4_matvec: qweight/y must be 16-byte, scales 8-byte aligned");
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
    p.units = K / group_size;
    const int MB = mb_for(M);
    return x_dtype == ST_F32 ? launch_i4<1, XM_F32>(ctx, p, MB) : launch_i4<1, XM_F16>(ctx, p, MB);
}

int st_gptq_i4_silu_matvec(st_context *ctx, const float *a, const float *b, const uint32_t *qweight,
                           const uint16_t *scales, const uint32_t *qzeros, const int32_t *perm, float *y,
                           int M, int K, int N, int group_size, uint32_t flags) {
    if (!ctx || !a || !b || !qweight || !scales || !y)
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_silu_matvec: NULL argument");
    if (int rc = check_i4("st_gptq_i4_silu_matvec", M, K, N, group_size, 32)) return rc;
    if (!st::aligned16(qweight) || !st::aligned16(y) || (reinterpret_cast<uintptr_t>(scales) & 7))
        return st::fail(ST_ERR_ALIGN, "st_gptq_i4_silu_matvec: qweight/y must be 16-byte, scales 8-byte aligned");
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
    p.units = K / group_size;
    return launch_i4<1, XM_SILU>(ctx, p, mb_for(M));
}

int st_gptq_i4_gate_up_silu(st_context *ctx, const void *x, int x_dtype, const uint32_t *qweight_gate,
                            const uint16_t *scales_gate, const uint32_t *qzeros_gate,
                            const uint32_t *qweight_up, const uint16_t *scales_up,
                            const uint32_t *qzeros_up, const int32_t *perm, float *y, int M, int K,
                            int N, int group_size, uint32_t flags) {
    if (!ctx || !x || !qweight_gate || !scales_gate || !qweight_up || !scales_up || !y)
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_gate_up_silu: NULL argument");
    if (int rc = check_i4("st_gptq_i4_gate_up_silu", M, K, N, group_size, 16)) return rc;
    if ((qzeros_gate == nullptr) != (qzeros_up == nullptr))
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_gate_up_silu: give qzeros for both or neither");
    if (!st::aligned16(qweight_gate) || !st::aligned16(qweight_up) || !st::aligned16(y) ||
        ((reinterpret_cast<uintptr_t>(scales_gate) | reinterpret_cast<uintptr_t>(scales_up)) & 7))
        return st::fail(ST_ERR_ALIGN, "st_gptq_i4_gate_up_silu: qweight/y must be 16-byte, scales 8-byte aligned");
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
    p.units = K / group_size;
    const int MB = mb_for(M);
    return x_dtype == ST_F32 ? launch_i4<2, XM_F32>(ctx, p, MB) : launch_i4<2, XM_F16>(ctx, p, MB);
}

int st_int8_matvec(st_context *ctx, const void *x, int x_dtype, const int8_t *w, const float *scale,
                   float *y, int M, int K, int N) {
    if (!ctx || !x || !w || !scale || !y) return st::fail(ST_ERR_INVALID, "st_int8_matvec: NULL argument");
    if (M < 1 || M > 32) return st::fail(ST_ERR_SHAPE, "st_int8_matvec: M=%d not in [1,32]", M);
    if (K <= 0 || K % 64) return st::fail(ST_ERR_SHAPE, "st_int8_matvec: K=%d not a positive multiple of 64", K);
    if (N <= 0 || N % 4) return st::fail(ST_ERR_SHAPE, "st_int8_matvec: N=%d not a positive multiple of 4", N);
    if (!st::aligned16(w)) return st::fail(ST_ERR_ALIGN, "st_int8_matvec: w must be 16-byte aligned");
    if (x_dtype != ST_F32 && x_dtype != ST_F16) return st::fail(ST_ERR_INVALID, "st_int8_matvec: x_dtype %d", x_dtype);
    // The INT8 K-slice shares one exponent per token; bound its length so the
    // int32 limb sums cannot overflow (|w| <= 127, |limb| <= 128).
    QmvParams p{};
    p.x = x;
    p.w8 = w;
    p.scale8 = scale;
    p.y = y;
    p.M = M;
    p.K = K;
    p.N = N;
    p.units = K / 64;
    const int MB = mb_for(M);
    Plan pl;
    if (int rc = plan(ctx, FMT_I8, 1, M, N, p.units, 1, MB, &pl)) return rc;
    if ((long long)pl.max_steps * 64 * 127 * 128 >= (1ll << 31))
        return st::fail(ST_ERR_SHAPE, "st_int8_matvec: K slice too long");
    p.splits = pl.splits;
    p.cblocks = pl.cblocks;
    p.max_steps = pl.max_steps;
    p.max_nb = pl.max_nb;
    p.partial = ctx->ws;
    p.counters = ctx->counters;
    if (x_dtype == ST_F32) return launch_mb<FMT_I8, 1, XM_F32, 1>(ctx, p, pl, MB);
    return launch_mb<FMT_I8, 1, XM_F16, 1>(ctx, p, pl, MB);
}

}  // extern "C"
