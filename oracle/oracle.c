/*
 * CPU oracle for the quantized-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or
 * calls this file. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may use it, and only as the checker (or, for the CPU
 * baseline, as the thing timed on the host cores).
 *
 * It restates the reference (tmzt/shady-thinker, Rust + WGSL) semantics in
 * plain C. Every function cites the reference file:line it follows. Paths
 * are relative to the reference repository root.
 *
 * Built with -ffp-contract=off so that every float operation rounds exactly
 * where the C source says; FMA contraction is applied only where a function
 * takes `contract` and calls fmaf() explicitly.
 *
 * Parity pins (what checks each function; the tests live in tests/):
 *   rng_*                 : golden first draws computed by hand from the
 *                           xorshift64 definition; Box-Muller mean/var.
 *   orc_f16_to_f32 / orc_f32_to_f16 / orc_f32_to_bf16
 *                         : exhaustive over all 65,536 f16 patterns against
 *                           numpy's float16 conversions; bf16 RNE against a
 *                           bit-level numpy restatement on random + edge cases.
 *   orc_dequant_i4        : exhaustive 16 x 16 x 65,536 KAT vs numpy float32
 *                           and vs the exact f64 product (exact in f32).
 *   orc_gptq_dequant_*    : one-hot columns, nibble-position patterns, numpy
 *                           restatement of weights.rs:257-313 transposition.
 *   orc_gptq_matvec_wgsl  : f64 truth (rel-L2 bound), integer-exact cases
 *                           where scales are 1.0 and x integer (bit-equal),
 *                           lane-split bookkeeping (1t == 4t when exact).
 *   orc_*_f64             : numpy float64 matmul on the dequantized matrix
 *                           (independent library routine), one-hot x,
 *                           brute force on tiny inputs.
 * The exact f32 bit results of the reference WGSL as compiled by naga 24 and
 * run by a particular driver (FMA contraction, exp ULPs) are NOT pinned:
 * neither wgpu, naga nor any Vulkan ICD exists in this image. Both
 * contraction choices are provided and tests accept either within tolerance.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ RNG */
/* xorshift64 exactly as src/lora.rs:80-92 (kaiming_init):
 *   state = seed ^ 0x5DEECE66D; state ^= state<<13; state ^= state>>7;
 *   state ^= state<<17; u = (state & 0xFFFFFFFF) / u32::MAX;
 *   z = sqrt(-2 ln(max(u1,1e-30))) * cos(2 pi u2)
 */
typedef struct { uint64_t s; } orc_rng;

static void rng_init(orc_rng *r, uint64_t seed) { r->s = seed ^ 0x5DEECE66DULL; }

static uint64_t rng_next(orc_rng *r) {
    r->s ^= r->s << 13;
    r->s ^= r->s >> 7;
    r->s ^= r->s << 17;
    return r->s;
}

static double rng_unit(orc_rng *r) {
    return (double)(rng_next(r) & 0xFFFFFFFFULL) / 4294967295.0;
}

static double rng_normal(orc_rng *r) {
    double u1 = rng_unit(r);
    double u2 = rng_unit(r);
    return sqrt(-2.0 * log(u1 > 1e-30 ? u1 : 1e-30)) * cos(2.0 * M_PI * u2);
}

/* Uniform integer in [lo, hi]: multiply-shift of the low 32 bits of one
 * xorshift draw (this build's convention; the reference draws no integers). */
static int64_t rng_int(orc_rng *r, int64_t lo, int64_t hi) {
    uint64_t span = (uint64_t)(hi - lo + 1);
    uint64_t u = rng_next(r) & 0xFFFFFFFFULL;
    return lo + (int64_t)((u * span) >> 32);
}

ORC_API uint64_t orc_rng_draws(uint64_t seed, uint64_t *out, int64_t n) {
    orc_rng r; rng_init(&r, seed);
    for (int64_t i = 0; i < n; i++) out[i] = rng_next(&r);
    return r.s;
}

/* ------------------------------------------------------- f16 / bf16 bits */
/* IEEE binary16 -> binary32, exact (WGSL unpack2x16float, used at
 * src/shaders/gptq_matvec.wgsl:44; half::f16::to_f32 at src/weights.rs:284). */
ORC_API float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24, renormalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400));
            man &= 0x3FF;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x400000u : 0);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even, overflow to inf, NaN kept
 * quiet. Used to generate fp16 scales/activations. */
ORC_API uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000;
    uint32_t absx = x & 0x7FFFFFFF;
    if (absx > 0x7F800000) return (uint16_t)(sign | 0x7E00 | ((absx >> 13) & 0x3FF));
    if (absx >= 0x477FF000) return (uint16_t)(sign | 0x7C00); /* >= 65520 rounds to inf */
    if (absx < 0x38800000) { /* below 2^-14: f16 subnormal or zero */
        if (absx < 0x33000000) return (uint16_t)sign; /* < 2^-25: rounds to 0 (tie at 2^-25 -> 0) */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7FFFFF) | 0x800000;
        uint32_t shift = 126 - e; /* value = m * 2^(e-150); unit 2^-24 -> shift = 126-e */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 127 + 15;
    uint32_t m = absx & 0x7FFFFF;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

/* binary32 -> bfloat16 RNE (half::bf16::from_f32, used at src/weights.rs:288). */
ORC_API uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFF) > 0x7F800000) return (uint16_t)((x >> 16) | 0x0040);
    uint32_t round = 0x7FFF + ((x >> 16) & 1);
    return (uint16_t)((x + round) >> 16);
}

/* --------------------------------------------------------- generators */
ORC_API void orc_gen_normal_f32(uint64_t seed, float *out, int64_t n, double mean, double std) {
    orc_rng r; rng_init(&r, seed);
    for (int64_t i = 0; i < n; i++) out[i] = (float)(mean + std * rng_normal(&r));
}

ORC_API void orc_gen_normal_f16(uint64_t seed, uint16_t *out, int64_t n, double mean, double std) {
    orc_rng r; rng_init(&r, seed);
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16((float)(mean + std * rng_normal(&r)));
}

/* |N(0, std)| rounded to f16 (GPTQ scales). */
ORC_API void orc_gen_abs_normal_f16(uint64_t seed, uint16_t *out, int64_t n, double std) {
    orc_rng r; rng_init(&r, seed);
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16((float)fabs(std * rng_normal(&r)));
}

/* |N(0, std)| as f32 (INT8 per-channel scales). */
ORC_API void orc_gen_abs_normal_f32(uint64_t seed, float *out, int64_t n, double std) {
    orc_rng r; rng_init(&r, seed);
    for (int64_t i = 0; i < n; i++) out[i] = (float)fabs(std * rng_normal(&r));
}

/* Eight nibbles uniform in [lo, hi] per u32, nibble j at bits 4j (low first),
 * which is the packing of src/shaders/gptq_matvec.wgsl:51-59. */
ORC_API void orc_gen_nibbles(uint64_t seed, uint32_t *out, int64_t nwords, int lo, int hi) {
    orc_rng r; rng_init(&r, seed);
    for (int64_t i = 0; i < nwords; i++) {
        uint32_t w = 0;
        for (int j = 0; j < 8; j++) w |= (uint32_t)rng_int(&r, lo, hi) << (4 * j);
        out[i] = w;
    }
}

ORC_API void orc_gen_int8(uint64_t seed, int8_t *out, int64_t n, int lo, int hi) {
    orc_rng r; rng_init(&r, seed);
    for (int64_t i = 0; i < n; i++) out[i] = (int8_t)rng_int(&r, lo, hi);
}

/* Fisher-Yates permutation of 0..n-1 (act-order g_idx source). */
ORC_API void orc_gen_perm(uint64_t seed, int32_t *out, int32_t n) {
    orc_rng r; rng_init(&r, seed);
    for (int32_t i = 0; i < n; i++) out[i] = i;
    for (int32_t i = n - 1; i > 0; i--) {
        int32_t j = (int32_t)rng_int(&r, 0, i);
        int32_t t = out[i]; out[i] = out[j]; out[j] = t;
    }
}

/* ------------------------------------------------------------ dequant */
/* One int4 weight: (f32(q) - f32(z)) * f32(scale). With z = 8 this is
 * src/shaders/gptq_matvec.wgsl:51 `(f32(packed & 0xF) - 8.0) * scale` and
 * src/weights.rs:286-287 `val * scale` before the bf16 rounding. Exact in
 * f32: |q - z| <= 15 needs 4 bits, an f16 significand 11. */
ORC_API float orc_dequant_i4(uint32_t q, uint32_t z, uint16_t scale_bits) {
    float v = (float)q - (float)z;
    return v * orc_f16_to_f32(scale_bits);
}

/* zero point of column n in group g from qzeros u32[G, N/8] (nibble n%8 of
 * word n/8); qzeros == NULL is the reference's symmetric z = 8
 * (src/weights.rs:372-374 drops .qzeros). zero_offset = 1 reads AutoGPTQ
 * v1 checkpoints, which store z - 1. */
static uint32_t zero_of(const uint32_t *qzeros, int g, int n, int N, int zero_offset) {
    if (!qzeros) return 8;
    uint32_t w = qzeros[(int64_t)g * (N / 8) + n / 8];
    return ((w >> (4 * (n % 8))) & 0xF) + (uint32_t)zero_offset;
}

static int group_of(const int32_t *g_idx, int k, int gs) { return g_idx ? g_idx[k] : k / gs; }

/* Dequantize to f32 [K, N] row-major. Generalises src/weights.rs:257-313
 * (dequant_gptq_to_bf16: [packed_rows, N] -> transposed [K, N]) with
 * zero points and act-order g_idx. */
ORC_API void orc_gptq_dequant_f32(const uint32_t *qweight, const uint16_t *scales,
                                  const uint32_t *qzeros, const int32_t *g_idx,
                                  int K, int N, int gs, int zero_offset, float *out) {
#pragma omp parallel for schedule(static)
    for (int k = 0; k < K; k++) {
        int g = group_of(g_idx, k, gs);
        for (int n = 0; n < N; n++) {
            uint32_t q = (qweight[(int64_t)(k / 8) * N + n] >> (4 * (k % 8))) & 0xF;
            out[(int64_t)k * N + n] =
                orc_dequant_i4(q, zero_of(qzeros, g, n, N, zero_offset), scales[(int64_t)g * N + n]);
        }
    }
}

/* src/weights.rs:257-313 verbatim semantics: symmetric, bf16 [K, N]. */
ORC_API void orc_gptq_dequant_bf16(const uint32_t *qweight, const uint16_t *scales,
                                   int K, int N, int gs, uint16_t *out) {
    for (int k = 0; k < K; k++) {
        int g = (k / 8 * 8) / gs; /* group = (pr * 8) / group_size, weights.rs:273 */
        for (int n = 0; n < N; n++) {
            uint32_t q = (qweight[(int64_t)(k / 8) * N + n] >> (4 * (k % 8))) & 0xF;
            out[(int64_t)k * N + n] = orc_f32_to_bf16(orc_dequant_i4(q, 8, scales[(int64_t)g * N + n]));
        }
    }
}

/* --------------------------------------------- WGSL-order f32 restatements */
static float silu_f32(float x) { return x / (1.0f + expf(-x)); } /* fused_silu_gptq.wgsl:19-21 */

static inline float acc_step(float sum, float a, float b, int contract) {
    return contract ? fmaf(a, b, sum) : sum + a * b;
}

/* Sum over packed rows [pr0, pr1) of one column in shader order:
 * t = (f32(nib) - 8) * scale; sum += t * input[row] (gptq_matvec.wgsl:52-59).
 * mode 0: x plain; mode 1: x = silu(a) * b applied as ((t * silu(a)) * b)
 * (fused_silu_gptq.wgsl:52-59). */
static float col_partial(const float *x, const float *b, const uint32_t *qw, const uint16_t *sc,
                         int N, int gs, int col, int pr0, int pr1, int mode, int contract) {
    float sum = 0.0f;
    for (int pr = pr0; pr < pr1; pr++) {
        int group = (pr * 8) / gs;
        float scale = orc_f16_to_f32(sc[(int64_t)group * N + col]);
        uint32_t packed = qw[(int64_t)pr * N + col];
        for (int j = 0; j < 8; j++) {
            float t = ((float)((packed >> (4 * j)) & 0xF) - 8.0f) * scale;
            int row = pr * 8 + j;
            if (mode == 0) {
                sum = acc_step(sum, t, x[row], contract);
            } else {
                float u = t * silu_f32(x[row]);
                sum = acc_step(sum, u, b[row], contract);
            }
        }
    }
    return sum;
}

/* gptq_matvec (variant 0, src/shaders/gptq_matvec.wgsl:17-82: one thread per
 * column, sequential over packed rows; the 4-row unroll does not change the
 * order) or gptq_matvec_4t (variant 1, gptq_matvec_4t.wgsl:37-85: 4 lanes,
 * remainder rows to the lower lanes, reduce (l0 + l2) + (l1 + l3)). */
ORC_API void orc_gptq_matvec_wgsl(const float *x, const uint32_t *qw, const uint16_t *sc, float *y,
                                  int K, int N, int gs, int variant, int contract) {
    int prs = K / 8;
#pragma omp parallel for schedule(static)
    for (int col = 0; col < N; col++) {
        if (variant == 0) {
            y[col] = col_partial(x, NULL, qw, sc, N, gs, col, 0, prs, 0, contract);
        } else {
            int chunk = prs / 4, rem = prs % 4;
            float l[4];
            for (int lane = 0; lane < 4; lane++) {
                int s = lane * chunk + (lane < rem ? lane : rem);
                int e = s + chunk + (lane < rem ? 1 : 0);
                l[lane] = col_partial(x, NULL, qw, sc, N, gs, col, s, e, 0, contract);
            }
            y[col] = (l[0] + l[2]) + (l[1] + l[3]);
        }
    }
}

/* fused_silu_gptq (variant 0, src/shaders/fused_silu_gptq.wgsl:23-88) or
 * fused_silu_gptq_4t (variant 1, fused_silu_gptq_4t.wgsl:26-81: chunk =
 * prs/4, lane 3 takes the remainder, reduce ((l0 + l1) + l2) + l3). */
ORC_API void orc_fused_silu_gptq_wgsl(const float *a, const float *b, const uint32_t *qw,
                                      const uint16_t *sc, float *y, int K, int N, int gs,
                                      int variant, int contract) {
    int prs = K / 8;
#pragma omp parallel for schedule(static)
    for (int col = 0; col < N; col++) {
        if (variant == 0) {
            y[col] = col_partial(a, b, qw, sc, N, gs, col, 0, prs, 1, contract);
        } else {
            int chunk = prs / 4;
            float l[4];
            for (int lane = 0; lane < 4; lane++) {
                int s = lane * chunk;
                int e = lane == 3 ? prs : s + chunk;
                l[lane] = col_partial(a, b, qw, sc, N, gs, col, s, e, 1, contract);
            }
            y[col] = ((l[0] + l[1]) + l[2]) + l[3];
        }
    }
}

/* fused_gate_up_silu (variant 0, src/shaders/fused_gate_up_silu.wgsl:26-102)
 * or fused_gate_up_silu_4t (variant 1, fused_gate_up_silu_4t.wgsl:28-91):
 * y = silu(gate) * up, each a GPTQ dot with `sum += dq * inp`. */
ORC_API void orc_gate_up_silu_wgsl(const float *x, const uint32_t *qg, const uint16_t *sg,
                                   const uint32_t *qu, const uint16_t *su, float *y,
                                   int K, int N, int gs, int variant, int contract) {
    int prs = K / 8;
#pragma omp parallel for schedule(static)
    for (int col = 0; col < N; col++) {
        float gl[4] = {0, 0, 0, 0}, ul[4] = {0, 0, 0, 0};
        int lanes = variant == 0 ? 1 : 4;
        int chunk = prs / lanes;
        for (int lane = 0; lane < lanes; lane++) {
            int s = lane * chunk;
            int e = lane == lanes - 1 ? prs : s + chunk;
            float gsum = 0.0f, usum = 0.0f;
            for (int pr = s; pr < e; pr++) {
                int group = (pr * 8) / gs;
                float scg = orc_f16_to_f32(sg[(int64_t)group * N + col]);
                float scu = orc_f16_to_f32(su[(int64_t)group * N + col]);
                uint32_t pg = qg[(int64_t)pr * N + col], pu = qu[(int64_t)pr * N + col];
                for (int j = 0; j < 8; j++) {
                    float dg = ((float)((pg >> (4 * j)) & 0xF) - 8.0f) * scg;
                    float du = ((float)((pu >> (4 * j)) & 0xF) - 8.0f) * scu;
                    float inp = x[pr * 8 + j];
                    gsum = acc_step(gsum, dg, inp, contract);
                    usum = acc_step(usum, du, inp, contract);
                }
            }
            gl[lane] = gsum;
            ul[lane] = usum;
        }
        float gt, ut;
        if (lanes == 1) { gt = gl[0]; ut = ul[0]; }
        else { gt = ((gl[0] + gl[1]) + gl[2]) + gl[3]; ut = ((ul[0] + ul[1]) + ul[2]) + ul[3]; }
        y[col] = silu_f32(gt) * ut;
    }
}

/* --------------------------------------------------------- f64 truth */
/* y[m, n] = sum_k dequant(k, n) * x[m, k], accumulated in f64, where dequant
 * is the exact f32 value (q - z) * s of orc_dequant_i4 and s is taken from
 * scales[g_idx[k], n] (act-order) or scales[k / gs, n]. Covers M > 1 (the
 * prefill GEMM: each row is this matvec). */
ORC_API void orc_gptq_matvec_f64(const double *x, const uint32_t *qw, const uint16_t *sc,
                                 const uint32_t *qzeros, const int32_t *g_idx, int M, int K,
                                 int N, int gs, int zero_offset, double *y) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        double *acc = (double *)calloc((size_t)M, sizeof(double));
        for (int k = 0; k < K; k++) {
            int g = group_of(g_idx, k, gs);
            uint32_t q = (qw[(int64_t)(k / 8) * N + n] >> (4 * (k % 8))) & 0xF;
            double w = (double)orc_dequant_i4(q, zero_of(qzeros, g, n, N, zero_offset),
                                              sc[(int64_t)g * N + n]);
            for (int m = 0; m < M; m++) acc[m] += w * x[(int64_t)m * K + k];
        }
        for (int m = 0; m < M; m++) y[(int64_t)m * N + n] = acc[m];
        free(acc);
    }
}

/* x = silu(a) * b in f64 (the fused down_proj input, fused_silu_gptq.wgsl:19-21,52). */
ORC_API void orc_silu_mul_f64(const float *a, const float *b, double *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        double v = (double)a[i];
        out[i] = v / (1.0 + exp(-v)) * (double)b[i];
    }
}

/* y = silu(g) * u in f64 over [M, N] (fused_gate_up_silu.wgsl:101). */
ORC_API void orc_silu_gate_f64(const double *g, const double *u, double *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
}

/* INT8 symmetric per-output-channel: y[m, n] = scale[n] * sum_k w[n, k] * x[m, k],
 * weights row-major [N, K] (nn.Linear layout). No reference counterpart. */
ORC_API void orc_int8_matvec_f64(const double *x, const int8_t *w, const float *scale, int M,
                                 int K, int N, double *y) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        for (int m = 0; m < M; m++) {
            double acc = 0.0;
            const int8_t *row = w + (int64_t)n * K;
            const double *xr = x + (int64_t)m * K;
            for (int k = 0; k < K; k++) acc += (double)row[k] * xr[k];
            y[(int64_t)m * N + n] = acc * (double)scale[n];
        }
    }
}

/* ----------------------------------------------------------- bf16 matvec */
/* src/shaders/bf16_matvec.wgsl:15-18,21-72 (lm_head / tied embeddings):
 * y[row] = sum_i bf16(W[row, i]) * x[i], W row-major [N, K] (two bf16 per u32,
 * low half first), in the shader's order: packed words in blocks of four, then
 * the remainder, one f32 multiply-add per element (contract = 1: fused, as a
 * driver contracting `sum += a * b`; 0: separate multiply and add). */
static inline float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

ORC_API void orc_bf16_matvec_wgsl(const float *x, const uint16_t *w, float *y, int K, int N, int contract) {
#pragma omp parallel for schedule(static)
    for (int row = 0; row < N; row++) {
        const uint16_t *wr = w + (int64_t)row * K;
        float sum = 0.0f;
        for (int i = 0; i < K; i++) {
            const float a = orc_bf16_to_f32(wr[i]);
            if (contract)
                sum = fmaf(a, x[i], sum);
            else {
                const volatile float prod = a * x[i];
                sum = sum + prod;
            }
        }
        y[row] = sum;
    }
}

/* f64 truth for the bf16 matvec, M rows of x ([M, K]) -> y [M, N]. */
ORC_API void orc_bf16_matvec_f64(const double *x, const uint16_t *w, int M, int K, int N, double *y) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const uint16_t *wr = w + (int64_t)n * K;
        for (int m = 0; m < M; m++) {
            const double *xr = x + (int64_t)m * K;
            double acc = 0.0;
            for (int k = 0; k < K; k++) acc += (double)orc_bf16_to_f32(wr[k]) * xr[k];
            y[(int64_t)m * N + n] = acc;
        }
    }
}

/* -------------------------------------------------------- CPU baseline */
/* gptq_matvec_4t restated (src/shaders/gptq_matvec_4t.wgsl:37-85), OpenMP
 * over columns on `threads` host threads; the timed CPU baseline when the
 * reference WGSL cannot run on a CPU Vulkan adapter. Returns threads used. */
ORC_API int orc_gptq_matvec_4t_omp(const float *x, const uint32_t *qw, const uint16_t *sc, float *y,
                                   int K, int N, int gs, int threads) {
    int used = 1;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
    {
#pragma omp single
        used = omp_get_num_threads();
    }
#endif
    orc_gptq_matvec_wgsl(x, qw, sc, y, K, N, gs, 1, 1);
    return used;
}
