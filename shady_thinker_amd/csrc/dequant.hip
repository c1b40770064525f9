// Upload-time GPTQ helpers: dequantization to f32/bf16 and act-order
// preparation (sorting K by g_idx).
#include "common.hpp"

#include <vector>

namespace {

// One thread per qweight word (8 consecutive k of one column n); writes the
// 8 dequantized values of out[k, n] (coalesced across n).
// (q - z) * scale is exact in f32 (src/weights.rs:286-287 with z = 8); the
// bf16 variant rounds to nearest even as half::bf16::from_f32 does
// (src/weights.rs:288).
template <int OUT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t *__restrict__ qw, const uint16_t *__restrict__ sc,
                                                      const uint32_t *__restrict__ qz, const int32_t *__restrict__ g_idx,
                                                      void *__restrict__ out, int K, int N, int gs, int zoff) {
    const long long word = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long nwords = (long long)(K / 8) * N;
    if (word >= nwords) return;
    const int pr = (int)(word / N), n = (int)(word % N);
    const uint32_t w = qw[word];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int k = pr * 8 + j;
        const int g = g_idx ? g_idx[k] : k / gs;
        const int q = (w >> (4 * j)) & 0xF;
        const int z = qz ? (int)((qz[(size_t)g * (N / 8) + n / 8] >> (4 * (n % 8))) & 0xF) + zoff : 8;
        const float s = (float)__builtin_bit_cast(_Float16, sc[(size_t)g * N + n]);
        const float v = (float)(q - z) * s;
        const size_t o = (size_t)k * N + n;
        if constexpr (OUT == ST_F32) {
            static_cast<float *>(out)[o] = v;
        } else {
            uint32_t b = __float_as_uint(v);
            uint16_t r = (b & 0x7FFFFFFFu) > 0x7F800000u ? (uint16_t)((b >> 16) | 0x40u)
                                                         : (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
            static_cast<uint16_t *>(out)[o] = r;
        }
    }
}

// qweight_out row j = qweight row perm[j] (nibble gather); one thread per
// output word.
__global__ __launch_bounds__(256) void act_order_gather(const uint32_t *__restrict__ qw, const int32_t *__restrict__ perm,
                                                        uint32_t *__restrict__ out, int K, int N) {
    const long long word = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long nwords = (long long)(K / 8) * N;
    if (word >= nwords) return;
    const int pr = (int)(word / N), n = (int)(word % N);
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int src = perm[pr * 8 + j];
        const uint32_t v = (qw[(size_t)(src / 8) * N + n] >> (4 * (src % 8))) & 0xFu;
        acc |= v << (4 * j);
    }
    out[word] = acc;
}

}  // namespace

extern "C" {

int st_gptq_i4_dequant(st_context *ctx, const uint32_t *qweight, const uint16_t *scales, const uint32_t *qzeros,
                       const int32_t *g_idx, void *out, int out_dtype, int K, int N, int group_size, uint32_t flags) {
    if (!ctx || !qweight || !scales || !out) return st::fail(ST_ERR_INVALID, "st_gptq_i4_dequant: NULL argument");
    if (group_size <= 0 || K <= 0 || K % 8 || (!g_idx && K % group_size) || N <= 0 || (qzeros && N % 8))
        return st::fail(ST_ERR_SHAPE, "st_gptq_i4_dequant: K=%d N=%d group_size=%d", K, N, group_size);
    const long long nwords = (long long)(K / 8) * N;
    const int zoff = (flags & ST_FLAG_ZEROS_PLUS_ONE) ? 1 : 0;
    dim3 grid((unsigned)((nwords + 255) / 256)), block(256);
    if (out_dtype == ST_F32)
        st::launch(ctx, dequant_kernel<ST_F32>, grid, block, 0, qweight, scales, qzeros, g_idx, out, K, N,
                           group_size, zoff);
    else if (out_dtype == ST_BF16)
        st::launch(ctx, dequant_kernel<ST_BF16>, grid, block, 0, qweight, scales, qzeros, g_idx, out, K, N,
                           group_size, zoff);
    else
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_dequant: out_dtype %d (F32 or BF16)", out_dtype);
    return st::launch_check("dequant_kernel");
}

int st_gptq_i4_act_order(st_context *ctx, const uint32_t *qweight, const int32_t *g_idx, uint32_t *qweight_out,
                         int32_t *perm_out, int K, int N, int group_size) {
    if (!ctx || !qweight || !g_idx || !qweight_out || !perm_out)
        return st::fail(ST_ERR_INVALID, "st_gptq_i4_act_order: NULL argument");
    if (group_size <= 0 || K <= 0 || K % group_size || K % 8 || N <= 0)
        return st::fail(ST_ERR_SHAPE, "st_gptq_i4_act_order: K=%d N=%d group_size=%d", K, N, group_size);
    if (qweight_out == qweight) return st::fail(ST_ERR_INVALID, "st_gptq_i4_act_order: in-place not supported");
    const int G = K / group_size;
    std::vector<int32_t> gi(K), perm(K);
    ST_HIP(hipMemcpyAsync(gi.data(), g_idx, sizeof(int32_t) * K, hipMemcpyDeviceToHost, ctx->stream));
    ST_HIP(hipStreamSynchronize(ctx->stream));
    // Stable counting sort by group.
    std::vector<int> start(G + 1, 0);
    for (int k = 0; k < K; ++k) {
        if (gi[k] < 0 || gi[k] >= G)
            return st::fail(ST_ERR_SHAPE, "st_gptq_i4_act_order: g_idx[%d]=%d outside [0,%d)", k, gi[k], G);
        start[gi[k] + 1]++;
    }
    for (int g = 0; g < G; ++g) {
        if (start[g + 1] != group_size)
            return st::fail(ST_ERR_SHAPE, "st_gptq_i4_act_order: group %d holds %d rows, expected %d", g, start[g + 1],
                            group_size);
        start[g + 1] += start[g];
    }
    for (int k = 0; k < K; ++k) perm[start[gi[k]]++] = k;
    ST_HIP(hipMemcpyAsync(perm_out, perm.data(), sizeof(int32_t) * K, hipMemcpyHostToDevice, ctx->stream));
    const long long nwords = (long long)(K / 8) * N;
    st::launch(ctx, act_order_gather, dim3((unsigned)((nwords + 255) / 256)), dim3(256), 0, qweight,
                       perm_out, qweight_out, K, N);
    if (int rc = st::launch_check("act_order_gather")) return rc;
    ST_HIP(hipStreamSynchronize(ctx->stream));
    return ST_OK;
}

}  // extern "C"
