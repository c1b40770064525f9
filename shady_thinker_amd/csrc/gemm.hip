// Prefill GEMM: not built yet; validates arguments and reports UNSUPPORTED.
#include "common.hpp"
extern "C" int st_gptq_i4_gemm(st_context *ctx, const uint16_t *a, const uint32_t *qweight, const uint16_t *scales,
                               const uint32_t *, const int32_t *, void *c, int, int, int, int, int, uint32_t) {
    if (!ctx || !a || !qweight || !scales || !c) return st::fail(ST_ERR_INVALID, "st_gptq_i4_gemm: NULL argument");
    return st::fail(ST_ERR_UNSUPPORTED, "st_gptq_i4_gemm: not built yet");
}
