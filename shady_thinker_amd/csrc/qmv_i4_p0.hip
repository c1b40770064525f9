// Decode kernel variants for FMT_I4, act-order false (one translation unit
// per weight format and act-order so the variants compile in parallel).
#include "qmv_kernel.hpp"

namespace st {
namespace qmv {
template <>
int dispatch<FMT_I4, false>(st_context *ctx, Params &p, int nsrc, int xm) {
    return dispatch_impl<FMT_I4, false>(ctx, p, nsrc, xm);
}
}  // namespace qmv
}  // namespace st
