// Decode kernel variants for FMT_I8T (tiled INT8), act-order false (one translation unit
// per weight format and act-order so the variants compile in parallel).
#include "qmv_kernel.hpp"

namespace st {
namespace qmv {
template <>
int dispatch<FMT_I8T, false>(st_context *ctx, Params &p, int nsrc, int xm) {
    return dispatch_impl<FMT_I8T, false>(ctx, p, nsrc, xm);
}
}  // namespace qmv
}  // namespace st
