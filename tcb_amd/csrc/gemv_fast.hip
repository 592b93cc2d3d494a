// gemv_fast.hip -- decode GEMV in the factored (tolerance-bound) order. Placeholder: routes to the exact
// kernels until the factored kernels land.
#include "trhip_internal.hpp"

namespace trhip {
int launch_gemv(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc,
                int mode);
int launch_gemv_fast(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     bool acc) {
    return launch_gemv(ctx, w, row0, N, x, c, acc, TRHIP_MODE_EXACT);
}
}  // namespace trhip
