// gemv_f16.hip -- the M = 1 kernels of gemv_impl.h instantiated for F16 weights
// (one translation unit per weight format, compiled in parallel).
#include "gemv_impl.h"

namespace janus {

int gemv_run_f16(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done) {
    return gemv_run<FF16>(ctx, a, mode, x_dt, done);
}

}  // namespace janus
