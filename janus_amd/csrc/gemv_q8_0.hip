// gemv_q8_0.hip -- the M = 1 kernels of gemv_impl.h instantiated for Q8_0 weights
// (one translation unit per weight format, compiled in parallel).
#include "gemv_impl.h"

namespace janus {

int gemv_run_q8_0(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done) {
    return gemv_run<FQ8_0>(ctx, a, mode, x_dt, done);
}

}  // namespace janus
