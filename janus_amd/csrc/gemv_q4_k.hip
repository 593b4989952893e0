// gemv_q4_k.hip -- the M = 1 kernels of gemv_impl.h instantiated for Q4_K weights
// (one translation unit per weight format, compiled in parallel).
#include "gemv_impl.h"

namespace janus {

int gemv_run_q4_k(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done) {
    return gemv_run<FQ4_K>(ctx, a, mode, x_dt, done);
}

}  // namespace janus
