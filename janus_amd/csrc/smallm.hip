// smallm.hip -- products with 2..64 activation rows (ragged decode batches).
#include "internal.h"

namespace janus {

int smallm_gemm_launch(janus_ctx *ctx, const void *a, int a_dt, const janus_weight *w, void *c, int c_dt,
                       uint32_t rows, const float *residual) {
    const size_t as = act_bytes(a_dt) * w->k, cs = act_bytes(c_dt) * w->n;
    for (uint32_t r = 0; r < rows; ++r) {
        int e = gemv_dispatch(ctx, (const uint8_t *)a + r * as, a_dt, w, (uint8_t *)c + r * cs, c_dt,
                              residual ? residual + (size_t)r * w->n : nullptr);
        if (e) return e;
    }
    return JANUS_OK;
}

}  // namespace janus
