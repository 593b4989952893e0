// gemv.hip -- M = 1 product dispatch: builds the launch arguments and hands
// them to the kernels of the weight's format (gemv_impl.h, instantiated once
// per format in gemv_q4_0.hip ... gemv_f16.hip).
//
// Replaces gemm_q8_0_into / gemm_q4_k_into / matmul::gemm at M=1
// (crates/janus-engine/src/compute/ops/quantized.rs:188-378,
// ops/matmul.rs:228-298) and adds Q4_0, Q5_K, which the reference cannot run
// (compute/engine.rs:833-838).
#include <cstring>

#include "gemv_impl.h"

namespace janus {

namespace {

// Units per row for a format, the format's runner, or null (unsupported type).
using RunFn = int (*)(janus_ctx *, const GemvArgs &, int, int, bool *);

RunFn runner(const janus_weight *w, uint32_t &units) {
    switch (w->type) {
    case JANUS_DT_Q4_0: units = w->k / 32; return gemv_run_q4_0;
    case JANUS_DT_Q8_0: units = w->k / 32; return gemv_run_q8_0;
    case JANUS_DT_Q4_K: units = w->k / 32; return gemv_run_q4_k;
    case JANUS_DT_Q5_K: units = w->k / 32; return gemv_run_q5_k;
    case JANUS_DT_F16: units = w->k % 8 ? 0 : w->k / 8; return gemv_run_f16;
    default: return nullptr;
    }
}

}  // namespace

int gemv_pair_dispatch(janus_ctx *ctx, const void *x, const janus_weight *w, int epi, void *y, int y_f16, void *kc,
                       void *vc, int kv_f16, const float *rope, const int32_t *d_pos, const int32_t *d_rowbase,
                       uint32_t q_pairs, uint32_t k_pairs, uint32_t half_hd, uint32_t kv_row, const float *gamma,
                       float eps, int x32) {
    GemvArgs a;
    std::memset(&a, 0, sizeof(a));
    a.gamma = gamma;
    a.eps = eps;
    a.w.qs = w->qs;
    a.w.sc = w->sc;
    a.x = x;
    a.y = y;
    a.n = w->n;
    a.k = w->k;
    a.out_f16 = y_f16;
    a.epi = epi == 0 ? EPI_QKV_ROPE : EPI_SWIGLU;
    a.kc = kc;
    a.vc = vc;
    a.kv_f16 = kv_f16;
    a.rope = rope;
    a.d_pos = d_pos;
    a.d_rowbase = d_rowbase;
    a.q_pairs = q_pairs;
    a.k_pairs = k_pairs;
    a.half_hd = half_hd;
    a.kv_row = kv_row;
    if (w->n % 2) return fail(ctx, JANUS_E_INVALID_DIM, "paired gemv: odd row count");
    const bool norm = gamma != nullptr;
    if (norm && w->k > 16u * 512u * NORM_MAXG) return fail(ctx, JANUS_E_INVALID_DIM, "paired gemv: normalised row too long");
    RunFn run = runner(w, a.units);
    if (!run) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "paired gemv: unsupported weight type");
    if (w->type == JANUS_DT_F16 && a.units == 0)
        return fail(ctx, JANUS_E_INVALID_DIM, "paired gemv: F16 rows need k % 8 == 0");
    bool done = false;
    const int e = run(ctx, a, GEMV_PAIR | (norm ? GEMV_NORM : 0) | (x32 ? GEMV_X32 : 0),
                      x32 ? JANUS_DT_F32 : JANUS_DT_F16, &done);
    if (!e && !done) return fail(ctx, JANUS_E_INVALID_DIM, "paired gemv: row too long");
    return e;
}

int gemv_norm_dispatch(janus_ctx *ctx, const float *x, const float *gamma, float eps, const janus_weight *w, float *y,
                       unsigned long long *best, const uint32_t *counts, const SamplerDev *sampler, int x32) {
    GemvArgs a;
    std::memset(&a, 0, sizeof(a));
    a.w.qs = w->qs;
    a.w.sc = w->sc;
    a.x = x;
    a.y = y;
    a.n = w->n;
    a.k = w->k;
    a.epi = best ? EPI_ARGMAX : EPI_STORE;
    a.best = best;
    a.counts = counts;
    a.sampler = sampler;
    a.gamma = gamma;
    a.eps = eps;
    if (w->k > 16u * 512u * NORM_MAXG) return fail(ctx, JANUS_E_INVALID_DIM, "normed gemv: row too long");
    RunFn run = runner(w, a.units);
    if (!run) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "normed gemv: unsupported weight type");
    if (w->type == JANUS_DT_F16 && a.units == 0)
        return fail(ctx, JANUS_E_INVALID_DIM, "normed gemv: F16 rows need k % 8 == 0");
    bool done = false;
    const int e = run(ctx, a, GEMV_NORM | (x32 ? GEMV_X32 : 0), JANUS_DT_F32, &done);
    if (!e && !done) return fail(ctx, JANUS_E_INVALID_DIM, "normed gemv: row too long");
    return e;
}

int gemv_dispatch(janus_ctx *ctx, const void *x, int x_dt, const janus_weight *w, void *y, int y_dt,
                  const float *residual) {
    GemvArgs a;
    std::memset(&a, 0, sizeof(a));
    a.w.qs = w->qs;
    a.w.sc = w->sc;
    a.x = x;
    a.y = y;
    a.resid = residual;
    a.n = w->n;
    a.k = w->k;
    a.out_f16 = (y_dt == JANUS_DT_F16);
    a.epi = residual ? EPI_RESIDUAL : EPI_STORE;
    RunFn run = runner(w, a.units);
    if (!run)
        return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE,
                    "FATAL: No compute kernel bound for tensor type " + std::to_string(w->type));
    bool done = false;
    const int e = run(ctx, a, GEMV_PLAIN, x_dt, &done);
    if (!e && !done) return fail(ctx, JANUS_E_INVALID_DIM, "gemv: row too long");
    return e;
}

}  // namespace janus
