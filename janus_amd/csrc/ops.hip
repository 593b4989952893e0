// ops.hip -- the extern "C" operator entry points: host-side validation
// (mirroring the reference's Result<_, ComputeError> checks) followed by the
// kernel launch on the context's stream.
#include <cmath>
#include <vector>

#include "internal.h"

namespace janus {

int gemm_dispatch(janus_ctx *ctx, const void *a, int a_dt, const janus_weight *w, void *c, int c_dt,
                  uint32_t rows, const float *residual) {
    if (rows == 1) return gemv_dispatch(ctx, a, a_dt, w, c, c_dt, residual);
    return smallm_gemm_launch(ctx, a, a_dt, w, c, c_dt, rows, residual);
}
}  // namespace janus

using namespace janus;

namespace {
int check_ctx(janus_ctx *ctx) { return ctx ? JANUS_OK : JANUS_E_INVALID_ARG; }
}  // namespace

extern "C" {

int janus_gemm_auto(janus_ctx *ctx, const void *a, int a_dt, const janus_weight *w, void *c, int c_dt,
                    uint32_t batch, uint32_t m, uint32_t k, uint32_t n) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!a || !w || !c) return fail(ctx, JANUS_E_INVALID_ARG, "gemm_auto: null buffer");
    if (!is_act_dtype(a_dt) || !is_act_dtype(c_dt))
        return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "gemm_auto: activations must be F32 or F16");
    if (k != w->k || n != w->n)
        return fail(ctx, JANUS_E_INVALID_DIM,
                    "gemm_auto: weight is [" + std::to_string(w->n) + "x" + std::to_string(w->k) + "], got k=" +
                        std::to_string(k) + " n=" + std::to_string(n));
    uint64_t rows = (uint64_t)batch * m;
    if (rows == 0) return fail(ctx, JANUS_E_INVALID_DIM, "gemm_auto: batch * m must be >= 1");
    if (rows > 64) return fail(ctx, JANUS_E_INVALID_DIM, "gemm_auto: at most 64 rows per call");
    if (int e = need_device(ctx)) return e;
    return gemm_dispatch(ctx, a, a_dt, w, c, c_dt, (uint32_t)rows, nullptr);
}

int janus_gemm_residual(janus_ctx *ctx, const void *a, int a_dt, const janus_weight *w, const float *residual,
                        float *c, uint32_t rows, uint32_t k, uint32_t n) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!a || !w || !c || !residual) return fail(ctx, JANUS_E_INVALID_ARG, "gemm_residual: null buffer");
    if (!is_act_dtype(a_dt)) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "gemm_residual: bad activation dtype");
    if (k != w->k || n != w->n) return fail(ctx, JANUS_E_INVALID_DIM, "gemm_residual: shape mismatch");
    if (rows == 0 || rows > 64) return fail(ctx, JANUS_E_INVALID_DIM, "gemm_residual: rows must be 1..64");
    if (int e = need_device(ctx)) return e;
    return gemm_dispatch(ctx, a, a_dt, w, c, JANUS_DT_F32, rows, residual);
}

int janus_rmsnorm(janus_ctx *ctx, const float *in, void *out, int out_dt, const float *gamma, uint32_t batch,
                  uint32_t hidden, float eps) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!in || !out || !gamma) return fail(ctx, JANUS_E_INVALID_ARG, "rmsnorm: null buffer");
    if (!is_act_dtype(out_dt)) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "rmsnorm: bad output dtype");
    if (batch == 0 || hidden == 0) return fail(ctx, JANUS_E_INVALID_DIM, "rmsnorm: empty input");
    if (int e = need_device(ctx)) return e;
    return rmsnorm_launch(ctx, in, out, out_dt, gamma, batch, hidden, eps);
}

static int ew(janus_ctx *ctx, int op, const float *a, const float *b, void *out, int out_dt, uint32_t n,
              const char *name) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!a || !out || (op != EW_SILU && !b)) return fail(ctx, JANUS_E_INVALID_ARG, std::string(name) + ": null buffer");
    if (n == 0) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    return elementwise_launch(ctx, op, a, b, out, out_dt, n);
}

int janus_silu(janus_ctx *ctx, const float *in, float *out, uint32_t size) {
    return ew(ctx, EW_SILU, in, nullptr, out, JANUS_DT_F32, size, "silu");
}
int janus_elementwise_mul(janus_ctx *ctx, const float *a, const float *b, float *out, uint32_t size) {
    return ew(ctx, EW_MUL, a, b, out, JANUS_DT_F32, size, "elementwise_mul");
}
int janus_add_tensors(janus_ctx *ctx, const float *a, const float *b, float *out, uint32_t size) {
    return ew(ctx, EW_ADD, a, b, out, JANUS_DT_F32, size, "add_tensors");
}
int janus_swiglu(janus_ctx *ctx, const float *gate, const float *up, void *out, int out_dt, uint32_t size) {
    if (ctx && !is_act_dtype(out_dt)) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "swiglu: bad output dtype");
    return ew(ctx, EW_SWIGLU, gate, up, out, out_dt, size, "swiglu");
}

int janus_rope_table(janus_ctx *ctx, float *d_table, uint32_t max_seq, uint32_t hd, float base) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!d_table) return fail(ctx, JANUS_E_INVALID_ARG, "rope_table: null buffer");
    if (hd == 0 || hd % 2 || max_seq == 0) return fail(ctx, JANUS_E_INVALID_DIM, "rope_table: head_dim must be even");
    if (int e = need_device(ctx)) return e;
    // model/transformer/constructor.rs:462-480 in binary32 with the C library's
    // powf/cosf/sinf (what Rust's f32 methods call on linux-gnu).
    const uint32_t half = hd / 2;
    std::vector<float> tab((size_t)max_seq * half * 2);
    for (uint32_t p = 0; p < max_seq; ++p)
        for (uint32_t i = 0; i < half; ++i) {
            float exponent = (float)(2 * i) / (float)hd;
            float theta = powf(base, exponent);
            float angle = (float)p / theta;
            tab[((size_t)p * half + i) * 2] = cosf(angle);
            tab[((size_t)p * half + i) * 2 + 1] = sinf(angle);
        }
    JANUS_HIP_CHECK(ctx, hipMemcpyAsync(d_table, tab.data(), tab.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
    return JANUS_OK;
}

int janus_rope(janus_ctx *ctx, const float *in, float *out, const float *d_table, uint32_t batch, uint32_t heads,
               uint32_t hd, uint32_t position, const int32_t *d_positions) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!in || !out || !d_table) return fail(ctx, JANUS_E_INVALID_ARG, "rope: null buffer");
    if (hd == 0 || hd % 2) return fail(ctx, JANUS_E_INVALID_DIM, "rope: head_dim must be even");
    if (batch == 0 || heads == 0) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    return rope_launch(ctx, in, out, d_table, batch, heads, hd, position, d_positions);
}

int janus_kv_update(janus_ctx *ctx, const float *k_new, const float *v_new, void *k_cache, void *v_cache,
                    int kv_dt, uint32_t batch, uint32_t kv_heads, uint32_t hd, uint32_t position,
                    uint32_t max_seq_len, const int32_t *d_row_base, const int32_t *d_positions) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!k_new || !v_new || !k_cache || !v_cache) return fail(ctx, JANUS_E_INVALID_ARG, "kv_update: null buffer");
    if (!is_act_dtype(kv_dt)) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "kv_update: kv dtype must be F32 or F16");
    if (!d_positions && position >= max_seq_len)
        return fail(ctx, JANUS_E_KV_OVERFLOW, "KV cache position " + std::to_string(position) +
                                                  " exceeds max_seq_len " + std::to_string(max_seq_len));
    if (batch == 0 || kv_heads == 0 || hd == 0) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    return kv_update_launch(ctx, k_new, v_new, k_cache, v_cache, kv_dt, batch, kv_heads * hd, position,
                            max_seq_len, d_row_base, d_positions);
}

namespace {
// Host checks shared by the two attention entry points (ops/attention.rs:78-235).
int attention_args(janus_ctx *ctx, const float *q, const void *k_cache, const void *v_cache, int kv_dt,
                   const float *out, uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t seq_len,
                   uint32_t max_seq_len, const int32_t *d_seq_lens) {
    if (!q || !k_cache || !v_cache || !out) return fail(ctx, JANUS_E_INVALID_ARG, "attention: null buffer");
    if (!is_act_dtype(kv_dt)) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "attention: kv dtype must be F32 or F16");
    if (kv_heads == 0 || heads == 0 || heads % kv_heads)
        return fail(ctx, JANUS_E_INVALID_DIM, "attention: heads must be a multiple of kv_heads");
    if (hd != 64 && hd != 128) return fail(ctx, JANUS_E_INVALID_DIM, "attention: head_dim must be 64 or 128");
    if (!d_seq_lens && seq_len > max_seq_len)
        return fail(ctx, JANUS_E_KV_OVERFLOW, "attention: seq_len exceeds max_seq_len");
    return JANUS_OK;
}
}  // namespace

int janus_attention(janus_ctx *ctx, const float *q, const void *k_cache, const void *v_cache, int kv_dt, float *out,
                    uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t seq_len,
                    uint32_t max_seq_len, const int32_t *d_row_base, const int32_t *d_seq_lens,
                    uint32_t max_len_hint, float scale) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (int e = attention_args(ctx, q, k_cache, v_cache, kv_dt, out, heads, kv_heads, hd, seq_len, max_seq_len,
                               d_seq_lens))
        return e;
    if (batch == 0) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    uint32_t max_len = d_seq_lens ? (max_len_hint ? max_len_hint : max_seq_len) : seq_len;
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)hd);
    return attention_launch(ctx, q, k_cache, v_cache, kv_dt, out, batch, heads, kv_heads, hd, seq_len, max_seq_len,
                            d_row_base, d_seq_lens, max_len, scale);
}

int janus_attention_noalloc(janus_ctx *ctx, const float *q, const void *k_cache, const void *v_cache, int kv_dt,
                            float *out, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                            uint32_t seq_len, uint32_t max_seq_len, const int32_t *d_row_base,
                            const int32_t *d_seq_lens, uint32_t max_len_hint, float scale) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (int e = attention_args(ctx, q, k_cache, v_cache, kv_dt, out, heads, kv_heads, hd, seq_len, max_seq_len,
                               d_seq_lens))
        return e;
    if (batch == 0) return JANUS_OK;
    const uint32_t max_len = d_seq_lens ? (max_len_hint ? max_len_hint : max_seq_len) : seq_len;
    // the same split plan as janus_attention, checked against the fixed scratch on the host
    const size_t need = attention_ws_bytes(ctx, batch, heads, kv_heads, hd, max_len, kv_dt == JANUS_DT_F16);
    if (need > kAttnScratchBytes)
        return fail(ctx, JANUS_E_INVALID_DIM,
                    "attention_noalloc: split partials need " + std::to_string(need) + " bytes, above the " +
                        std::to_string(kAttnScratchBytes) + "-byte fixed scratch; use janus_attention");
    if (int e = need_device(ctx)) return e;
    if (!ctx->attn_scratch)
        return fail(ctx, JANUS_E_HIP, "attention_noalloc: no fixed scratch on this device: " + ctx->attn_scratch_error);
    if (scale <= 0.0f) scale = 1.0f / sqrtf((float)hd);
    return attention_launch(ctx, q, k_cache, v_cache, kv_dt, out, batch, heads, kv_heads, hd, seq_len, max_seq_len,
                            d_row_base, d_seq_lens, max_len, scale, 0, ctx->attn_scratch, kAttnScratchBytes);
}

int janus_embed(janus_ctx *ctx, const janus_weight *table, const uint32_t *h_ids, uint32_t batch, float *out) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!table || !h_ids || !out) return fail(ctx, JANUS_E_INVALID_ARG, "embed: null argument");
    if (table->type != JANUS_DT_F16) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "embed: table must be F16");
    for (uint32_t i = 0; i < batch; ++i)
        if (h_ids[i] >= table->n)
            return fail(ctx, JANUS_E_TOKEN_RANGE, "Token ID " + std::to_string(h_ids[i]) + " at batch index " +
                                                      std::to_string(i) + " exceeds vocab size " +
                                                      std::to_string(table->n));
    if (batch == 0) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    return embed_launch(ctx, table, h_ids, nullptr, batch, out);
}

int janus_embed_device(janus_ctx *ctx, const janus_weight *table, const int32_t *d_ids, uint32_t batch, float *out) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!table || !d_ids || !out) return fail(ctx, JANUS_E_INVALID_ARG, "embed_device: null argument");
    if (table->type != JANUS_DT_F16) return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "embed: table must be F16");
    if (batch == 0) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    return embed_launch(ctx, table, nullptr, d_ids, batch, out);
}

int janus_argmax(janus_ctx *ctx, const float *logits, int32_t *d_out, uint32_t vocab, uint32_t batch, int tie) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!logits || !d_out) return fail(ctx, JANUS_E_INVALID_ARG, "argmax: null buffer");
    if (tie != JANUS_TIE_LAST && tie != JANUS_TIE_WGSL) return fail(ctx, JANUS_E_INVALID_ARG, "argmax: bad tie rule");
    if (vocab == 0) return fail(ctx, JANUS_E_INVALID_DIM, "argmax: empty vocabulary");
    if (batch == 0) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    return argmax_launch(ctx, logits, d_out, vocab, batch, tie);
}

int janus_repetition_penalty(janus_ctx *ctx, float *logits, uint32_t vocab, const int32_t *d_context,
                             uint32_t n_context, float penalty) {
    if (check_ctx(ctx)) return JANUS_E_INVALID_ARG;
    if (!logits || (n_context && !d_context)) return fail(ctx, JANUS_E_INVALID_ARG, "penalty: null buffer");
    if (n_context == 0) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    return penalty_launch(ctx, logits, vocab, d_context, n_context, penalty);
}

}  // extern "C"
