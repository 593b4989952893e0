// model.hip -- the C++ decode driver (include/janus_model.h).
//
// Reference call stack mirrored here (crates/janus-engine/src/):
//   Model::forward            model/transformer/forward.rs:25-119
//   Model::forward_batch      model/transformer/forward.rs:141-245
//   TransformerBlock::forward model/block.rs:190-458 (op order per layer)
//   Model::generate           model/transformer/generation.rs:129-323
//   Model::generate_batch     model/transformer/generation.rs:673-870
//   Sampler::sample (greedy)  model/sampler.rs:146-209, 599-613, 784-795
//   Sampler::sample_batch     model/sampler.rs:379-428
// Differences by design: the o-proj and down-proj residual adds are fused
// into the products' epilogues (same f32 addition), SiLU and the gate*up
// product are one kernel, K/V may be stored as binary16, every sequence of a
// batch carries its own position (the reference shares one, rope.wgsl:64-66)
// and its own KV slot (a row-base table), and sampling runs on the device.
//
// Decode state lives on the device, one entry per batch row: the token the
// next step consumes, its position, the KV row base, the prompt still to
// prefill, the generated tokens, their occurrence counts (the repetition
// penalty's context) and a done flag. One step (forward, greedy choice,
// advance) is either enqueued directly or captured per row count and
// context-length bucket into a HIP graph and replayed; generate and
// generate_batch both run on replays.
#include <climits>
#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/janus_model.h"
#include "internal.h"

using namespace janus;

namespace {

// Per-row control block of the device-side decode loop.
struct RowDev {
    int32_t prompt_len;   // prompt tokens at prompts[row][0, prompt_len); 0: decode from the first step
    int32_t max_new;      // the row is done after this many generated tokens
    int32_t nout;         // generated tokens so far (out[row][0, nout))
    int32_t done;
    int32_t eos_mode;     // EOS_* below
    int32_t nan;          // set (with done) when the step's logits held a NaN under the CPU-path rules
};

// What a generated 128001 / 128009 (LLAMA3_END_OF_TEXT_ID / LLAMA3_EOT_ID) does.
enum { EOS_IGNORE = 0, EOS_STOP_DROP = 1, EOS_STOP_KEEP = 2 };

constexpr int kMaxRows = 64;

}  // namespace

struct janus_model {
    janus_ctx *ctx = nullptr;
    janus_model_config cfg{};
    struct Layer {
        float *attn_norm = nullptr, *ffn_norm = nullptr;
        janus_weight *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
        janus_weight *gate = nullptr, *up = nullptr, *down = nullptr;
        // fused copies for the single-sequence path (built by ensure_fused)
        janus_weight *qkv = nullptr;   // rows: q RoPE pairs, k RoPE pairs, v
        janus_weight *gu = nullptr;    // rows: gate_0, up_0, gate_1, up_1, ...
    };
    bool fused_ready = false;
    bool tiles_ready = false;   // T32 tile copies of the batched products built
    std::vector<Layer> layers;
    janus_weight *tok_embd = nullptr, *lm_head = nullptr;
    float *out_norm = nullptr;
    // activations (max_batch rows each)
    float *hidden = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *h1 = nullptr;
    float *gate = nullptr, *up = nullptr, *logits = nullptr;
    void *xn = nullptr, *act = nullptr;   // act_dtype
    void *attn16 = nullptr;               // attention output as binary16 (act_dtype F16)
    void *kcache = nullptr, *vcache = nullptr;
    bool kv_external = false;
    size_t layer_kv_elems = 0;
    float *rope = nullptr;
    // device decode state, max_batch rows
    int32_t *d_pos = nullptr, *d_lens = nullptr, *d_tokens = nullptr, *d_rowbase = nullptr;
    int32_t *d_feed = nullptr;   // the token each row consumes in the next step
    RowDev *d_rows = nullptr;
    int32_t *d_prompts = nullptr;   // [max_batch][max_seq_len]
    int32_t *d_out = nullptr;       // [max_batch][max_seq_len]
    uint32_t *d_counts = nullptr;   // [max_batch][vocab]
    unsigned long long *d_best = nullptr;   // greedy key per row (zero between steps)
    SamplerDev *d_sampler = nullptr;
    SamplerDev h_sampler{1.0f, SAMPLE_ARGMAX};
    // captured steps, one per row count and length bucket: graphs[nseq * nbuckets + b]
    std::vector<hipGraphExec_t> graphs;
    uint32_t nbuckets = 1;
    std::vector<uint32_t> h_pos;   // graph_run: host mirror of the rows' positions
    uint32_t graph_nseq = 0;
    hipStream_t cap_stream = nullptr;
    // generate_stream: pinned slots the steps' outcomes are copied to, and
    // the events that mark them written
    struct StreamSlot {
        RowDev row;
        int32_t token;
    } *h_stream = nullptr;
    hipEvent_t stream_ev[2] = {nullptr, nullptr};
};

namespace {

size_t kv_elem_bytes(int dt) { return dt == JANUS_DT_F16 ? 2 : 4; }

int parse_layer_name(const std::string &name, uint32_t *layer, std::string *rest) {
    if (name.rfind("blk.", 0) != 0) return 0;
    size_t dot = name.find('.', 4);
    if (dot == std::string::npos) return 0;
    *layer = (uint32_t)std::stoul(name.substr(4, dot - 4));
    *rest = name.substr(dot + 1);
    return 1;
}

struct AdvanceArgs {
    int32_t *pos, *lens, *tokens, *feed;
    RowDev *rows;
    const int32_t *prompts;
    int32_t *out;
    uint32_t *counts;
    unsigned long long *best;
    const SamplerDev *sampler;
    uint32_t n, max_seq, vocab;
};

// End of a decode step, one lane per row. The step consumed tokens[r] at
// position pos[r]; the next token is the next prompt token while the prompt
// lasts, the last prompt token again right after it (the first decode step
// re-feeds it at position n, generation.rs:176,217), and from then on the
// greedy choice of this step (best[r]). A chosen token is appended to the
// row's generated list and counted for the repetition penalty. tokens[r] is
// the last token chosen (or the next prompt token); feed[r] the token the
// next step consumes. A row that is done keeps its feed token, position and
// length, so a later replay recomputes its last step exactly and rewrites
// that position's K/V rows with the values they hold.
__global__ void advance_kernel(AdvanceArgs a) {
    const uint32_t r = threadIdx.x;
    if (r >= a.n) return;
    const unsigned long long key = a.best[r];
    a.best[r] = 0;
    RowDev c = a.rows[r];
    if (c.done) return;
    const int32_t p = a.pos[r];
    int32_t next;
    if (p + 1 < c.prompt_len) {
        next = a.prompts[(size_t)r * a.max_seq + p + 1];
    } else if (p + 1 == c.prompt_len) {
        next = a.prompts[(size_t)r * a.max_seq + p];
    } else if (key == kNanKey) {
        next = a.tokens[r];   // nothing is chosen: the row stops with its NaN flag
        c.nan = 1;
        c.done = 1;
    } else {
        next = (int32_t)sampler_key_index(key, a.sampler->mode);
        if ((uint32_t)next >= a.vocab) next = 0;
        const bool eos = next == 128001 || next == 128009;
        if (!(eos && c.eos_mode == EOS_STOP_DROP)) {
            if ((uint32_t)c.nout < a.max_seq) a.out[(size_t)r * a.max_seq + c.nout] = next;
            c.nout += 1;
            a.counts[(size_t)r * a.vocab + next] += 1;
        }
        if ((eos && c.eos_mode != EOS_IGNORE) || c.nout >= c.max_new) c.done = 1;
    }
    a.tokens[r] = next;
    if (!c.done) {
        if ((uint32_t)p + 1 >= a.max_seq) {
            c.done = 1;   // no room for another position (generation.rs:200-205)
        } else {
            a.pos[r] = p + 1;
            a.lens[r] = p + 2;
            a.feed[r] = next;
        }
    }
    a.rows[r] = c;
}

// One decode step over nseq rows whose ids are either host ids or device ids
// and whose positions / lengths / row bases are already on the device.
int forward_rows(janus_model *m, const uint32_t *h_ids, const int32_t *d_ids, uint32_t nseq, uint32_t max_len) {
    janus_ctx *ctx = m->ctx;
    const janus_model_config &c = m->cfg;
    const uint32_t kvd = c.kv_heads * c.head_dim;
    int e;
    if ((e = embed_launch(ctx, m->tok_embd, h_ids, d_ids, nseq, m->hidden))) return e;
    for (uint32_t l = 0; l < c.layers; ++l) {
        const janus_model::Layer &L = m->layers[l];
        void *kc = (uint8_t *)m->kcache + (size_t)l * m->layer_kv_elems * kv_elem_bytes(c.kv_dtype);
        void *vc = (uint8_t *)m->vcache + (size_t)l * m->layer_kv_elems * kv_elem_bytes(c.kv_dtype);
        // attention block (block.rs:223-355)
        if ((e = rmsnorm_launch(ctx, m->hidden, m->xn, c.act_dtype, L.attn_norm, nseq, c.hidden, c.rms_eps))) return e;
        if ((e = gemm_dispatch(ctx, m->xn, c.act_dtype, L.q, m->q, JANUS_DT_F32, nseq, nullptr))) return e;
        if ((e = gemm_dispatch(ctx, m->xn, c.act_dtype, L.k, m->k, JANUS_DT_F32, nseq, nullptr))) return e;
        if ((e = gemm_dispatch(ctx, m->xn, c.act_dtype, L.v, m->v, JANUS_DT_F32, nseq, nullptr))) return e;
        if ((e = rope_launch(ctx, m->q, m->q, m->rope, nseq, c.heads, c.head_dim, 0, m->d_pos))) return e;
        if ((e = rope_launch(ctx, m->k, m->k, m->rope, nseq, c.kv_heads, c.head_dim, 0, m->d_pos))) return e;
        if ((e = kv_update_launch(ctx, m->k, m->v, kc, vc, c.kv_dtype, nseq, kvd, 0, c.max_seq_len, m->d_rowbase,
                                  m->d_pos)))
            return e;
        // attention output in the products' activation dtype
        const bool a16 = c.act_dtype == JANUS_DT_F16;
        void *att = a16 ? m->attn16 : (void *)m->attn;
        if ((e = attention_launch(ctx, m->q, kc, vc, c.kv_dtype, att, nseq, c.heads, c.kv_heads, c.head_dim, 0,
                                  c.max_seq_len, m->d_rowbase, m->d_lens, max_len, 1.0f / sqrtf((float)c.head_dim),
                                  a16)))
            return e;
        // o-proj with the residual add fused: h1 = hidden + attn . Wo^T
        if ((e = gemm_dispatch(ctx, att, c.act_dtype, L.o, m->h1, JANUS_DT_F32, nseq, m->hidden))) return e;
        // feed-forward block (block.rs:370-447)
        if ((e = rmsnorm_launch(ctx, m->h1, m->xn, c.act_dtype, L.ffn_norm, nseq, c.hidden, c.rms_eps))) return e;
        if ((e = gemm_dispatch(ctx, m->xn, c.act_dtype, L.gate, m->gate, JANUS_DT_F32, nseq, nullptr))) return e;
        if ((e = gemm_dispatch(ctx, m->xn, c.act_dtype, L.up, m->up, JANUS_DT_F32, nseq, nullptr))) return e;
        if ((e = elementwise_launch(ctx, EW_SWIGLU, m->gate, m->up, m->act, c.act_dtype, nseq * c.ffn))) return e;
        if ((e = gemm_dispatch(ctx, m->act, c.act_dtype, L.down, m->hidden, JANUS_DT_F32, nseq, m->h1))) return e;
    }
    // final norm + LM head (forward.rs:87-111)
    if ((e = rmsnorm_launch(ctx, m->hidden, m->xn, c.act_dtype, m->out_norm, nseq, c.hidden, c.rms_eps))) return e;
    return gemm_dispatch(ctx, m->xn, c.act_dtype, m->lm_head, m->logits, JANUS_DT_F32, nseq, nullptr);
}

// Copies `height` rows of a weight (quants and scales) from src rows
// [s0, s0 + height) to dst rows d0, d0 + dstep, ...
int copy_rows(janus_ctx *ctx, janus_weight *dst, uint32_t d0, uint32_t dstep, const janus_weight *src, uint32_t s0,
              uint32_t height) {
    const size_t qb = weight_qs_row_bytes(src->type, src->k), sb = weight_sc_row_elems(src->type, src->k) * 2;
    JANUS_HIP_CHECK(ctx, hipMemcpy2DAsync((uint8_t *)dst->qs + (size_t)d0 * qb, dstep * qb, src->qs + (size_t)s0 * qb,
                                          qb, qb, height, hipMemcpyDeviceToDevice, ctx->stream));
    if (sb)
        JANUS_HIP_CHECK(ctx, hipMemcpy2DAsync((uint8_t *)dst->sc + (size_t)d0 * sb, dstep * sb,
                                              (const uint8_t *)src->sc + (size_t)s0 * sb, sb, sb, height,
                                              hipMemcpyDeviceToDevice, ctx->stream));
    return JANUS_OK;
}

// Builds the fused QKV and gate/up weights of every layer once all tensors
// are present. QKV rows are ordered so each consecutive pair is a RoPE pair
// (i, i + hd/2) of one head (q heads, then k heads) followed by v in order;
// gate/up rows alternate gate_j, up_j. Layers whose tensors differ in type
// keep the unfused path.
int ensure_fused(janus_model *m) {
    if (m->fused_ready) return JANUS_OK;
    janus_ctx *ctx = m->ctx;
    const janus_model_config &c = m->cfg;
    const uint32_t hd = c.head_dim, half = hd / 2, kvd = c.kv_heads * hd;
    for (auto &L : m->layers) {
        const janus_weight *q = L.q, *k = L.k, *v = L.v;
        bool same = q->type == k->type && q->type == v->type && q->flags == k->flags && q->flags == v->flags &&
                    (q->type != JANUS_DT_F16 || q->k % 8 == 0);
        if (same && !L.qkv) {
            janus_weight *w = nullptr;
            if (int e = weight_alloc(ctx, q->type, c.hidden + 2 * kvd, c.hidden, q->flags, &w)) return e;
            for (uint32_t h = 0; h < c.heads; ++h) {
                if (int e = copy_rows(ctx, w, h * hd, 2, q, h * hd, half)) return e;
                if (int e = copy_rows(ctx, w, h * hd + 1, 2, q, h * hd + half, half)) return e;
            }
            for (uint32_t h = 0; h < c.kv_heads; ++h) {
                if (int e = copy_rows(ctx, w, c.hidden + h * hd, 2, k, h * hd, half)) return e;
                if (int e = copy_rows(ctx, w, c.hidden + h * hd + 1, 2, k, h * hd + half, half)) return e;
            }
            if (int e = copy_rows(ctx, w, c.hidden + kvd, 1, v, 0, kvd)) return e;
            L.qkv = w;
        }
        const janus_weight *g = L.gate, *u = L.up;
        same = g->type == u->type && g->flags == u->flags && (g->type != JANUS_DT_F16 || g->k % 8 == 0);
        if (same && !L.gu) {
            janus_weight *w = nullptr;
            if (int e = weight_alloc(ctx, g->type, 2 * c.ffn, c.hidden, g->flags, &w)) return e;
            if (int e = copy_rows(ctx, w, 0, 2, g, 0, c.ffn)) return e;
            if (int e = copy_rows(ctx, w, 1, 2, u, 0, c.ffn)) return e;
            L.gu = w;
        }
    }
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
    m->fused_ready = true;
    return JANUS_OK;
}

// The LM head runs as one LDS-staged GEMV with the final RMSNorm fused in
// (and optionally the greedy choice) when its rows fit that kernel.
bool can_fold_head(const janus_model *m) {
    const janus_weight *w = m->lm_head;
    if (w->type != JANUS_DT_F16 || w->k % 8) return false;
    return (w->k / 8 + 63) / 64 <= 8;
}

// Single-sequence step over the fused weights (binary16 or binary32 activations): per layer
// QKV (with the attention RMSNorm in its prologue and RoPE + KV append in its
// epilogue), attention, o-proj + residual, gate/up (FFN RMSNorm prologue,
// SwiGLU epilogue), down-proj + residual; the final RMSNorm runs in the LM
// head's prologue, and with fold_sample the greedy choice in its epilogue.
int forward_fused1(janus_model *m, const uint32_t *h_ids, const int32_t *d_ids, uint32_t max_len,
                   bool fold_sample = false) {
    janus_ctx *ctx = m->ctx;
    const janus_model_config &c = m->cfg;
    const uint32_t kvd = c.kv_heads * c.head_dim, half = c.head_dim / 2;
    const int kv16 = c.kv_dtype == JANUS_DT_F16;
    const int f32 = c.act_dtype == JANUS_DT_F32;   // the reference's dtype: every product reads binary32 x
    int e;
    if ((e = embed_launch(ctx, m->tok_embd, h_ids, d_ids, 1, m->hidden))) return e;
    for (uint32_t l = 0; l < c.layers; ++l) {
        const janus_model::Layer &L = m->layers[l];
        void *kc = (uint8_t *)m->kcache + (size_t)l * m->layer_kv_elems * kv_elem_bytes(c.kv_dtype);
        void *vc = (uint8_t *)m->vcache + (size_t)l * m->layer_kv_elems * kv_elem_bytes(c.kv_dtype);
        if ((e = gemv_pair_dispatch(ctx, m->hidden, L.qkv, 0, m->q, 0, kc, vc, kv16, m->rope, m->d_pos, m->d_rowbase,
                                    c.heads * half, c.kv_heads * half, half, kvd, L.attn_norm, c.rms_eps, f32)))
            return e;
        void *att = f32 ? (void *)m->attn : m->attn16;
        if ((e = attention_launch(ctx, m->q, kc, vc, c.kv_dtype, att, 1, c.heads, c.kv_heads, c.head_dim, 0,
                                  c.max_seq_len, m->d_rowbase, m->d_lens, max_len, 1.0f / sqrtf((float)c.head_dim),
                                  f32 ? 0 : 1)))
            return e;
        if ((e = gemm_dispatch(ctx, att, c.act_dtype, L.o, m->h1, JANUS_DT_F32, 1, m->hidden))) return e;
        if ((e = gemv_pair_dispatch(ctx, m->h1, L.gu, 1, m->act, f32 ? 0 : 1, nullptr, nullptr, 0, nullptr, nullptr,
                                    nullptr, 0, 0, 0, 0, L.ffn_norm, c.rms_eps, f32)))
            return e;
        if ((e = gemm_dispatch(ctx, m->act, c.act_dtype, L.down, m->hidden, JANUS_DT_F32, 1, m->h1))) return e;
    }
    if (can_fold_head(m))
        return gemv_norm_dispatch(ctx, m->hidden, m->out_norm, c.rms_eps, m->lm_head, m->logits,
                                  fold_sample ? m->d_best : nullptr, m->d_counts, m->d_sampler, f32);
    if ((e = rmsnorm_launch(ctx, m->hidden, m->xn, c.act_dtype, m->out_norm, 1, c.hidden, c.rms_eps))) return e;
    return gemm_dispatch(ctx, m->xn, c.act_dtype, m->lm_head, m->logits, JANUS_DT_F32, 1, nullptr);
}

bool use_fused1(const janus_model *m, uint32_t nseq) {
    // the fused norms stage x in registers: hidden <= 8192
    if (nseq != 1 || !m->fused_ready || m->cfg.hidden > 8192 || !m->ctx->fused_step) return false;
    for (const auto &L : m->layers)
        if (!L.qkv || !L.gu) return false;
    return true;
}

// The batched fused step needs binary16 activations, the fused weights of
// every layer on the MFMA path and rows the one-workgroup norm can hold.
bool fused_batch_ok(const janus_model *m) {
    const janus_model_config &c = m->cfg;
    if (c.act_dtype != JANUS_DT_F16 || c.max_batch < 2 || !m->fused_ready || !resnorm_supported(c.hidden) ||
        !m->ctx->fused_step)
        return false;
    for (const auto &L : m->layers)
        if (!L.qkv || !L.gu || !mfma_gemm_supported(JANUS_DT_F16, L.qkv) || !mfma_gemm_supported(JANUS_DT_F16, L.gu) ||
            !mfma_gemm_supported(JANUS_DT_F16, L.o) || !mfma_gemm_supported(JANUS_DT_F16, L.down))
            return false;
    return true;
}

bool use_fused_batch(const janus_model *m, uint32_t nseq) { return nseq > 1 && fused_batch_ok(m); }

// Batched step over the fused weights: per layer the QKV product (RoPE and
// the K/V append in its epilogue), attention, o-proj (residual add and the
// FFN RMSNorm in its epilogue), gate/up (SwiGLU epilogue) and down-proj
// (residual add and the next layer's attention RMSNorm, or the final norm,
// in its epilogue). Same operations and order as forward_rows.
int forward_batch(janus_model *m, const uint32_t *h_ids, const int32_t *d_ids, uint32_t nseq, uint32_t max_len) {
    janus_ctx *ctx = m->ctx;
    const janus_model_config &c = m->cfg;
    const uint32_t kvd = c.kv_heads * c.head_dim, half = c.head_dim / 2;
    const int kv16 = c.kv_dtype == JANUS_DT_F16;
    int e;
    if ((e = embed_launch(ctx, m->tok_embd, h_ids, d_ids, nseq, m->hidden))) return e;
    if ((e = rmsnorm_launch(ctx, m->hidden, m->xn, JANUS_DT_F16, m->layers[0].attn_norm, nseq, c.hidden, c.rms_eps)))
        return e;
    for (uint32_t l = 0; l < c.layers; ++l) {
        const janus_model::Layer &L = m->layers[l];
        void *kc = (uint8_t *)m->kcache + (size_t)l * m->layer_kv_elems * kv_elem_bytes(c.kv_dtype);
        void *vc = (uint8_t *)m->vcache + (size_t)l * m->layer_kv_elems * kv_elem_bytes(c.kv_dtype);
        const QkvEpilogue qe{m->q, kc, vc, m->rope, m->d_pos, m->d_rowbase, c.heads * half, c.kv_heads * half, half,
                             kvd, c.max_seq_len};
        if ((e = gemm_qkv_rope(ctx, m->xn, L.qkv, nseq, qe, kv16))) return e;
        if ((e = attention_launch(ctx, m->q, kc, vc, c.kv_dtype, m->attn16, nseq, c.heads, c.kv_heads, c.head_dim, 0,
                                  c.max_seq_len, m->d_rowbase, m->d_lens, max_len, 1.0f / sqrtf((float)c.head_dim),
                                  1)))
            return e;
        if ((e = gemm_residual_norm(ctx, m->attn16, L.o, nseq, m->hidden, m->h1, L.ffn_norm, c.rms_eps, m->xn)))
            return e;
        if ((e = gemm_swiglu(ctx, m->xn, L.gu, nseq, m->act))) return e;
        const float *next = l + 1 < c.layers ? m->layers[l + 1].attn_norm : m->out_norm;
        if ((e = gemm_residual_norm(ctx, m->act, L.down, nseq, m->h1, m->hidden, next, c.rms_eps, m->xn))) return e;
    }
    return gemm_dispatch(ctx, m->xn, JANUS_DT_F16, m->lm_head, m->logits, JANUS_DT_F32, nseq, nullptr);
}

int forward_any(janus_model *m, const uint32_t *h_ids, const int32_t *d_ids, uint32_t nseq, uint32_t max_len,
                bool fold_sample) {
    if (use_fused1(m, nseq)) return forward_fused1(m, h_ids, d_ids, max_len, fold_sample);
    if (use_fused_batch(m, nseq)) return forward_batch(m, h_ids, d_ids, nseq, max_len);
    return forward_rows(m, h_ids, d_ids, nseq, max_len);
}

// One full decode step over rows 0..nseq-1 from the device state: forward
// (attention planned for rows up to max_len long), greedy choice (folded
// into the single-sequence LM head, or keyed over the logits), advance.
int step_launch(janus_model *m, uint32_t nseq, uint32_t max_len) {
    janus_ctx *ctx = m->ctx;
    const bool fold = use_fused1(m, nseq) && can_fold_head(m);
    int e = forward_any(m, nullptr, m->d_feed, nseq, max_len, fold);
    if (!e && !fold) e = argmax_keys_launch(ctx, m->logits, m->d_best, m->cfg.vocab, nseq, m->d_counts, m->d_sampler);
    if (e) return e;
    AdvanceArgs a;
    a.pos = m->d_pos;
    a.lens = m->d_lens;
    a.tokens = m->d_tokens;
    a.feed = m->d_feed;
    a.rows = m->d_rows;
    a.prompts = m->d_prompts;
    a.out = m->d_out;
    a.counts = m->d_counts;
    a.best = m->d_best;
    a.sampler = m->d_sampler;
    a.n = nseq;
    a.max_seq = m->cfg.max_seq_len;
    a.vocab = m->cfg.vocab;
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(kMaxRows), 0, ctx->stream, a);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

struct RowInit {
    int32_t token[kMaxRows], pos[kMaxRows], rowbase[kMaxRows];
    RowDev ctl[kMaxRows];
    uint32_t mask[2];   // rows to set (bit r of mask[r / 32])
    uint32_t set_ctl;   // also write the control blocks
};

// Sets the device state of the masked rows from kernel arguments, ordered on
// the stream behind any step still reading the old values.
__global__ void set_rows_kernel(RowInit in, int32_t *tokens, int32_t *feed, int32_t *pos, int32_t *lens,
                                int32_t *rowbase, RowDev *rows) {
    const uint32_t r = threadIdx.x;
    if (r >= kMaxRows || !((in.mask[r / 32] >> (r % 32)) & 1u)) return;
    tokens[r] = in.token[r];
    feed[r] = in.token[r];
    pos[r] = in.pos[r];
    lens[r] = in.pos[r] + 1;
    rowbase[r] = in.rowbase[r];
    if (in.set_ctl) rows[r] = in.ctl[r];
}

int set_rows(janus_model *m, const RowInit &in) {
    hipLaunchKernelGGL(set_rows_kernel, dim3(1), dim3(kMaxRows), 0, m->ctx->stream, in, m->d_tokens, m->d_feed, m->d_pos,
                       m->d_lens, m->d_rowbase, m->d_rows);
    JANUS_LAUNCH_CHECK(m->ctx);
    return JANUS_OK;
}

// Validates tokens / positions / slots of an eager step and stores them
// into rows 0..nseq-1. slots == NULL: row s uses slot s.
int upload_step(janus_model *m, const uint32_t *tokens, const uint32_t *positions, const uint32_t *slots,
                uint32_t nseq, uint32_t *max_len) {
    const janus_model_config &c = m->cfg;
    RowInit in;
    std::memset(&in, 0, sizeof(in));
    uint64_t used = 0;
    *max_len = 0;
    for (uint32_t i = 0; i < nseq; ++i) {
        if (positions[i] >= c.max_seq_len)
            return fail(m->ctx, JANUS_E_KV_OVERFLOW, "KV cache position " + std::to_string(positions[i]) +
                                                         " exceeds max_seq_len " + std::to_string(c.max_seq_len));
        if (tokens && tokens[i] >= c.vocab)
            return fail(m->ctx, JANUS_E_TOKEN_RANGE, "Token ID " + std::to_string(tokens[i]) + " exceeds vocab size");
        const uint32_t s = slots ? slots[i] : i;
        if (s >= c.max_batch)
            return fail(m->ctx, JANUS_E_INVALID_ARG, "KV slot " + std::to_string(s) + " exceeds max_batch");
        if ((used >> s) & 1u) return fail(m->ctx, JANUS_E_INVALID_ARG, "KV slot " + std::to_string(s) + " used twice");
        used |= 1ull << s;
        in.token[i] = tokens ? (int32_t)tokens[i] : 0;
        in.pos[i] = (int32_t)positions[i];
        in.rowbase[i] = (int32_t)(s * c.max_seq_len);
        in.mask[i / 32] |= 1u << (i % 32);
        *max_len = positions[i] + 1 > *max_len ? positions[i] + 1 : *max_len;
    }
    return set_rows(m, in);
}

int upload_sampler(janus_model *m) {
    JANUS_HIP_CHECK(m->ctx, hipMemcpyAsync(m->d_sampler, &m->h_sampler, sizeof(SamplerDev), hipMemcpyHostToDevice,
                                           m->ctx->stream));
    return JANUS_OK;
}

void free_graphs(janus_model *m) {
    for (auto &g : m->graphs) {
        if (g) (void)hipGraphExecDestroy(g);
        g = nullptr;
    }
    m->graph_nseq = 0;
}

// Captured steps are planned for a length bucket: the attention of a step
// whose longest row attends `len` positions runs with the plan for the
// smallest of 256, 512, 1024, ... (or max_seq_len, the last bucket) that is
// at least len. A plan for a longer length is correct for any shorter one
// (lengths are read from the device), so a replay may use any bucket at or
// above its rows' lengths; the host picks the smallest, from positions it
// knows to be upper bounds.
constexpr uint32_t kBucket0 = 256;

uint32_t bucket_count(uint32_t max_seq) {
    uint32_t n = 1;
    while (((uint64_t)kBucket0 << (n - 1)) < max_seq) ++n;
    return n;   // kBucket0 << (n - 2) < max_seq <= INT_MAX, so every bucket length fits
}

uint32_t bucket_len(const janus_model *m, uint32_t b) {
    return b + 1 < m->nbuckets ? kBucket0 << b : m->cfg.max_seq_len;
}

uint32_t bucket_of(const janus_model *m, uint32_t len) {
    uint32_t b = 0;
    while (b + 1 < m->nbuckets && (kBucket0 << b) < len) ++b;
    return b;
}

// The captured step for nseq rows and length bucket b, captured on first use.
// Capture follows one eager forward over the same rows (it sets kernel
// attributes and grows the GEMM workspace outside the capture; it writes the
// K/V rows the next step writes again with the same values), so it is called
// only between steps, where the device state is the next step's.
int ensure_graph(janus_model *m, uint32_t nseq, uint32_t b) {
    hipGraphExec_t &slot = m->graphs[(size_t)nseq * m->nbuckets + b];
    if (slot) return JANUS_OK;
    janus_ctx *ctx = m->ctx;
    const uint32_t max_len = bucket_len(m, b);
    if (int e = forward_any(m, nullptr, m->d_feed, nseq, max_len, false)) return e;
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
    // Capture on the model's own stream (the caller's may be the legacy
    // default stream, which cannot be captured); the graph is launched on the
    // caller's stream afterwards.
    if (!m->cap_stream) JANUS_HIP_CHECK(ctx, hipStreamCreateWithFlags(&m->cap_stream, hipStreamNonBlocking));
    hipStream_t user = ctx->stream;
    ctx->stream = m->cap_stream;
    hipError_t be = hipStreamBeginCapture(m->cap_stream, hipStreamCaptureModeThreadLocal);
    if (be != hipSuccess) {
        ctx->stream = user;
        return hip_fail(ctx, be, "hipStreamBeginCapture");
    }
    int e = step_launch(m, nseq, max_len);
    hipGraph_t g = nullptr;
    hipError_t ce = hipStreamEndCapture(m->cap_stream, &g);
    ctx->stream = user;
    if (e) {
        if (g) (void)hipGraphDestroy(g);
        return e;
    }
    if (ce != hipSuccess) return hip_fail(ctx, ce, "hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess) return hip_fail(ctx, ie, "hipGraphInstantiate");
    slot = ge;
    return JANUS_OK;
}

// The reference's CPU sampler panics on NaN logits (sampler.rs:191-193,
// 397-399); here the call that ran the step returns an error.
int nan_fail(janus_ctx *ctx, uint32_t row) {
    return fail(ctx, JANUS_E_NAN_LOGITS,
                "GPU returned NaN logits (batch row " + std::to_string(row) + "): no token was sampled");
}

// Captures the steps for nseq rows of every bucket from the one of length
// lo to the one of length hi.
int replay_prepare(janus_model *m, uint32_t nseq, uint32_t lo, uint32_t hi) {
    for (uint32_t b = bucket_of(m, lo), e = bucket_of(m, hi); b <= e; ++b)
        if (int st = ensure_graph(m, nseq, b)) return st;
    return JANUS_OK;
}

// `steps` replays of the captured step for nseq rows. len0 bounds the
// attention length of the first step's longest row; each step adds at most
// one position, so step s runs the bucket of min(len0 + s, max_seq_len).
// Every bucket the replays need is captured before the first is launched.
int replay(janus_model *m, uint32_t nseq, uint32_t steps, uint32_t len0) {
    if (!steps) return JANUS_OK;
    const uint32_t cap = m->cfg.max_seq_len;
    auto len_at = [&](uint32_t s) -> uint32_t {
        const uint64_t l = (uint64_t)len0 + s;
        return l < cap ? (uint32_t)l : cap;
    };
    if (int e = replay_prepare(m, nseq, len_at(0), len_at(steps - 1))) return e;
    hipGraphExec_t *row = &m->graphs[(size_t)nseq * m->nbuckets];
    for (uint32_t s = 0; s < steps; ++s)
        JANUS_HIP_CHECK(m->ctx, hipGraphLaunch(row[bucket_of(m, len_at(s))], m->ctx->stream));
    return JANUS_OK;
}

struct Request {
    const uint32_t *prompt;
    uint32_t n;
};

// The prompt checks of Model::generate (generation.rs:146-150; positions 0..n-1, :161-173).
int check_request(janus_model *m, const Request &q) {
    const janus_model_config &c = m->cfg;
    if (q.n == 0) return fail(m->ctx, JANUS_E_INVALID_ARG, "Empty prompt after tokenization");
    if (q.n > c.max_seq_len)
        return fail(m->ctx, JANUS_E_KV_OVERFLOW, "prompt of " + std::to_string(q.n) +
                                                     " tokens exceeds max_seq_len " + std::to_string(c.max_seq_len));
    for (uint32_t t = 0; t < q.n; ++t)
        if (q.prompt[t] >= c.vocab)
            return fail(m->ctx, JANUS_E_TOKEN_RANGE, "Token ID " + std::to_string(q.prompt[t]) + " exceeds vocab size");
    return JANUS_OK;
}

// Puts request q into row r of `in`: its prompt copied to the device, its
// occurrence counts cleared, its first prompt token at position 0 of KV slot r.
int admit_row(janus_model *m, uint32_t r, const Request &q, uint32_t max_tokens, int eos_mode, RowInit &in,
              std::vector<int32_t> &tmp) {
    janus_ctx *ctx = m->ctx;
    const janus_model_config &c = m->cfg;
    tmp.assign(q.prompt, q.prompt + q.n);
    JANUS_HIP_CHECK(ctx, hipMemcpyAsync(m->d_prompts + (size_t)r * c.max_seq_len, tmp.data(), q.n * 4,
                                        hipMemcpyHostToDevice, ctx->stream));
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));   // tmp is reused
    JANUS_HIP_CHECK(ctx, hipMemsetAsync(m->d_counts + (size_t)r * c.vocab, 0, (size_t)c.vocab * 4, ctx->stream));
    in.token[r] = (int32_t)q.prompt[0];
    in.pos[r] = 0;
    in.rowbase[r] = (int32_t)(r * c.max_seq_len);
    in.ctl[r] = RowDev{(int32_t)q.n, (int32_t)max_tokens, 0, 0, eos_mode, 0};
    in.mask[r / 32] |= 1u << (r % 32);
    return JANUS_OK;
}

// The device-side generation loop for a list of requests, at most max_batch
// at a time: a request takes the lowest free row (its KV slot), prefills and
// decodes on graph replays in chunks, and frees the row when done; the next
// request is admitted between chunks. Nothing is copied between KV slots.
int run_requests(janus_model *m, const std::vector<Request> &reqs, uint32_t max_tokens, int eos_mode,
                 uint32_t *out_tokens, uint32_t *n_out) {
    janus_ctx *ctx = m->ctx;
    const janus_model_config &c = m->cfg;
    const uint32_t B = c.max_batch;
    for (size_t i = 0; i < reqs.size(); ++i) {
        n_out[i] = 0;
        if (int e = check_request(m, reqs[i])) return e;
    }
    if (int e = janus_model_validate(m)) return e;
    if (int e = upload_sampler(m)) return e;
    m->graph_nseq = 0;   // the rows are about to hold this loop's state, not a graph_begin's
    std::vector<int> row_req(B, -1);
    std::vector<uint8_t> parked(B, 0);
    std::vector<RowDev> hrows(B);
    std::vector<int32_t> hpos(B, 0);
    std::vector<int32_t> tmp;
    size_t next_req = 0;
    for (;;) {
        // admission: free rows take the next requests
        RowInit in;
        std::memset(&in, 0, sizeof(in));
        in.set_ctl = 1;
        bool any_new = false;
        for (uint32_t r = 0; r < B && next_req < reqs.size(); ++r) {
            if (row_req[r] >= 0) continue;
            row_req[r] = (int)next_req;
            parked[r] = 0;
            if (int e = admit_row(m, r, reqs[next_req++], max_tokens, eos_mode, in, tmp)) return e;
            hrows[r] = in.ctl[r];
            hpos[r] = 0;
            any_new = true;
        }
        uint32_t nrows = 0;
        for (uint32_t r = 0; r < B; ++r)
            if (row_req[r] >= 0) nrows = r + 1;
        if (nrows == 0) break;
        // A free row below nrows still runs through every replay: park it at
        // position 0 of its own (free) slot with one row of attention, so it
        // costs little until a request takes it.
        for (uint32_t r = 0; r < nrows; ++r) {
            if (row_req[r] >= 0 || parked[r]) continue;
            in.token[r] = 0;
            in.pos[r] = 0;
            in.rowbase[r] = (int32_t)(r * c.max_seq_len);
            in.ctl[r] = RowDev{0, 0, 0, 1, EOS_IGNORE, 0};
            in.mask[r / 32] |= 1u << (r % 32);
            parked[r] = 1;
            hpos[r] = 0;
            any_new = true;
        }
        if (any_new)
            if (int e = set_rows(m, in)) return e;
        // steps until the first row can be done without an EOS: its prompt,
        // its tokens, or its capacity
        uint32_t k = 16;
        for (uint32_t r = 0; r < nrows; ++r) {
            if (row_req[r] < 0 || hrows[r].done) continue;
            const int64_t left_prompt = hrows[r].prompt_len - hpos[r];   // steps still prefilling
            int64_t need = (left_prompt > 0 ? left_prompt : 0) + (hrows[r].max_new - hrows[r].nout);
            const int64_t cap = (int64_t)c.max_seq_len - hpos[r];
            if (cap < need) need = cap;
            if (need < 1) need = 1;
            if ((uint64_t)need < k) k = (uint32_t)need;
        }
        // hpos holds each row's position (admitted and parked rows start at 0)
        int32_t top = 0;
        for (uint32_t r = 0; r < nrows; ++r) top = hpos[r] > top ? hpos[r] : top;
        if (int e = replay(m, nrows, k, (uint32_t)top + 1)) return e;
        JANUS_HIP_CHECK(ctx, hipMemcpyAsync(hrows.data(), m->d_rows, nrows * sizeof(RowDev), hipMemcpyDeviceToHost,
                                            ctx->stream));
        JANUS_HIP_CHECK(ctx, hipMemcpyAsync(hpos.data(), m->d_pos, nrows * 4, hipMemcpyDeviceToHost, ctx->stream));
        JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
        for (uint32_t r = 0; r < nrows; ++r)
            if (row_req[r] >= 0 && hrows[r].nan) return nan_fail(ctx, r);
        // retirement: finished rows hand back their tokens and free the row
        for (uint32_t r = 0; r < nrows; ++r) {
            if (row_req[r] < 0 || !hrows[r].done) continue;
            const int i = row_req[r];
            const uint32_t n = (uint32_t)hrows[r].nout < max_tokens ? (uint32_t)hrows[r].nout : max_tokens;
            tmp.resize(n ? n : 1);
            if (n)
                JANUS_HIP_CHECK(ctx, hipMemcpy(tmp.data(), m->d_out + (size_t)r * c.max_seq_len, n * 4,
                                               hipMemcpyDeviceToHost));
            for (uint32_t t = 0; t < n; ++t) out_tokens[(size_t)i * max_tokens + t] = (uint32_t)tmp[t];
            n_out[i] = n;
            row_req[r] = -1;
        }
    }
    return JANUS_OK;
}

// The streaming form of run_requests for one request in row 0: the prompt
// on replays of the captured step, then one replay per token with the row's
// control block and its token copied behind it to pinned host memory; the
// host hands step i's token to the callback while step i + 1 runs.
int run_stream(janus_model *m, const Request &q, uint32_t max_tokens, janus_token_callback cb, void *user,
               uint32_t *out_tokens, uint32_t *n_out) {
    janus_ctx *ctx = m->ctx;
    if (int e = check_request(m, q)) return e;
    if (int e = janus_model_validate(m)) return e;
    if (int e = upload_sampler(m)) return e;
    if (!m->h_stream) {
        void *h = nullptr;
        JANUS_HIP_CHECK(ctx, hipHostMalloc(&h, 2 * sizeof(janus_model::StreamSlot), hipHostMallocDefault));
        m->h_stream = (janus_model::StreamSlot *)h;
    }
    for (hipEvent_t &ev : m->stream_ev)
        if (!ev) JANUS_HIP_CHECK(ctx, hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    m->graph_nseq = 0;   // row 0 is about to hold this loop's state, not a graph_begin's
    RowInit in;
    std::memset(&in, 0, sizeof(in));
    in.set_ctl = 1;
    std::vector<int32_t> tmp;
    if (int e = admit_row(m, 0, q, max_tokens, EOS_STOP_DROP, in, tmp)) return e;
    if (int e = set_rows(m, in)) return e;
    // every bucket the request can reach, captured before the first step so
    // that no capture stalls the stream of tokens
    {
        const uint64_t reach = (uint64_t)q.n + max_tokens + 1;
        if (int e = replay_prepare(m, 1, 1, reach < m->cfg.max_seq_len ? (uint32_t)reach : m->cfg.max_seq_len))
            return e;
    }
    // prefill: positions 0 .. n-1; the last of these steps queues the re-fed
    // last prompt token at position n (or ends the row at max_seq_len)
    if (int e = replay(m, 1, q.n, 1)) return e;
    // step i samples token i (the step at position n + i at most); at most
    // max_tokens steps can sample one
    auto issue = [&](uint32_t i) -> int {
        janus_model::StreamSlot *slot = m->h_stream + (i & 1);
        if (int e = replay(m, 1, 1, q.n + i + 1)) return e;
        JANUS_HIP_CHECK(ctx, hipMemcpyAsync(&slot->row, m->d_rows, sizeof(RowDev), hipMemcpyDeviceToHost, ctx->stream));
        JANUS_HIP_CHECK(ctx, hipMemcpyAsync(&slot->token, m->d_tokens, 4, hipMemcpyDeviceToHost, ctx->stream));
        JANUS_HIP_CHECK(ctx, hipEventRecord(m->stream_ev[i & 1], ctx->stream));
        return JANUS_OK;
    };
    uint32_t n = 0;
    int status = JANUS_OK;
    if (int e = issue(0)) return e;
    for (uint32_t i = 0;; ++i) {
        // queue step i + 1 before waiting for step i (its slot was read in
        // iteration i - 1)
        if (i + 1 < max_tokens)
            if ((status = issue(i + 1))) break;
        hipError_t we = hipEventSynchronize(m->stream_ev[i & 1]);
        if (we != hipSuccess) {
            status = hip_fail(ctx, we, "hipEventSynchronize");
            break;
        }
        const janus_model::StreamSlot got = m->h_stream[i & 1];
        if (got.row.nan) {
            status = nan_fail(ctx, 0);
            break;
        }
        bool stop = got.row.done || i + 1 >= max_tokens;
        if ((uint32_t)got.row.nout > n) {   // this step pushed a token (a stop token is not pushed)
            out_tokens[n] = (uint32_t)got.token;
            ++n;
            if (cb && !cb(user, (uint32_t)got.token, n - 1)) stop = true;
        }
        if (stop) break;
    }
    *n_out = n;
    // the step queued behind the last one read still runs; leave the stream idle
    const hipError_t se = hipStreamSynchronize(ctx->stream);
    if (status == JANUS_OK && se != hipSuccess) status = hip_fail(ctx, se, "hipStreamSynchronize");
    return status;
}

}  // namespace

extern "C" {

int janus_model_create(janus_ctx *ctx, const janus_model_config *cfg, janus_model **out) {
    if (!ctx || !cfg || !out) return JANUS_E_INVALID_ARG;
    *out = nullptr;
    const janus_model_config &c = *cfg;
    if (!c.hidden || !c.heads || !c.kv_heads || !c.head_dim || !c.ffn || !c.vocab || !c.layers || !c.max_seq_len)
        return fail(ctx, JANUS_E_INVALID_DIM, "model: zero dimension in config");
    if (c.heads % c.kv_heads) return fail(ctx, JANUS_E_INVALID_DIM, "model: heads must be a multiple of kv_heads");
    if (c.head_dim * c.heads != c.hidden) return fail(ctx, JANUS_E_INVALID_DIM, "model: head_dim * heads != hidden");
    if (c.max_batch == 0 || c.max_batch > kMaxRows) return fail(ctx, JANUS_E_INVALID_DIM, "model: max_batch must be 1..64");
    if (c.vocab >= (1u << 24)) return fail(ctx, JANUS_E_INVALID_DIM, "model: vocab must be below 2^24");
    if ((uint64_t)c.max_batch * c.max_seq_len > (uint64_t)INT_MAX)
        return fail(ctx, JANUS_E_INVALID_DIM, "model: max_batch * max_seq_len exceeds the row index range");
    if (!is_act_dtype(c.kv_dtype) || !is_act_dtype(c.act_dtype))
        return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "model: kv/act dtype must be F32 or F16");
    if (int e = need_device(ctx)) return e;
    janus_model *m = new janus_model();
    m->ctx = ctx;
    m->cfg = c;
    m->layers.resize(c.layers);
    m->nbuckets = ctx->graph_buckets ? bucket_count(c.max_seq_len) : 1;
    m->graphs.assign((size_t)(c.max_batch + 1) * m->nbuckets, nullptr);
    const size_t B = c.max_batch, kvd = (size_t)c.kv_heads * c.head_dim, S = c.max_seq_len;
    auto alloc = [&](void **p, size_t bytes) { return hipMalloc(p, bytes < 256 ? 256 : bytes) == hipSuccess; };
    bool ok = alloc((void **)&m->hidden, B * c.hidden * 4) && alloc((void **)&m->q, B * c.hidden * 4) &&
              alloc((void **)&m->k, B * kvd * 4) && alloc((void **)&m->v, B * kvd * 4) &&
              alloc((void **)&m->attn, B * c.hidden * 4) && alloc((void **)&m->h1, B * c.hidden * 4) &&
              alloc((void **)&m->gate, B * c.ffn * 4) && alloc((void **)&m->up, B * c.ffn * 4) &&
              alloc((void **)&m->logits, B * c.vocab * 4) && alloc(&m->xn, B * c.hidden * 4) &&
              alloc(&m->act, B * c.ffn * 4) && alloc(&m->attn16, B * c.hidden * 2) &&
              alloc((void **)&m->rope, S * c.head_dim * 4) && alloc((void **)&m->d_pos, kMaxRows * 4) &&
              alloc((void **)&m->d_lens, kMaxRows * 4) && alloc((void **)&m->d_tokens, kMaxRows * 4) &&
              alloc((void **)&m->d_feed, kMaxRows * 4) &&
              alloc((void **)&m->d_rowbase, kMaxRows * 4) && alloc((void **)&m->d_rows, kMaxRows * sizeof(RowDev)) &&
              alloc((void **)&m->d_prompts, B * S * 4) && alloc((void **)&m->d_out, B * S * 4) &&
              alloc((void **)&m->d_counts, B * c.vocab * 4) && alloc((void **)&m->d_best, kMaxRows * 8) &&
              alloc((void **)&m->d_sampler, sizeof(SamplerDev));
    ok = ok && hipMemset(m->d_best, 0, kMaxRows * 8) == hipSuccess &&
         hipMemset(m->d_rows, 0, kMaxRows * sizeof(RowDev)) == hipSuccess &&
         hipMemset(m->d_counts, 0, B * c.vocab * 4) == hipSuccess &&
         hipMemset(m->d_pos, 0, kMaxRows * 4) == hipSuccess && hipMemset(m->d_tokens, 0, kMaxRows * 4) == hipSuccess &&
         hipMemset(m->d_feed, 0, kMaxRows * 4) == hipSuccess &&
         hipMemcpy(m->d_sampler, &m->h_sampler, sizeof(SamplerDev), hipMemcpyHostToDevice) == hipSuccess;
    if (ok) {
        std::vector<int32_t> base(kMaxRows, 0), ones(kMaxRows, 1);
        for (size_t r = 0; r < B; ++r) base[r] = (int32_t)(r * S);
        ok = hipMemcpy(m->d_rowbase, base.data(), kMaxRows * 4, hipMemcpyHostToDevice) == hipSuccess &&
             hipMemcpy(m->d_lens, ones.data(), kMaxRows * 4, hipMemcpyHostToDevice) == hipSuccess;
    }
    m->layer_kv_elems = B * S * kvd;
    size_t kv_bytes = (size_t)c.layers * m->layer_kv_elems * kv_elem_bytes(c.kv_dtype);
    ok = ok && alloc(&m->kcache, kv_bytes) && alloc(&m->vcache, kv_bytes);
    if (!ok) {
        janus_model_destroy(m);
        return fail(ctx, JANUS_E_OOM, "model: device allocation failed");
    }
    if (int e = janus_rope_table(ctx, m->rope, c.max_seq_len, c.head_dim, c.rope_theta)) {
        janus_model_destroy(m);
        return e;
    }
    // The attention workspace for every row count and every captured step's
    // length bucket, so no step ever needs to grow it.
    size_t need = 0;
    for (uint32_t b = 1; b <= c.max_batch; ++b)
        for (uint32_t k = 0; k < m->nbuckets; ++k) {
            const size_t n = attention_ws_bytes(ctx, b, c.heads, c.kv_heads, c.head_dim, bucket_len(m, k),
                                                c.kv_dtype == JANUS_DT_F16);
            need = n > need ? n : need;
        }
    if (need)
        if (int e = ensure_attn_ws(ctx, need)) {
            janus_model_destroy(m);
            return e;
        }
    *out = m;
    return JANUS_OK;
}

void janus_model_destroy(janus_model *m) {
    if (!m) return;
    (void)hipStreamSynchronize(m->ctx->stream);
    free_graphs(m);
    if (m->cap_stream) (void)hipStreamDestroy(m->cap_stream);
    for (hipEvent_t ev : m->stream_ev)
        if (ev) (void)hipEventDestroy(ev);
    if (m->h_stream) (void)hipHostFree(m->h_stream);
    for (auto &L : m->layers) {
        for (janus_weight *w : {L.q, L.k, L.v, L.o, L.gate, L.up, L.down, L.qkv, L.gu}) janus_weight_free(m->ctx, w);
        (void)hipFree(L.attn_norm);
        (void)hipFree(L.ffn_norm);
    }
    janus_weight_free(m->ctx, m->tok_embd);
    janus_weight_free(m->ctx, m->lm_head);
    for (void *p : {(void *)m->out_norm, (void *)m->hidden, (void *)m->q, (void *)m->k, (void *)m->v,
                    (void *)m->attn, m->attn16, (void *)m->h1, (void *)m->gate, (void *)m->up, (void *)m->logits, m->xn,
                    m->act, m->kv_external ? nullptr : m->kcache, m->kv_external ? nullptr : m->vcache,
                    (void *)m->rope, (void *)m->d_pos, (void *)m->d_lens, (void *)m->d_tokens, (void *)m->d_feed, (void *)m->d_rowbase,
                    (void *)m->d_rows, (void *)m->d_prompts, (void *)m->d_out, (void *)m->d_counts,
                    (void *)m->d_best, (void *)m->d_sampler})
        if (p) (void)hipFree(p);
    delete m;
}

int janus_model_set_tensor(janus_model *m, const char *cname, int type, uint32_t n, uint32_t k, const void *bytes,
                           size_t nbytes) {
    if (!m || !cname || !bytes) return JANUS_E_INVALID_ARG;
    janus_ctx *ctx = m->ctx;
    const janus_model_config &c = m->cfg;
    const std::string name(cname);
    auto set_vec = [&](float **dst, uint32_t len) -> int {
        if (type != JANUS_DT_F32 || k != 0 || n != len || nbytes != (size_t)len * 4)
            return fail(ctx, JANUS_E_INVALID_DIM, name + ": expected F32 vector of " + std::to_string(len));
        if (!*dst) JANUS_HIP_CHECK(ctx, hipMalloc((void **)dst, (size_t)len * 4));
        JANUS_HIP_CHECK(ctx, hipMemcpy(*dst, bytes, nbytes, hipMemcpyHostToDevice));
        return JANUS_OK;
    };
    auto set_w = [&](janus_weight **dst, uint32_t rows, uint32_t cols, uint32_t flags) -> int {
        if (n != rows || k != cols)
            return fail(ctx, JANUS_E_INVALID_DIM, name + ": expected [" + std::to_string(rows) + "x" +
                                                      std::to_string(cols) + "]");
        // 2-D float weights follow allocate_tensors: binary16 storage decoded with
        // f16_to_f32_safe (shaders/gemm.wgsl:18-31, embed.wgsl:11-20).
        // Q6_K is loaded as binary16 (engine.rs:800-831) and takes the same path.
        if (type == JANUS_DT_F32 || type == JANUS_DT_F16 || type == JANUS_DT_Q6_K) flags |= JANUS_WEIGHT_FTZ_F16;
        if (type == JANUS_DT_Q4_K) flags |= JANUS_WEIGHT_FTZ_F16;   // gemm_q4_k.wgsl:62-65
        janus_weight *w = nullptr;
        if (int e = janus_weight_upload(ctx, type, n, k, bytes, nbytes, flags, &w)) return e;
        janus_weight_free(ctx, *dst);
        *dst = w;
        return JANUS_OK;
    };
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
    free_graphs(m);
    m->fused_ready = false;
    m->tiles_ready = false;
    for (auto &L : m->layers) {
        janus_weight_free(ctx, L.qkv);
        janus_weight_free(ctx, L.gu);
        L.qkv = L.gu = nullptr;
    }
    // Q6_K tensors arrive as binary16 whatever their role (engine.rs:800-831).
    if (name == "token_embd.weight") {
        if (type != JANUS_DT_F32 && type != JANUS_DT_F16 && type != JANUS_DT_Q6_K)
            return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "token_embd.weight must be F32, F16 or Q6_K");
        return set_w(&m->tok_embd, c.vocab, c.hidden, 0);
    }
    if (name == "output_norm.weight") return set_vec(&m->out_norm, c.hidden);
    if (name == "output.weight") {
        // The LM head is always the f16 GEMM (model/transformer/forward.rs:101-111).
        if (type != JANUS_DT_F32 && type != JANUS_DT_F16 && type != JANUS_DT_Q6_K)
            return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "output.weight must be F32, F16 or Q6_K");
        return set_w(&m->lm_head, c.vocab, c.hidden, 0);
    }
    uint32_t l;
    std::string rest;
    if (!parse_layer_name(name, &l, &rest) || l >= c.layers)
        return fail(ctx, JANUS_E_INVALID_ARG, "unknown tensor " + name);
    janus_model::Layer &L = m->layers[l];
    const uint32_t kvd = c.kv_heads * c.head_dim;
    if (rest == "attn_norm.weight") return set_vec(&L.attn_norm, c.hidden);
    if (rest == "ffn_norm.weight") return set_vec(&L.ffn_norm, c.hidden);
    if (rest == "attn_q.weight") return set_w(&L.q, c.hidden, c.hidden, 0);
    if (rest == "attn_k.weight") return set_w(&L.k, kvd, c.hidden, 0);
    if (rest == "attn_v.weight") return set_w(&L.v, kvd, c.hidden, 0);
    if (rest == "attn_output.weight") return set_w(&L.o, c.hidden, c.hidden, 0);
    if (rest == "ffn_gate.weight") return set_w(&L.gate, c.ffn, c.hidden, 0);
    if (rest == "ffn_up.weight") return set_w(&L.up, c.ffn, c.hidden, 0);
    if (rest == "ffn_down.weight") return set_w(&L.down, c.hidden, c.ffn, 0);
    return fail(ctx, JANUS_E_INVALID_ARG, "unknown tensor " + name);
}

int janus_model_validate(janus_model *m) {
    if (!m) return JANUS_E_INVALID_ARG;
    if (!m->tok_embd || !m->lm_head || !m->out_norm) return fail(m->ctx, JANUS_E_INVALID_ARG, "model: missing global tensor");
    for (size_t l = 0; l < m->layers.size(); ++l) {
        const auto &L = m->layers[l];
        if (!L.attn_norm || !L.ffn_norm || !L.q || !L.k || !L.v || !L.o || !L.gate || !L.up || !L.down)
            return fail(m->ctx, JANUS_E_INVALID_ARG, "model: missing tensor in block " + std::to_string(l));
    }
    if (int e = ensure_fused(m)) return e;   // the fused single-sequence step, either activation dtype
    if (m->cfg.act_dtype != JANUS_DT_F16) return JANUS_OK;
    if (m->cfg.max_batch > 1 && !m->tiles_ready) {
        // tile copies for the batched MFMA products, built before any graph
        // capture: the fused QKV and gate/up weights where the fused batched
        // step runs, the separate ones otherwise
        const bool fb = fused_batch_ok(m);
        for (auto &L : m->layers) {
            std::vector<const janus_weight *> ws{L.o, L.down};
            if (fb) ws.insert(ws.end(), {L.qkv, L.gu});
            else ws.insert(ws.end(), {L.q, L.k, L.v, L.gate, L.up});
            for (const janus_weight *w : ws)
                if (mfma_gemm_supported(JANUS_DT_F16, w))
                    if (int e = mfma_gemm_prepare(m->ctx, w)) return e;
        }
        if (mfma_gemm_supported(JANUS_DT_F16, m->lm_head))
            if (int e = mfma_gemm_prepare(m->ctx, m->lm_head)) return e;
        m->tiles_ready = true;
    }
    return JANUS_OK;
}

int janus_model_set_kv_cache(janus_model *m, void *d_k, void *d_v, size_t bytes_each) {
    if (!m || !d_k || !d_v) return JANUS_E_INVALID_ARG;
    const size_t need = (size_t)m->cfg.layers * m->layer_kv_elems * kv_elem_bytes(m->cfg.kv_dtype);
    if (bytes_each < need)
        return fail(m->ctx, JANUS_E_INVALID_DIM, "set_kv_cache: buffers hold " + std::to_string(bytes_each) +
                                                     " bytes, need " + std::to_string(need));
    JANUS_HIP_CHECK(m->ctx, hipStreamSynchronize(m->ctx->stream));
    free_graphs(m);
    if (!m->kv_external) {
        (void)hipFree(m->kcache);
        (void)hipFree(m->vcache);
    }
    m->kcache = d_k;
    m->vcache = d_v;
    m->kv_external = true;
    return JANUS_OK;
}

int janus_model_reset(janus_model *m) {
    if (!m) return JANUS_E_INVALID_ARG;
    // KVCache::reset only rewinds the position; stale rows are never read
    // because attention reads rows [0, pos + 1).
    m->graph_nseq = 0;
    return JANUS_OK;
}

int janus_model_forward_slots(janus_model *m, const uint32_t *tokens, const uint32_t *positions,
                              const uint32_t *slots, uint32_t nseq) {
    if (!m || !tokens || !positions) return JANUS_E_INVALID_ARG;
    if (nseq == 0 || nseq > m->cfg.max_batch) return fail(m->ctx, JANUS_E_INVALID_DIM, "forward: bad batch size");
    if (int e = janus_model_validate(m)) return e;
    uint32_t max_len = 0;
    if (int e = upload_step(m, tokens, positions, slots, nseq, &max_len)) return e;
    m->graph_nseq = 0;   // the rows no longer hold a graph decode's state
    return forward_any(m, tokens, nullptr, nseq, max_len, false);
}

int janus_model_forward(janus_model *m, const uint32_t *tokens, const uint32_t *positions, uint32_t nseq) {
    return janus_model_forward_slots(m, tokens, positions, nullptr, nseq);
}

const float *janus_model_logits(const janus_model *m) { return m ? m->logits : nullptr; }

void *janus_model_kv_cache(const janus_model *m, int which) {
    if (!m) return nullptr;
    return which == 0 ? m->kcache : m->vcache;
}

int janus_model_read_logits(janus_model *m, float *h_out, uint32_t nseq) {
    if (!m || !h_out) return JANUS_E_INVALID_ARG;
    if (nseq > m->cfg.max_batch) return fail(m->ctx, JANUS_E_INVALID_DIM, "read_logits: more rows than max_batch");
    return janus_d2h(m->ctx, h_out, m->logits, (size_t)nseq * m->cfg.vocab * 4);
}

int janus_model_set_sampler(janus_model *m, int mode, float penalty) {
    if (!m) return JANUS_E_INVALID_ARG;
    if (mode != JANUS_SAMPLER_ARGMAX && mode != JANUS_SAMPLER_PENALTY && mode != JANUS_SAMPLER_WGSL)
        return fail(m->ctx, JANUS_E_INVALID_ARG, "set_sampler: unknown mode");
    if (!(penalty > 0.0f) || !std::isfinite(penalty))
        return fail(m->ctx, JANUS_E_INVALID_ARG, "set_sampler: penalty must be positive and finite");
    m->h_sampler.mode = mode == JANUS_SAMPLER_PENALTY ? SAMPLE_PENALTY : mode == JANUS_SAMPLER_WGSL ? SAMPLE_WGSL
                                                                                                  : SAMPLE_ARGMAX;
    m->h_sampler.penalty = penalty;
    return upload_sampler(m);
}

int janus_model_generate(janus_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_tokens,
                         float penalty, uint32_t *out_tokens, uint32_t *n_out) {
    if (!m || !prompt || !out_tokens || !n_out) return JANUS_E_INVALID_ARG;
    *n_out = 0;
    if (n_prompt == 0) return fail(m->ctx, JANUS_E_INVALID_ARG, "Empty prompt after tokenization");
    if (!(penalty > 0.0f) || !std::isfinite(penalty))
        return fail(m->ctx, JANUS_E_INVALID_ARG, "generate: penalty must be positive and finite");
    // Sampler::sample: with the penalty within 0.01 of 1 the reference takes
    // the GPU argmax (its tie rule, no penalty); otherwise the penalty and the
    // last-max argmax (sampler.rs:154-160, 188-206).
    m->h_sampler.mode = std::fabs(penalty - 1.0f) < 0.01f ? SAMPLE_WGSL : SAMPLE_PENALTY;
    m->h_sampler.penalty = penalty;
    if (max_tokens == 0) {
        // prefill only (generation.rs:161-173), then a loop of zero steps
        for (uint32_t i = 0; i < n_prompt; ++i)
            if (int e = janus_model_forward(m, &prompt[i], &i, 1)) return e;
        return upload_sampler(m);
    }
    std::vector<Request> reqs{Request{prompt, n_prompt}};
    return run_requests(m, reqs, max_tokens, EOS_STOP_DROP, out_tokens, n_out);
}

int janus_model_generate_stream(janus_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_tokens,
                                float penalty, janus_token_callback cb, void *user, uint32_t *out_tokens,
                                uint32_t *n_out) {
    if (!m || !prompt || !out_tokens || !n_out) return JANUS_E_INVALID_ARG;
    *n_out = 0;
    if (n_prompt == 0) return fail(m->ctx, JANUS_E_INVALID_ARG, "Empty prompt after tokenization");
    if (!(penalty > 0.0f) || !std::isfinite(penalty))
        return fail(m->ctx, JANUS_E_INVALID_ARG, "generate_stream: penalty must be positive and finite");
    // the same sampler as generate (Sampler::sample, sampler.rs:154-160, 188-206)
    m->h_sampler.mode = std::fabs(penalty - 1.0f) < 0.01f ? SAMPLE_WGSL : SAMPLE_PENALTY;
    m->h_sampler.penalty = penalty;
    if (max_tokens == 0) return janus_model_generate(m, prompt, n_prompt, 0, penalty, out_tokens, n_out);
    return run_stream(m, Request{prompt, n_prompt}, max_tokens, cb, user, out_tokens, n_out);
}

int janus_model_generate_batch(janus_model *m, const uint32_t *prompts, const uint32_t *prompt_lens, uint32_t nreq,
                               uint32_t max_tokens, float penalty, uint32_t *out_tokens, uint32_t *n_out) {
    if (!m || (nreq && (!prompts || !prompt_lens || !out_tokens || !n_out))) return JANUS_E_INVALID_ARG;
    if (nreq == 0 || max_tokens == 0) {
        for (uint32_t i = 0; i < nreq; ++i) n_out[i] = 0;
        return JANUS_OK;
    }
    if (!(penalty > 0.0f) || !std::isfinite(penalty))
        return fail(m->ctx, JANUS_E_INVALID_ARG, "generate_batch: penalty must be positive and finite");
    // Sampler::sample_batch applies the penalty and the last-max argmax to
    // every sequence (sampler.rs:379-428).
    m->h_sampler.mode = SAMPLE_PENALTY;
    m->h_sampler.penalty = penalty;
    std::vector<Request> reqs(nreq);
    size_t off = 0;
    for (uint32_t i = 0; i < nreq; ++i) {
        reqs[i] = Request{prompts + off, prompt_lens[i]};
        off += prompt_lens[i];
    }
    return run_requests(m, reqs, max_tokens, EOS_STOP_KEEP, out_tokens, n_out);
}

int janus_model_graph_begin_slots(janus_model *m, const uint32_t *tokens, const uint32_t *positions,
                                  const uint32_t *slots, uint32_t nseq) {
    if (!m || !tokens || !positions) return JANUS_E_INVALID_ARG;
    if (nseq == 0 || nseq > m->cfg.max_batch) return fail(m->ctx, JANUS_E_INVALID_DIM, "graph: bad batch size");
    janus_ctx *ctx = m->ctx;
    if (int e = janus_model_validate(m)) return e;
    uint32_t max_len = 0;
    if (int e = upload_step(m, tokens, positions, slots, nseq, &max_len)) return e;
    // plain decode rows: no prompt, no stop, a fresh penalty context
    RowInit in;
    std::memset(&in, 0, sizeof(in));
    in.set_ctl = 1;
    for (uint32_t i = 0; i < nseq; ++i) {
        in.token[i] = (int32_t)tokens[i];
        in.pos[i] = (int32_t)positions[i];
        in.rowbase[i] = (int32_t)((slots ? slots[i] : i) * m->cfg.max_seq_len);
        in.ctl[i] = RowDev{0, INT_MAX, 0, 0, EOS_IGNORE, 0};
        in.mask[i / 32] |= 1u << (i % 32);
    }
    if (int e = set_rows(m, in)) return e;
    JANUS_HIP_CHECK(ctx, hipMemsetAsync(m->d_counts, 0, (size_t)nseq * m->cfg.vocab * 4, ctx->stream));
    if (int e = upload_sampler(m)) return e;
    // every bucket from these rows' lengths up, so graph_run never captures
    if (int e = replay_prepare(m, nseq, max_len, m->cfg.max_seq_len)) return e;
    m->h_pos.assign(positions, positions + nseq);
    m->graph_nseq = nseq;
    return JANUS_OK;
}

int janus_model_graph_begin(janus_model *m, const uint32_t *tokens, const uint32_t *positions, uint32_t nseq) {
    return janus_model_graph_begin_slots(m, tokens, positions, nullptr, nseq);
}

int janus_model_graph_run(janus_model *m, uint32_t steps) {
    if (!m) return JANUS_E_INVALID_ARG;
    const uint32_t n = m->graph_nseq;
    if (!n) return fail(m->ctx, JANUS_E_INVALID_ARG, "graph: call janus_model_graph_begin first");
    uint32_t top = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if ((uint64_t)m->h_pos[i] + steps > m->cfg.max_seq_len)
            return fail(m->ctx, JANUS_E_KV_OVERFLOW, "graph: steps would exceed max_seq_len");
        top = m->h_pos[i] > top ? m->h_pos[i] : top;
    }
    if (int e = replay(m, n, steps, top + 1)) return e;
    for (auto &p : m->h_pos) p += steps;
    // a row whose step met NaN logits is stopped on the device; report it
    RowDev rows[kMaxRows];
    if (int e = janus_d2h(m->ctx, rows, m->d_rows, (size_t)n * sizeof(RowDev))) return e;
    for (uint32_t r = 0; r < n; ++r)
        if (rows[r].nan) return nan_fail(m->ctx, r);
    return JANUS_OK;
}

int janus_model_graph_read_tokens(janus_model *m, uint32_t *h_tokens, uint32_t nseq) {
    if (!m || !h_tokens || nseq > m->cfg.max_batch) return JANUS_E_INVALID_ARG;
    return janus_d2h(m->ctx, h_tokens, m->d_tokens, (size_t)nseq * 4);
}

int janus_model_read_generated(janus_model *m, uint32_t row, uint32_t *h_tokens, uint32_t cap, uint32_t *n) {
    if (!m || !n || (cap && !h_tokens)) return JANUS_E_INVALID_ARG;
    if (row >= m->cfg.max_batch) return fail(m->ctx, JANUS_E_INVALID_ARG, "read_generated: row out of range");
    RowDev c;
    if (int e = janus_d2h(m->ctx, &c, m->d_rows + row, sizeof(RowDev))) return e;
    uint32_t total = (uint32_t)c.nout < m->cfg.max_seq_len ? (uint32_t)c.nout : m->cfg.max_seq_len;
    *n = total;
    const uint32_t take = total < cap ? total : cap;
    if (take) return janus_d2h(m->ctx, h_tokens, m->d_out + (size_t)row * m->cfg.max_seq_len, (size_t)take * 4);
    return JANUS_OK;
}

}  // extern "C"
