/*
 * janus_model.h -- C++ host-side decode driver over libjanus_hip.
 *
 * Mirrors the reference's model layer (paths relative to
 * crates/janus-engine/src/): Model::new (model/transformer/constructor.rs:23-437),
 * Model::forward (model/transformer/forward.rs:25-119) / forward_batch
 * (:141-245), TransformerBlock::forward (model/block.rs:190-458) and the
 * generate loop (model/transformer/generation.rs:129-323). Each forward
 * enqueues the per-layer operator sequence on the context's stream; a decode
 * step can also be captured once into a HIP graph and replayed.
 */
#ifndef JANUS_MODEL_H
#define JANUS_MODEL_H

#include "janus_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ModelConfig (model/transformer/mod.rs:79-110) plus the build's layout and
 * precision choices. */
typedef struct janus_model_config {
    uint32_t hidden;        /* embedding_length */
    uint32_t heads;         /* attention.head_count */
    uint32_t kv_heads;      /* attention.head_count_kv */
    uint32_t head_dim;      /* hidden / heads (config.rs:437) */
    uint32_t ffn;           /* feed_forward_length */
    uint32_t vocab;
    uint32_t layers;        /* block_count */
    uint32_t max_seq_len;   /* KV capacity per sequence */
    uint32_t max_batch;     /* sequences per decode step (1 .. 64) */
    float rms_eps;          /* attention.layer_norm_rms_epsilon */
    float rope_theta;       /* rope.freq_base */
    int kv_dtype;           /* JANUS_DT_F32 (the reference's cache, core.rs:60-88) or JANUS_DT_F16 */
    int act_dtype;          /* activations entering the matrix products: F32 (reference) or F16 */
} janus_model_config;

typedef struct janus_model janus_model;

int janus_model_create(janus_ctx *ctx, const janus_model_config *cfg, janus_model **out);
void janus_model_destroy(janus_model *m);
/* Load one GGUF tensor by its GGUF name: token_embd.weight, output_norm.weight,
 * output.weight, blk.N.{attn_norm,attn_q,attn_k,attn_v,attn_output,ffn_norm,
 * ffn_gate,ffn_up,ffn_down}.weight. 1-D tensors (norms) must be F32. The
 * embedding and LM head follow allocate_tensors (compute/engine.rs:471-500):
 * F32 -> binary16 RNE, decoded with f16_to_f32_safe (FTZ). Shapes are given
 * in PyTorch [out][in] order (n rows, k columns; k = 0 for 1-D). */
int janus_model_set_tensor(janus_model *m, const char *name, int ggml_type, uint32_t n, uint32_t k,
                           const void *bytes, size_t nbytes);
/* Missing tensors -> JANUS_E_INVALID_ARG (validate_config, mod.rs:270-368). */
int janus_model_validate(janus_model *m);
/* KVCache::reset (compute/cache/core.rs). */
int janus_model_reset(janus_model *m);
/* Use caller-owned K and V cache buffers (each layers * max_batch * max_seq_len
 * * kv_heads * head_dim elements of kv_dtype, layout [layer][row][kvh][hd])
 * instead of the model's own; the model's allocation is released. Lets a
 * caller place or pre-fill the cache (the reference's caller-owned buffers,
 * model/transformer/constructor.rs:148-344). */
int janus_model_set_kv_cache(janus_model *m, void *d_k, void *d_v, size_t bytes_each);
/* One decode step for nseq sequences: sequence s consumes tokens[s] at
 * position positions[s] (its KV rows start at s * max_seq_len). Logits land
 * in janus_model_logits()[s][vocab]. */
int janus_model_forward(janus_model *m, const uint32_t *tokens, const uint32_t *positions, uint32_t nseq);
const float *janus_model_logits(const janus_model *m);        /* device pointer */
void *janus_model_kv_cache(const janus_model *m, int which);  /* 0 = K, 1 = V; [layers][rows][kvh][hd] */
int janus_model_read_logits(janus_model *m, float *h_out, uint32_t nseq);
/* Greedy generation with the reference's loop semantics (generation.rs:129-323):
 * prefill token by token, then re-feed the last prompt token at position n
 * and sample with the repetition penalty over generated tokens and the
 * last-max argmax (model/sampler.rs:146-209,599-613,784-795). Stops at
 * max_tokens, at 128001/128009 (generation.rs:241-260) or at max_seq_len. */
int janus_model_generate(janus_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_tokens,
                         float repetition_penalty, uint32_t *out_tokens, uint32_t *n_out);

/* Graph decode: capture one greedy decode step (embed from device ids ->
 * forward -> argmax written back as the next ids, positions advanced on the
 * device) for nseq sequences, then replay it `steps` times. Device state:
 * janus_model_device_tokens() [nseq] int32, janus_model_device_positions()
 * [nseq] int32, initialised by janus_model_graph_begin. */
int janus_model_graph_begin(janus_model *m, const uint32_t *tokens, const uint32_t *positions, uint32_t nseq);
int janus_model_graph_run(janus_model *m, uint32_t steps);
int janus_model_graph_read_tokens(janus_model *m, uint32_t *h_tokens, uint32_t nseq);

#ifdef __cplusplus
}
#endif
#endif /* JANUS_MODEL_H */
