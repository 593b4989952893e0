/*
 * janus_model.h -- C++ host-side decode driver over libjanus_hip.
 *
 * Mirrors the reference's model layer (paths relative to
 * crates/janus-engine/src/): Model::new (model/transformer/constructor.rs:23-437),
 * Model::forward (model/transformer/forward.rs:25-119) / forward_batch
 * (:141-245), TransformerBlock::forward (model/block.rs:190-458) and the
 * generate loop (model/transformer/generation.rs:129-323). Each forward
 * enqueues the per-layer operator sequence on the context's stream; a decode
 * step can also be captured into a HIP graph (per sequence count and
 * context-length bucket) and replayed.
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
 * in janus_model_logits()[s][vocab]. Model::forward_batch
 * (model/transformer/forward.rs:141-245), with a position per sequence. */
int janus_model_forward(janus_model *m, const uint32_t *tokens, const uint32_t *positions, uint32_t nseq);
/* As janus_model_forward, with sequence s in KV slot slots[s] (its rows start
 * at slots[s] * max_seq_len; slots distinct, each < max_batch): a sequence
 * keeps its cache wherever it sits in the batch, so sequences can join and
 * leave a batch without copying KV. */
int janus_model_forward_slots(janus_model *m, const uint32_t *tokens, const uint32_t *positions,
                              const uint32_t *slots, uint32_t nseq);
const float *janus_model_logits(const janus_model *m);        /* device pointer */
void *janus_model_kv_cache(const janus_model *m, int which);  /* 0 = K, 1 = V; [layers][rows][kvh][hd] */
int janus_model_read_logits(janus_model *m, float *h_out, uint32_t nseq);
/* Greedy generation with the reference's loop semantics (generation.rs:129-323):
 * prefill token by token, then re-feed the last prompt token at position n
 * and sample as Sampler::sample does with temperature 0 (model/sampler.rs:
 * 146-209): with |repetition_penalty - 1| < 0.01 the GPU argmax and its tie
 * rule (shaders/argmax.wgsl:26-126), otherwise the penalty over the generated
 * tokens (:599-613) and the last-max argmax (:784-795). Stops at max_tokens,
 * at max_seq_len, or at 128001/128009 (generation.rs:241-260; the stop token
 * is not returned, as the reference does not push it). Runs on the device:
 * the decode step is captured (per context-length bucket) and replayed, the penalty's context is
 * kept as occurrence counts on the device and the sampled tokens are read
 * back in chunks. Sets the model's sampler (janus_model_set_sampler).
 * Under the penalty rule a NaN among a step's logits ends the call with
 * JANUS_E_NAN_LOGITS, where the reference's CPU sampler panics
 * (sampler.rs:191-193); the GPU-argmax rule ignores NaN as argmax.wgsl does. */
int janus_model_generate(janus_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_tokens,
                         float repetition_penalty, uint32_t *out_tokens, uint32_t *n_out);
/* Per-token callback of janus_model_generate_stream: `token` is the
 * index-th generated token (0-based). Return nonzero to go on, 0 to stop
 * with this token kept. It must not call into the same model. */
typedef int (*janus_token_callback)(void *user, uint32_t token, uint32_t index);
/* Model::generate_with_callback (generation.rs:340-604) at the token level:
 * janus_model_generate's prefill, sampler and stop rules, with every
 * generated token handed to cb once its step has run, in order, while the
 * next step runs on the GPU. cb returning 0 ends generation after that token,
 * which stays in the output (the reference pushes a token before its
 * callback and stops when the callback returns false, generation.rs:481-509);
 * a stop token 128001/128009 is neither returned nor passed to cb
 * (:462-479). Text-level work (detokenising, stop strings, the UTF-8 stream
 * decoder) belongs to the caller's callback, since token ids cross this
 * boundary. The step queued behind the one whose token ended generation
 * still runs (it writes one more position's K/V rows of this sequence) and
 * its token is dropped. cb may be NULL. Tokens land in out_tokens[0, *n_out) as in
 * janus_model_generate; the same NaN rule applies. */
int janus_model_generate_stream(janus_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_tokens,
                                float repetition_penalty, janus_token_callback cb, void *user, uint32_t *out_tokens,
                                uint32_t *n_out);
/* Model::generate_batch (generation.rs:673-870) with continuous batching:
 * request i is prompt_lens[i] token ids, the prompts back to back in
 * `prompts`. Up to max_batch requests run at once, each in its own KV slot
 * and at its own position (prefill token by token, then the re-fed last
 * prompt token, then decode). A request leaves when it has max_tokens
 * tokens, hits 128001/128009 (kept in its output, as the reference pushes
 * it before the check, generation.rs:810-833) or fills max_seq_len, and a
 * waiting request takes its slot without any KV copy. Sampling follows
 * Sampler::sample_batch (sampler.rs:379-428): the penalty over that
 * request's generated tokens, then the last-max argmax. Output: request i's
 * tokens at out_tokens[i * max_tokens], n_out[i] of them. Sets the model's
 * sampler. A NaN among any row's logits ends the call with
 * JANUS_E_NAN_LOGITS (sample_batch panics, sampler.rs:397-399). */
int janus_model_generate_batch(janus_model *m, const uint32_t *prompts, const uint32_t *prompt_lens, uint32_t nreq,
                               uint32_t max_tokens, float repetition_penalty, uint32_t *out_tokens, uint32_t *n_out);

/* Greedy rule of the device-side decode step (graph decode, generate). */
#define JANUS_SAMPLER_ARGMAX 0   /* last maximal logit, no penalty */
#define JANUS_SAMPLER_PENALTY 1  /* repetition penalty over the generated tokens, then last-max
                                    (sampler.rs:599-613, 784-795) */
#define JANUS_SAMPLER_WGSL 2     /* no penalty, the tie rule of shaders/argmax.wgsl:26-126 */
int janus_model_set_sampler(janus_model *m, int mode, float repetition_penalty);

/* Graph decode: capture one greedy decode step (embed from device ids ->
 * forward -> greedy choice under the model's sampler written back as the next
 * ids, positions advanced on the device) for nseq sequences once, then replay
 * it `steps` times. janus_model_graph_begin sets sequence s to token
 * tokens[s] at position positions[s] in KV slot s (or slots[s]) and clears
 * its generated tokens. A step is captured per sequence count and per
 * context-length bucket (256, 512, 1024, ... positions, the last one
 * max_seq_len; its attention is planned for the bucket's length), and kept
 * until a tensor or the KV cache is replaced; each replay runs the smallest
 * bucket that covers its sequences. graph_begin captures every bucket from
 * the sequences' current lengths up to max_seq_len, so graph_run never
 * captures. */
int janus_model_graph_begin(janus_model *m, const uint32_t *tokens, const uint32_t *positions, uint32_t nseq);
int janus_model_graph_begin_slots(janus_model *m, const uint32_t *tokens, const uint32_t *positions,
                                  const uint32_t *slots, uint32_t nseq);
/* graph_run returns once the steps have run (it synchronises the context's
 * stream). Under JANUS_SAMPLER_ARGMAX or _PENALTY a NaN among a sequence's
 * logits stops that sequence (its generated tokens end before that step) and
 * the call returns JANUS_E_NAN_LOGITS (sampler.rs:191-193, 397-399). */
int janus_model_graph_run(janus_model *m, uint32_t steps);
/* The token each sequence consumes next (the last one chosen). */
int janus_model_graph_read_tokens(janus_model *m, uint32_t *h_tokens, uint32_t nseq);
/* The tokens generated so far by batch row `row` since its graph_begin or
 * admission: up to cap of them into h_tokens, their total in *n. */
int janus_model_read_generated(janus_model *m, uint32_t row, uint32_t *h_tokens, uint32_t cap, uint32_t *n);

#ifdef __cplusplus
}
#endif
#endif /* JANUS_MODEL_H */
