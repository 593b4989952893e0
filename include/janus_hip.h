/*
 * janus_hip.h -- C ABI of the MI355X (gfx950) decode hot path.
 *
 * This library replaces the wgpu backend behind janus-engine's operator
 * layer (the crates/janus-engine/src/compute/ops module). Each entry point below
 * names the reference function it stands in for (paths relative to
 * crates/janus-engine/src/). Conventions shared by every call:
 *
 *  - Every function returns a janus_status; on failure janus_last_error()
 *    holds a message. Argument and dimension checks happen on the host
 *    before anything is enqueued, so they are testable without a GPU.
 *  - Pointers named d_* or documented as "device" are HIP device pointers
 *    owned by the caller (the reference's caller-owned wgpu::Buffers,
 *    model/transformer/constructor.rs:148-344). Weights are library-owned
 *    janus_weight handles (the reference's GpuTensor, compute/tensor.rs:4-7).
 *  - Calls enqueue on the context's current stream and return without
 *    waiting (the reference records into a CommandEncoder and submits once,
 *    model/transformer/forward.rs:116). janus_sync and janus_d2h block.
 *  - A context is used from one thread at a time, like the reference's
 *    Arc<tokio::Mutex<Model>> (src/app.rs:17).
 *  - No entry point allocates device memory on the per-token path except
 *    where it says so (workspaces grow on first use and are then reused).
 */
#ifndef JANUS_HIP_H
#define JANUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JANUS_ABI_VERSION 1

/* Status codes. Reference error type: compute/error.rs:5-35. */
typedef enum janus_status {
    JANUS_OK = 0,
    JANUS_E_INVALID_ARG = 1,       /* null pointer, zero size, bad enum */
    JANUS_E_INVALID_DIM = 2,       /* ComputeError::InvalidDimensions (ops/quantized.rs:199-204,327-332) */
    JANUS_E_UNSUPPORTED_DTYPE = 3, /* replaces panic! (ops/quantized.rs:181) and engine.rs:833-838 */
    JANUS_E_KV_OVERFLOW = 4,       /* ComputeError::Other (compute/cache/core.rs:283-288) */
    JANUS_E_TOKEN_RANGE = 5,       /* token id >= vocab (model/transformer/embedding.rs:33-39) */
    JANUS_E_HIP = 6,               /* ComputeError::KernelExecutionFailed */
    JANUS_E_OOM = 7,               /* ComputeError::BufferCreationFailed */
    JANUS_E_NO_DEVICE = 8,         /* no adapter (compute/engine.rs:32-39) */
    JANUS_E_NAN_LOGITS = 9         /* NaN logits under the CPU-path greedy rules; the reference
                                      panics (model/sampler.rs:191-193, 397-399) */
} janus_status;

/* Tensor element types use GGML's type ids (formats/gguf/types.rs:80-187). */
typedef enum janus_dtype {
    JANUS_DT_F32 = 0,
    JANUS_DT_F16 = 1,
    JANUS_DT_Q4_0 = 2,
    JANUS_DT_Q8_0 = 8,
    JANUS_DT_Q4_K = 12,
    JANUS_DT_Q5_K = 13,
    JANUS_DT_Q6_K = 14
} janus_dtype;

/* janus_weight_upload flags. */
#define JANUS_WEIGHT_FTZ_F16 0x1u  /* decode binary16 values (F16 weights, Q4_K d/dmin)
                                      with f16_to_f32_safe semantics: subnormals -> +-0
                                      (shaders/gemm_q4_k.wgsl:30-43, shaders/gemm.wgsl:18-31) */
#define JANUS_WEIGHT_Q6K_REF_ORDER 0x2u  /* Q6_K: the element order of the reference loader's
                                            q6_k_to_f32 (compute/engine.rs:198-248) instead of
                                            GGML's dequantize_row_q6_K order */

/* argmax tie rules. */
#define JANUS_TIE_LAST 0  /* Sampler::argmax, model/sampler.rs:784-795: last maximal index */
#define JANUS_TIE_WGSL 1  /* shaders/argmax.wgsl:26-126: smallest (bitrev8(i % 256), i) among ties */

typedef struct janus_ctx janus_ctx;
typedef struct janus_weight janus_weight;

/* ---- context: ComputeEngine::new (compute/engine.rs:27-83) ------------ */
int janus_create(int hip_device, janus_ctx **out);
void janus_destroy(janus_ctx *ctx);
const char *janus_last_error(const janus_ctx *ctx);
const char *janus_status_string(int status);
int janus_abi_version(void);
/* Run subsequent calls on `hip_stream` (a hipStream_t) exactly as given:
 * NULL selects the legacy default stream. A new context runs on its own
 * non-blocking stream, which janus_get_stream returns before any change. */
int janus_set_stream(janus_ctx *ctx, void *hip_stream);
void *janus_get_stream(janus_ctx *ctx);
int janus_sync(janus_ctx *ctx);                      /* device.poll(wait) */
/* Current sizes of the context's attention and small-M GEMM workspaces (the
 * library-owned split-K partials; diagnostics, no reference counterpart).
 * A workspace that grows keeps its old buffer until janus_destroy, because a
 * captured HIP graph may still use it. */
int janus_workspace_bytes(const janus_ctx *ctx, size_t *attn_bytes, size_t *gemm_bytes);
int janus_device_count(int *count);
/* Buffer helpers for callers without their own allocator (Buffer,
 * compute/buffer.rs): plain device memory. */
int janus_alloc(janus_ctx *ctx, size_t bytes, void **d_ptr);
int janus_free(janus_ctx *ctx, void *d_ptr);
int janus_h2d(janus_ctx *ctx, void *d_dst, const void *h_src, size_t bytes);
int janus_d2h(janus_ctx *ctx, void *h_dst, const void *d_src, size_t bytes); /* blocks */

/* ---- weights: ComputeEngine::allocate_tensors (compute/engine.rs:424-858) */
/* Upload one 2-D GGUF tensor of logical shape [n rows][k cols] (the PyTorch
 * [out, in] order the reference's gemm_auto consumes, ops/quantized.rs:63-74).
 * `bytes` holds the tensor exactly as stored in a GGUF file:
 *   F32  -> converted to binary16 RNE (engine.rs:471-500), FTZ if flagged;
 *   F16  -> binary16 (engine.rs:539-566), FTZ if flagged;
 *   Q4_0 -> 18-byte GGML blocks (no reference kernel: engine.rs:833-838);
 *   Q8_0 -> 34-byte GGML blocks (engine.rs:772-797, read with the GGML
 *           34-byte stride rather than the shader's 36, gemm_q8_0.wgsl:79);
 *   Q4_K -> 144-byte GGML block_q4_K (engine.rs:662-687);
 *   Q5_K -> 176-byte GGML block_q5_K, kept raw as the reference keeps it
 *           (engine.rs:717-742) but read in GGML order (its shader,
 *           gemm_q5_k.wgsl:6-23, reads the bytes at other offsets);
 *   Q6_K -> 210-byte GGML block_q6_K, dequantised on the host to binary16
 *           exactly as engine.rs:800-831 does; the handle then reports F16.
 * The library repacks into its own HBM layout. k must be a multiple of the
 * block width (32, or 256 for the K-quants): JANUS_E_INVALID_DIM otherwise. */
int janus_weight_upload(janus_ctx *ctx, int ggml_type, uint32_t n, uint32_t k,
                        const void *bytes, size_t nbytes, uint32_t flags,
                        janus_weight **out);
int janus_weight_free(janus_ctx *ctx, janus_weight *w);
int janus_weight_info(const janus_weight *w, int *ggml_type, uint32_t *n, uint32_t *k,
                      size_t *device_bytes);
/* Dequantise the stored weight into d_out[n*k] (f32, row-major) with exactly
 * the arithmetic the matrix kernels use; the bit-exactness check of the
 * dequantised weights. */
int janus_weight_dequant(janus_ctx *ctx, const janus_weight *w, float *d_out);

/* ---- matrix products: gemm_auto (ops/quantized.rs:63-186) -------------- */
/* C[b, i, :] = A[b, i, :] . W^T for b < batch, i < m; A is [batch*m][k] of
 * a_dtype (F32 or F16), C is [batch*m][n] of c_dtype (F32 or F16). Rows
 * batch*m == 1 run the GEMV kernels; up to 64 rows run the small-M MFMA GEMM
 * (the reference's M>1 quantized fallback, quantized.rs:77-90, is replaced
 * by a correct product). k and n must match the weight. */
int janus_gemm_auto(janus_ctx *ctx, const void *a, int a_dtype, const janus_weight *w,
                    void *c, int c_dtype, uint32_t batch, uint32_t m, uint32_t k,
                    uint32_t n);
/* As janus_gemm_auto, then C += R (R: [rows][n] f32, may alias C): the
 * o-proj / down-proj residual adds of model/block.rs:355,447 fused into the
 * product's epilogue. */
int janus_gemm_residual(janus_ctx *ctx, const void *a, int a_dtype, const janus_weight *w,
                        const float *residual, float *c, uint32_t rows, uint32_t k,
                        uint32_t n);

/* ---- elementwise and normalisation (ops/activation.rs, ops/elementwise.rs) */
/* rmsnorm (ops/activation.rs:58-123): out = x / sqrt(mean(x^2) + eps) * gamma,
 * per row of `hidden`; out_dtype F32 or F16. */
int janus_rmsnorm(janus_ctx *ctx, const float *in, void *out, int out_dtype,
                  const float *gamma, uint32_t batch, uint32_t hidden, float eps);
int janus_silu(janus_ctx *ctx, const float *in, float *out, uint32_t size);   /* activation.rs:137-196 */
int janus_elementwise_mul(janus_ctx *ctx, const float *a, const float *b, float *out,
                          uint32_t size);                                        /* elementwise.rs:107-164 */
int janus_add_tensors(janus_ctx *ctx, const float *a, const float *b, float *out,
                      uint32_t size);                                            /* elementwise.rs:36-93 */
/* silu(gate) * up in one pass (model/block.rs:411-430, two reference
 * dispatches); out_dtype F32 or F16. */
int janus_swiglu(janus_ctx *ctx, const float *gate, const float *up, void *out,
                 int out_dtype, uint32_t size);

/* ---- RoPE (ops/rope.rs:48-115; table: model/transformer/constructor.rs:454-489) */
/* Fill d_table[max_seq][head_dim/2][2] = (cos, sin) of pos / base^(2i/hd),
 * computed on the host in binary32 as the reference does, then uploaded. */
int janus_rope_table(janus_ctx *ctx, float *d_table, uint32_t max_seq, uint32_t head_dim,
                     float theta_base);
/* Half-split rotation of in[batch][heads][head_dim] into out (may alias).
 * d_positions == NULL: every row uses `position` (the reference's shared
 * position, shaders/rope.wgsl:64-66); otherwise row b uses d_positions[b]. */
int janus_rope(janus_ctx *ctx, const float *in, float *out, const float *d_table,
               uint32_t batch, uint32_t heads, uint32_t head_dim, uint32_t position,
               const int32_t *d_positions);

/* ---- KV cache (compute/cache/core.rs:261-469) ------------------------- */
/* Append one token of K and V per sequence:
 *   k_cache[row_base[b] + pos_b][kvh][hd] = k_new[b][kvh][hd] (same for v),
 * stored as kv_dtype (F32 as the reference, or F16). The cache pointers
 * address one layer's slice. d_row_base == NULL means row_base[b] =
 * b * max_seq_len; d_positions == NULL means pos_b = position, which must
 * be < max_seq_len (JANUS_E_KV_OVERFLOW otherwise, core.rs:283-288). */
int janus_kv_update(janus_ctx *ctx, const float *k_new, const float *v_new, void *k_cache,
                    void *v_cache, int kv_dtype, uint32_t batch, uint32_t kv_heads,
                    uint32_t head_dim, uint32_t position, uint32_t max_seq_len,
                    const int32_t *d_row_base, const int32_t *d_positions);

/* ---- decode attention: compute_attention (ops/attention.rs:78-235) ----- */
/* One query token per sequence, q[batch][heads][head_dim] f32, against
 * keys/values at rows [row_base[b], row_base[b] + len_b) of k_cache/v_cache
 * ([rows][kv_heads][head_dim], kv_dtype F32 or F16). Query head h reads KV
 * head (h * kv_heads) / heads (shaders/attention.wgsl:243). len_b =
 * d_seq_lens[b], or seq_len for all when d_seq_lens is NULL; d_row_base NULL
 * means b * max_seq_len. Long contexts are split across workgroups and
 * merged with a log-sum-exp reduction; the workspace grows on first use.
 * scale <= 0 selects 1/sqrt(head_dim) (ops/attention.rs:98). */
int janus_attention(janus_ctx *ctx, const float *q, const void *k_cache, const void *v_cache,
                    int kv_dtype, float *out, uint32_t batch, uint32_t heads,
                    uint32_t kv_heads, uint32_t head_dim, uint32_t seq_len,
                    uint32_t max_seq_len, const int32_t *d_row_base,
                    const int32_t *d_seq_lens, uint32_t max_len_hint, float scale);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): janus_attention with the same arguments, kernels and
 * results, whose split partials go to a fixed per-device scratch of
 * JANUS_ATTN_SCRATCH_BYTES held for the life of the process, so the call
 * allocates nothing. A shape whose partials need more than that is rejected
 * with JANUS_E_INVALID_DIM before anything is enqueued. Every call on a
 * device shares that device's scratch: calls that overlap on one GPU (two
 * streams, or two contexts on different threads) race on it. */
#define JANUS_ATTN_SCRATCH_BYTES (16u << 20)
int janus_attention_noalloc(janus_ctx *ctx, const float *q, const void *k_cache, const void *v_cache,
                            int kv_dtype, float *out, uint32_t batch, uint32_t heads,
                            uint32_t kv_heads, uint32_t head_dim, uint32_t seq_len,
                            uint32_t max_seq_len, const int32_t *d_row_base,
                            const int32_t *d_seq_lens, uint32_t max_len_hint, float scale);

/* ---- embedding (model/transformer/embedding.rs:16-198) ---------------- */
/* out[b][:] = table[ids[b]][:] decoded as the table's binary16 values.
 * h_ids are host token ids checked against the vocabulary. */
int janus_embed(janus_ctx *ctx, const janus_weight *table, const uint32_t *h_ids,
                uint32_t batch, float *out);
/* Device-id variant for graph capture; ids >= vocab produce zero rows. */
int janus_embed_device(janus_ctx *ctx, const janus_weight *table, const int32_t *d_ids,
                       uint32_t batch, float *out);

/* ---- greedy sampling (model/sampler.rs:146-209; ops/argmax.rs:50-107) -- */
/* d_out[b] = argmax of logits[b][vocab] under tie_rule (JANUS_TIE_*). */
int janus_argmax(janus_ctx *ctx, const float *logits, int32_t *d_out, uint32_t vocab,
                 uint32_t batch, int tie_rule);
/* Repetition penalty (sampler.rs:599-613) applied in context order, so a
 * repeated id is divided (or multiplied) once per occurrence. */
int janus_repetition_penalty(janus_ctx *ctx, float *logits, uint32_t vocab,
                             const int32_t *d_context, uint32_t n_context, float penalty);

#ifdef __cplusplus
}
#endif
#endif /* JANUS_HIP_H */
