/*
 * janus_oracle.h -- CPU restatement of janus-engine's per-token decode
 * arithmetic, used ONLY as the checker for the HIP path.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or the
 * CPU baseline -- never as the product path.
 *
 * Every function restates one reference routine; the citation names the
 * reference file:line (paths relative to crates/janus-engine/src/).
 * Arithmetic is plain IEEE binary32 in the reference's operation order and
 * the file is compiled with -ffp-contract=off, so no FMA is formed unless a
 * function says so.
 */
#ifndef JANUS_ORACLE_H
#define JANUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- binary16 conversions --------------------------------------------- */
/* IEEE-exact decode (subnormals kept, inf/nan kept): GGML_FP16_TO_FP32 and
 * the `half` crate's f16::to_f32 (compute/engine.rs:392). */
float jo_f16_to_f32_exact(uint16_t h);
/* compute/shaders/gemm_q8_0.wgsl:33-60: subnormals kept, exponent 31 -> +-1e38. */
float jo_f16_to_f32_q8(uint16_t h);
/* f16_to_f32_safe, compute/shaders/gemm_q4_k.wgsl:30-43 (also gemm.wgsl:18-31,
 * embed.wgsl:11-20): subnormals flushed to signed zero. */
float jo_f16_to_f32_ftz(uint16_t h);
/* f32 -> binary16, round to nearest even: `half` f16::from_f32 used by
 * compute/engine.rs:133-136. */
uint16_t jo_f32_to_f16_rne(float f);
void jo_f32_to_f16_rne_n(const float *in, uint16_t *out, size_t n);
void jo_f16_to_f32_n(const uint16_t *in, float *out, size_t n, int mode); /* 0 exact,1 q8,2 ftz */

/* ---- block dequantisation (GGUF byte layouts) ------------------------- */
/* Q8_0: 34-byte GGML block {f16 d; int8 q[32]}; w = d*q with the q8 decode of d
 * (gemm_q8_0.wgsl:74-105 read with the GGML 34-byte stride, as
 * compute/engine.rs:377-409 does). */
void jo_dequant_q8_0(const uint8_t *blocks, size_t nblocks, float *out);
/* Q4_0: 18-byte GGML block {f16 d; uint8 qs[16]}: element j = (qs[j]&15)-8,
 * element j+16 = (qs[j]>>4)-8, w = d*q (GGML closed form; the reference has
 * no Q4_0 kernel, formats/gguf/types.rs:12,87). */
void jo_dequant_q4_0(const uint8_t *blocks, size_t nblocks, float *out);
/* Q4_K: 144-byte GGML block_q4_K {f16 d, dmin; u8 scales[12]; u8 qs[128]}
 * decoded as gemm_q4_k.wgsl:55-147: w = (d*sc)*q - (dmin*m); ftz!=0 decodes
 * d/dmin with f16_to_f32_safe (the shader's behaviour), ftz==0 exactly. */
void jo_dequant_q4_k(const uint8_t *blocks, size_t nblocks, int ftz, float *out);
/* get_scale_min_k4 restated from extract_6bit_from_packed, gemm_q4_k.wgsl:120-147 */
void jo_q4_k_scale_min(const uint8_t *scales12, int j, uint8_t *sc, uint8_t *mn);
/* Q5_K: 176-byte GGML block_q5_K {f16 d, dmin; u8 scales[12]; u8 qh[32];
 * u8 qs[128]} in GGML element order (ggml-quants.c dequantize_row_q5_K, the
 * published llama.cpp layout; the reference's shaders/gemm_q5_k.wgsl:6-23
 * reads these bytes at other offsets, so GGML defines it here): for chunk
 * j = 0..3, b = 0..31, with (sc, m) from jo_q4_k_scale_min:
 *   w[64j+b]    = (d*sc[2j])   * (qs[32j+b] & 15 | bit 2j   of qh[b] << 4) - dmin*m[2j]
 *   w[64j+32+b] = (d*sc[2j+1]) * (qs[32j+b] >> 4 | bit 2j+1 of qh[b] << 4) - dmin*m[2j+1]
 * rounded as the Q4_K form (product, then difference); ftz as for Q4_K. */
void jo_dequant_q5_k(const uint8_t *blocks, size_t nblocks, int ftz, float *out);
/* Q5_K product, the Q4_K accumulation order (per 64-chunk, per byte: low
 * then high element). */
void jo_gemv_q5_k(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k, int ftz);
/* Q6_K: 210-byte block {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}.
 * ref_order == 0: GGML element order (ggml-quants.c dequantize_row_q6_K): half
 * h = 0,1 uses ql[64h..], qh[32h..], scales[8h..]; for l = 0..31, is = l/16:
 *   w[128h+l]    = (d*sc[is])   * ((ql[l]    & 15 | (qh[l]     & 3) << 4) - 32)
 *   w[128h+l+32] = (d*sc[is+2]) * ((ql[l+32] & 15 | (qh[l]>>2 & 3) << 4) - 32)
 *   w[128h+l+64] = (d*sc[is+4]) * ((ql[l]    >> 4 | (qh[l]>>4 & 3) << 4) - 32)
 *   w[128h+l+96] = (d*sc[is+6]) * ((ql[l+32] >> 4 | (qh[l]>>6 & 3) << 4) - 32)
 * ref_order != 0: the reference's own loader order, compute/engine.rs:198-248:
 * element i takes nibble i%2 of ql[i/2], bits 2(i%4) of qh[i/4], scale
 * scales[i/16]: w = (d*s)*(q-32). d decoded exactly (engine.rs:221).
 * Pinned by special values, single-bit brute force and a hand-worked
 * reference-order known answer; GGML element placement beyond the spot
 * checks of element l and l+96: parity unpinned (no GGML build here). */
void jo_dequant_q6_k(const uint8_t *blocks, size_t nblocks, int ref_order, float *out);

/* ---- matrix-vector products in the reference's accumulation order ------ */
/* gemm_q8_0.wgsl:74-128: per element sum += (d*q)*x; per block row += sum. */
void jo_gemv_q8_0(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k);
/* gemm_q4_k.wgsl:55-170 order: per 64-chunk, per byte: low then high nibble. */
void jo_gemv_q4_k(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k, int ftz);
/* Q4_0 in the same per-block order as the Q8_0 shader (no reference kernel). */
void jo_gemv_q4_0(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k);
/* gemm.wgsl:58-147: C[b,m,n] = sum_k A[b,m,k]*ftz(B[n,k]), B binary16 [N,K];
 * sequential k order (the 16-wide tiles preserve it). */
void jo_gemm_f16(const float *a, const uint16_t *b, float *c, uint32_t batch,
                 uint32_t m, uint32_t k, uint32_t n);
/* Double-precision reference y = W x with W already dequantised (n x k). */
void jo_gemv_f64(const float *w, const float *x, double *y, uint32_t n, uint32_t k);

/* ---- glue ops ---------------------------------------------------------- */
/* activations.wgsl:67-134: 256-lane strided partial sums, tree reduction,
 * rms = sqrt(sum/H + eps), y = (x / rms) * gamma. */
void jo_rmsnorm(const float *in, float *out, const float *gamma, uint32_t batch,
                uint32_t hidden, float eps);
/* activations.wgsl:20-35: x * (1 / (1 + exp(-x))). */
void jo_silu(const float *in, float *out, size_t n);
void jo_mul(const float *a, const float *b, float *out, size_t n);  /* elementwise_mul.wgsl:15-24 */
void jo_add(const float *a, const float *b, float *out, size_t n);  /* add_tensors.wgsl:15-24 */
/* model/transformer/constructor.rs:454-489: [max_seq][hd/2][cos,sin]. */
void jo_rope_table(float *table, uint32_t max_seq, uint32_t head_dim, float theta_base);
/* rope.wgsl:33-77 half-split rotation at one shared position. */
void jo_rope(const float *in, float *out, const float *table, uint32_t batch,
             uint32_t heads, uint32_t head_dim, uint32_t position);
/* attention.wgsl:62-186 + softmax.wgsl:18-51 for one sequence:
 * q [H][hd], k/v [len][kvh][hd] (f32), out [H][hd]. */
void jo_attention(const float *q, const float *k, const float *v, float *out,
                  uint32_t len, uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                  float scale);
/* embed.wgsl:31-63: out[b,:] = ftz(f16 table[id]). Returns -1 if id >= vocab
 * (model/transformer/embedding.rs:33-39), else 0. */
int jo_embed(const uint16_t *table, const uint32_t *ids, float *out, uint32_t batch,
             uint32_t hidden, uint32_t vocab);

/* ---- sampling ---------------------------------------------------------- */
/* model/sampler.rs:599-613: for each context token, logit /= p if > 0 else *= p. */
void jo_repetition_penalty(float *logits, uint32_t vocab, const uint32_t *ctx, size_t nctx,
                           float penalty);
/* model/sampler.rs:784-795: Iterator::max_by -> the LAST maximal index. */
uint32_t jo_argmax_last(const float *logits, uint32_t vocab);
/* argmax.wgsl:26-126: 256 lanes, strict '>' -> smallest (bitrev8(i%256), i) among ties. */
uint32_t jo_argmax_wgsl(const float *logits, uint32_t vocab);

/* ---- CPU baseline helpers (OpenMP over rows when built with it) -------- */
int jo_num_threads(void);
void jo_gemv_q4_0_mt(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k);

#ifdef __cplusplus
}
#endif
#endif
