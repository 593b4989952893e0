// internal.h -- shared host/device definitions of libjanus_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/janus_hip.h"

// ---------------------------------------------------------------------------
// host-side context and weight handles
// ---------------------------------------------------------------------------

struct janus_ctx {
    int device = 0;
    int num_cus = 256;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string last_error;
    // binary16 M = 1 products with long rows use the LDS-staged kernel
    // (JANUS_GEMV_KERNEL=reg selects the register-resident one instead).
    bool gemv_lds = true;
    // M = 1 products: most resident wavefronts per CU the grids ask for, for
    // the register kernel and the LDS-staged kernel (JANUS_GEMV_WPC,
    // JANUS_GEMV_LDS_WPC)
    uint32_t gemv_wpc = 16;
    uint32_t gemv_lds_wpc = 16;
    uint32_t gemv_lds_threads = 0;   // LDS GEMV workgroup size (0: chosen per launch)
    bool gemv_f16_rows2 = true;      // F16 rows of 8 units per lane: two rows per step
    // binary16-cache attention scores on MFMA (JANUS_ATTN_KERNEL=valu selects
    // the all-VALU kernel instead, for comparisons).
    bool attn_valu = false;
    // attention context split: about this many wavefronts per CU (JANUS_ATTN_WPC)
    uint32_t attn_wpc = 8;
    // binary16-cache attention piece length in positions (0: planned; JANUS_ATTN_TASK)
    uint32_t attn_task = 0;
    // ragged binary16-cache batches with 4 or 8 KV heads of 128 dims stream
    // whole cache rows through LDS, one workgroup per CU (JANUS_ATTN_ROWS:
    // 0 never, 1 whenever the shape allows, unset: planned)
    int attn_rows = -1;
    bool fused_step = true;          // JANUS_FUSED=0: models take the per-operator step (A/B and parity probes)
    // wavefronts per workgroup of the per-query-head attention launch (short
    // contexts, few sequences): 4, 8 or 16 (JANUS_ATTN_QH_NW; 0: planned)
    uint32_t attn_qh_nw = 0;
    // small-M quantised GEMMs over several K passes per workgroup use the
    // cross-pass pipelined kernel (JANUS_GEMM_PIPE=0 selects the single-buffered one)
    bool gemm_pipe = true;
    bool epi_split = true;           // batched residual + RMSNorm in two spread launches
    // captured decode steps, one per context-length bucket (JANUS_GRAPH_BUCKETS=0:
    // one step planned for max_seq_len, for comparisons)
    bool graph_buckets = true;
    // small-M GEMM pass length / K split forced for every product (0: planned)
    uint32_t gemm_kr = 0, gemm_ks = 0;
    // Attention split-K partials; grows on first use and is then reused.
    void *attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    // Small-M GEMM split-K partials; grows on first use.
    void *gemm_ws = nullptr;
    size_t gemm_ws_bytes = 0;
    // Workspaces replaced by a larger one. A captured graph may still write
    // them, so they are freed only by janus_destroy.
    std::vector<void *> retired;
    // Device address of this device's fixed attention scratch (the
    // allocation-free entry point), or null if the lookup failed.
    float *attn_scratch = nullptr;
    std::string attn_scratch_error;
};

// Size of the fixed attention scratch: one per device, held for the life of
// the process. Split partials of up to this many bytes run allocation-free.
constexpr size_t kAttnScratchBytes = JANUS_ATTN_SCRATCH_BYTES;
constexpr int kMaxScratchDevices = 64;

// Greedy sampler state in device memory, read by the argmax kernels, so a
// captured decode step follows a change without being captured again.
//  SAMPLE_ARGMAX : last maximal index, no penalty.
//  SAMPLE_PENALTY: repetition penalty over the generated tokens, then the
//                  last maximal index (model/sampler.rs:146-209,599-613,784-795).
//  SAMPLE_WGSL   : the GPU argmax of shaders/argmax.wgsl:26-126, which the
//                  reference takes when |penalty - 1| < 0.01 (sampler.rs:154-160).
enum { SAMPLE_ARGMAX = 0, SAMPLE_PENALTY = 1, SAMPLE_WGSL = 2 };
struct SamplerDev {
    float penalty;
    int32_t mode;
};


// HBM layout of an uploaded weight. Rows are the output dimension n.
//  Q4_0 : qs  = n * nb * 16 bytes (GGML nibble order per block), 16-B aligned
//         sc  = n * nb binary16 scales (nb = k / 32)
//  Q8_0 : qs  = n * nb * 32 bytes (int8), sc = n * nb binary16 scales
//  Q4_K : qs  = the GGML 144-byte super-blocks, 256-B aligned base, with the
//         12 scale bytes rewritten as chunk-pair fields (kquant_pack_scales,
//         read by kq_group)
//  Q5_K : qs  = the GGML 176-byte super-blocks, scale bytes as Q4_K, with
//         qh[32] rewritten as one 32-bit word of high bits per 16-byte quant
//         chunk (q5k_pack_high_bits)
//  F16  : qs  = n * k binary16, row-major, FTZ applied at upload when flagged
struct janus_weight {
    int type = 0;
    uint32_t n = 0, k = 0;
    uint32_t flags = 0;
    void *base = nullptr;     // single allocation
    size_t bytes = 0;
    const uint8_t *qs = nullptr;
    const uint16_t *sc = nullptr;
    // MFMA tile copy for the small-M GEMM (smallm.hip), built on first use.
    void *t32 = nullptr;
    const uint8_t *t32_qs = nullptr;
    const uint8_t *t32_side = nullptr;
    const uint32_t *t32_q5h = nullptr;   // Q5_K: the fifth bits, one word per lane and chunk
    uint32_t t32_chunks = 0;
};

namespace janus {

// Records `msg` as the context's last error and returns `code`.
int fail(janus_ctx *ctx, int code, const std::string &msg);
int hip_fail(janus_ctx *ctx, hipError_t e, const char *what);

#define JANUS_HIP_CHECK(ctx, expr)                                  \
    do {                                                            \
        hipError_t _e = (expr);                                     \
        if (_e != hipSuccess) return ::janus::hip_fail(ctx, _e, #expr); \
    } while (0)

#define JANUS_LAUNCH_CHECK(ctx)                                     \
    do {                                                            \
        hipError_t _e = hipGetLastError();                          \
        if (_e != hipSuccess) return ::janus::hip_fail(ctx, _e, "kernel launch"); \
    } while (0)

inline bool is_act_dtype(int dt) { return dt == JANUS_DT_F32 || dt == JANUS_DT_F16; }
inline size_t act_bytes(int dt) { return dt == JANUS_DT_F16 ? 2 : 4; }

// Grows the context's attention workspace to at least `bytes`.
int ensure_attn_ws(janus_ctx *ctx, size_t bytes);
// Grows the small-M GEMM split-K partials to at least `bytes`.
int ensure_gemm_ws(janus_ctx *ctx, size_t bytes);
// Returns JANUS_E_NO_DEVICE for a validation-only context (device < 0).
int need_device(janus_ctx *ctx);

// M = 1 product (gemv.hip). residual may be null; when set, y must be F32.
int gemv_dispatch(janus_ctx *ctx, const void *x, int x_dt, const janus_weight *w, void *y, int y_dt,
                  const float *residual);
// Paired-row M = 1 products: epi 0 = fused QKV with RoPE and KV append (q
// rotated into y, f32; K/V land in cache row rowbase[0] + pos[0], rowbase may
// be null for 0), epi 1 = fused gate/up with SwiGLU into y. x is f16, or,
// with gamma set, the f32 residual stream RMS-normalised in the kernel. x32:
// the products read binary32 x (f32 x, or its RMSNorm kept in f32: the
// reference's dtype) instead of binary16.
int gemv_pair_dispatch(janus_ctx *ctx, const void *x, const janus_weight *w, int epi, void *y, int y_f16, void *kc,
                       void *vc, int kv_f16, const float *rope, const int32_t *d_pos, const int32_t *d_rowbase,
                       uint32_t q_pairs, uint32_t k_pairs, uint32_t half_hd, uint32_t kv_row,
                       const float *gamma = nullptr, float eps = 0.0f, int x32 = 0);
// M = 1 product of RMSNorm(x, gamma, eps) (x f32) into y (f32). With best
// set, the outputs are also folded into *best as the running maximum of
// sampler_key (counts: the row's occurrence counts of generated tokens, or
// null); *best must be 0 before the launch.
int gemv_norm_dispatch(janus_ctx *ctx, const float *x, const float *gamma, float eps, const janus_weight *w, float *y,
                       unsigned long long *best, const uint32_t *counts = nullptr,
                       const SamplerDev *sampler = nullptr, int x32 = 0);
// Row layout of an uploaded weight (bytes of quants, binary16 scales per row).
size_t weight_qs_row_bytes(int type, uint32_t k);
size_t weight_sc_row_elems(int type, uint32_t k);
// Device allocation of an empty weight of the given type and shape.
int weight_alloc(janus_ctx *ctx, int type, uint32_t n, uint32_t k, uint32_t flags, janus_weight **out);
// rows >= 1 product (small-M MFMA GEMM for rows > 1).
int gemm_dispatch(janus_ctx *ctx, const void *a, int a_dt, const janus_weight *w, void *c,
                  int c_dt, uint32_t rows, const float *residual);
int smallm_gemm_launch(janus_ctx *ctx, const void *a, int a_dt, const janus_weight *w, void *c, int c_dt,
                       uint32_t rows, const float *residual);
// The MFMA GEMM takes binary16 activations and k % 8 == 0; prepare builds the
// weight's tile copy (allocates: call outside graph capture).
bool mfma_gemm_supported(int a_dt, const janus_weight *w);
int mfma_gemm_prepare(janus_ctx *ctx, const janus_weight *w);

// Split-K partials of one MFMA product: ws[ksplit][mpad][npad] (f32), and
// beside them in the same workspace a small per-row area for the epilogues
// (ss: kEpiSlices floats per row).
constexpr uint32_t kEpiSlices = 16;
struct GemmPartials {
    const float *ws;
    uint32_t ksplit, mpad, npad;
    float *ss;
};
// Batched products (binary16 rows, 1..64) whose epilogue kernel sums the
// partials and finishes the step:
//  gemm_qkv_rope: rows of the fused QKV weight (RoPE pairs of the q heads,
//    of the k heads, then v) -> q rotated (f32 [rows][q_pairs * 2]), k rotated
//    and v appended to the cache row rowbase[m] + pos[m] (kv_row elements;
//    m * max_seq + pos[m] when rowbase is null).
//  gemm_swiglu: interleaved gate/up rows -> act (binary16 [rows][n / 2]).
//  gemm_residual_norm: out = resid + product (f32, may alias resid), then
//    xn = RMSNorm(out) * gamma (binary16), one workgroup per row.
struct QkvEpilogue {
    float *q;
    void *kc, *vc;
    const float *rope;
    const int32_t *pos;
    const int32_t *rowbase;   // KV row base per row (null: m * max_seq)
    uint32_t q_pairs, k_pairs, half_hd, kv_row, max_seq;
};
int gemm_qkv_rope(janus_ctx *ctx, const void *a16, const janus_weight *w, uint32_t rows, const QkvEpilogue &e,
                  int kv_f16);
int gemm_swiglu(janus_ctx *ctx, const void *a16, const janus_weight *w, uint32_t rows, void *act16);
bool resnorm_supported(uint32_t hidden);
int gemm_residual_norm(janus_ctx *ctx, const void *a16, const janus_weight *w, uint32_t rows, const float *resid,
                       float *out, const float *gamma, float eps, void *xn16);

enum { EW_SILU = 0, EW_MUL = 1, EW_ADD = 2, EW_SWIGLU = 3 };
int rmsnorm_launch(janus_ctx *ctx, const float *in, void *out, int out_dt, const float *gamma, uint32_t batch,
                   uint32_t hidden, float eps);
int elementwise_launch(janus_ctx *ctx, int op, const float *a, const float *b, void *out, int out_dt, uint32_t n);
int rope_launch(janus_ctx *ctx, const float *in, float *out, const float *table, uint32_t batch, uint32_t heads,
                uint32_t hd, uint32_t position, const int32_t *positions);
int kv_update_launch(janus_ctx *ctx, const float *k_new, const float *v_new, void *kc, void *vc, int kv_dt,
                     uint32_t batch, uint32_t row_elems, uint32_t position, uint32_t max_seq,
                     const int32_t *row_base, const int32_t *positions);
// Attention split sizing shared by the launch and workspace reservation.
// rows: 1 when the row-streaming kernel runs (chunk then counts 16-position blocks).
void attention_plan(const janus_ctx *ctx, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                    uint32_t max_len, int kv_f16, uint32_t *chunk, uint32_t *nw, uint32_t *splits,
                    uint32_t *qh_div, uint32_t *rows);
// Bytes of split partials a launch of this shape writes (0: no split).
size_t attention_ws_bytes(const janus_ctx *ctx, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                          uint32_t max_len, int kv_f16);
int attention_reserve(janus_ctx *ctx, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                      uint32_t max_len, int kv_f16);
// out is f32, or binary16 when out_f16 is set. With fixed_ws set the split
// partials go there (JANUS_E_INVALID_DIM when they need more than
// fixed_ws_bytes) and nothing is allocated; otherwise into the context's
// workspace, grown on demand.
int attention_launch(janus_ctx *ctx, const float *q, const void *kc, const void *vc, int kv_dt, void *out,
                     uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t seq_len,
                     uint32_t max_seq, const int32_t *row_base, const int32_t *seq_lens, uint32_t max_len,
                     float scale, int out_f16 = 0, float *fixed_ws = nullptr, size_t fixed_ws_bytes = 0);
// Looks up, once per device, the device address of the fixed attention
// scratch (kAttnScratchBytes) and stores it in ctx->attn_scratch. Called by
// janus_create with the context's device current.
int attention_scratch_init(janus_ctx *ctx);
int embed_launch(janus_ctx *ctx, const janus_weight *table, const uint32_t *h_ids, const int32_t *d_ids,
                 uint32_t batch, float *out);
int argmax_launch(janus_ctx *ctx, const float *logits, int32_t *out, uint32_t vocab, uint32_t batch, int tie);
// Greedy choice of each row as a running atomicMax of sampler_key into
// best[row] (zero before the call; the caller reads and clears it), the
// rows split over many workgroups. counts: [batch][vocab] occurrence counts
// of the generated tokens (read under SAMPLE_PENALTY), or null; sampler
// null means SAMPLE_ARGMAX.
int argmax_keys_launch(janus_ctx *ctx, const float *logits, unsigned long long *best, uint32_t vocab,
                       uint32_t batch, const uint32_t *counts = nullptr, const SamplerDev *sampler = nullptr);
// Repetition penalty over a token list in list order (sampler.rs:599-613),
// parallel over distinct ids: each id's occurrences are applied in sequence
// by one lane.
int penalty_launch(janus_ctx *ctx, float *logits, uint32_t vocab, const int32_t *ids, uint32_t n, float penalty);

}  // namespace janus

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

typedef _Float16 jh2 __attribute__((ext_vector_type(2)));
typedef _Float16 jh4 __attribute__((ext_vector_type(4)));
typedef float jf2 __attribute__((ext_vector_type(2)));
// 0x64006400 (binary16 pair 1024, 1024) materialised in a VGPR: with the
// constant in a register, (x & mask) | c compiles to one v_and_or_b32 (VOP3
// takes no literal on gfx9). Not volatile, so it is hoisted and shared.
__device__ __forceinline__ uint32_t vgpr_const_6400() {
    uint32_t m;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(m));
    return m;
}
typedef float jf4 __attribute__((ext_vector_type(4)));
typedef uint32_t ju4 __attribute__((ext_vector_type(4)));

// 128-bit streaming load (non-temporal: weights are read once per launch).
__device__ __forceinline__ uint4 ld_stream(const void *p) {
#if !defined(JANUS_GEMV_NT) || JANUS_GEMV_NT
    ju4 v = __builtin_nontemporal_load((const ju4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return *(const uint4 *)p;
#endif
}

// Exact binary16 -> binary32 (subnormals kept). Hardware conversion is exact
// with f16 denormals enabled (the gfx950 default for HIP).
__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// K-quant (Q4_K / Q5_K) scales in HBM. Bytes 0-3 of a super-block are d and
// dmin (binary16), as in GGML. The 12 bytes after them, little-endian words
// s0, s1, s2 (96 bits), hold for chunk pair j = 0..3 (quant bytes 32j ..
// 32j + 31, sub-blocks 2j and 2j + 1) the 24-bit field at bit 24j:
// sc(2j), sc(2j + 1), m(2j), m(2j + 1), six bits each from the low end. GGML
// spreads sub-blocks 4..7 over three bytes each (get_scale_min_k4); here one
// funnel shift gives a chunk its whole field. Returns that field in bits 0-23.
__device__ __forceinline__ uint32_t kq_group(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j) {
    const uint32_t lo = j < 2 ? s0 : (j == 2 ? s1 : s2);
    const uint32_t hi = j < 2 ? s1 : s2;
    return __builtin_amdgcn_alignbit(hi, lo, (32u - 8u * j) & 31u);   // bits 24j.. of s2:s1:s0
}

// Q8_0 scale decode of shaders/gemm_q8_0.wgsl:33-60: exact, but exponent 31
// (inf/nan) becomes +-1e38.
__device__ __forceinline__ float h2f_q8(uint16_t h) {
    float v = h2f(h);
    return ((h & 0x7c00u) == 0x7c00u) ? ((h & 0x8000u) ? -1e38f : 1e38f) : v;
}

__device__ __forceinline__ uint16_t f2h_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // round to nearest even
}

template <typename T> __device__ __forceinline__ T shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// Order-preserving key of a float (larger value -> larger key); NaN maps to 0
// so it never wins. Packed with the index below it, the maximum key is the
// largest value and, among equal values, the last index (argmax "last max").
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t k = (v != v) ? 0u : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
    return ((uint64_t)k << 32) | idx;
}

// Key of a NaN logit under SAMPLE_ARGMAX and SAMPLE_PENALTY: above every
// other key, so a row's running maximum carries it to the step's consumer,
// which refuses the step (the reference's CPU sampler panics on NaN logits,
// sampler.rs:191-193 and 397-399). SAMPLE_WGSL never produces it.
constexpr uint64_t kNanKey = ~0ull;

// Argmax key of logit v at index idx under the sampler state s.
//  SAMPLE_ARGMAX / SAMPLE_PENALTY: a NaN v gives kNanKey.
//  SAMPLE_PENALTY: v first takes the repetition penalty once per occurrence
//    of idx among the generated tokens (count; sampler.rs:599-613:
//    divide when positive, else multiply). Occurrences of one id are applied
//    in order and ids do not interact, so this equals the reference's loop
//    over the context. Then the last-max key.
//  SAMPLE_WGSL: among equal values the smallest (bitrev8(idx % 256), idx)
//    wins, and values not above -1e38 (or NaN) count as -1e38 at index 0:
//    the per-lane strict '>' scan from -1e38 and the strict '>' tree of
//    shaders/argmax.wgsl:26-126. Index below 2^24.
__device__ __forceinline__ uint64_t sampler_key(float v, uint32_t idx, uint32_t count, int mode,
                                                float penalty) {
    if (mode == SAMPLE_WGSL) {
        if (!(v > -1e38f)) {
            v = -1e38f;
            idx = 0;
        }
        const uint32_t u = __float_as_uint(v);
        const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
        const uint32_t pri = (__builtin_bitreverse32(idx & 255u) & 0xff000000u) | idx;
        return ((uint64_t)k << 32) | (uint32_t)~pri;
    }
    if (v != v) return kNanKey;
    if (mode == SAMPLE_PENALTY)
        for (uint32_t c = count; c; --c) v = v > 0.0f ? v / penalty : v * penalty;
    return argmax_key(v, idx);
}

// Token index held by a nonzero sampler_key.
__device__ __forceinline__ uint32_t sampler_key_index(uint64_t key, int mode) {
    return mode == SAMPLE_WGSL ? (~(uint32_t)key) & 0xffffffu : (uint32_t)key;
}

// Sum over all 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor(v, o);
    return v;
}

// The same total with permlane swaps and DPP row rotations (no LDS traffic,
// no wait between the steps; a different summation order than wave_sum).
__device__ __forceinline__ float wave_sum_dpp(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));   // row_ror:8
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false));   // row_ror:4
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xf, 0xf, false));   // row_ror:2
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false));   // row_ror:1
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, shfl_xor(v, o));
    return v;
}
