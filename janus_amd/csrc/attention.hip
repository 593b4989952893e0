// attention.hip -- split-K GQA decode attention (one query token per sequence).
//
// Replaces compute_attention (crates/janus-engine/src/compute/ops/attention.rs:78-235:
// compute_qk_scores + softmax + apply_attention in attention.wgsl:62-186 and
// softmax.wgsl:18-51). Those three passes materialise scores/probabilities in
// HBM and run the softmax on one thread per head; here:
//  * grid = (split, kv_head, sequence). A workgroup owns the G = H / KVH query
//    heads that share one KV head and a contiguous chunk of positions.
//  * K/V tiles of 64 positions are staged through LDS with 128-bit loads (K
//    rows padded so per-position dot products read conflict-free), scores are
//    computed in fp32 from fp16 or fp32 keys, and an online (running max /
//    running sum) softmax accumulates P.V in fp32 registers.
//  * Each split writes (m, l, o[D]) partials; a merge kernel combines splits
//    with the log-sum-exp rule. A sequence covered by one split writes its
//    output directly.
//  * Ragged batches: per-sequence row offsets and lengths are device tables,
//    so all sequences share one launch.
#include "internal.h"

namespace janus {

namespace {

constexpr int TP = 64;        // positions per tile
constexpr int THREADS = 256;

template <typename KV> struct KVPad;
template <> struct KVPad<_Float16> { static constexpr int P = 8; };
template <> struct KVPad<float> { static constexpr int P = 4; };

struct AttnArgs {
    const float *q;
    const void *kc, *vc;
    void *out;              // [B][H][D] f32, or binary16 when out_f16
    float *ws;              // [B][H][S][D + 2]
    const int32_t *row_base;
    const int32_t *seq_lens;
    uint32_t batch, heads, kv_heads;
    uint32_t seq_len, max_seq;
    uint32_t chunk;         // positions per split (multiple of TP)
    uint32_t splits;        // S
    float scale;
    int out_f16;
};

__device__ __forceinline__ void put_out(const AttnArgs &a, size_t at, float v) {
    if (a.out_f16) ((uint16_t *)a.out)[at] = f2h_bits(v);
    else ((float *)a.out)[at] = v;
}

__device__ __forceinline__ float to_f(float v) { return v; }
__device__ __forceinline__ float to_f(_Float16 v) { return (float)v; }

template <typename KV, int D, int G>
__global__ __launch_bounds__(THREADS) void attn_partial_kernel(AttnArgs a) {
    constexpr int KP = D + KVPad<KV>::P;                 // padded K row (elements)
    constexpr int NPART = G >= 4 ? 1 : 4 / G;            // D-parts per (head, position) in QK
    constexpr int DP = D / NPART;
    constexpr int TPH = THREADS / G;                     // PV threads per head
    constexpr int DPT = TPH >= D ? 1 : D / TPH;          // dims per PV thread
    constexpr int PS = TPH >= D ? TPH / D : 1;           // position interleave in PV

    __shared__ __align__(16) KV kt[TP * KP];
    __shared__ __align__(16) KV vt[TP * D];
    __shared__ __align__(16) float qs[G * D];
    __shared__ float spart[G * NPART * TP];
    __shared__ float prob[G * TP];
    __shared__ float st_m[G], st_l[G], st_alpha[G];
    __shared__ float comb[PS > 1 ? THREADS * DPT : 1];

    const uint32_t split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    // lengths beyond the planned splits (or the capacity) are clamped, never read past
    const uint32_t len = min(min(a.seq_lens ? (uint32_t)a.seq_lens[b] : a.seq_len, a.max_seq), a.splits * a.chunk);
    const uint32_t start = split * a.chunk;
    if (start >= len && !(split == 0 && len == 0)) return;   // len 0: split 0 writes zeros
    const uint32_t end = min(len, start + a.chunk);
    const size_t row0 = (size_t)(a.row_base ? (uint32_t)a.row_base[b] : b * a.max_seq);
    const uint32_t kvrow = a.kv_heads * D;                // elements per cache row
    const KV *kc = (const KV *)a.kc + row0 * kvrow + (size_t)kvh * D;
    const KV *vc = (const KV *)a.vc + row0 * kvrow + (size_t)kvh * D;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

    // q for the G heads of this KV group
    for (int i = t; i < G * D; i += THREADS) qs[i] = a.q[((size_t)b * a.heads + kvh * G) * D + i];
    if (t < G) { st_m[t] = -INFINITY; st_l[t] = 0.0f; }

    // PV ownership: head pg, dims [pd, pd + DPT), positions p % PS == pps
    const int pg = t / TPH, pr = t % TPH;
    const int pd = (pr % (D / DPT)) * DPT, pps = pr / (D / DPT);
    float acc[DPT];
#pragma unroll
    for (int i = 0; i < DPT; ++i) acc[i] = 0.0f;

    constexpr int VEC = 16 / sizeof(KV);                  // elements per 128-bit load
    constexpr int CPR = D / VEC;                          // 128-bit chunks per row
    for (uint32_t p0 = start; p0 < end; p0 += TP) {
        const int np = (int)min((uint32_t)TP, end - p0);
        __syncthreads();   // previous tile fully consumed
        for (int c = t; c < TP * CPR; c += THREADS) {
            int p = c / CPR, cc = c % CPR;
            uint4 kv4 = {0u, 0u, 0u, 0u}, vv4 = {0u, 0u, 0u, 0u};
            if (p < np) {
                kv4 = *(const uint4 *)(kc + (size_t)(p0 + p) * kvrow + cc * VEC);
                vv4 = *(const uint4 *)(vc + (size_t)(p0 + p) * kvrow + cc * VEC);
            }
            *(uint4 *)(kt + p * KP + cc * VEC) = kv4;
            *(uint4 *)(vt + p * D + cc * VEC) = vv4;
        }
        __syncthreads();
        // QK partial dots: item -> (head g, part, position p)
        for (int it = t; it < G * NPART * TP; it += THREADS) {
            int g = it / (NPART * TP), rest = it % (NPART * TP);
            int part = rest / TP, p = rest % TP;
            const KV *kr = kt + p * KP + part * DP;
            const float *qr = qs + g * D + part * DP;
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int d = 0; d < DP; d += 2) {
                s0 = fmaf(qr[d], to_f(kr[d]), s0);
                s1 = fmaf(qr[d + 1], to_f(kr[d + 1]), s1);
            }
            spart[it] = s0 + s1;
        }
        __syncthreads();
        // softmax statistics: wave w < G owns head w (and w + 4 for G = 8)
        for (int g = wave; g < G; g += THREADS / 64) {
            float s = 0.0f;
#pragma unroll
            for (int part = 0; part < NPART; ++part) s += spart[(g * NPART + part) * TP + lane];
            s = lane < np ? s * a.scale : -INFINITY;
            float mt = wave_max(s);
            float m_old = st_m[g];
            float m_new = fmaxf(m_old, mt);
            float e = lane < np ? expf(s - m_new) : 0.0f;
            prob[g * TP + lane] = e;
            float lt = wave_sum(e);
            if (lane == 0) {
                float alpha = expf(m_old - m_new);
                st_alpha[g] = alpha;
                st_l[g] = st_l[g] * alpha + lt;
                st_m[g] = m_new;
            }
        }
        __syncthreads();
        // P.V
        {
            const float alpha = st_alpha[pg];
#pragma unroll
            for (int i = 0; i < DPT; ++i) acc[i] *= alpha;
            const float *pr_ = prob + pg * TP;
            for (int p = pps; p < np; p += PS) {
                float w = pr_[p];
                const KV *vr = vt + p * D + pd;
#pragma unroll
                for (int i = 0; i < DPT; ++i) acc[i] = fmaf(w, to_f(vr[i]), acc[i]);
            }
        }
    }
    // combine the PS position-interleaved partial accumulators
    if (PS > 1) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < DPT; ++i) comb[t * DPT + i] = acc[i];
        __syncthreads();
        if (pps == 0) {
            for (int s = 1; s < PS; ++s) {
                int src = pg * TPH + s * (D / DPT) + pr;
#pragma unroll
                for (int i = 0; i < DPT; ++i) acc[i] += comb[src * DPT + i];
            }
        }
    }
    __syncthreads();
    if (pps != 0) return;
    const uint32_t h = kvh * G + pg;
    const float m = st_m[pg], l = st_l[pg];
    if (a.splits == 1 || len <= a.chunk) {
        float inv = 1.0f / fmaxf(l, 1e-20f);
        const size_t o = ((size_t)b * a.heads + h) * D + pd;
#pragma unroll
        for (int i = 0; i < DPT; ++i) put_out(a, o + i, acc[i] * inv);
    } else {
        float *w = a.ws + (((size_t)b * a.heads + h) * a.splits + split) * (D + 2);
        if (pd == 0) { w[0] = m; w[1] = l; }
#pragma unroll
        for (int i = 0; i < DPT; ++i) w[2 + pd + i] = acc[i];
    }
}

// Merge: o = sum_s o_s e^{m_s - M} / sum_s l_s e^{m_s - M}.
template <int D>
__global__ __launch_bounds__(D) void attn_merge_kernel(AttnArgs a) {
    const uint32_t h = blockIdx.x, b = blockIdx.y;
    // lengths beyond the planned splits (or the capacity) are clamped, never read past
    const uint32_t len = min(min(a.seq_lens ? (uint32_t)a.seq_lens[b] : a.seq_len, a.max_seq), a.splits * a.chunk);
    if (len <= a.chunk) return;   // written directly by the partial kernel
    const uint32_t ns = (len + a.chunk - 1) / a.chunk;
    const float *w = a.ws + ((size_t)b * a.heads + h) * a.splits * (D + 2);
    float M = -INFINITY;
    for (uint32_t s = 0; s < ns; ++s) M = fmaxf(M, w[s * (D + 2)]);
    float L = 0.0f, o = 0.0f;
    for (uint32_t s = 0; s < ns; ++s) {
        const float *ws = w + s * (D + 2);
        float f = expf(ws[0] - M);
        L = fmaf(ws[1], f, L);
        o = fmaf(ws[2 + threadIdx.x], f, o);
    }
    put_out(a, ((size_t)b * a.heads + h) * D + threadIdx.x, o / fmaxf(L, 1e-20f));
}

template <typename KV, int D>
int launch_d(janus_ctx *ctx, const AttnArgs &a, uint32_t G) {
    dim3 grid(a.splits, a.kv_heads, a.batch), block(THREADS);
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_partial_kernel<KV, D, 1>), grid, block, 0, ctx->stream, a); break;
    case 2: hipLaunchKernelGGL((attn_partial_kernel<KV, D, 2>), grid, block, 0, ctx->stream, a); break;
    case 4: hipLaunchKernelGGL((attn_partial_kernel<KV, D, 4>), grid, block, 0, ctx->stream, a); break;
    case 8: hipLaunchKernelGGL((attn_partial_kernel<KV, D, 8>), grid, block, 0, ctx->stream, a); break;
    default: return fail(ctx, JANUS_E_INVALID_DIM, "attention: heads / kv_heads must be 1, 2, 4 or 8");
    }
    JANUS_LAUNCH_CHECK(ctx);
    if (a.splits > 1) {
        hipLaunchKernelGGL((attn_merge_kernel<D>), dim3(a.heads, a.batch), dim3(D), 0, ctx->stream, a);
        JANUS_LAUNCH_CHECK(ctx);
    }
    return JANUS_OK;
}

}  // namespace

// Chooses the split size so the launch has roughly 2 workgroups per CU.
void attention_plan(const janus_ctx *ctx, uint32_t batch, uint32_t kv_heads, uint32_t max_len, uint32_t *chunk_out,
                    uint32_t *splits_out) {
    if (max_len == 0) max_len = 1;
    uint64_t groups = (uint64_t)batch * kv_heads;
    uint64_t want = (uint64_t)ctx->num_cus * 2;
    uint32_t splits = (uint32_t)((want + groups - 1) / groups);
    uint32_t max_splits = (max_len + TP - 1) / TP;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    uint32_t chunk = (max_len + splits - 1) / splits;
    chunk = (chunk + TP - 1) / TP * TP;
    *chunk_out = chunk;
    *splits_out = (max_len + chunk - 1) / chunk;
}

int attention_reserve(janus_ctx *ctx, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                      uint32_t max_len) {
    uint32_t chunk, splits;
    attention_plan(ctx, batch, kv_heads, max_len, &chunk, &splits);
    if (splits <= 1) return JANUS_OK;
    return ensure_attn_ws(ctx, (size_t)batch * heads * splits * (hd + 2) * sizeof(float));
}

int attention_launch(janus_ctx *ctx, const float *q, const void *kc, const void *vc, int kv_dt, void *out,
                     uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t seq_len,
                     uint32_t max_seq, const int32_t *row_base, const int32_t *seq_lens, uint32_t max_len,
                     float scale, int out_f16) {
    AttnArgs a;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.out = out;
    a.row_base = row_base;
    a.seq_lens = seq_lens;
    a.batch = batch;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.seq_len = seq_len;
    a.max_seq = max_seq;
    a.scale = scale;
    a.out_f16 = out_f16;
    uint32_t chunk, splits;
    attention_plan(ctx, batch, kv_heads, max_len, &chunk, &splits);
    a.chunk = chunk;
    a.splits = splits;
    a.ws = nullptr;
    if (splits > 1) {
        size_t bytes = (size_t)batch * heads * splits * (hd + 2) * sizeof(float);
        if (int e = ensure_attn_ws(ctx, bytes)) return e;
        a.ws = (float *)ctx->attn_ws;
    }
    const uint32_t G = heads / kv_heads;
    if (kv_dt == JANUS_DT_F16) {
        if (hd == 64) return launch_d<_Float16, 64>(ctx, a, G);
        if (hd == 128) return launch_d<_Float16, 128>(ctx, a, G);
    } else {
        if (hd == 64) return launch_d<float, 64>(ctx, a, G);
        if (hd == 128) return launch_d<float, 128>(ctx, a, G);
    }
    return fail(ctx, JANUS_E_INVALID_DIM, "attention: head_dim must be 64 or 128");
}

}  // namespace janus
