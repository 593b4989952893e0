// glue.hip -- normalisation, activation, RoPE, KV append, embedding and
// greedy-sampling kernels around the matrix products.
//
// Reference kernels (crates/janus-engine/src/compute/shaders/):
// activations.wgsl (rmsnorm :67-134, silu :20-35), elementwise_mul.wgsl,
// add_tensors.wgsl, rope.wgsl, update_cache.wgsl, embed.wgsl, argmax.wgsl;
// sampler penalty: model/sampler.rs:599-613.
#include "internal.h"

namespace janus {

// ---- RMSNorm: one workgroup per row ---------------------------------------
// y = (x / sqrt(sum(x^2)/H + eps)) * gamma  -- division by the root, as the
// reference writes it (activations.wgsl:114,128).
// Rows of up to 256 * 4 * NV elements are held in registers: every thread
// issues all of its 16-byte loads at once, so the kernel costs one memory
// round trip instead of one per strided iteration.
template <bool OUT_F16, int NV>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ in, void *__restrict__ out,
                                                      const float *__restrict__ gamma, uint32_t hidden,
                                                      float eps) {
    __shared__ float red[4];
    const float *x = in + (size_t)blockIdx.x * hidden;
    const bool vec = (hidden & 3) == 0;
    float v[NV][4];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = 4 * (threadIdx.x + 256u * j);
        if (vec && i < hidden) {
            jf4 t = *(const jf4 *)(x + i);
            v[j][0] = t.x; v[j][1] = t.y; v[j][2] = t.z; v[j][3] = t.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) v[j][c] = (i + c < hidden) ? x[i + c] : 0.0f;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) s = fmaf(v[j][c], v[j][c], s);
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = sqrtf(tot / (float)hidden + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = 4 * (threadIdx.x + 256u * j);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (i + c < hidden) {
                float r = (v[j][c] / rms) * gamma[i + c];
                if (OUT_F16) ((uint16_t *)out)[(size_t)blockIdx.x * hidden + i + c] = f2h_bits(r);
                else ((float *)out)[(size_t)blockIdx.x * hidden + i + c] = r;
            }
        }
    }
}

// Rows too long for registers: strided loops.
template <bool OUT_F16>
__global__ __launch_bounds__(256) void rmsnorm_long_kernel(const float *__restrict__ in, void *__restrict__ out,
                                                           const float *__restrict__ gamma, uint32_t hidden,
                                                           float eps) {
    __shared__ float red[4];
    const float *x = in + (size_t)blockIdx.x * hidden;
    float s = 0.0f;
    for (uint32_t i = threadIdx.x; i < hidden; i += 256u) s = fmaf(x[i], x[i], s);
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float rms = sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)hidden + eps);
    for (uint32_t i = threadIdx.x; i < hidden; i += 256u) {
        float v = (x[i] / rms) * gamma[i];
        if (OUT_F16) ((uint16_t *)out)[(size_t)blockIdx.x * hidden + i] = f2h_bits(v);
        else ((float *)out)[(size_t)blockIdx.x * hidden + i] = v;
    }
}

template <bool H>
static void rmsnorm_dispatch(janus_ctx *ctx, const float *in, void *out, const float *gamma, uint32_t batch,
                             uint32_t hidden, float eps) {
    if (hidden <= 1024) hipLaunchKernelGGL((rmsnorm_kernel<H, 1>), dim3(batch), dim3(256), 0, ctx->stream, in, out, gamma, hidden, eps);
    else if (hidden <= 4096) hipLaunchKernelGGL((rmsnorm_kernel<H, 4>), dim3(batch), dim3(256), 0, ctx->stream, in, out, gamma, hidden, eps);
    else if (hidden <= 8192) hipLaunchKernelGGL((rmsnorm_kernel<H, 8>), dim3(batch), dim3(256), 0, ctx->stream, in, out, gamma, hidden, eps);
    else hipLaunchKernelGGL((rmsnorm_long_kernel<H>), dim3(batch), dim3(256), 0, ctx->stream, in, out, gamma, hidden, eps);
}

int rmsnorm_launch(janus_ctx *ctx, const float *in, void *out, int out_dt, const float *gamma,
                   uint32_t batch, uint32_t hidden, float eps) {
    if (out_dt == JANUS_DT_F16) rmsnorm_dispatch<true>(ctx, in, out, gamma, batch, hidden, eps);
    else rmsnorm_dispatch<false>(ctx, in, out, gamma, batch, hidden, eps);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// ---- elementwise ------------------------------------------------------------
__device__ __forceinline__ float silu_f(float x) { return x * (1.0f / (1.0f + expf(-x))); }

template <int OP, bool OUT_F16>
__global__ __launch_bounds__(256) void elementwise_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                                          void *__restrict__ out, uint32_t n) {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    float v;
    if (OP == EW_SILU) v = silu_f(a[i]);
    else if (OP == EW_MUL) v = a[i] * b[i];
    else if (OP == EW_ADD) v = a[i] + b[i];
    else v = silu_f(a[i]) * b[i];
    if (OUT_F16) ((uint16_t *)out)[i] = f2h_bits(v);
    else ((float *)out)[i] = v;
}

int elementwise_launch(janus_ctx *ctx, int op, const float *a, const float *b, void *out, int out_dt,
                       uint32_t n) {
    dim3 grid((n + 255) / 256), block(256);
    bool h = out_dt == JANUS_DT_F16;
    switch (op) {
    case EW_SILU: hipLaunchKernelGGL((elementwise_kernel<EW_SILU, false>), grid, block, 0, ctx->stream, a, b, out, n); break;
    case EW_MUL: hipLaunchKernelGGL((elementwise_kernel<EW_MUL, false>), grid, block, 0, ctx->stream, a, b, out, n); break;
    case EW_ADD: hipLaunchKernelGGL((elementwise_kernel<EW_ADD, false>), grid, block, 0, ctx->stream, a, b, out, n); break;
    default:
        if (h) hipLaunchKernelGGL((elementwise_kernel<EW_SWIGLU, true>), grid, block, 0, ctx->stream, a, b, out, n);
        else hipLaunchKernelGGL((elementwise_kernel<EW_SWIGLU, false>), grid, block, 0, ctx->stream, a, b, out, n);
    }
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// ---- RoPE (half-split, host cos/sin table) ---------------------------------
// One thread per (row, head, pair): y0 = x0*c - x1*s, y1 = x0*s + x1*c
// (rope.wgsl:71-72). In-place is safe: each thread owns its pair.
__global__ __launch_bounds__(256) void rope_kernel(const float *in, float *out, const float *__restrict__ table,
                                                   uint32_t batch, uint32_t heads, uint32_t hd,
                                                   uint32_t position, const int32_t *__restrict__ positions) {
    const uint32_t half = hd / 2;
    uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= batch * heads * half) return;
    uint32_t b = idx / (heads * half), rem = idx % (heads * half);
    uint32_t h = rem / half, i = rem % half;
    uint32_t pos = positions ? (uint32_t)positions[b] : position;
    size_t base = ((size_t)b * heads + h) * hd;
    float x0 = in[base + i], x1 = in[base + i + half];
    float c = table[((size_t)pos * half + i) * 2], s = table[((size_t)pos * half + i) * 2 + 1];
    out[base + i] = x0 * c - x1 * s;
    out[base + i + half] = x0 * s + x1 * c;
}

int rope_launch(janus_ctx *ctx, const float *in, float *out, const float *table, uint32_t batch, uint32_t heads,
                uint32_t hd, uint32_t position, const int32_t *positions) {
    uint32_t n = batch * heads * (hd / 2);
    hipLaunchKernelGGL(rope_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, in, out, table, batch, heads,
                       hd, position, positions);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// ---- KV append ----------------------------------------------------------------
template <typename KV>
__global__ __launch_bounds__(256) void kv_update_kernel(const float *__restrict__ k_new, const float *__restrict__ v_new,
                                                        KV *__restrict__ kc, KV *__restrict__ vc, uint32_t batch,
                                                        uint32_t row_elems, uint32_t position, uint32_t max_seq,
                                                        const int32_t *__restrict__ row_base,
                                                        const int32_t *__restrict__ positions) {
    uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= batch * row_elems) return;
    uint32_t b = idx / row_elems, e = idx % row_elems;
    const uint32_t pos = positions ? (uint32_t)positions[b] : position;
    if (pos >= max_seq) return;   // device-side positions past capacity are dropped
    size_t row = (size_t)(row_base ? (uint32_t)row_base[b] : b * max_seq) + pos;
    kc[row * row_elems + e] = (KV)k_new[idx];
    vc[row * row_elems + e] = (KV)v_new[idx];
}

int kv_update_launch(janus_ctx *ctx, const float *k_new, const float *v_new, void *kc, void *vc, int kv_dt,
                     uint32_t batch, uint32_t row_elems, uint32_t position, uint32_t max_seq,
                     const int32_t *row_base, const int32_t *positions) {
    uint32_t n = batch * row_elems;
    dim3 grid((n + 255) / 256), block(256);
    if (kv_dt == JANUS_DT_F16)
        hipLaunchKernelGGL(kv_update_kernel<_Float16>, grid, block, 0, ctx->stream, k_new, v_new, (_Float16 *)kc,
                           (_Float16 *)vc, batch, row_elems, position, max_seq, row_base, positions);
    else
        hipLaunchKernelGGL(kv_update_kernel<float>, grid, block, 0, ctx->stream, k_new, v_new, (float *)kc,
                           (float *)vc, batch, row_elems, position, max_seq, row_base, positions);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// ---- embedding gather ---------------------------------------------------------
// Token ids either travel as kernel arguments (host ids, up to 64 per launch)
// or are read from device memory.
struct EmbedIds {
    int32_t id[64];
};

__global__ __launch_bounds__(256) void embed_kernel(const uint16_t *__restrict__ table, EmbedIds ids,
                                                    const int32_t *__restrict__ d_ids, float *__restrict__ out,
                                                    uint32_t hidden, uint32_t vocab) {
    const uint32_t b = blockIdx.y;
    const int32_t id = d_ids ? d_ids[b] : ids.id[b];
    float *o = out + (size_t)b * hidden;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < hidden; i += gridDim.x * 256u)
        o[i] = ((uint32_t)id < vocab) ? h2f(table[(size_t)id * hidden + i]) : 0.0f;
}

int embed_launch(janus_ctx *ctx, const janus_weight *table, const uint32_t *h_ids, const int32_t *d_ids,
                 uint32_t batch, float *out) {
    const uint32_t hidden = table->k, vocab = table->n;
    const uint32_t gx = (hidden + 255) / 256 < 16 ? (hidden + 255) / 256 : 16;
    for (uint32_t b0 = 0; b0 < batch; b0 += 64) {
        uint32_t nb = batch - b0 < 64 ? batch - b0 : 64;
        EmbedIds ids;
        std::memset(&ids, 0, sizeof(ids));
        if (h_ids)
            for (uint32_t i = 0; i < nb; ++i) ids.id[i] = (int32_t)h_ids[b0 + i];
        hipLaunchKernelGGL(embed_kernel, dim3(gx, nb), dim3(256), 0, ctx->stream, (const uint16_t *)table->qs, ids,
                           d_ids ? d_ids + b0 : nullptr, out + (size_t)b0 * hidden, hidden, vocab);
        JANUS_LAUNCH_CHECK(ctx);
    }
    return JANUS_OK;
}

// ---- greedy argmax --------------------------------------------------------------
// TIE_LAST: the last maximal index (Iterator::max_by, model/sampler.rs:784-795);
// NaN entries never win. TIE_WGSL: the 256-lane scan and strict '>' tree of
// argmax.wgsl:26-126 reproduced lane for lane.
__global__ __launch_bounds__(1024) void argmax_last_kernel(const float *__restrict__ logits, int32_t *__restrict__ out,
                                                           uint32_t vocab) {
    __shared__ float sv[16];
    __shared__ int32_t si[16];
    const float *l = logits + (size_t)blockIdx.x * vocab;
    float bv = -INFINITY;
    int32_t bi = -1;
    for (uint32_t i = threadIdx.x; i < vocab; i += 1024u) {
        float v = l[i];
        if (v > bv || (v == bv && (int32_t)i > bi)) { bv = v; bi = (int32_t)i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = shfl_xor(bv, o);
        int32_t oi = shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi > bi)) { bv = ov; bi = oi; }
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (sv[w] > bv || (sv[w] == bv && si[w] > bi)) { bv = sv[w]; bi = si[w]; }
        out[blockIdx.x] = bi < 0 ? 0 : bi;
    }
}

__global__ __launch_bounds__(256) void argmax_wgsl_kernel(const float *__restrict__ logits, int32_t *__restrict__ out,
                                                          uint32_t vocab) {
    __shared__ float sv[256];
    __shared__ int32_t si[256];
    const float *l = logits + (size_t)blockIdx.x * vocab;
    const uint32_t t = threadIdx.x;
    float mv = -1e38f;
    int32_t mi = 0;
    for (uint32_t i = t; i < vocab; i += 256)
        if (l[i] > mv) { mv = l[i]; mi = (int32_t)i; }
    sv[t] = mv;
    si[t] = mi;
    __syncthreads();
    for (uint32_t stride = 128; stride >= 2; stride >>= 1) {
        if (t < stride && sv[t + stride] > sv[t]) { sv[t] = sv[t + stride]; si[t] = si[t + stride]; }
        __syncthreads();
    }
    if (t == 0) out[blockIdx.x] = sv[1] > sv[0] ? si[1] : si[0];
}

int argmax_launch(janus_ctx *ctx, const float *logits, int32_t *out, uint32_t vocab, uint32_t batch, int tie) {
    if (tie == JANUS_TIE_WGSL)
        hipLaunchKernelGGL(argmax_wgsl_kernel, dim3(batch), dim3(256), 0, ctx->stream, logits, out, vocab);
    else
        hipLaunchKernelGGL(argmax_last_kernel, dim3(batch), dim3(1024), 0, ctx->stream, logits, out, vocab);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// Each 1024-thread workgroup scans 32768 logits of one row (8 float4 per
// thread, all loads in flight together), reduces its keys through LDS and
// posts one atomicMax: a row's slot takes one device-scope atomic per
// workgroup (4 for a 128k vocabulary) rather than one per wavefront. The key
// is sampler_key under the sampler state (SAMPLE_ARGMAX when null).
__global__ __launch_bounds__(1024) void argmax_keys_kernel(const float *__restrict__ logits,
                                                           unsigned long long *best, uint32_t vocab,
                                                           const uint32_t *__restrict__ counts,
                                                           const SamplerDev *__restrict__ sampler) {
    __shared__ uint64_t wbest[16];
    const uint32_t row = blockIdx.y;
    const float *l = logits + (size_t)row * vocab;
    const uint32_t *cnt = counts ? counts + (size_t)row * vocab : nullptr;
    int mode = SAMPLE_ARGMAX;
    float pen = 1.0f;
    if (sampler) {
        mode = sampler->mode;
        pen = sampler->penalty;
    }
    const uint32_t base = blockIdx.x * 32768u + threadIdx.x * 4u;
    uint64_t key = 0;
    float4 v[8];
    uint4 c[8];
    const bool vec = (vocab & 3u) == 0;
    const bool counted = mode == SAMPLE_PENALTY && cnt;
    // logits and (under the penalty) their counts requested together
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t i = base + 4096u * j;
        c[j] = make_uint4(0u, 0u, 0u, 0u);
        if (vec && i + 4 <= vocab) {
            v[j] = *(const float4 *)(l + i);
            if (counted) c[j] = *(const uint4 *)(cnt + i);
        } else {
            v[j].x = i < vocab ? l[i] : -INFINITY;
            v[j].y = i + 1 < vocab ? l[i + 1] : -INFINITY;
            v[j].z = i + 2 < vocab ? l[i + 2] : -INFINITY;
            v[j].w = i + 3 < vocab ? l[i + 3] : -INFINITY;
            if (counted) {
                c[j].x = i < vocab ? cnt[i] : 0u;
                c[j].y = i + 1 < vocab ? cnt[i + 1] : 0u;
                c[j].z = i + 2 < vocab ? cnt[i + 2] : 0u;
                c[j].w = i + 3 < vocab ? cnt[i + 3] : 0u;
            }
        }
    }
    auto take = [&](float x, uint32_t i, uint32_t n) {
        if (i < vocab) {
            const uint64_t k = sampler_key(x, i, n, mode, pen);
            key = k > key ? k : key;
        }
    };
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t i = base + 4096u * j;
        take(v[j].x, i, c[j].x);
        take(v[j].y, i + 1, c[j].y);
        take(v[j].z, i + 2, c[j].z);
        take(v[j].w, i + 3, c[j].w);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t other = ((uint64_t)(uint32_t)shfl_xor((int)(key >> 32), o) << 32) |
                               (uint32_t)shfl_xor((int)(key & 0xffffffffu), o);
        key = other > key ? other : key;
    }
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t k = 0;
        for (int w = 0; w < 16; ++w) k = wbest[w] > k ? wbest[w] : k;
        if (k) atomicMax(best + row, (unsigned long long)k);
    }
}

int argmax_keys_launch(janus_ctx *ctx, const float *logits, unsigned long long *best, uint32_t vocab,
                       uint32_t batch, const uint32_t *counts, const SamplerDev *sampler) {
    hipLaunchKernelGGL(argmax_keys_kernel, dim3((vocab + 32767) / 32768, batch), dim3(1024), 0, ctx->stream, logits,
                       best, vocab, counts, sampler);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// Repetition penalty over a token list (sampler.rs:599-613). Thread i owns
// list entry i when it is the first occurrence of its id: it counts the
// id's occurrences and applies that many divides (positive logit) or
// multiplies (otherwise) in sequence. The sign of a logit never changes
// under either operation, so the result equals the reference's pass over
// the list in order; distinct ids touch distinct logits.
__global__ __launch_bounds__(256) void penalty_kernel(float *logits, uint32_t vocab, const int32_t *__restrict__ ids,
                                                      uint32_t n, float penalty) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const int32_t t = ids[i];
    if ((uint32_t)t >= vocab) return;
    bool first = true;
    for (uint32_t j = 0; j < i && first; ++j) first = ids[j] != t;
    if (!first) return;
    uint32_t c = 1;
    for (uint32_t j = i + 1; j < n; ++j) c += ids[j] == t ? 1u : 0u;
    float v = logits[t];
    for (; c; --c) v = v > 0.0f ? v / penalty : v * penalty;
    logits[t] = v;
}

int penalty_launch(janus_ctx *ctx, float *logits, uint32_t vocab, const int32_t *ids, uint32_t n, float penalty) {
    if (n == 0) return JANUS_OK;
    hipLaunchKernelGGL(penalty_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, logits, vocab, ids, n,
                       penalty);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

}  // namespace janus
