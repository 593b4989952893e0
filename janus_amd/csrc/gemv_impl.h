// gemv_impl.h -- dequant-fused matrix-vector products for gfx950 (wave64).
// Kernel templates shared by one translation unit per weight format
// (gemv_q4_0.hip, gemv_q8_0.hip, gemv_q4_k.hip, gemv_q5_k.hip, gemv_f16.hip);
// gemv.hip holds the dispatch.
//
// Replaces gemm_q8_0_into / gemm_q4_k_into / matmul::gemm at M=1
// (crates/janus-engine/src/compute/ops/quantized.rs:188-378,
// ops/matmul.rs:228-298; shaders gemm_q8_0.wgsl, gemm_q4_k.wgsl, gemm.wgsl)
// and adds Q4_0, which the reference cannot run (compute/engine.rs:833-838).
//
// Design (one launch per product, HBM-bound):
//  * The activation vector x is staged once per workgroup into LDS, padded
//    per 32-element block (no bank conflicts on 16-byte LDS reads), together
//    with its 16-element partial sums (used by the Q4_K mins and the Q4_0 /
//    Q8_0 offset terms).
//  * LPR lanes cooperate on a row; each lane owns the row's units
//    u = lane, lane + LPR, ... and reads each unit's quants with one or two
//    128-bit loads, so a wavefront's load covers LPR*16 contiguous bytes.
//  * A wavefront processes R rows at once: x registers loaded from LDS are
//    reused for all R rows, and all R*units weight loads are issued before
//    any arithmetic so the wave keeps many KB in flight.
//  * Nibbles are unpacked in registers: f32 activations use
//    v_cvt_f32_ubyte{0..3} + FMA; f16 activations build binary16 pairs with
//    the 0x6400 exponent trick and reduce with v_dot2_f32_f16 (exact
//    products, fp32 accumulation).
//  * The R partial sums are reduced across the LPR lanes with a transposed
//    butterfly (log2 R exchange steps that halve the live values, then a
//    plain xor butterfly), so the reduction costs O(R + log LPR) shuffles.
#pragma once
#include <atomic>
#include <type_traits>

#include "internal.h"

namespace janus {

struct WPtr {
    const uint8_t *qs;
    const uint16_t *sc;
};

enum { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_QKV_ROPE = 2, EPI_SWIGLU = 3, EPI_ARGMAX = 4 };

struct GemvArgs {
    WPtr w;
    const void *x;       // activation [k]
    void *y;             // output [n] (EPI_SWIGLU: [n / 2])
    const float *resid;  // residual [n] (EPI_RESIDUAL)
    unsigned long long *best;   // EPI_ARGMAX: running max of sampler_key, reset by the consumer
    const uint32_t *counts;     // EPI_ARGMAX: occurrence counts of generated tokens (SAMPLE_PENALTY), or null
    const SamplerDev *sampler;  // EPI_ARGMAX: sampler state, or null for SAMPLE_ARGMAX
    uint32_t n, k;
    uint32_t units;      // units per row (0: F16 rows with k % 8 != 0)
    // threads per workgroup of the launch (the kernels read it from here:
    // blockDim.x costs a global load and a full wait at the kernel's start)
    uint32_t threads;
    int out_f16;
    int epi;
    // EPI_QKV_ROPE: row pairs are (i, i + hd/2) of a q head, then of a k head,
    // then consecutive v elements; q is rotated into y (f32), k is rotated and
    // v copied into the cache row d_rowbase[0] + d_pos[0] (d_rowbase may be null).
    void *kc, *vc;
    const float *rope;
    const int32_t *d_pos;
    const int32_t *d_rowbase;
    uint32_t q_pairs, k_pairs, half_hd, kv_row;
    int kv_f16;
    // fused RMSNorm of x (f32) with gamma, eps (the LDS kernel)
    const float *gamma;
    float eps;
};

// kinds of product: plain (x as given), or x RMS-normalised on staging
// (GEMV_NORM), with paired-row epilogues (GEMV_PAIR, two rows per step)
// (GEMV_X32: x staged as binary32, the reference's activation dtype)
enum { GEMV_PLAIN = 0, GEMV_NORM = 1, GEMV_PAIR = 2, GEMV_X32 = 4 };

// One launch of the product `a` for one weight format (the format's own
// translation unit); *done = false when no kernel covers the row length.
int gemv_run_q4_0(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done);
int gemv_run_q8_0(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done);
int gemv_run_q4_k(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done);
int gemv_run_q5_k(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done);
int gemv_run_f16(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done);

}  // namespace janus

namespace {

using janus::GemvArgs;
using janus::WPtr;
using janus::EPI_STORE;
using janus::EPI_RESIDUAL;
using janus::EPI_QKV_ROPE;
using janus::EPI_SWIGLU;
using janus::EPI_ARGMAX;

#ifndef JANUS_GEMV_NT
#define JANUS_GEMV_NT 1      // stream weights with non-temporal loads
#endif

constexpr int XB = 32;                 // activation elements per LDS block
constexpr int NORM_MAXG = 1;           // normalised LDS staging: k <= 16 * 512 * NORM_MAXG
template <typename XT> struct XLayout;
template <> struct XLayout<float> {    // 32 floats + 4 pad = 144 B
    static constexpr int STRIDE = 36;
};
template <> struct XLayout<_Float16> { // 32 halves + 8 pad = 80 B
    static constexpr int STRIDE = 40;
};

__device__ __forceinline__ float cvt_b0(uint32_t u) { return (float)(u & 0xffu); }
__device__ __forceinline__ float cvt_b1(uint32_t u) { return (float)((u >> 8) & 0xffu); }
__device__ __forceinline__ float cvt_b2(uint32_t u) { return (float)((u >> 16) & 0xffu); }
__device__ __forceinline__ float cvt_b3(uint32_t u) { return (float)(u >> 24); }

__device__ __forceinline__ jh2 as_h2(uint32_t u) { return __builtin_bit_cast(jh2, u); }
__device__ __forceinline__ float dot2(jh2 a, jh2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
// The first product of a chain: v_dot2_f32_f16 with an inline-constant zero
// accumulator (the builtin with 0.0f costs a register move for the zero).
__device__ __forceinline__ float dot2z(jh2 a, jh2 b) {
    float r;
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// The first product of a chain that starts from a value still needed
// afterwards: the three-operand form (the builtin becomes a register copy plus
// the destructive two-operand form).
__device__ __forceinline__ float dot2a(jh2 a, jh2 b, float c) {
    float r;
    asm("v_dot2_f32_f16 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Quantised values enter v_dot2_f32_f16 as exact binary16 integers with
// normal encodings. The masked nibble (or byte) under the magic exponent
// 0x6400 is 1024 + q (or 1024 + 16 q for a high nibble left in place); one
// packed add or packed FMA then removes the 1024 (and the format's offset)
// exactly. v_dot2_f32_f16 does not keep subnormal operands exact: with
// q * 2^-24 encodings it returned results below the correctly rounded sum by
// ~50 ulp on average, an error shared by every row of a product.
__device__ __forceinline__ jh2 nib_lo(uint32_t u, uint32_t m6400, _Float16 off) {
    const jh2 o = {off, off};
    return as_h2((u & 0x000f000fu) | m6400) - o;   // (1024 + q) - off
}
__device__ __forceinline__ jh2 nib_hi(uint32_t u, uint32_t m6400, _Float16 off) {
    const jh2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const _Float16 cb = (_Float16)(960.0f - (float)off);
    const jh2 c = {cb, cb};
    return __builtin_elementwise_fma(as_h2((u & 0x00f000f0u) | m6400), s16, c);   // (1024 + 16 q) / 16 + 960 - off
}

// Bytes 2S and 2S + 1 of v, each below 16, as the exact binary16 integers
// (natural pair order). A byte b < 16 read as OCP e4m3 is b * 2^-9 (the
// subnormals m * 2^-9 below 8, the lowest normal binade (8 + m) * 2^-9 from
// 8), and v_cvt_scalef32_pk_f16_fp8 scales it by 512 exactly: one instruction
// per pair against an AND-OR plus a packed add or FMA for the 0x6400 form.
template <bool S> __device__ __forceinline__ jh2 nib8(uint32_t v) {
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v, 512.0f, S);
}

// (x0,x1),(x2,x3) -> (x0,x2),(x1,x3): the pair order the nibble unpack produces.
__device__ __forceinline__ void perm4(uint32_t w01, uint32_t w23, jh2 &even, jh2 &odd) {
    even = as_h2(__builtin_amdgcn_perm(w23, w01, 0x05040100u));
    odd = as_h2(__builtin_amdgcn_perm(w23, w01, 0x07060302u));
}

// 16 halves at p (16-byte aligned) -> 8 permuted pairs, plus their fp32 sum
// (v_dot2 against (1, 1): exact products, fp32 sums).
__device__ __forceinline__ float load16h_perm(const _Float16 *p, jh2 *dst) {
    const uint4 *q = (const uint4 *)p;
    const jh2 one = {(_Float16)1.0f, (_Float16)1.0f};
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint4 t = q[i];
        perm4(t.x, t.y, dst[4 * i + 0], dst[4 * i + 1]);
        perm4(t.z, t.w, dst[4 * i + 2], dst[4 * i + 3]);
        s0 = dot2(as_h2(t.x), one, s0);
        s1 = dot2(as_h2(t.y), one, s1);
        s0 = dot2(as_h2(t.z), one, s0);
        s1 = dot2(as_h2(t.w), one, s1);
    }
    return s0 + s1;
}

// 16 halves at p (16-byte aligned) -> 8 pairs in order, plus their fp32 sum.
__device__ __forceinline__ float load16h(const _Float16 *p, jh2 *dst) {
    const uint4 *q = (const uint4 *)p;
    const jh2 one = {(_Float16)1.0f, (_Float16)1.0f};
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint4 t = q[i];
        dst[4 * i + 0] = as_h2(t.x);
        dst[4 * i + 1] = as_h2(t.y);
        dst[4 * i + 2] = as_h2(t.z);
        dst[4 * i + 3] = as_h2(t.w);
        s0 = dot2(as_h2(t.x), one, s0);
        s1 = dot2(as_h2(t.y), one, s1);
        s0 = dot2(as_h2(t.z), one, s0);
        s1 = dot2(as_h2(t.w), one, s1);
    }
    return s0 + s1;
}

// ---------------------------------------------------------------------------
// x staging
// ---------------------------------------------------------------------------
// Writes x[0..k) into LDS: element e goes to block e/32, slot e%32. For f16
// with PERM, each group of four (a,b,c,d) is stored as (a,c,b,d) so a u32 of
// packed nibbles maps onto (x[i], x[i+2]) pairs. sx16[g] = sum of the stored
// values x[16g..16g+16). With NORM the stored value is (x / rms) * gamma,
// the RMSNorm of shaders/activations.wgsl:114,128.
template <typename XIN, typename XT, bool PERM, bool NORM = false>
__device__ void stage_x(const XIN *__restrict__ x, uint32_t k, XT *xs, float *sx16, int nt,
                        const float *__restrict__ gamma = nullptr, float rms = 1.0f) {
    const int groups = (int)((k + 15) / 16);
    for (int g = threadIdx.x; g < groups; g += nt) {
        float v[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            uint32_t e = (uint32_t)g * 16 + t;
            float f = e < k ? (float)x[e] : 0.0f;
            if (NORM) f = e < k ? (f / rms) * gamma[e] : 0.0f;
            v[t] = (float)(XT)f;   // the value the products will read
        }
        float s = 0.0f;
#pragma unroll
        for (int t = 0; t < 16; ++t) s += v[t];
        sx16[g] = s;
        int blk = g >> 1, off = (g & 1) * 16;
        XT *dst = xs + blk * XLayout<XT>::STRIDE + off;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (PERM) {
                dst[4 * q + 0] = (XT)v[4 * q + 0];
                dst[4 * q + 1] = (XT)v[4 * q + 2];
                dst[4 * q + 2] = (XT)v[4 * q + 1];
                dst[4 * q + 3] = (XT)v[4 * q + 3];
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) dst[4 * q + t] = (XT)v[4 * q + t];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// formats. Each provides: UNIT (weights per lane-unit), a weight register
// record W with load(), an x register record per activation type with
// loadx(), and dot(W, X) returning the unit's contribution in fp32.
// ---------------------------------------------------------------------------

// ---- Q4_0: 16 B nibbles (GGML order) + binary16 scale per 32 weights -------
struct FQ4_0 {
    static constexpr int UNIT = 32;
    static constexpr bool XREREAD = false;   // long rows re-read x from LDS per row group
    static constexpr bool PERM = false;      // binary16 x staged in element order (nib8 pairs)
    struct W { uint4 q; uint16_t d; };
    __device__ static W load(WPtr w, size_t unit) {
        W r;
        r.q = ld_stream((const uint4 *)w.qs + unit);
        r.d = w.sc[unit];
        return r;
    }
    // unit u of the row starting at unit ru (ru uniform over the wavefront:
    // a scalar row base plus a 32-bit lane offset)
    __device__ static W load_row(WPtr w, size_t ru, uint32_t u) {
        W r;
        r.q = ld_stream(w.qs + ru * 16 + u * 16u);
        r.d = *(const uint16_t *)((const uint8_t *)w.sc + ru * 2 + u * 2u);
        return r;
    }
    struct XF { jf4 v[8]; float s; };          // x[0..32) and sum(x)
    __device__ static XF loadx(const float *xs, const float *sx16, int u) {
        XF r;
        const jf4 *p = (const jf4 *)(xs + u * XLayout<float>::STRIDE);
#pragma unroll
        for (int i = 0; i < 8; ++i) r.v[i] = p[i];
        r.s = sx16[2 * u] + sx16[2 * u + 1];
        return r;
    }
    // binary32 x: the nibbles become the exact binary16 integers q (nib8,
    // two per instruction) and each product is one mixed-precision FMA
    // (v_fma_mix_f32: binary16 weight, binary32 x and accumulator); the
    // offset enters as -8 * sum(x) at the head of the first chain. 15
    // instructions per 8 weights, against 17 with the 0x6400 form and 19
    // with per-byte conversions.
    __device__ static float dot(const W &w, const XF &x) {
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        float s0 = -8.0f * x.s, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = q[i] & 0x0f0f0f0fu, hi = (q[i] >> 4) & 0x0f0f0f0fu;
            const jf4 xl = x.v[i], xh = x.v[4 + i];   // elements 4i..4i+3 and 16+4i..
            const jh2 a = nib8<false>(lo), c = nib8<true>(lo);   // (4i, 4i+1), (4i+2, 4i+3)
            const jh2 b = nib8<false>(hi), e = nib8<true>(hi);   // 16 + the same
            s0 = fmaf((float)a.x, xl.x, s0);
            s1 = fmaf((float)a.y, xl.y, s1);
            s0 = fmaf((float)c.x, xl.z, s0);
            s1 = fmaf((float)c.y, xl.w, s1);
            s0 = fmaf((float)b.x, xh.x, s0);
            s1 = fmaf((float)b.y, xh.y, s1);
            s0 = fmaf((float)e.x, xh.z, s0);
            s1 = fmaf((float)e.y, xh.w, s1);
        }
        return h2f(w.d) * (s0 + s1);
    }
    // x[0..32) as pairs in element order and the sums of its two halves
    struct XH { jh2 v[16]; float s0, s1; };
    __device__ static XH loadx(const _Float16 *xs, const float *sx16, int u) {
        XH r;
        const uint4 *p = (const uint4 *)(xs + u * XLayout<_Float16>::STRIDE);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint4 t = p[i];
            r.v[4 * i + 0] = as_h2(t.x);
            r.v[4 * i + 1] = as_h2(t.y);
            r.v[4 * i + 2] = as_h2(t.z);
            r.v[4 * i + 3] = as_h2(t.w);
        }
        r.s0 = sx16[2 * u];
        r.s1 = sx16[2 * u + 1];
        return r;
    }
    // register-resident x, read straight from global memory
    __device__ static XF loadx_g(const float *x, int u) {
        XF r;
        const jf4 *p = (const jf4 *)(x + (size_t)u * 32);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            r.v[i] = p[i];
            s += (r.v[i].x + r.v[i].y) + (r.v[i].z + r.v[i].w);
        }
        r.s = s;
        return r;
    }
    __device__ static XH loadx_g(const _Float16 *x, int u) {
        XH r;
        r.s0 = load16h(x + (size_t)u * 32, r.v);
        r.s1 = load16h(x + (size_t)u * 32 + 16, r.v + 8);
        return r;
    }
    // Each nibble pair becomes the exact binary16 integers q (nib8), so every
    // v_dot2_f32_f16 product is exact; the offset enters as -8 * sum(x) at
    // the head of each chain (low nibbles: x[0..16), high: x[16..32)), and
    // the two chains are added once per block and scaled by d.
    __device__ static float dot(const W &w, const XH &x) {
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        float s = 0.0f, t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = q[i] & 0x0f0f0f0fu, hi = (q[i] >> 4) & 0x0f0f0f0fu;
            // (4i, 4i+1) and (16+4i, 16+4i+1); the chain heads keep -8 * sum
            // intact (x and its sums are often loop-invariant)
            s = i == 0 ? dot2a(nib8<false>(lo), x.v[0], -8.0f * x.s0) : dot2(nib8<false>(lo), x.v[2 * i], s);
            t = i == 0 ? dot2a(nib8<false>(hi), x.v[8], -8.0f * x.s1) : dot2(nib8<false>(hi), x.v[8 + 2 * i], t);
            s = dot2(nib8<true>(lo), x.v[2 * i + 1], s);     // (4i+2, 4i+3)
            t = dot2(nib8<true>(hi), x.v[8 + 2 * i + 1], t);
        }
        return h2f(w.d) * (s + t);
    }
};

// ---- Q8_0: 32 B int8 + binary16 scale (exp 31 -> 1e38) per 32 weights ------
struct FQ8_0 {
    static constexpr int UNIT = 32;
    static constexpr bool XREREAD = false;   // long rows re-read x from LDS per row group
    static constexpr bool PERM = true;
    struct W { uint4 q0, q1; uint16_t d; };
    __device__ static W load(WPtr w, size_t unit) {
        W r;
        const uint4 *p = (const uint4 *)w.qs + 2 * unit;
        r.q0 = ld_stream(p);
        r.q1 = ld_stream(p + 1);
        r.d = w.sc[unit];
        return r;
    }
    __device__ static W load_row(WPtr w, size_t ru, uint32_t u) {
        W r;
        const uint8_t *p = w.qs + ru * 32 + u * 32u;
        r.q0 = ld_stream(p);
        r.q1 = ld_stream(p + 16);
        r.d = *(const uint16_t *)((const uint8_t *)w.sc + ru * 2 + u * 2u);
        return r;
    }
    using XF = FQ4_0::XF;
    using XH = FQ4_0::XH;
    __device__ static XF loadx(const float *xs, const float *sx16, int u) { return FQ4_0::loadx(xs, sx16, u); }
    __device__ static XH loadx(const _Float16 *xs, const float *sx16, int u) { return FQ4_0::loadx(xs, sx16, u); }
    __device__ static XF loadx_g(const float *x, int u) { return FQ4_0::loadx_g(x, u); }
    __device__ static XH loadx_g(const _Float16 *x, int u) { return FQ4_0::loadx_g(x, u); }
    __device__ static float dot(const W &w, const XF &x) {
        const uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t u = q[i] ^ 0x80808080u;   // int8 q -> unsigned q + 128
            jf4 xv = x.v[i];
            s0 = fmaf(cvt_b0(u), xv.x, s0);
            s1 = fmaf(cvt_b1(u), xv.y, s1);
            s0 = fmaf(cvt_b2(u), xv.z, s0);
            s1 = fmaf(cvt_b3(u), xv.w, s1);
        }
        return h2f_q8(w.d) * fmaf(-128.0f, x.s, s0 + s1);
    }
    // The biased bytes q + 128 (0..255) go under the exponent byte 0x64 with
    // one v_perm_b32 per pair (1024 + q + 128, exact normal binary16), and a
    // packed add of -1152 leaves the exact integers q: every v_dot2_f32_f16
    // product is exact (see nib_lo).
    __device__ static float dot(const W &w, const XH &x) {
        const uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        const jh2 o = {(_Float16)1152.0f, (_Float16)1152.0f};
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = q[i] ^ 0x80808080u;
            // bytes 4-7 of the pool are 0x64: (byte 0 | 0x64 << 8, byte 2 | 0x64 << 8) and bytes 1, 3
            const jh2 a = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04020400u)) - o;   // (4i, 4i+2)
            const jh2 c = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030401u)) - o;   // (4i+1, 4i+3)
            s0 = i == 0 ? dot2z(a, x.v[0]) : dot2(a, x.v[2 * i], s0);
            s1 = i == 0 ? dot2z(c, x.v[1]) : dot2(c, x.v[2 * i + 1], s1);
        }
        return h2f_q8(w.d) * (s0 + s1);
    }
};

// ---- Q4_K: GGML 144-byte super-blocks; a unit is one 16-byte quant chunk ----
// Chunk c (0..7) of a super-block covers qs bytes 16c..16c+15, i.e. j = c/2,
// h = c%2: low nibbles -> elements 64j+16h+t (sub-block 2j), high nibbles ->
// 64j+32+16h+t (sub-block 2j+1), t = 0..15. Weight = (d*sc)*q - dmin*m
// (shaders/gemm_q4_k.wgsl:82-113).
struct FQ4_K {
    static constexpr int UNIT = 32;
    static constexpr bool XREREAD = true;   // long rows re-read x from LDS per row group
    static constexpr bool PERM = false;     // binary16 x staged in element order (nib8 pairs)
    // The 16-byte super-block header (d, dmin, the scale fields of kq_group
    // in words 1-3) is shared by the 8 units of a super-block, which sit on 8
    // consecutive lanes in every kernel, unit c on lane p = lane & 7 (units
    // are lane-contiguous from a multiple of 8 and a row holds a multiple of
    // 8). Lane p keeps header word hword(p) = {0, 1, 1, 2, 0, 2, 3, 3}[p]:
    // quad DPP reads of lanes [0,0,0,0], [1,1,2,2] and [3,3,3,3] then hand
    // every lane d / dmin and the words (lo, hi) = (1, 2) for chunk pairs
    // j = 0, 1 (first quad), (2, 3) for j = 2 and (3, 3) for j = 3 (second
    // quad), whose funnel shift by (32 - 8j) & 31 is the lane's field. One
    // VGPR of header per unit, three DPP moves and one shift at use.
    struct W { uint4 q; uint32_t hw; };
    __device__ static uint32_t hword() { return (0x33202110u >> (4u * (__lane_id() & 7u))) & 15u; }
    __device__ static W load(WPtr w, size_t unit) {
        size_t sb = unit >> 3;
        int c = (int)(unit & 7);
        const uint4 *blk = (const uint4 *)(w.qs + sb * 144);
        W r;
        r.hw = ((const uint32_t *)blk)[hword()];
        r.q = ld_stream(blk + 1 + c);
        return r;
    }
    // ru: first unit of the row (a multiple of 8, uniform), u: unit in the row
    __device__ static W load_row(WPtr w, size_t ru, uint32_t u) {
        const uint8_t *row = w.qs + (ru >> 3) * 144;   // uniform; one 32-bit lane offset per load
        const uint32_t ob = (u >> 3) * 144u;
        W r;
        r.hw = *(const uint32_t *)(row + (ob + 4u * hword()));
        r.q = ld_stream(row + (ob + 16u + 16u * (u & 7u)));
        return r;
    }
    template <int PERM> __device__ static uint32_t quad_read(uint32_t v) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, PERM, 0xf, 0xf, false);
    }
    // x for one chunk: 16 low-nibble elements and 16 high-nibble elements.
    struct XF { jf4 lo[4], hi[4]; float slo, shi; };
    __device__ static XF loadx(const float *xs, const float *sx16, int u) {
        int sb = u >> 3, c = u & 7, j = c >> 1, h = c & 1;
        int blo = sb * 8 + 2 * j, bhi = blo + 1;   // 32-element LDS blocks
        XF r;
        const jf4 *pl = (const jf4 *)(xs + blo * XLayout<float>::STRIDE + 16 * h);
        const jf4 *ph = (const jf4 *)(xs + bhi * XLayout<float>::STRIDE + 16 * h);
#pragma unroll
        for (int i = 0; i < 4; ++i) { r.lo[i] = pl[i]; r.hi[i] = ph[i]; }
        r.slo = sx16[2 * blo + h];
        r.shi = sx16[2 * bhi + h];
        return r;
    }
    struct XH { jh2 lo[8], hi[8]; float slo, shi; };
    __device__ static XH loadx(const _Float16 *xs, const float *sx16, int u) {
        int sb = u >> 3, c = u & 7, j = c >> 1, h = c & 1;
        int blo = sb * 8 + 2 * j, bhi = blo + 1;
        XH r;
        const uint4 *pl = (const uint4 *)(xs + blo * XLayout<_Float16>::STRIDE + 16 * h);
        const uint4 *ph = (const uint4 *)(xs + bhi * XLayout<_Float16>::STRIDE + 16 * h);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint4 a = pl[i], b = ph[i];
            r.lo[4 * i + 0] = as_h2(a.x); r.lo[4 * i + 1] = as_h2(a.y);
            r.lo[4 * i + 2] = as_h2(a.z); r.lo[4 * i + 3] = as_h2(a.w);
            r.hi[4 * i + 0] = as_h2(b.x); r.hi[4 * i + 1] = as_h2(b.y);
            r.hi[4 * i + 2] = as_h2(b.z); r.hi[4 * i + 3] = as_h2(b.w);
        }
        r.slo = sx16[2 * blo + h];
        r.shi = sx16[2 * bhi + h];
        return r;
    }
    __device__ static XF loadx_g(const float *x, int u) {
        int sb = u >> 3, c = u & 7, j = c >> 1, h = c & 1;
        const float *base = x + (size_t)sb * 256 + 64 * j + 16 * h;
        XF r;
        float sl = 0.0f, sh = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.lo[i] = ((const jf4 *)base)[i];
            r.hi[i] = ((const jf4 *)(base + 32))[i];
            sl += (r.lo[i].x + r.lo[i].y) + (r.lo[i].z + r.lo[i].w);
            sh += (r.hi[i].x + r.hi[i].y) + (r.hi[i].z + r.hi[i].w);
        }
        r.slo = sl;
        r.shi = sh;
        return r;
    }
    __device__ static XH loadx_g(const _Float16 *x, int u) {
        int sb = u >> 3, c = u & 7, j = c >> 1, h = c & 1;
        const _Float16 *base = x + (size_t)sb * 256 + 64 * j + 16 * h;
        XH r;
        r.slo = load16h(base, r.lo);
        r.shi = load16h(base + 32, r.hi);
        return r;
    }
    template <class WW, class X>
    __device__ static float finish(const WW &w, const X &x, float qlo, float qhi) {
        const uint32_t dd = quad_read<0x00>(w.hw);   // quad_perm [0,0,0,0]
        const uint32_t lo = quad_read<0xa5>(w.hw);   // [1,1,2,2]
        const uint32_t hi = quad_read<0xff>(w.hw);   // [3,3,3,3]
        const uint32_t g = __builtin_amdgcn_alignbit(hi, lo, (0u - 4u * (__lane_id() & 6u)) & 31u);
        const float d = h2f((uint16_t)(dd & 0xffffu)), dmin = h2f((uint16_t)(dd >> 16));
        const float sl = (float)(g & 63u), sh = (float)((g >> 6) & 63u);
        const float ml = (float)((g >> 12) & 63u), mh = (float)((g >> 18) & 63u);
        // d (sc_lo q_lo + sc_hi q_hi) - dmin (m_lo sum_lo + m_hi sum_hi)
        const float a = fmaf(sh, qhi, sl * qlo), b = fmaf(mh, x.shi, ml * x.slo);
        return fmaf(d, a, -(dmin * b));
    }
    __device__ static float dot(const W &w, const XF &x) {
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        float l0 = 0.0f, l1 = 0.0f, h0 = 0.0f, h1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo = q[i] & 0x0f0f0f0fu, hi = (q[i] >> 4) & 0x0f0f0f0fu;
            l0 = fmaf(cvt_b0(lo), x.lo[i].x, l0);
            l1 = fmaf(cvt_b1(lo), x.lo[i].y, l1);
            l0 = fmaf(cvt_b2(lo), x.lo[i].z, l0);
            l1 = fmaf(cvt_b3(lo), x.lo[i].w, l1);
            h0 = fmaf(cvt_b0(hi), x.hi[i].x, h0);
            h1 = fmaf(cvt_b1(hi), x.hi[i].y, h1);
            h0 = fmaf(cvt_b2(hi), x.hi[i].z, h0);
            h1 = fmaf(cvt_b3(hi), x.hi[i].w, h1);
        }
        return finish(w, x, l0 + l1, h0 + h1);
    }
    // Nibbles as the exact binary16 integers q (nib8, pairs in element order).
    __device__ static float dot(const W &w, const XH &x) {
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        float l = 0.0f, h = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = q[i] & 0x0f0f0f0fu, hi = (q[i] >> 4) & 0x0f0f0f0fu;
            l = i == 0 ? dot2z(nib8<false>(lo), x.lo[0]) : dot2(nib8<false>(lo), x.lo[2 * i], l);
            h = i == 0 ? dot2z(nib8<false>(hi), x.hi[0]) : dot2(nib8<false>(hi), x.hi[2 * i], h);
            l = dot2(nib8<true>(lo), x.lo[2 * i + 1], l);
            h = dot2(nib8<true>(hi), x.hi[2 * i + 1], h);
        }
        return finish(w, x, l, h);
    }
};

// ---- Q5_K: GGML 176-byte super-blocks {d, dmin, scales[12], qh, qs[128]} ----
// Same header, sub-block scales and element order as Q4_K (a unit is one
// 16-byte chunk of qs, x layout shared), plus a fifth bit per element
// (ggml-quants.c dequantize_row_q5_K). The upload rewrites qh as one word per
// chunk (bytes 16 + 4c), bit 8 (t % 4) + t / 4 (+ 4 for the high nibble) for
// quant byte t, so (w >> i) & 0x01010101 sits under the bytes of quant word
// i. Weight = (d*sc)*q - dmin*m with q in 0..31.
struct FQ5_K : FQ4_K {
    // 5-bit values do not fit e4m3's linear range: the 0x6400 form, whose
    // pairs are (x[i], x[i+2]), so binary16 x is staged permuted.
    static constexpr bool PERM = true;
    using FQ4_K::loadx_g;
    __device__ static XH loadx_g(const _Float16 *x, int u) {
        int sb = u >> 3, c = u & 7, j = c >> 1, h = c & 1;
        const _Float16 *base = x + (size_t)sb * 256 + 64 * j + 16 * h;
        XH r;
        r.slo = load16h_perm(base, r.lo);
        r.shi = load16h_perm(base + 32, r.hi);
        return r;
    }
    struct W { uint4 q; uint32_t qh; uint32_t hw; };
    __device__ static W load_row(WPtr w, size_t ru, uint32_t u) {
        const uint8_t *row = w.qs + (ru >> 3) * 176;   // uniform; one 32-bit lane offset per load
        const uint32_t ob = (u >> 3) * 176u, c = u & 7u;
        W r;
        r.hw = *(const uint32_t *)(row + (ob + 4u * hword()));
#if !defined(JANUS_GEMV_NT) || JANUS_GEMV_NT
        r.qh = __builtin_nontemporal_load((const uint32_t *)(row + (ob + 16u + 4u * c)));
#else
        r.qh = *(const uint32_t *)(row + (ob + 16u + 4u * c));
#endif
        r.q = ld_stream(row + (ob + 48u + 16u * c));
        return r;
    }
    __device__ static W load(WPtr w, size_t unit) {
        size_t sb = unit >> 3;
        int c = (int)(unit & 7);
        const uint4 *blk = (const uint4 *)(w.qs + sb * 176);
        W r;
        r.hw = ((const uint32_t *)blk)[hword()];
#if !defined(JANUS_GEMV_NT) || JANUS_GEMV_NT
        r.qh = __builtin_nontemporal_load((const uint32_t *)blk + 4 + c);
#else
        r.qh = ((const uint32_t *)blk)[4 + c];
#endif
        r.q = ld_stream(blk + 3 + c);
        return r;
    }
    // 5-bit values of the four bytes of quant word i: low (lo) and high (hi) elements
    __device__ static void q5(const W &w, int i, uint32_t &lo, uint32_t &hi) {
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        lo = (q[i] & 0x0f0f0f0fu) | (((w.qh >> i) & 0x01010101u) << 4);
        hi = ((q[i] >> 4) & 0x0f0f0f0fu) | (((w.qh >> (4 + i)) & 0x01010101u) << 4);
    }
    __device__ static float dot(const W &w, const XF &x) {
        float l0 = 0.0f, l1 = 0.0f, h0 = 0.0f, h1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo, hi;
            q5(w, i, lo, hi);
            l0 = fmaf(cvt_b0(lo), x.lo[i].x, l0);
            l1 = fmaf(cvt_b1(lo), x.lo[i].y, l1);
            l0 = fmaf(cvt_b2(lo), x.lo[i].z, l0);
            l1 = fmaf(cvt_b3(lo), x.lo[i].w, l1);
            h0 = fmaf(cvt_b0(hi), x.hi[i].x, h0);
            h1 = fmaf(cvt_b1(hi), x.hi[i].y, h1);
            h0 = fmaf(cvt_b2(hi), x.hi[i].z, h0);
            h1 = fmaf(cvt_b3(hi), x.hi[i].w, h1);
        }
        return finish(w, x, l0 + l1, h0 + h1);
    }
    __device__ static float dot(const W &w, const XH &x) {
        const uint32_t m = vgpr_const_6400();
        const jh2 o = {(_Float16)1024.0f, (_Float16)1024.0f};
        float l = 0.0f, h = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo, hi;
            q5(w, i, lo, hi);
            // bytes 0, 2 and 1, 3 of each word as the exact binary16 integers
            // q <= 31: (1024 + q) - 1024 (see nib_lo)
            const jh2 a = as_h2((lo & 0x001f001fu) | m) - o;
            const jh2 c = as_h2(((lo >> 8) & 0x001f001fu) | m) - o;
            const jh2 b = as_h2((hi & 0x001f001fu) | m) - o;
            const jh2 e = as_h2(((hi >> 8) & 0x001f001fu) | m) - o;
            l = i == 0 ? dot2z(a, x.lo[0]) : dot2(a, x.lo[2 * i], l);
            h = i == 0 ? dot2z(b, x.hi[0]) : dot2(b, x.hi[2 * i], h);
            l = dot2(c, x.lo[2 * i + 1], l);
            h = dot2(e, x.hi[2 * i + 1], h);
        }
        return finish(w, x, l, h);
    }
};

// ---- F16 weights: a unit is 8 binary16 weights (one 16-byte load) ----------
struct FF16 {
    static constexpr int UNIT = 8;
    static constexpr bool XREREAD = false;   // long rows re-read x from LDS per row group
    static constexpr bool PERM = false;
    struct W { uint4 q; };
    __device__ static W load(WPtr w, size_t unit) {
        W r;
        r.q = ld_stream((const uint4 *)w.qs + unit);
        return r;
    }
    __device__ static W load_row(WPtr w, size_t ru, uint32_t u) {
        W r;
        r.q = ld_stream(w.qs + ru * 16 + u * 16u);
        return r;
    }
    struct XF { jf4 a, b; };
    __device__ static XF loadx(const float *xs, const float *, int u) {
        const jf4 *p = (const jf4 *)(xs + (u >> 2) * XLayout<float>::STRIDE + (u & 3) * 8);
        XF r;
        r.a = p[0];
        r.b = p[1];
        return r;
    }
    struct XH { uint4 v; };
    __device__ static XH loadx(const _Float16 *xs, const float *, int u) {
        XH r;
        r.v = *(const uint4 *)(xs + (u >> 2) * XLayout<_Float16>::STRIDE + (u & 3) * 8);
        return r;
    }
    __device__ static XF loadx_g(const float *x, int u) {
        const jf4 *p = (const jf4 *)(x + (size_t)u * 8);
        XF r;
        r.a = p[0];
        r.b = p[1];
        return r;
    }
    __device__ static XH loadx_g(const _Float16 *x, int u) {
        XH r;
        r.v = *(const uint4 *)(x + (size_t)u * 8);
        return r;
    }
    __device__ static float dot(const W &w, const XF &x) {
        jh2 p0 = as_h2(w.q.x), p1 = as_h2(w.q.y), p2 = as_h2(w.q.z), p3 = as_h2(w.q.w);
        float s0 = (float)p0.x * x.a.x;
        float s1 = (float)p0.y * x.a.y;
        s0 = fmaf((float)p1.x, x.a.z, s0);
        s1 = fmaf((float)p1.y, x.a.w, s1);
        s0 = fmaf((float)p2.x, x.b.x, s0);
        s1 = fmaf((float)p2.y, x.b.y, s1);
        s0 = fmaf((float)p3.x, x.b.z, s0);
        s1 = fmaf((float)p3.y, x.b.w, s1);
        return s0 + s1;
    }
    __device__ static float dot(const W &w, const XH &x) {
        float s = dot2z(as_h2(w.q.x), as_h2(x.v.x));
        s = dot2(as_h2(w.q.y), as_h2(x.v.y), s);
        s = dot2(as_h2(w.q.z), as_h2(x.v.z), s);
        return dot2(as_h2(w.q.w), as_h2(x.v.w), s);
    }
};

// ---------------------------------------------------------------------------
// cross-lane reduction of R row partials over LPR lanes
// ---------------------------------------------------------------------------
// On return, lanes whose (li % (LPR/R)) == 0 hold the total of row `ridx`.
template <int LPR, int R>
__device__ __forceinline__ float reduce_rows(float (&v)[R], int li, int &ridx) {
    int base = 0;
#pragma unroll
    for (int c = R, o = LPR / 2; c > 1; c >>= 1, o >>= 1) {
        const bool upper = (li & o) != 0;
#pragma unroll
        for (int j = 0; j < c / 2; ++j) {
            float send = upper ? v[j] : v[j + c / 2];
            float keep = upper ? v[j + c / 2] : v[j];
            v[j] = keep + shfl_xor(send, o);
        }
        if (upper) base += c / 2;
    }
    float s = v[0];
#pragma unroll
    for (int o = LPR / (2 * R); o > 0; o >>= 1) s += shfl_xor(s, o);
    ridx = base;
    return s;
}

template <class F, typename XIN, typename XT, int LPR, int R, int BPL_MAX>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nblk = (a.k + XB - 1) / XB;
    XT *xs = (XT *)smem;
    float *sx16 = (float *)(smem + ((nblk * XLayout<XT>::STRIDE * sizeof(XT) + 15) & ~15u));

    constexpr int SUB = 64 / LPR;   // row groups per wavefront
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane % LPR, sg = lane / LPR;
    const int waves = 4;   // 256-thread workgroups
    const uint32_t rows_per_wave = SUB * R;
    const uint32_t wave_id = blockIdx.x * waves + wave;
    const uint32_t row0 = wave_id * rows_per_wave + sg * R;
    const int units = (int)a.units;

    // Issue the weight loads first: they do not depend on x.
    typename F::W wr[BPL_MAX][R];
#pragma unroll
    for (int i = 0; i < BPL_MAX; ++i) {
        int u = li + i * LPR;
        if (u < units) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t row = row0 + r;
                row = row < a.n ? row : a.n - 1;
                wr[i][r] = F::load(a.w, (size_t)row * units + u);
            }
        }
    }

    stage_x<XIN, XT, F::PERM && sizeof(XT) == 2>((const XIN *)a.x, a.k, xs, sx16, 256);
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < BPL_MAX; ++i) {
        int u = li + i * LPR;
        if (u < units) {
            auto xr = F::loadx((const XT *)xs, sx16, u);
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] += F::dot(wr[i][r], xr);
        }
    }

    int ridx;
    float s = reduce_rows<LPR, R>(acc, li, ridx);
    uint32_t row = row0 + ridx;
    if ((li % (LPR / R)) == 0 && row < a.n) {
        if (a.epi == EPI_RESIDUAL) s += a.resid[row];
        if (a.out_f16) ((uint16_t *)a.y)[row] = f2h_bits(s);
        else ((float *)a.y)[row] = s;
    }
}

// Cross-lane reduction for a full wavefront per row (LPR = 64), R <= 4 rows:
// v_permlane32_swap / v_permlane16_swap exchange halves of two row partials
// at once (the transposed steps), DPP row rotations finish each 16-lane row.
// On return every lane holds the total of row `ridx`; lanes with
// lane % (64 / R) == 0 are the writers.
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float swap32_sum(float a, float b) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float swap16_sum(float a, float b) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
template <int R>
__device__ __forceinline__ float reduce_wave_rows(float (&v)[R], int lane, int &ridx) {
    static_assert(R == 1 || R == 2 || R == 4, "R must be 1, 2 or 4");
    float s;
    if (R == 1) {
        s = swap16_sum(v[0], v[0]);
        s = swap32_sum(s, s);
        ridx = 0;
    } else if (R == 2) {
        s = swap32_sum(v[0], v[1]);          // lanes < 32: row 0, lanes >= 32: row 1
        s = swap16_sum(s, s);
        ridx = lane >> 5;
    } else {
        float a = swap32_sum(v[0], v[2]);    // rows 0 | 2
        float b = swap32_sum(v[1], v[3]);    // rows 1 | 3
        s = swap16_sum(a, b);                // rows 0,1 | 2,3 by 16-lane row
        ridx = ((lane >> 5) << 1) | ((lane >> 4) & 1);
    }
    s += dpp_f<0x128>(s);   // row_ror:8
    s += dpp_f<0x124>(s);   // row_ror:4
    s += dpp_f<0x122>(s);   // row_ror:2
    s += dpp_f<0x121>(s);   // row_ror:1
    return s;
}

// Register-resident variant: each lane keeps x for its units in registers
// (read once per wavefront from global memory, no LDS, no barriers) and every
// wavefront walks row groups g, g + W, ... (W = wavefronts in the grid). The
// steady-state loop is branch-free: the next group's weights are loaded while
// the current group is reduced, so the loads of one stage stay in flight
// behind the arithmetic of the other.
// XMODE 0: each lane keeps its units of x in registers, read once from global
// memory. XMODE 1: the same, read once from the LDS staging (xs, sx16) that
// stage() fills. XMODE 2: x is read from LDS per unit at every use (long rows,
// where x in registers would cost occupancy). stage() is called by every
// wavefront of the workgroup after the first weight loads are issued.
// DB = false drops the second weight buffer: the next row group is requested
// only after the current one is reduced (long rows whose registers would
// otherwise spill, where a wavefront rarely owns more than one group).
// pre() (if given) runs before the first weight loads are requested.
template <class F, typename XT, int BPL, int R, bool FULL, int XMODE = 0, class StageFn = int, bool DB = true,
          class PreFn = int>
__device__ __forceinline__ void gemv_reg_body(const GemvArgs &a, const XT *xs = nullptr,
                                              const float *sx16 = nullptr, StageFn stage = 0, PreFn pre = 0,
                                              uint64_t *lbest = nullptr) {
    const int lane = threadIdx.x & 63;
    // wavefront-uniform: row bases then live in scalar registers
    const uint32_t wg_waves = a.threads >> 6;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * wg_waves + (threadIdx.x >> 6));
    const uint32_t nwaves = gridDim.x * wg_waves;
    const int units = (int)a.units;
    const uint32_t groups = (a.n + R - 1) / R;
    using XR = std::conditional_t<sizeof(XT) == 2, typename F::XH, typename F::XF>;
    using WT = typename F::W;

    int uu[BPL];
    bool ok[BPL];
#pragma unroll
    for (int i = 0; i < BPL; ++i) {
        const int u = lane + 64 * i;
        ok[i] = FULL || u < units;
        uu[i] = ok[i] ? u : units - 1;   // clamped: always a valid address
    }
    WT wa[BPL][R], wb[BPL][R];
    auto load = [&](WT (&w)[BPL][R], uint32_t g) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t row = g * R + r;
            row = row < a.n ? row : a.n - 1;
            const size_t ru = (size_t)row * (uint32_t)units;   // uniform
#pragma unroll
            for (int i = 0; i < BPL; ++i) {
                uint32_t u = (uint32_t)uu[i];
                // long rows: the lane offsets are rebuilt per group from u (the
                // compiler would otherwise hold a 64-bit offset per load across
                // the group loop, and spill them)
                if constexpr (BPL >= 5) asm volatile("" : "+v"(u));
                w[i][r] = F::load_row(a.w, ru, u);
            }
        }
    };
    const bool has = wave < groups;
    const uint32_t mine = has ? (groups - 1 - wave) / nwaves + 1 : 0;   // groups this wavefront owns
    // The RoPE position and cache row base are requested before anything
    // else (the position selects the cos/sin row of the first group, requested
    // right after the staging), as vector loads through an index the compiler
    // cannot see is zero: a scalar load shares its counter with the staging's
    // LDS accesses, whose waits would then wait for it as well. Other
    // epilogues read a weight word instead (always a valid address).
    uint32_t zv;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zv));
    const bool qkv = a.epi == EPI_QKV_ROPE;
    const int32_t *pos_p = qkv ? a.d_pos : (const int32_t *)a.w.qs;
    const int32_t *rb_p = (qkv && a.d_rowbase) ? a.d_rowbase : pos_p;
    const int32_t pos_v = pos_p[zv], rb_v = rb_p[zv];
    // Row written by this lane after the reduction (a static function of the lane).
    const int my_ridx = R == 1 ? 0 : R == 2 ? (lane >> 5) : (((lane >> 5) << 1) | ((lane >> 4) & 1));
    // the first group's residual, requested ahead of x for the same reason
    float res0 = 0.0f;
    if (a.epi == EPI_RESIDUAL) {
        const uint32_t row = wave * R + my_ridx;
        res0 = row < a.n ? a.resid[row] : 0.0f;
    }
    if constexpr (!std::is_same<PreFn, int>::value) pre();
    // Wavefronts without a group (the last workgroup of the LDS kernel) still
    // request a real one and discard it: every wavefront then issues the same
    // loads, so the wait for x in stage() counts exactly and does not also
    // wait for the weights.
    load(wa, has ? wave : groups - 1);
    if constexpr (XMODE != 0) stage();
    if (!has) return;

    XR xr[XMODE == 2 ? 1 : BPL];
    if constexpr (XMODE == 0) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) xr[i] = F::loadx_g((const XT *)a.x, uu[i]);
    } else if constexpr (XMODE == 1) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) xr[i] = F::loadx(xs, sx16, uu[i]);
    }

    const bool writer = (lane & (64 / R - 1)) == 0;
    const uint32_t pos = qkv ? (uint32_t)__builtin_amdgcn_readfirstlane(pos_v) : 0u;
    const uint32_t kvbase = (qkv && a.d_rowbase) ? (uint32_t)__builtin_amdgcn_readfirstlane(rb_v) : 0u;
    const size_t kvrow = (size_t)kvbase + pos;
    int smode = SAMPLE_ARGMAX;
    float spen = 1.0f;
    if (a.epi == EPI_ARGMAX && a.sampler) {
        smode = a.sampler->mode;
        spen = a.sampler->penalty;
    }
    // Per-group side data (the residual, or the RoPE cos/sin pair) is read
    // before the next group's weights are requested, so waiting for it never
    // waits for the prefetch.
    auto load_side = [&](uint32_t g) -> float2 {
        if (a.epi == EPI_RESIDUAL) {
            const uint32_t row = g * R + my_ridx;
            return make_float2(row < a.n ? a.resid[row] : 0.0f, 0.0f);
        }
        if (a.epi == EPI_QKV_ROPE && g < a.q_pairs + a.k_pairs) {
            const uint32_t i = (g < a.q_pairs ? g : g - a.q_pairs) % a.half_hd;
            return *(const float2 *)(a.rope + 2 * ((size_t)pos * a.half_hd + i));
        }
        if (a.epi == EPI_ARGMAX && smode == SAMPLE_PENALTY && a.counts) {
            // the row's occurrence count rides in .y (.x is added to the row)
            const uint32_t row = g * R + my_ridx;
            return make_float2(0.0f, __uint_as_float(row < a.n ? a.counts[row] : 0u));
        }
        return make_float2(0.0f, 0.0f);
    };
    uint64_t best = 0;   // EPI_ARGMAX: this lane's running maximum key
    auto consume = [&](WT (&w)[BPL][R], uint32_t g, float2 side) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            XR xv;
            if constexpr (XMODE == 2) {
                int u = uu[i];
                // Q4_K: x does not change between row groups and the compiler
                // would hoist every unit's read out of the group loop, keeping
                // them all live (spills on long rows); an opaque index keeps
                // each read next to its use
                if constexpr (F::XREREAD || sizeof(XT) == 4) asm volatile("" : "+v"(u));
                xv = F::loadx(xs, sx16, u);
            } else {
                xv = xr[i];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float d = F::dot(w[i][r], xv);
                acc[r] = ok[i] ? acc[r] + d : acc[r];
            }
            if constexpr (XMODE == 2 && (F::XREREAD || sizeof(XT) == 4)) __builtin_amdgcn_sched_barrier(0);
        }
        int ridx;
        float s = reduce_wave_rows<R>(acc, lane, ridx);
        // the paired-row epilogues only (EPI_ARGMAX rides the per-row store below)
        if (R == 2 && (a.epi == EPI_QKV_ROPE || a.epi == EPI_SWIGLU)) {
            // both row totals in every lane: lanes < 32 hold row 0, lanes >= 32 row 1
            auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
            const float r0 = __uint_as_float(p[0]), r1 = __uint_as_float(p[1]);
            if (lane == 0 && 2 * g < a.n) {
                if (a.epi == EPI_SWIGLU) {
                    // rows (2g, 2g + 1) = (gate_g, up_g): act_g = silu(gate) * up
                    const float v = r0 * (1.0f / (1.0f + expf(-r0))) * r1;
                    if (a.out_f16) ((uint16_t *)a.y)[g] = f2h_bits(v);
                    else ((float *)a.y)[g] = v;
                } else if (g < a.q_pairs + a.k_pairs) {
                    // rope.wgsl:71-72 on the pair (x0, x1) = (r0, r1)
                    const float y0 = r0 * side.x - r1 * side.y;
                    const float y1 = r0 * side.y + r1 * side.x;
                    if (g < a.q_pairs) {
                        const uint32_t h = g / a.half_hd, i = g % a.half_hd;
                        float *q = (float *)a.y + (size_t)h * 2 * a.half_hd + i;
                        q[0] = y0;
                        q[a.half_hd] = y1;
                    } else {
                        const uint32_t gk = g - a.q_pairs, h = gk / a.half_hd, i = gk % a.half_hd;
                        const size_t at = kvrow * a.kv_row + (size_t)h * 2 * a.half_hd + i;
                        if (a.kv_f16) {
                            ((_Float16 *)a.kc)[at] = (_Float16)y0;
                            ((_Float16 *)a.kc)[at + a.half_hd] = (_Float16)y1;
                        } else {
                            ((float *)a.kc)[at] = y0;
                            ((float *)a.kc)[at + a.half_hd] = y1;
                        }
                    }
                } else {
                    const size_t at = kvrow * a.kv_row + 2 * (size_t)(g - a.q_pairs - a.k_pairs);
                    if (a.kv_f16) {
                        ((_Float16 *)a.vc)[at] = (_Float16)r0;
                        ((_Float16 *)a.vc)[at + 1] = (_Float16)r1;
                    } else {
                        ((float *)a.vc)[at] = r0;
                        ((float *)a.vc)[at + 1] = r1;
                    }
                }
            }
            return;
        }
        const uint32_t row = g * R + ridx;
        if (writer && row < a.n) {
            s += side.x;
            if (a.out_f16) ((uint16_t *)a.y)[row] = f2h_bits(s);
            else ((float *)a.y)[row] = s;
            if (a.epi == EPI_ARGMAX) {
                const uint64_t key = sampler_key(s, row, __float_as_uint(side.y), smode, spen);
                best = key > best ? key : best;
            }
        }
    };

    uint32_t it = 0, g = wave;
    float2 ra = a.epi == EPI_RESIDUAL ? make_float2(res0, 0.0f) : load_side(g), rb;
    if constexpr (!DB) {
        for (;;) {
            consume(wa, g, ra);
            if (++it >= mine) break;
            g += nwaves;
            ra = load_side(g);
            load(wa, g);
        }
        it = mine;   // the double-buffered tail below has nothing left
    }
    for (; DB && it + 2 < mine; it += 2, g += 2 * nwaves) {
        rb = load_side(g + nwaves);
        load(wb, g + nwaves);
        consume(wa, g, ra);
        ra = load_side(g + 2 * nwaves);
        load(wa, g + 2 * nwaves);
        consume(wb, g + nwaves, rb);
    }
    if (DB && it + 1 < mine) {
        rb = load_side(g + nwaves);
        load(wb, g + nwaves);
        consume(wa, g, ra);
        consume(wb, g + nwaves, rb);
    } else if (it < mine) {
        consume(wa, g, ra);
    }
    if (a.epi == EPI_ARGMAX) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint64_t other = ((uint64_t)(uint32_t)shfl_xor((int)(best >> 32), o) << 32) |
                                   (uint32_t)shfl_xor((int)(best & 0xffffffffu), o);
            best = other > best ? other : best;
        }
        if (lane == 0) {
            if (lbest) {
                // Workgroup maximum in LDS (lbest[0], zeroed by the staging
                // before its barrier, with the arrival count in lbest[1]); the
                // last of the workgroup's wavefronts that own groups folds it
                // into the global key: one global atomic per workgroup.
                const uint32_t wg0 = blockIdx.x * wg_waves;
                const uint32_t owners = groups > wg0 ? min(wg_waves, groups - wg0) : 0u;
                __hip_atomic_fetch_max(lbest, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                const uint64_t n = __hip_atomic_fetch_add(lbest + 1, (uint64_t)1, __ATOMIC_ACQ_REL,
                                                          __HIP_MEMORY_SCOPE_WORKGROUP);
                if (n + 1 == owners) {
                    const uint64_t wb = __hip_atomic_load(lbest, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    if (wb) atomicMax(a.best, (unsigned long long)wb);
                }
            } else if (best) {
                atomicMax(a.best, (unsigned long long)best);
            }
        }
    }
}

template <class F, typename XT, int BPL, int R>
__global__ __launch_bounds__(256) void gemv_reg_kernel(GemvArgs a) {
    const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6);   // 256-thread workgroups
    if (wave >= (a.n + R - 1) / R) return;
    if (a.units == 64u * BPL) gemv_reg_body<F, XT, BPL, R, true>(a);
    else gemv_reg_body<F, XT, BPL, R, false>(a);
}

// Rounds 16 staged values (group g of x) to binary16, writes them to LDS in
// the layout of stage_x and their sum to sx16[g].
template <bool PERM>
__device__ __forceinline__ void store_x16(const float (&v)[16], uint32_t g, _Float16 *xs, float *sx16) {
    const uint32_t e0 = g * 16;
    _Float16 hv[16];
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        hv[t] = (_Float16)v[t];
        s += (float)hv[t];
    }
    sx16[g] = s;
    _Float16 *dst = xs + (e0 / 32) * XLayout<_Float16>::STRIDE + (e0 % 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const jh4 o = PERM ? (jh4){hv[4 * q], hv[4 * q + 2], hv[4 * q + 1], hv[4 * q + 3]}
                           : (jh4){hv[4 * q], hv[4 * q + 1], hv[4 * q + 2], hv[4 * q + 3]};
        *(jh4 *)(dst + 4 * q) = o;
    }
}

// RMS-normalised staging of f32 x (workgroups of 512 to 1024 threads,
// k <= 16 * 512 * MAXG). Thread t holds the float4 slots s = t + nt * j
// (elements 4s..4s+3), so each load instruction of a wavefront reads 1 KiB of
// consecutive bytes, and a 16-element group of the staging is one lane quad.
// All loads are in flight together; the sum of squares is reduced in a fixed
// order (the thread's slots, the wavefront by permlane / DPP steps, then
// wavefront order), then x * (1 / rms) * gamma is staged.
// The loads (norm_load) are requested before the weights: loads return in
// issue order, so x requested after the weights would hold the reduction and
// its barriers until every weight load had landed.
template <int MAXG> struct NormRegs { jf4 v[4 * MAXG], gm[4 * MAXG]; };

template <int MAXG>
__device__ __forceinline__ void norm_load(const float *__restrict__ x, const float *__restrict__ gamma, uint32_t k,
                                          uint32_t nt, NormRegs<MAXG> &r) {
    // x and gamma are requested together: one round trip before the reduction
#pragma unroll
    for (int j = 0; j < 4 * MAXG; ++j) {
        // Rounds with no slot of the staging load nothing (a workgroup-uniform
        // branch; their registers are never read). k % 8 == 0 for every weight
        // format these kernels take, so a slot is whole or past the end; slots
        // past the end load the last slot again and are zeroed in the staging
        // (a per-lane conditional load makes the compiler merge registers and
        // wait for the load before the weights are requested).
        if (nt * j < 4 * ((k + 15) / 16)) {
            const uint32_t sl = min(threadIdx.x + nt * j, k / 4 - 1);
            r.v[j] = *(const jf4 *)(x + 4 * sl);
            r.gm[j] = *(const jf4 *)(gamma + 4 * sl);
        }
    }
}

template <bool PERM, int MAXG>
__device__ void stage_x16_norm(NormRegs<MAXG> &r, uint32_t k, uint32_t nt, _Float16 *xs, float *sx16, float eps,
                               float *red) {
    const uint32_t nslot = 4 * ((k + 15) / 16);   // whole 16-element groups (zeros past k)
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4 * MAXG; ++j) {
        if (nt * j >= nslot) break;   // uniform: the round loaded nothing
        if (4 * (threadIdx.x + nt * j) >= k) r.v[j] = (jf4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; ++t) ss = fmaf(r.v[j][t], r.v[j][t], ss);
    }
    float sv[1] = {ss};
    int ridx;
    ss = reduce_wave_rows<1>(sv, threadIdx.x & 63, ridx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (uint32_t w = 0; w < (nt >> 6); ++w) tot += red[w];
    // (x / rms) * gamma, the reference's formula (activations.wgsl:128)
    const float rms = sqrtf(tot / (float)k + eps);
#pragma unroll
    for (int j = 0; j < 4 * MAXG; ++j) {
        if (nt * j >= nslot) break;   // uniform: no slot of this round is staged
        const uint32_t sl = threadIdx.x + nt * j, e0 = 4 * sl;
        _Float16 hv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) hv[t] = (_Float16)((r.v[j][t] / rms) * r.gm[j][t]);
        // the group's sum of its binary16 values: lane, then lane pairs of the quad
        float q = (((float)hv[0] + (float)hv[1]) + (float)hv[2]) + (float)hv[3];
        q += dpp_f<0xb1>(q);   // quad_perm [1,0,3,2]
        q += dpp_f<0x4e>(q);   // quad_perm [2,3,0,1]
        if (sl < nslot) {
            if ((threadIdx.x & 3) == 0) sx16[sl >> 2] = q;
            const jh4 o = PERM ? (jh4){hv[0], hv[2], hv[1], hv[3]} : (jh4){hv[0], hv[1], hv[2], hv[3]};
            *(jh4 *)(xs + (e0 / 32) * XLayout<_Float16>::STRIDE + (e0 % 32)) = o;
        }
    }
}

// The same staging in binary32 (the reference's dtype): (x / rms) * gamma
// stored unrounded in the f32 LDS layout (natural element order), with the
// 16-element sums beside it.
template <int MAXG>
__device__ void stage_x32_norm(NormRegs<MAXG> &r, uint32_t k, uint32_t nt, float *xs, float *sx16, float eps,
                               float *red) {
    const uint32_t nslot = 4 * ((k + 15) / 16);
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4 * MAXG; ++j) {
        if (nt * j >= nslot) break;
        if (4 * (threadIdx.x + nt * j) >= k) r.v[j] = (jf4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; ++t) ss = fmaf(r.v[j][t], r.v[j][t], ss);
    }
    float sv[1] = {ss};
    int ridx;
    ss = reduce_wave_rows<1>(sv, threadIdx.x & 63, ridx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (uint32_t w = 0; w < (nt >> 6); ++w) tot += red[w];
    const float rms = sqrtf(tot / (float)k + eps);
#pragma unroll
    for (int j = 0; j < 4 * MAXG; ++j) {
        if (nt * j >= nslot) break;
        const uint32_t sl = threadIdx.x + nt * j, e0 = 4 * sl;
        jf4 v;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = (r.v[j][t] / rms) * r.gm[j][t];
        float q = ((v[0] + v[1]) + v[2]) + v[3];
        q += dpp_f<0xb1>(q);   // quad_perm [1,0,3,2]
        q += dpp_f<0x4e>(q);   // quad_perm [2,3,0,1]
        if (sl < nslot) {
            if ((threadIdx.x & 3) == 0) sx16[sl >> 2] = q;
            *(jf4 *)(xs + (e0 / 32) * XLayout<float>::STRIDE + (e0 % 32)) = v;
        }
    }
}

// Plain binary32 x of the f32 staging, requested before the weights: thread
// t holds the float4 slots t + nt * j (j < 8, so k <= 32 * nt), a 16-element
// group being one lane quad, as in norm_load.
struct X32Regs { jf4 v[8]; };

__device__ __forceinline__ void x32_load(const float *__restrict__ x, uint32_t k, uint32_t nt, X32Regs &r) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if (nt * j < 4 * ((k + 15) / 16)) {   // workgroup-uniform
            const uint32_t sl = min(threadIdx.x + nt * j, k / 4 - 1);
            r.v[j] = *(const jf4 *)(x + 4 * sl);
        }
}

__device__ void x32_store(X32Regs &r, uint32_t k, uint32_t nt, float *xs, float *sx16) {
    const uint32_t nslot = 4 * ((k + 15) / 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (nt * j >= nslot) break;
        const uint32_t sl = threadIdx.x + nt * j, e0 = 4 * sl;
        const jf4 v = e0 < k ? r.v[j] : (jf4){0.0f, 0.0f, 0.0f, 0.0f};
        float q = ((v[0] + v[1]) + v[2]) + v[3];
        q += dpp_f<0xb1>(q);   // quad_perm [1,0,3,2]
        q += dpp_f<0x4e>(q);   // quad_perm [2,3,0,1]
        if (sl < nslot) {
            if ((threadIdx.x & 3) == 0) sx16[sl >> 2] = q;
            *(jf4 *)(xs + (e0 / 32) * XLayout<float>::STRIDE + (e0 % 32)) = v;
        }
    }
}

// binary16 x of the plain (not normalised) LDS staging, requested before the
// weights like norm_load: every thread's groups of 16 (k <= 16 * 2 * threads)
// held in registers until the weights are in flight.
struct X16Regs { uint4 u[2][2]; };

__device__ __forceinline__ void x16_load(const _Float16 *__restrict__ x, uint32_t k, uint32_t nt, X16Regs &r) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t e0 = (threadIdx.x + nt * j) * 16;
        const bool full = e0 + 16 <= k;
        r.u[j][0] = full ? *(const uint4 *)(x + e0) : make_uint4(0u, 0u, 0u, 0u);
        r.u[j][1] = full ? *(const uint4 *)(x + e0 + 8) : make_uint4(0u, 0u, 0u, 0u);
    }
}

// Stores the groups of x16_load in the layout of stage_x: full groups are
// copied as they are (the pair permutation is a byte select) with their sums
// taken by v_dot2_f32_f16 against (1, 1); a ragged last group goes through
// store_x16.
template <bool PERM>
__device__ void x16_store(const X16Regs &r, const _Float16 *__restrict__ x, uint32_t k, uint32_t nt, _Float16 *xs,
                          float *sx16) {
    const uint32_t g16 = (k + 15) / 16;
    const jh2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t g = threadIdx.x + nt * j, e0 = g * 16;
        if (g >= g16) continue;
        if (e0 + 16 <= k) {
            float s0 = 0.0f, s1 = 0.0f;
            uint4 o[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint4 u = r.u[j][q];
                s0 = dot2(as_h2(u.x), one, s0);
                s1 = dot2(as_h2(u.y), one, s1);
                s0 = dot2(as_h2(u.z), one, s0);
                s1 = dot2(as_h2(u.w), one, s1);
                if (PERM) {
                    o[q] = make_uint4(__builtin_amdgcn_perm(u.y, u.x, 0x05040100u), __builtin_amdgcn_perm(u.y, u.x, 0x07060302u),
                                      __builtin_amdgcn_perm(u.w, u.z, 0x05040100u), __builtin_amdgcn_perm(u.w, u.z, 0x07060302u));
                } else {
                    o[q] = u;
                }
            }
            sx16[g] = s0 + s1;
            uint4 *dst = (uint4 *)(xs + (g >> 1) * XLayout<_Float16>::STRIDE + (g & 1) * 16);
            dst[0] = o[0];
            dst[1] = o[1];
        } else {
            float v[16];
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = e0 + t < k ? (float)x[e0 + t] : 0.0f;
            store_x16<PERM>(v, g, xs, sx16);
        }
    }
}

// Vectorised staging of binary16 x for the LDS kernel: each thread handles
// groups of 16 elements (16-byte global loads of x, and of gamma when
// normalising) and writes them with 8-byte LDS stores in the layout of
// stage_x; sx16 gets the 16-element sums of the stored values.
template <bool PERM, bool NORM>
__device__ void stage_x16(const void *__restrict__ xin, uint32_t k, uint32_t nt, _Float16 *xs, float *sx16,
                          const float *__restrict__ gamma, float rms) {
    const uint32_t g16 = (k + 15) / 16;
    for (uint32_t g = threadIdx.x; g < g16; g += nt) {
        float v[16];
        const uint32_t e0 = g * 16;
        if (NORM) {
            const float *x = (const float *)xin;
            if (e0 + 16 <= k) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const jf4 xa = *(const jf4 *)(x + e0 + 4 * q), ga = *(const jf4 *)(gamma + e0 + 4 * q);
#pragma unroll
                    for (int t = 0; t < 4; ++t) v[4 * q + t] = (xa[t] / rms) * ga[t];
                }
            } else {
#pragma unroll
                for (int t = 0; t < 16; ++t) v[t] = e0 + t < k ? (x[e0 + t] / rms) * gamma[e0 + t] : 0.0f;
            }
        } else {
            const _Float16 *x = (const _Float16 *)xin;
            if (e0 + 16 <= k) {
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const uint4 u = *(const uint4 *)(x + e0 + 8 * q);
                    const jh2 h[4] = {as_h2(u.x), as_h2(u.y), as_h2(u.z), as_h2(u.w)};
#pragma unroll
                    for (int t = 0; t < 4; ++t) { v[8 * q + 2 * t] = (float)h[t].x; v[8 * q + 2 * t + 1] = (float)h[t].y; }
                }
            } else {
#pragma unroll
                for (int t = 0; t < 16; ++t) v[t] = e0 + t < k ? (float)x[e0 + t] : 0.0f;
            }
        }
        store_x16<PERM>(v, g, xs, sx16);
    }
}

// Largest workgroup of the LDS kernel: 1024 threads (16 wavefronts, x staged
// once per CU at 16 wavefronts per CU) where the body fits 128 VGPRs, else 512.
template <class F, int BPL>
constexpr int lds_max_threads() {
    return ((BPL == 1 && !std::is_same<F, FQ5_K>::value) ||
            (BPL == 2 && (std::is_same<F, FQ4_0>::value || std::is_same<F, FF16>::value)))
               ? 1024
               : 512;
}

// LDS-staged variant for binary16 products: workgroups of 512 or 1024
// threads, x staged once per workgroup (optionally RMS-normalised on the way:
// the sum of squares is reduced over the workgroup in a fixed order, then
// x / rms * gamma is rounded to binary16). x is requested before the weights
// (loads return in issue order: x requested after them would hold the staging
// and its barrier until the first weights had landed). Up to 4 units per lane,
// each lane then keeps its units in registers; longer rows read their units
// from LDS at every use.
template <class F, int BPL, int R, bool NORM>
__global__ __launch_bounds__((lds_max_threads<F, BPL>())) void gemv_lds_kernel(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nblk = (a.k + XB - 1) / XB;
    _Float16 *xs = (_Float16 *)smem;
    float *sx16 = (float *)(smem + ((nblk * XLayout<_Float16>::STRIDE * 2 + 15) & ~15u));
    float *red = sx16 + (((a.k + 15) / 16 + 3) & ~3u);
    uint64_t *lbest = (uint64_t *)(red + 16);   // folded argmax key and arrival count
    NormRegs<NORM_MAXG> nr;
    // Plain binary16 x is requested first too, except on long K-quant and F16
    // rows (no registers to spare there)
    constexpr bool XPRE = !NORM && (BPL <= 4 || (!F::XREREAD && !std::is_same<F, FF16>::value));
    X16Regs xr;
    const uint32_t nt = a.threads;
    const bool xpre = XPRE && a.k <= 16u * 2u * nt;
    auto pre = [&]() {
        if constexpr (NORM) norm_load<NORM_MAXG>((const float *)a.x, a.gamma, a.k, nt, nr);
        if constexpr (XPRE)
            if (xpre) x16_load((const _Float16 *)a.x, a.k, nt, xr);
    };
    auto stage = [&]() {
        if constexpr (NORM) {
            stage_x16_norm<F::PERM, NORM_MAXG>(nr, a.k, nt, xs, sx16, a.eps, red);
        } else if (XPRE && xpre) {
            x16_store<F::PERM>(xr, (const _Float16 *)a.x, a.k, nt, xs, sx16);
        } else {
            stage_x16<F::PERM, false>(a.x, a.k, nt, xs, sx16, nullptr, 1.0f);
        }
        if (threadIdx.x == 0) lbest[0] = lbest[1] = 0;
        __syncthreads();
    };
    constexpr int XMODE = BPL <= 4 ? 1 : 2;
    // long rows single-buffered (the 512-thread workgroup caps a lane at 128
    // VGPRs; at these shapes a wavefront owns one row group): K-quants, whose
    // two buffers of chunks plus headers spill, and long Q4_0 / Q8_0 rows,
    // which spend the freed registers on x requested before the weights
    // (single-buffered alone measured slower: 4096x14336 10.6 against 9.8 us;
    // with x first 9.05 us)
    constexpr bool DB = BPL <= 4 || (!F::XREREAD && !XPRE);
    if (a.units == 64u * BPL)
        gemv_reg_body<F, _Float16, BPL, R, true, XMODE, decltype(stage), DB, decltype(pre)>(a, xs, sx16, stage, pre,
                                                                                           lbest);
    else
        gemv_reg_body<F, _Float16, BPL, R, false, XMODE, decltype(stage), DB, decltype(pre)>(a, xs, sx16, stage, pre,
                                                                                            lbest);
}

// The LDS-staged product on binary32 x (the reference's dtype; the fused
// single-sequence step with f32 activations): x, or its RMSNorm (requested
// before the weights), is staged once per workgroup as f32 and each unit's
// 32 values are read from LDS next to their use (an f32 unit is 32 VGPRs).
// 512-thread workgroups; the format's binary32 dot (exact integer weights,
// fp32 FMAs) as in the register kernel.
template <class F, int BPL, int R, bool NORM>
__global__ __launch_bounds__(512) void gemv_lds32_kernel(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nblk = (a.k + XB - 1) / XB;
    float *xs = (float *)smem;
    float *sx16 = (float *)(smem + ((nblk * XLayout<float>::STRIDE * 4 + 15) & ~15u));
    float *red = sx16 + (((a.k + 15) / 16 + 3) & ~3u);
    uint64_t *lbest = (uint64_t *)(red + 16);   // folded argmax key and arrival count
    NormRegs<NORM_MAXG> nr;
    X32Regs xr;
    const uint32_t nt = a.threads;
    const bool xpre = !NORM && a.k <= 32u * nt;
    auto pre = [&]() {
        if constexpr (NORM) norm_load<NORM_MAXG>((const float *)a.x, a.gamma, a.k, nt, nr);
        else if (xpre) x32_load((const float *)a.x, a.k, nt, xr);
    };
    auto stage = [&]() {
        if constexpr (NORM) stage_x32_norm<NORM_MAXG>(nr, a.k, nt, xs, sx16, a.eps, red);
        else if (xpre) x32_store(xr, a.k, nt, xs, sx16);
        else stage_x<float, float, false>((const float *)a.x, a.k, xs, sx16, (int)nt);
        if (threadIdx.x == 0) lbest[0] = lbest[1] = 0;
        __syncthreads();
    };
    constexpr bool DB = BPL <= 4;
    if (a.units == 64u * BPL)
        gemv_reg_body<F, float, BPL, R, true, 2, decltype(stage), DB, decltype(pre)>(a, xs, sx16, stage, pre, lbest);
    else
        gemv_reg_body<F, float, BPL, R, false, 2, decltype(stage), DB, decltype(pre)>(a, xs, sx16, stage, pre, lbest);
}

// Generic fallback for F16 weights whose k is not a multiple of 8: one
// wavefront per row, scalar loads (the tiny-model ffn_down case, k = 688).
template <typename XIN>
__global__ __launch_bounds__(256) void gemv_f16_any_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);   // 256-thread workgroups
    if (row >= a.n) return;
    const uint16_t *w = (const uint16_t *)a.w.qs + (size_t)row * a.k;
    const XIN *x = (const XIN *)a.x;
    float s = 0.0f;
    for (uint32_t i = lane; i < a.k; i += 64) s = fmaf(h2f(w[i]), (float)x[i], s);
    s = wave_sum(s);
    if (lane == 0) {
        if (a.epi == EPI_RESIDUAL) s += a.resid[row];
        if (a.out_f16) ((uint16_t *)a.y)[row] = f2h_bits(s);
        else ((float *)a.y)[row] = s;
    }
}

// ---------------------------------------------------------------------------
// launch selection
// ---------------------------------------------------------------------------

template <class F, typename XIN, typename XT, int LPR, int R, int BPL>
int launch_one(janus_ctx *ctx, const GemvArgs &a) {
    const int threads = 256, waves = threads / 64;
    const uint32_t rows_per_block = (uint32_t)waves * (64 / LPR) * R;
    const uint32_t grid = (a.n + rows_per_block - 1) / rows_per_block;
    const uint32_t nblk = (a.k + XB - 1) / XB;
    size_t lds = ((nblk * XLayout<XT>::STRIDE * sizeof(XT) + 15) & ~(size_t)15) + ((a.k + 15) / 16) * 4;
    if (lds > 160 * 1024) return janus::fail(ctx, JANUS_E_INVALID_DIM, "gemv: k too large for LDS staging");
    // allow > 64 KiB of dynamic LDS (gfx950 has 160 KiB per CU); thread-safe one-time set-up
    static const bool attr_set = [] {
        (void)hipFuncSetAttribute((const void *)gemv_kernel<F, XIN, XT, LPR, R, BPL>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        return true;
    }();
    (void)attr_set;
    hipLaunchKernelGGL((gemv_kernel<F, XIN, XT, LPR, R, BPL>), dim3(grid), dim3(threads), lds, ctx->stream, a);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// Chooses lanes-per-row, rows-per-wave and the unrolled units-per-lane bound
// from the row length. Large rows use the whole wavefront per row.
template <class F, typename XIN, typename XT>
int launch_fmt(janus_ctx *ctx, const GemvArgs &a) {
    const int u = (int)a.units;
    if (u <= 8) return launch_one<F, XIN, XT, 8, 4, 1>(ctx, a);
    if (u <= 16) return launch_one<F, XIN, XT, 16, 4, 1>(ctx, a);
    if (u <= 64) return launch_one<F, XIN, XT, 64, 4, 1>(ctx, a);
    if (u <= 128) return launch_one<F, XIN, XT, 64, 4, 2>(ctx, a);
    if (u <= 256) return launch_one<F, XIN, XT, 64, 2, 4>(ctx, a);
    if (u <= 512) return launch_one<F, XIN, XT, 64, 2, 8>(ctx, a);
    if (u <= 1024) return launch_one<F, XIN, XT, 64, 1, 16>(ctx, a);
    if (u <= 2048) return launch_one<F, XIN, XT, 64, 1, 32>(ctx, a);
    return janus::fail(ctx, JANUS_E_INVALID_DIM, "gemv: row too long");
}

// Persistent grid: as many workgroups as can be resident at once (from the
// occupancy the compiled kernel allows, capped at ctx->gemv_wpc wavefronts
// per CU); each wavefront then walks several row groups.
template <class F, typename XT, int BPL, int R>
int launch_reg(janus_ctx *ctx, const GemvArgs &a) {
    // host threads may launch at once: the cached value is relaxed-atomic (a
    // race only repeats the same occupancy query)
    static std::atomic<int> occ_cache{0};
    int occ = occ_cache.load(std::memory_order_relaxed);
    if (occ == 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, gemv_reg_kernel<F, XT, BPL, R>, 256, 0) != hipSuccess ||
            nb < 1)
            nb = 1;
        occ = nb;
        occ_cache.store(occ, std::memory_order_relaxed);
    }
    int per_cu = occ < (int)ctx->gemv_wpc / 4 ? occ : (int)ctx->gemv_wpc / 4;
    if (per_cu < 1) per_cu = 1;
    const uint32_t groups = (a.n + R - 1) / R;
    uint32_t blocks = (groups + 3) / 4;
    const uint32_t cap = (uint32_t)ctx->num_cus * per_cu;
    if (blocks > cap) blocks = cap;
    GemvArgs b = a;
    b.threads = 256;
    hipLaunchKernelGGL((gemv_reg_kernel<F, XT, BPL, R>), dim3(blocks), dim3(256), 0, ctx->stream, b);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// Units per lane = ceil(units / 64); R rows per wavefront step keep at least
// ~4 KB of weights in flight per stage. x must fit ~128 VGPRs per lane.
template <class F, typename XT>
int launch_reg_fmt(janus_ctx *ctx, const GemvArgs &a, bool &done) {
    constexpr int XREGS = sizeof(std::conditional_t<sizeof(XT) == 2, typename F::XH, typename F::XF>) / 4;
    const int bpl = (int)((a.units + 63) / 64);
    done = bpl * XREGS <= 132 && a.units >= 64;
    if (!done) return JANUS_OK;
    switch (bpl) {
    case 1: return launch_reg<F, XT, 1, 4>(ctx, a);
    case 2: return launch_reg<F, XT, 2, 2>(ctx, a);
    case 3: return launch_reg<F, XT, 3, 1>(ctx, a);
    case 4: return launch_reg<F, XT, 4, 1>(ctx, a);
    case 5: return launch_reg<F, XT, (XREGS * 5 <= 132 ? 5 : 1), 1>(ctx, a);
    case 6: return launch_reg<F, XT, (XREGS * 6 <= 132 ? 6 : 1), 1>(ctx, a);
    case 7: return launch_reg<F, XT, (XREGS * 7 <= 132 ? 7 : 1), 1>(ctx, a);
    case 8: return launch_reg<F, XT, (XREGS * 8 <= 132 ? 8 : 1), 1>(ctx, a);
    default: break;
    }
    if (bpl <= 16 && XREGS * 16 <= 132) return launch_reg<F, XT, (XREGS * 16 <= 132 ? 16 : 1), 1>(ctx, a);
    if (bpl <= 32 && XREGS * 32 <= 132) return launch_reg<F, XT, (XREGS * 32 <= 132 ? 32 : 1), 1>(ctx, a);
    done = false;
    return JANUS_OK;
}

// LDS-staged kernel: grid = the workgroups that fit at once (occupancy of the
// compiled kernel), each wavefront walking several row groups.
template <class F, int BPL, int R>
int launch_lds(janus_ctx *ctx, const GemvArgs &a, bool norm) {
    constexpr int TMAX = lds_max_threads<F, BPL>();
    const uint32_t groups = (a.n + R - 1) / R;
    // Q4_0 / F16 rows of one or two units per lane in at most 16 row groups
    // per CU (batch-1 QKV and o-proj): one 512-thread workgroup per CU, so a
    // wavefront owns about two groups (the second group's weights are
    // requested before the first is consumed) and x is staged once per CU.
    // Otherwise 512-thread workgroups, two per CU, whose stagings and
    // barriers do not hold each other's wavefronts (Q4_0 14336x4096 7.8 ->
    // 7.35 us, gate/up 28672x4096 14.6 -> 13.2; K-quant rows, VALU-heavier,
    // and the long down-proj rows measured slower at one per CU).
    // JANUS_GEMV_LDS_THREADS sets the size (up to 1024 where the body fits)
    // and the JANUS_GEMV_LDS_WPC cap applies to it.
    int threads = 512;
    int one_per_cu = TMAX == 1024 && groups <= 16u * ctx->num_cus;
    if (ctx->gemv_lds_threads && (int)ctx->gemv_lds_threads <= TMAX) {
        threads = (int)ctx->gemv_lds_threads;
        one_per_cu = 0;
    }
    const int wg_waves = threads / 64;
    // resident workgroups per CU for this kernel at this LDS size (4 KB steps)
    static std::atomic<int> per_cu[2][17][17] = {};   // relaxed, as in launch_reg
    const void *kern = norm ? (const void *)gemv_lds_kernel<F, BPL, R, true> : (const void *)gemv_lds_kernel<F, BPL, R, false>;
    const uint32_t nblk = (a.k + XB - 1) / XB;
    const size_t lds = ((nblk * XLayout<_Float16>::STRIDE * 2 + 15) & ~(size_t)15) + ((((a.k + 15) / 16) + 3) & ~3u) * 4 + 80;
    if (lds > 64 * 1024) return janus::fail(ctx, JANUS_E_INVALID_DIM, "gemv: k too large for LDS staging");
    const size_t lds_step = (lds + 4095) / 4096;
    std::atomic<int> &occ_cache = per_cu[norm ? 1 : 0][wg_waves][lds_step];
    int occ = occ_cache.load(std::memory_order_relaxed);
    if (occ == 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, threads, lds_step * 4096) != hipSuccess || nb < 1)
            nb = 1;
        occ = nb;
        occ_cache.store(occ, std::memory_order_relaxed);
    }
    const int wg_cap = one_per_cu ? 1 : (int)ctx->gemv_lds_wpc / wg_waves;
    int pc = occ < wg_cap ? occ : wg_cap;
    if (pc < 1) pc = 1;
    uint32_t blocks = (groups + wg_waves - 1) / wg_waves;
    const uint32_t cap = (uint32_t)ctx->num_cus * pc;
    if (blocks > cap) blocks = cap;
    GemvArgs b = a;
    b.threads = (uint32_t)threads;
    if (norm) hipLaunchKernelGGL((gemv_lds_kernel<F, BPL, R, true>), dim3(blocks), dim3(threads), lds, ctx->stream, b);
    else hipLaunchKernelGGL((gemv_lds_kernel<F, BPL, R, false>), dim3(blocks), dim3(threads), lds, ctx->stream, b);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

// binary32 x: one 512-thread workgroup per CU, each wavefront walking several
// row groups, x staged once per CU. Against two per CU (the bs=1 step with
// the reference's dtypes, Llama-3-8B shapes, traced): QKV + gate/up 24.3
// against 25.3 us, down 10.4 against 11.5, o-proj 5.1 against 5.3, F16 LM
// head 160.9 against 166.2; 1.640-1.645 against 1.717-1.720 ms/token.
template <class F, int BPL, int R>
int launch_lds32(janus_ctx *ctx, const GemvArgs &a, bool norm) {
    const int threads = 512, wg_waves = 8;
    const uint32_t groups = (a.n + R - 1) / R;
    const uint32_t nblk = (a.k + XB - 1) / XB;
    const size_t lds = ((nblk * XLayout<float>::STRIDE * 4 + 15) & ~(size_t)15) + ((((a.k + 15) / 16) + 3) & ~3u) * 4 + 80;
    if (lds > 160 * 1024) return janus::fail(ctx, JANUS_E_INVALID_DIM, "gemv: k too large for f32 LDS staging");
    static const bool attr_set = [] {   // > 64 KiB of dynamic LDS for long rows; thread-safe one-time set-up
        (void)hipFuncSetAttribute((const void *)gemv_lds32_kernel<F, BPL, R, true>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void *)gemv_lds32_kernel<F, BPL, R, false>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        return true;
    }();
    (void)attr_set;
    uint32_t blocks = (groups + wg_waves - 1) / wg_waves;
    if (blocks > (uint32_t)ctx->num_cus) blocks = (uint32_t)ctx->num_cus;
    GemvArgs b = a;
    b.threads = (uint32_t)threads;
    if (norm) hipLaunchKernelGGL((gemv_lds32_kernel<F, BPL, R, true>), dim3(blocks), dim3(threads), lds, ctx->stream, b);
    else hipLaunchKernelGGL((gemv_lds32_kernel<F, BPL, R, false>), dim3(blocks), dim3(threads), lds, ctx->stream, b);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

template <class F>
int launch_lds32_fmt(janus_ctx *ctx, const GemvArgs &a, bool norm, bool pair, bool &done) {
    const int bpl = (int)((a.units + 63) / 64);
    done = bpl <= 8;
    if (!done) return JANUS_OK;
    if (pair) {
        switch (bpl) {
        case 1: return launch_lds32<F, 1, 2>(ctx, a, norm);
        case 2: return launch_lds32<F, 2, 2>(ctx, a, norm);
        case 3: return launch_lds32<F, 3, 2>(ctx, a, norm);
        case 4: return launch_lds32<F, 4, 2>(ctx, a, norm);
        default: done = false; return JANUS_OK;
        }
    }
    switch (bpl) {
    case 1: return launch_lds32<F, 1, 4>(ctx, a, norm);
    case 2: return launch_lds32<F, 2, 1>(ctx, a, norm);
    case 3: return launch_lds32<F, 3, 1>(ctx, a, norm);
    case 4: return launch_lds32<F, 4, 1>(ctx, a, norm);
    case 5: return launch_lds32<F, 5, 1>(ctx, a, norm);
    case 6: return launch_lds32<F, 6, 1>(ctx, a, norm);
    case 7: return launch_lds32<F, 7, 1>(ctx, a, norm);
    default: return launch_lds32<F, 8, 1>(ctx, a, norm);
    }
}

// Units per lane = ceil(units / 64), up to 8. Rows per wavefront step: four
// at one unit per lane, one at two (each wavefront's last row group, whose
// arithmetic runs after the stream has ended, is half as long: Q4_0
// 14336x4096 8.1 -> 7.8 us, 4096x4096 4.0 -> 3.7), two at three and four,
// one beyond; always two for the paired-row epilogues.
template <class F>
int launch_lds_fmt(janus_ctx *ctx, const GemvArgs &a, bool norm, bool pair, bool &done) {
    const int bpl = (int)((a.units + 63) / 64);
    done = bpl <= 8;
    if (!done) return JANUS_OK;
    if (pair) {
        switch (bpl) {
        case 1: return launch_lds<F, 1, 2>(ctx, a, norm);
        case 2: return launch_lds<F, 2, 2>(ctx, a, norm);
        case 3: return launch_lds<F, 3, 2>(ctx, a, norm);
        case 4: return launch_lds<F, 4, 2>(ctx, a, norm);
        case 5: return launch_lds<F, 5, 2>(ctx, a, norm);
        case 6: return launch_lds<F, 6, 2>(ctx, a, norm);
        case 7: return launch_lds<F, 7, 2>(ctx, a, norm);
        default: return launch_lds<F, 8, 2>(ctx, a, norm);
        }
    }
    // F16 rows of 8 units per lane (the LM head): two rows per step halve the
    // cross-lane reductions per row and double the bytes in flight (the body
    // fits: 4 VGPRs per unit, double-buffered)
    if (std::is_same<F, FF16>::value && bpl == 8 && ctx->gemv_f16_rows2) return launch_lds<F, 8, 2>(ctx, a, norm);
    switch (bpl) {
    case 1: return launch_lds<F, 1, 4>(ctx, a, norm);
    case 2: return launch_lds<F, 2, 1>(ctx, a, norm);
    case 3: return launch_lds<F, 3, 2>(ctx, a, norm);
    case 4: return launch_lds<F, 4, 2>(ctx, a, norm);
    case 5: return launch_lds<F, 5, 1>(ctx, a, norm);
    case 6: return launch_lds<F, 6, 1>(ctx, a, norm);
    case 7: return launch_lds<F, 7, 1>(ctx, a, norm);
    default: return launch_lds<F, 8, 1>(ctx, a, norm);
    }
}

template <class F>
int launch_gemv(janus_ctx *ctx, GemvArgs a, int x_dt) {
    bool done = false;
    int e;
    // binary16 x: LDS staging, once per workgroup (short rows), and out of
    // the registers (long rows: more wavefronts per SIMD)
    if (x_dt == JANUS_DT_F16 && ctx->gemv_lds && a.units >= 64) {
        e = launch_lds_fmt<F>(ctx, a, false, false, done);
        if (done || e) return e;
    }
    // binary32 x: the f32 LDS staging, once per workgroup
    if (x_dt == JANUS_DT_F32 && ctx->gemv_lds && a.units >= 64) {
        e = launch_lds32_fmt<F>(ctx, a, false, false, done);
        if (done || e) return e;
    }
    if (x_dt == JANUS_DT_F16) e = launch_reg_fmt<F, _Float16>(ctx, a, done);
    else e = launch_reg_fmt<F, float>(ctx, a, done);
    if (done || e) return e;
    if (x_dt == JANUS_DT_F16) return launch_fmt<F, _Float16, _Float16>(ctx, a);
    return launch_fmt<F, float, float>(ctx, a);
}

// One product of format F: plain products pick the register, LDS or
// per-launch kernel by row length; normalised and paired-row products run
// the LDS kernel. F16 rows with k % 8 != 0 (units == 0) take the scalar kernel.
template <class F>
int gemv_run(janus_ctx *ctx, const GemvArgs &a, int mode, int x_dt, bool *done) {
    *done = true;
    if constexpr (std::is_same<F, FF16>::value) {
        if (a.units == 0) {
            if (mode != janus::GEMV_PLAIN) {
                *done = false;
                return JANUS_OK;
            }
            const uint32_t grid = (a.n + 3) / 4;
            if (x_dt == JANUS_DT_F16)
                hipLaunchKernelGGL(gemv_f16_any_kernel<_Float16>, dim3(grid), dim3(256), 0, ctx->stream, a);
            else
                hipLaunchKernelGGL(gemv_f16_any_kernel<float>, dim3(grid), dim3(256), 0, ctx->stream, a);
            JANUS_LAUNCH_CHECK(ctx);
            return JANUS_OK;
        }
    }
    if (mode == janus::GEMV_PLAIN) return launch_gemv<F>(ctx, a, x_dt);
    if (mode & janus::GEMV_X32)
        return launch_lds32_fmt<F>(ctx, a, (mode & janus::GEMV_NORM) != 0, (mode & janus::GEMV_PAIR) != 0, *done);
    return launch_lds_fmt<F>(ctx, a, (mode & janus::GEMV_NORM) != 0, (mode & janus::GEMV_PAIR) != 0, *done);
}

}  // namespace
