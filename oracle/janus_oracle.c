/*
 * janus_oracle.c -- CPU restatement of the reference decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the CPU
 * baseline of bench.py. Nothing in the product library links or calls it.
 * Compiled with -O2 -ffp-contract=off (see oracle/Makefile) so every
 * binary32 operation rounds where the reference's WGSL source rounds.
 *
 * Reference paths are relative to crates/janus-engine/src/.
 */
#include "janus_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------------------ */
/* binary16                                                                 */
/* ------------------------------------------------------------------------ */

float jo_f16_to_f32_exact(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        float v = ldexpf((float)m, -24);
        return bits_to_f32(f32_to_bits(v) | sign);
    }
    if (e == 31) return bits_to_f32(sign | 0x7f800000u | (m << 13));
    return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

float jo_f16_to_f32_q8(uint16_t h)
{
    /* gemm_q8_0.wgsl:33-60. Subnormal branch: f32(m)/1024 * 2^-14 == m*2^-24
     * exactly; exponent 31 maps to +-1e38 instead of inf/nan. */
    uint32_t e = (h >> 10) & 0x1fu;
    if (e == 31) return (h & 0x8000u) ? -1e38f : 1e38f;
    return jo_f16_to_f32_exact(h);
}

float jo_f16_to_f32_ftz(uint16_t h)
{
    /* gemm_q4_k.wgsl:30-43 */
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h & 0x7c00u) >> 10, m = h & 0x3ffu;
    if (e == 0) return bits_to_f32(s);
    if (e == 31) return bits_to_f32(s | 0x7f800000u | (m << 13));
    return bits_to_f32(s | ((e + 112u) << 23) | (m << 13));
}

uint16_t jo_f32_to_f16_rne(float f)
{
    uint32_t x = f32_to_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                 /* inf / nan */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);   /* quiet nan */
    }
    if (ax >= 0x477ff000u) return sign | 0x7c00u;   /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                 /* normal binary16 result */
        uint32_t e = (ax >> 23) - 112u;      /* rebias 127 -> 15 */
        uint32_t m = ax & 0x7fffffu;
        uint32_t r = (e << 10) | (m >> 13);
        uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1u;  /* carry may bump e */
        return sign | (uint16_t)r;
    }
    /* subnormal (or zero) binary16 result: q = round(|f| / 2^-24) */
    uint32_t E = ax >> 23;
    uint32_t mant = (E == 0) ? (ax & 0x7fffffu) : ((ax & 0x7fffffu) | 0x800000u);
    uint32_t shift = (E == 0) ? 126u : (126u - E);
    if (shift >= 25u) return sign;           /* < 2^-25 (or a tie to even 0) */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return sign | (uint16_t)q;
}

void jo_f32_to_f16_rne_n(const float *in, uint16_t *out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = jo_f32_to_f16_rne(in[i]);
}

void jo_f16_to_f32_n(const uint16_t *in, float *out, size_t n, int mode)
{
    for (size_t i = 0; i < n; ++i)
        out[i] = mode == 0 ? jo_f16_to_f32_exact(in[i])
               : mode == 1 ? jo_f16_to_f32_q8(in[i]) : jo_f16_to_f32_ftz(in[i]);
}

/* ------------------------------------------------------------------------ */
/* dequantisation                                                           */
/* ------------------------------------------------------------------------ */

void jo_dequant_q8_0(const uint8_t *blocks, size_t nblocks, float *out)
{
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = blocks + b * 34;
        float d = jo_f16_to_f32_q8(rd16(blk));
        for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
    }
}

void jo_dequant_q4_0(const uint8_t *blocks, size_t nblocks, float *out)
{
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = blocks + b * 18;
        float d = jo_f16_to_f32_exact(rd16(blk));
        for (int j = 0; j < 16; ++j) {
            out[b * 32 + j] = d * (float)((int)(blk[2 + j] & 15) - 8);
            out[b * 32 + j + 16] = d * (float)((int)(blk[2 + j] >> 4) - 8);
        }
    }
}

void jo_q4_k_scale_min(const uint8_t *q, int j, uint8_t *sc, uint8_t *mn)
{
    /* extract_6bit_from_packed (gemm_q4_k.wgsl:120-147): indices 0..7 are the
     * sub-block scales, 8..15 the mins. */
    if (j < 4) {
        *sc = q[j] & 63u;
        *mn = q[j + 4] & 63u;
    } else {
        *sc = (uint8_t)((q[j + 4] & 15u) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Dequantise one Q4_K super-block exactly as gemm_q4_k.wgsl:82-113 forms w. */
static void q4k_block(const uint8_t *blk, int ftz, float *w /*256*/)
{
    float d = ftz ? jo_f16_to_f32_ftz(rd16(blk)) : jo_f16_to_f32_exact(rd16(blk));
    float dmin = ftz ? jo_f16_to_f32_ftz(rd16(blk + 2)) : jo_f16_to_f32_exact(rd16(blk + 2));
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    for (int j = 0; j < 4; ++j) {
        uint8_t sl, ml, sh, mh;
        jo_q4_k_scale_min(scales, 2 * j, &sl, &ml);
        jo_q4_k_scale_min(scales, 2 * j + 1, &sh, &mh);
        float scale_lo = d * (float)sl, min_lo = dmin * (float)ml;
        float scale_hi = d * (float)sh, min_hi = dmin * (float)mh;
        for (int b = 0; b < 32; ++b) {
            uint8_t byte = qs[32 * j + b];
            w[64 * j + b] = scale_lo * (float)(byte & 15u) - min_lo;
            w[64 * j + 32 + b] = scale_hi * (float)(byte >> 4) - min_hi;
        }
    }
}

void jo_dequant_q4_k(const uint8_t *blocks, size_t nblocks, int ftz, float *out)
{
    for (size_t b = 0; b < nblocks; ++b) q4k_block(blocks + b * 144, ftz, out + b * 256);
}

/* Q5_K, GGML dequantize_row_q5_K: the Q4_K header and element order with a
 * fifth bit per element from qh (bit 2j / 2j+1 of qh[b] for chunk j). */
static void q5k_block(const uint8_t *blk, int ftz, float *w /*256*/)
{
    float d = ftz ? jo_f16_to_f32_ftz(rd16(blk)) : jo_f16_to_f32_exact(rd16(blk));
    float dmin = ftz ? jo_f16_to_f32_ftz(rd16(blk + 2)) : jo_f16_to_f32_exact(rd16(blk + 2));
    const uint8_t *scales = blk + 4, *qh = blk + 16, *qs = blk + 48;
    for (int j = 0; j < 4; ++j) {
        uint8_t sl, ml, sh, mh;
        jo_q4_k_scale_min(scales, 2 * j, &sl, &ml);
        jo_q4_k_scale_min(scales, 2 * j + 1, &sh, &mh);
        float scale_lo = d * (float)sl, min_lo = dmin * (float)ml;
        float scale_hi = d * (float)sh, min_hi = dmin * (float)mh;
        for (int b = 0; b < 32; ++b) {
            uint8_t byte = qs[32 * j + b];
            unsigned lo = (byte & 15u) | (((qh[b] >> (2 * j)) & 1u) << 4);
            unsigned hi = (byte >> 4) | (((qh[b] >> (2 * j + 1)) & 1u) << 4);
            w[64 * j + b] = scale_lo * (float)lo - min_lo;
            w[64 * j + 32 + b] = scale_hi * (float)hi - min_hi;
        }
    }
}

void jo_dequant_q5_k(const uint8_t *blocks, size_t nblocks, int ftz, float *out)
{
    for (size_t b = 0; b < nblocks; ++b) q5k_block(blocks + b * 176, ftz, out + b * 256);
}

void jo_dequant_q6_k(const uint8_t *blocks, size_t nblocks, int ref_order, float *out)
{
    for (size_t bi = 0; bi < nblocks; ++bi) {
        const uint8_t *blk = blocks + bi * 210;
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        float d = jo_f16_to_f32_exact(rd16(blk + 208));
        float *w = out + bi * 256;
        if (ref_order) {
            /* compute/engine.rs:221-241 */
            for (int i = 0; i < 256; ++i) {
                unsigned lo = (i % 2 == 0) ? (ql[i / 2] & 15u) : (ql[i / 2] >> 4);
                unsigned hi = (qh[i / 4] >> (2 * (i % 4))) & 3u;
                int q = (int)((hi << 4) | lo) - 32;
                w[i] = d * (float)sc[i / 16] * (float)q;
            }
            continue;
        }
        for (int h = 0; h < 2; ++h) {
            const uint8_t *l8 = ql + 64 * h, *h8 = qh + 32 * h;
            const int8_t *s8 = sc + 8 * h;
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                int q1 = (int)((l8[l] & 15u) | ((h8[l] & 3u) << 4)) - 32;
                int q2 = (int)((l8[l + 32] & 15u) | (((h8[l] >> 2) & 3u) << 4)) - 32;
                int q3 = (int)((l8[l] >> 4) | (((h8[l] >> 4) & 3u) << 4)) - 32;
                int q4 = (int)((l8[l + 32] >> 4) | (((h8[l] >> 6) & 3u) << 4)) - 32;
                w[128 * h + l] = d * (float)s8[is] * (float)q1;
                w[128 * h + l + 32] = d * (float)s8[is + 2] * (float)q2;
                w[128 * h + l + 64] = d * (float)s8[is + 4] * (float)q3;
                w[128 * h + l + 96] = d * (float)s8[is + 6] * (float)q4;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* matrix-vector products                                                   */
/* ------------------------------------------------------------------------ */

void jo_gemv_q8_0(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k)
{
    uint32_t nb = k / 32;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if ((uint64_t)n * k > (1u << 18))
#endif
    for (long long r = 0; r < (long long)n; ++r) {
        float row = 0.0f;
        for (uint32_t b = 0; b < nb; ++b) {
            const uint8_t *blk = w + ((size_t)r * nb + b) * 34;
            float d = jo_f16_to_f32_q8(rd16(blk));
            float s = 0.0f;
            for (int i = 0; i < 32; ++i) {
                float wv = d * (float)(int8_t)blk[2 + i];
                s += wv * x[b * 32 + i];
            }
            row += s;
        }
        y[r] = row;
    }
}

static float q4_0_row(const uint8_t *row_blocks, const float *x, uint32_t nb)
{
    float row = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = row_blocks + (size_t)b * 18;
        float d = jo_f16_to_f32_exact(rd16(blk));
        float s = 0.0f;
        for (int j = 0; j < 32; ++j) {
            int q = j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4);
            float wv = d * (float)(q - 8);
            s += wv * x[b * 32 + j];
        }
        row += s;
    }
    return row;
}

void jo_gemv_q4_0(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k)
{
    uint32_t nb = k / 32;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if ((uint64_t)n * k > (1u << 18))
#endif
    for (long long r = 0; r < (long long)n; ++r) y[r] = q4_0_row(w + (size_t)r * nb * 18, x, nb);
}

void jo_gemv_q4_0_mt(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k)
{
    uint32_t nb = k / 32;
    long long rows = (long long)n;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (long long r = 0; r < rows; ++r) y[r] = q4_0_row(w + (size_t)r * nb * 18, x, nb);
}

int jo_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void jo_gemv_q5_k(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k, int ftz)
{
    uint32_t nb = k / 256;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if ((uint64_t)n * k > (1u << 18))
#endif
    for (long long r = 0; r < (long long)n; ++r) {
        float wv[256];
        float row = 0.0f;
        for (uint32_t b = 0; b < nb; ++b) {
            q5k_block(w + ((size_t)r * nb + b) * 176, ftz, wv);
            const float *xv = x + (size_t)b * 256;
            float s = 0.0f;
            for (int j = 0; j < 4; ++j)
                for (int bi = 0; bi < 32; ++bi) {
                    s = s + wv[64 * j + bi] * xv[64 * j + bi];
                    s = s + wv[64 * j + 32 + bi] * xv[64 * j + 32 + bi];
                }
            row += s;
        }
        y[r] = row;
    }
}

void jo_gemv_q4_k(const uint8_t *w, const float *x, float *y, uint32_t n, uint32_t k, int ftz)
{
    uint32_t nb = k / 256;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if ((uint64_t)n * k > (1u << 18))
#endif
    for (long long r = 0; r < (long long)n; ++r) {
        float row = 0.0f;
        for (uint32_t b = 0; b < nb; ++b) {
            const uint8_t *blk = w + ((size_t)r * nb + b) * 144;
            float d = ftz ? jo_f16_to_f32_ftz(rd16(blk)) : jo_f16_to_f32_exact(rd16(blk));
            float dmin = ftz ? jo_f16_to_f32_ftz(rd16(blk + 2)) : jo_f16_to_f32_exact(rd16(blk + 2));
            const uint8_t *scales = blk + 4, *qs = blk + 16;
            const float *xv = x + (size_t)b * 256;
            float s = 0.0f;
            for (int j = 0; j < 4; ++j) {
                uint8_t sl, ml, sh, mh;
                jo_q4_k_scale_min(scales, 2 * j, &sl, &ml);
                jo_q4_k_scale_min(scales, 2 * j + 1, &sh, &mh);
                float scale_lo = d * (float)sl, min_lo = dmin * (float)ml;
                float scale_hi = d * (float)sh, min_hi = dmin * (float)mh;
                for (int bi = 0; bi < 32; ++bi) {
                    uint8_t byte = qs[32 * j + bi];
                    float wl = scale_lo * (float)(byte & 15u) - min_lo;
                    float wh = scale_hi * (float)(byte >> 4) - min_hi;
                    s = s + wl * xv[64 * j + bi];
                    s = s + wh * xv[64 * j + 32 + bi];
                }
            }
            row += s;
        }
        y[r] = row;
    }
}

void jo_gemm_f16(const float *a, const uint16_t *b, float *c, uint32_t batch,
                 uint32_t m, uint32_t k, uint32_t n)
{
    for (uint32_t bi = 0; bi < batch; ++bi)
        for (uint32_t i = 0; i < m; ++i)
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if ((uint64_t)n * k > (1u << 18))
#endif
            for (long long j = 0; j < (long long)n; ++j) {
                const float *arow = a + ((size_t)bi * m + i) * k;
                const uint16_t *brow = b + (size_t)j * k;
                float s = 0.0f;
                for (uint32_t kk = 0; kk < k; ++kk) s = s + arow[kk] * jo_f16_to_f32_ftz(brow[kk]);
                c[((size_t)bi * m + i) * n + j] = s;
            }
}

void jo_gemv_f64(const float *w, const float *x, double *y, uint32_t n, uint32_t k)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if ((uint64_t)n * k > (1u << 18))
#endif
    for (long long r = 0; r < (long long)n; ++r) {
        double s = 0.0;
        for (uint32_t i = 0; i < k; ++i) s += (double)w[(size_t)r * k + i] * (double)x[i];
        y[r] = s;
    }
}

/* ------------------------------------------------------------------------ */
/* glue                                                                     */
/* ------------------------------------------------------------------------ */

void jo_rmsnorm(const float *in, float *out, const float *gamma, uint32_t batch,
                uint32_t hidden, float eps)
{
    float part[256];
    for (uint32_t b = 0; b < batch; ++b) {
        const float *x = in + (size_t)b * hidden;
        for (uint32_t t = 0; t < 256; ++t) {
            float acc = 0.0f;
            for (uint32_t i = t; i < hidden; i += 256) acc = acc + x[i] * x[i];
            part[t] = acc;
        }
        for (uint32_t stride = 128; stride > 0; stride /= 2)
            for (uint32_t t = 0; t < stride; ++t) part[t] = part[t] + part[t + stride];
        float rms = sqrtf(part[0] / (float)hidden + eps);
        for (uint32_t i = 0; i < hidden; ++i) out[(size_t)b * hidden + i] = (x[i] / rms) * gamma[i];
    }
}

void jo_silu(const float *in, float *out, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        float x = in[i];
        out[i] = x * (1.0f / (1.0f + expf(-x)));
    }
}

void jo_mul(const float *a, const float *b, float *out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

void jo_add(const float *a, const float *b, float *out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

void jo_rope_table(float *table, uint32_t max_seq, uint32_t head_dim, float theta_base)
{
    uint32_t half = head_dim / 2;
    for (uint32_t p = 0; p < max_seq; ++p)
        for (uint32_t i = 0; i < half; ++i) {
            float exponent = (float)(2 * i) / (float)head_dim;
            float theta = powf(theta_base, exponent);
            float angle = (float)p / theta;
            table[((size_t)p * half + i) * 2] = cosf(angle);
            table[((size_t)p * half + i) * 2 + 1] = sinf(angle);
        }
}

void jo_rope(const float *in, float *out, const float *table, uint32_t batch,
             uint32_t heads, uint32_t head_dim, uint32_t position)
{
    uint32_t half = head_dim / 2;
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t h = 0; h < heads; ++h)
            for (uint32_t i = 0; i < half; ++i) {
                size_t base = ((size_t)b * heads + h) * head_dim;
                float x0 = in[base + i], x1 = in[base + i + half];
                float c = table[((size_t)position * half + i) * 2];
                float s = table[((size_t)position * half + i) * 2 + 1];
                out[base + i] = x0 * c - x1 * s;
                out[base + i + half] = x0 * s + x1 * c;
            }
}

void jo_attention(const float *q, const float *k, const float *v, float *out,
                  uint32_t len, uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                  float scale)
{
    float *sc = (float *)malloc(sizeof(float) * (len ? len : 1));
    size_t pos_stride = (size_t)kv_heads * head_dim;
    for (uint32_t h = 0; h < heads; ++h) {
        uint32_t kvh = (h * kv_heads) / heads;          /* attention.wgsl:243 */
        const float *qh = q + (size_t)h * head_dim;
        for (uint32_t p = 0; p < len; ++p) {
            const float *kp = k + p * pos_stride + (size_t)kvh * head_dim;
            float dot = 0.0f;
            for (uint32_t d = 0; d < head_dim; ++d) dot += qh[d] * kp[d];
            sc[p] = dot * scale;
        }
        /* softmax.wgsl:30-50 */
        float mx = -999999.0f;
        for (uint32_t p = 0; p < len; ++p) if (sc[p] > mx) mx = sc[p];
        float sum = 0.0f;
        for (uint32_t p = 0; p < len; ++p) { sc[p] = expf(sc[p] - mx); sum = sum + sc[p]; }
        float safe = sum > 1e-20f ? sum : 1e-20f;
        for (uint32_t p = 0; p < len; ++p) sc[p] = sc[p] / safe;
        /* attention.wgsl:172-181 */
        for (uint32_t d = 0; d < head_dim; ++d) {
            float acc = 0.0f;
            for (uint32_t p = 0; p < len; ++p)
                acc += sc[p] * v[p * pos_stride + (size_t)kvh * head_dim + d];
            out[(size_t)h * head_dim + d] = acc;
        }
    }
    free(sc);
}

int jo_embed(const uint16_t *table, const uint32_t *ids, float *out, uint32_t batch,
             uint32_t hidden, uint32_t vocab)
{
    for (uint32_t b = 0; b < batch; ++b)
        if (ids[b] >= vocab) return -1;
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t i = 0; i < hidden; ++i)
            out[(size_t)b * hidden + i] = jo_f16_to_f32_ftz(table[(size_t)ids[b] * hidden + i]);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* sampling                                                                 */
/* ------------------------------------------------------------------------ */

void jo_repetition_penalty(float *logits, uint32_t vocab, const uint32_t *ctx, size_t nctx,
                           float penalty)
{
    for (size_t i = 0; i < nctx; ++i) {
        uint32_t t = ctx[i];
        if (t < vocab) {
            if (logits[t] > 0.0f) logits[t] /= penalty;
            else logits[t] *= penalty;
        }
    }
}

uint32_t jo_argmax_last(const float *logits, uint32_t vocab)
{
    /* fold(first, |x, y| if x > y { x } else { y }) */
    if (vocab == 0) return 0;
    uint32_t best = 0;
    for (uint32_t i = 1; i < vocab; ++i)
        if (!(logits[best] > logits[i])) best = i;
    return best;
}

uint32_t jo_argmax_wgsl(const float *logits, uint32_t vocab)
{
    float val[256];
    uint32_t idx[256];
    for (uint32_t t = 0; t < 256; ++t) {
        float mv = -1e38f;
        uint32_t mi = 0;
        for (uint32_t i = t; i < vocab; i += 256)
            if (logits[i] > mv) { mv = logits[i]; mi = i; }
        val[t] = mv;
        idx[t] = mi;
    }
    for (uint32_t stride = 128; stride >= 2; stride /= 2)
        for (uint32_t t = 0; t < stride; ++t)
            if (val[t + stride] > val[t]) { val[t] = val[t + stride]; idx[t] = idx[t + stride]; }
    return val[1] > val[0] ? idx[1] : idx[0];
}
