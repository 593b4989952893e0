// smallm.hip -- products with 2..64 activation rows (ragged decode batches):
// the dequant-fused fp16 MFMA GEMM.
//
// Replaces the reference's M>1 quantised path, which hands quantised bytes
// to the f16 GEMM (crates/janus-engine/src/compute/ops/quantized.rs:77-90,
// 104-117, 131-144; shaders/gemm.wgsl) and so has no correct result to match;
// parity is "equal to M stacked GEMVs" within fp32 accumulation tolerance.
//
// Weight tiles ("T32", built once per weight on first use from the GEMV
// layout): rows are grouped by 32 and K by chunks; for row group g and chunk c
// the 64 lanes of a wavefront each load 16 contiguous bytes (1 KiB per
// wavefront load) that are already the lane's B operand of
// v_mfma_f32_32x32x16_f16: lane l holds weight row 32g + (l % 32) and the
// K-half h = l / 32 of each 16-wide MFMA step.
//   Q4_0 / Q4_K: chunk = 64 K (two 32-element blocks). Per block two words:
//     elements 8h..8h+7 and 16+8h..16+8h+7, nibbles stored in the order
//     e0,e2,e4,e6,e1,e3,e5,e7 so that (w >> 4t) & 0x000f000f yields the
//     natural pair (e_2t, e_2t+1) as binary16 1024 + q.
//     Q4_0 side data: [g][c][32] u32 = the two blocks' binary16 scales.
//     Q4_K side data: [g][super-block][32] 16-byte headers as uploaded (d,
//     dmin, scale fields of kq_group).
//   Q5_K: as Q4_K (nibbles and headers), plus the fifth bits: one word per
//     lane and chunk [g][c][64], bit 4 * slot + i for the element in nibble
//     slot `slot` of the lane's word i (176 bytes per 256 weights, the GGUF
//     size).
//   Q8_0: chunk = 32 K (one block): bytes of elements 8h..8h+7 then
//     16+8h..16+8h+7; side data [g][c][32] binary16 scales.
//   F16: chunk = 16 K: the eight binary16 weights 8h..8h+7 of the chunk.
// Padding rows and K are zero (zero scale), so they add nothing.
//
// Kernel: a workgroup is 16 wavefronts, 4 K slices of 4 consecutive row groups
// (128 weight rows), over a range of K "passes". Per pass the activations
// A[rows][kr] (binary16) are staged in LDS once and shared by all wavefronts;
// each wavefront streams the weight chunks of its row group and K slice with 128-bit non-temporal loads,
// unpacks them in registers into exact binary16 integers, runs
// 32x32x16 MFMAs with fp32 accumulation per quantisation block, and applies
// the block scale to the fp32 block result (so products and scales round
// exactly as the M=1 kernels do). The K slices of a row group are added in
// slice order through LDS at the end. When there are too few row tiles to fill
// the GPU, K is split over workgroups; the partial tiles go to a workspace
// and a second kernel adds them in fixed split order, so results do not
// depend on scheduling.
#include "internal.h"

namespace janus {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));

constexpr int WAVES = 4;   // row groups per workgroup

__device__ __forceinline__ jh2 as_h2(uint32_t u) { return __builtin_bit_cast(jh2, u); }

// 8 permuted nibbles -> 8 binary16 (1024 + q) - off, natural element order.
// Slots 0/4 and 2/6 (mask 0x000f000f) become 1024 + q; slots 1/5 and 3/7
// (mask 0x00f000f0) become 1024 + 16 q, scaled back exactly by one FMA
// ((1024 + 16 q) / 16 - 64 - (off - 1024) = q - (off - 1024)). The magic
// exponent sits in a VGPR so each mask-and-merge is one v_and_or_b32.
__device__ __forceinline__ h8 unpack_nib8(uint32_t u, _Float16 off) {
    const jh2 o = {off, off};
    const jh2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const _Float16 cb = (_Float16)(960.0f - (float)off);
    const jh2 c = {cb, cb};
    const uint32_t m = vgpr_const_6400();
    const uint32_t u8 = u >> 8;
    const jh2 p0 = as_h2((u & 0x000f000fu) | m) - o;
    const jh2 p1 = __builtin_elementwise_fma(as_h2((u & 0x00f000f0u) | m), s16, c);
    const jh2 p2 = as_h2((u8 & 0x000f000fu) | m) - o;
    const jh2 p3 = __builtin_elementwise_fma(as_h2((u8 & 0x00f000f0u) | m), s16, c);
    return (h8){p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// unpack_nib8 with off = 1024 for 5-bit values: the fifth bits of the word's
// 8 elements (Q5_K layout above, word I of the lane) are OR-ed into the
// binary16 mantissas: bit 4 of 1024 + q (slots 0/4, 2/6) or bit 8 of
// 1024 + 16 q (slots 1/5, 3/7), so the values are q in 0..31, exact.
template <int I>
__device__ __forceinline__ h8 unpack_nib8_q5(uint32_t u, uint32_t fifth) {
    const jh2 o = {(_Float16)1024.0f, (_Float16)1024.0f};
    const jh2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const jh2 c = {(_Float16)-64.0f, (_Float16)-64.0f};
    const uint32_t m = vgpr_const_6400();
    const uint32_t u8 = u >> 8;
    const uint32_t ta = fifth << (4 - I), tb = fifth >> (4 + I);   // slot s of word I -> bit 4 s + 4, 4 s - 4
    const jh2 p0 = as_h2((u & 0x000f000fu) | m | (ta & 0x00100010u)) - o;
    const jh2 p1 = __builtin_elementwise_fma(as_h2((u & 0x00f000f0u) | m | (ta & 0x01000100u)), s16, c);
    const jh2 p2 = as_h2((u8 & 0x000f000fu) | m | (tb & 0x00100010u)) - o;
    const jh2 p3 = __builtin_elementwise_fma(as_h2((u8 & 0x00f000f0u) | m | (tb & 0x01000100u)), s16, c);
    return (h8){p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// 8 int8 (two words) -> 8 binary16 integers, natural order.
__device__ __forceinline__ h8 unpack_i8x8(uint32_t lo, uint32_t hi) {
    const jh2 o = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t c64 = 0x64646464u;
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
    jh2 p0 = as_h2(__builtin_amdgcn_perm(lo, c64, 0x00050004u)) - o;
    jh2 p1 = as_h2(__builtin_amdgcn_perm(lo, c64, 0x00070006u)) - o;
    jh2 p2 = as_h2(__builtin_amdgcn_perm(hi, c64, 0x00050004u)) - o;
    jh2 p3 = as_h2(__builtin_amdgcn_perm(hi, c64, 0x00070006u)) - o;
    return (h8){p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

__device__ __forceinline__ f16x mfma(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h8 lds_h8(const _Float16 *p) { return *(const h8 *)p; }

struct GemmArgs {
    const uint8_t *qs;     // T32 quant chunks [G][C][64][16 B]
    const uint8_t *side;   // T32 side data (scales / headers)
    const uint32_t *q5h;   // Q5_K fifth bits [G][C][64]
    const _Float16 *a;     // activations [rows][k]
    void *c;               // output [rows][n]
    const float *resid;    // [rows][n] or null (may alias c)
    float *ws;             // split-K partials [ksplit][Mpad][Npad]
    uint32_t rows, n, k;
    uint32_t chunks;       // C: chunks per row group
    uint32_t pass_chunks;  // chunks per LDS pass
    uint32_t passes_per_wg;
    uint32_t total_passes;
    uint32_t ksplit;
    uint32_t pitch;        // LDS row pitch of A, in halves
    int c_f16;
    int to_ws;             // write partials to ws even when ksplit == 1 (epilogue kernels read them)
    uint32_t seg_shift;    // log2 of the 8-half A segments per row of a pass (pass length / 8)
    int swiglu;            // ksplit == 1 only: rows (2j, 2j+1) are (gate_j, up_j); c = silu(gate)*up, binary16 [rows][n/2]
};

// ---- formats ------------------------------------------------------------------
// W: one chunk of one lane. load() reads it; mma() adds its contribution for
// MT M-tiles given the LDS A slice (row stride pitch) at chunk offset kl.

// Block results whose scale is applied one block later: the scale FMAs of a
// block then run while the next block's MFMAs are in flight instead of
// waiting for their own (the same FMAs in the same order).
template <int MT> struct Deferred {
    f16x t[MT];   // the last block's MFMA results
    float d;      // and its scale (0 before the first block)
};

struct GQ4_0 {
    static constexpr int CK = 64;
    static constexpr bool DEFER = true;
    struct W { uint4 q; uint32_t s; };
    // g and c are wavefront-uniform: the chunk base is scalar, the lane adds
    // a 32-bit offset
    __device__ static W load(const GemmArgs &a, uint32_t g, uint32_t c, int lane) {
        const size_t ch = (size_t)g * a.chunks + c;
        W w;
        w.q = ld_stream(a.qs + ch * 1024 + (uint32_t)lane * 16u);
        w.s = *(const uint32_t *)(a.side + ch * 128 + (uint32_t)(lane & 31) * 4u);
        return w;
    }
    template <int MT>
    __device__ static void mma_deferred(const W &w, const _Float16 *As, uint32_t pitch, uint32_t kl, int lane,
                                        f16x (&acc)[MT], Deferred<MT> &pend) {
        const int h = lane >> 5, r = lane & 31;
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const h8 b0 = unpack_nib8(q[2 * b], (_Float16)1032.0f);
            const h8 b1 = unpack_nib8(q[2 * b + 1], (_Float16)1032.0f);
            const float d = h2f((uint16_t)(b ? (w.s >> 16) : (w.s & 0xffffu)));
            f16x t[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const _Float16 *ap = As + (size_t)(mt * 32 + r) * pitch + kl + b * 32 + 8 * h;
                t[mt] = mfma(lds_h8(ap), b0, (f16x){});
                t[mt] = mfma(lds_h8(ap + 16), b1, t[mt]);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[mt][v] = fmaf(pend.d, pend.t[mt][v], acc[mt][v]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) pend.t[mt] = t[mt];
            pend.d = d;
        }
    }
    template <int MT>
    __device__ static void mma(const W &w, const _Float16 *As, uint32_t pitch, uint32_t kl, int lane,
                               const float *, uint32_t, f16x (&acc)[MT]) {
        const int h = lane >> 5, r = lane & 31;
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const h8 b0 = unpack_nib8(q[2 * b], (_Float16)1032.0f);
            const h8 b1 = unpack_nib8(q[2 * b + 1], (_Float16)1032.0f);
            const float d = h2f((uint16_t)(b ? (w.s >> 16) : (w.s & 0xffffu)));
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const _Float16 *ap = As + (size_t)(mt * 32 + r) * pitch + kl + b * 32 + 8 * h;
                f16x t = mfma(lds_h8(ap), b0, (f16x){});
                t = mfma(lds_h8(ap + 16), b1, t);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[mt][v] = fmaf(d, t[v], acc[mt][v]);
            }
        }
    }
};

struct GQ8_0 {
    static constexpr int CK = 32;
    struct W { uint4 q; uint16_t s; };
    __device__ static W load(const GemmArgs &a, uint32_t g, uint32_t c, int lane) {
        const size_t ch = (size_t)g * a.chunks + c;
        W w;
        w.q = ld_stream(a.qs + (ch * 64 + lane) * 16);
        w.s = ((const uint16_t *)a.side)[ch * 32 + (lane & 31)];
        return w;
    }
    template <int MT>
    __device__ static void mma(const W &w, const _Float16 *As, uint32_t pitch, uint32_t kl, int lane,
                               const float *, uint32_t, f16x (&acc)[MT]) {
        const int h = lane >> 5, r = lane & 31;
        const h8 b0 = unpack_i8x8(w.q.x, w.q.y);
        const h8 b1 = unpack_i8x8(w.q.z, w.q.w);
        const float d = h2f_q8(w.s);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const _Float16 *ap = As + (size_t)(mt * 32 + r) * pitch + kl + 8 * h;
            f16x t = mfma(lds_h8(ap), b0, (f16x){});
            t = mfma(lds_h8(ap + 16), b1, t);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[mt][v] = fmaf(d, t[v], acc[mt][v]);
        }
    }
};

// Q4_K: w = (d*sc)*q - dmin*m per 32-element sub-block (shaders/gemm_q4_k.wgsl:82-113);
// the m term uses the per-(row, sub-block) activation sums staged in LDS.
struct GQ4_K {
    static constexpr int CK = 64;
    struct W { uint4 q; uint4 hdr; };
    __device__ static W load(const GemmArgs &a, uint32_t g, uint32_t c, int lane) {
        const size_t ch = (size_t)g * a.chunks + c;
        W w;
        w.q = ld_stream(a.qs + (ch * 64 + lane) * 16);
        const size_t sb = (size_t)g * (a.chunks / 4) + c / 4;
        w.hdr = *(const uint4 *)(a.side + (sb * 32 + (lane & 31)) * 16);
        return w;
    }
    // (sc, m) of sub-block `sub` (uniform) from the packed scale words hdr.y..w
    __device__ static void scale_min(const uint4 &hdr, int sub, float &sc, float &mn) {
        const uint32_t g = kq_group(hdr.y, hdr.z, hdr.w, (uint32_t)sub >> 1), o = 6u * (uint32_t)(sub & 1);
        sc = (float)((g >> o) & 63u);
        mn = (float)((g >> (12u + o)) & 63u);
    }
    template <int MT>
    __device__ static void mma(const W &w, const _Float16 *As, uint32_t pitch, uint32_t kl, int lane,
                               const float *Ss, uint32_t sub0, f16x (&acc)[MT]) {
        const int h = lane >> 5, r = lane & 31;
        const uint32_t q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        const float d = h2f((uint16_t)(w.hdr.x & 0xffffu)), dmin = h2f((uint16_t)(w.hdr.x >> 16));
        const int j = (int)((kl / 64 + sub0 / 2) & 3);   // chunk index within the super-block
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float sc, mn;
            scale_min(w.hdr, 2 * j + b, sc, mn);
            const float ds = d * sc, dm = dmin * mn;
            const h8 b0 = unpack_nib8(q[2 * b], (_Float16)1024.0f);
            const h8 b1 = unpack_nib8(q[2 * b + 1], (_Float16)1024.0f);
            const uint32_t sub = kl / 32 + b;   // sub-block index within the pass
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const _Float16 *ap = As + (size_t)(mt * 32 + r) * pitch + kl + b * 32 + 8 * h;
                f16x t = mfma(lds_h8(ap), b0, (f16x){});
                t = mfma(lds_h8(ap + 16), b1, t);
                const float *sx = Ss + (size_t)sub * (MT * 32) + mt * 32 + 4 * h;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const jf4 s4 = *(const jf4 *)(sx + 8 * jj);
                    acc[mt][4 * jj + 0] = fmaf(-dm, s4.x, fmaf(ds, t[4 * jj + 0], acc[mt][4 * jj + 0]));
                    acc[mt][4 * jj + 1] = fmaf(-dm, s4.y, fmaf(ds, t[4 * jj + 1], acc[mt][4 * jj + 1]));
                    acc[mt][4 * jj + 2] = fmaf(-dm, s4.z, fmaf(ds, t[4 * jj + 2], acc[mt][4 * jj + 2]));
                    acc[mt][4 * jj + 3] = fmaf(-dm, s4.w, fmaf(ds, t[4 * jj + 3], acc[mt][4 * jj + 3]));
                }
            }
        }
    }
};

// Q5_K (GGML block_q5_K): the Q4_K tiles (nibbles, 16-byte headers) plus the
// fifth bits of the lane's 32 elements in one word per chunk; w = (d*sc)*q -
// dmin*m with q in 0..31, the m term from the staged activation sums.
struct GQ5_K {
    static constexpr int CK = 64;
    struct W { uint4 q; uint4 hdr; uint32_t fifth; };
    __device__ static W load(const GemmArgs &a, uint32_t g, uint32_t c, int lane) {
        const size_t ch = (size_t)g * a.chunks + c;
        W w;
        w.q = ld_stream(a.qs + (ch * 64 + lane) * 16);
        w.fifth = __builtin_nontemporal_load(a.q5h + ch * 64 + lane);
        const size_t sb = (size_t)g * (a.chunks / 4) + c / 4;
        w.hdr = *(const uint4 *)(a.side + (sb * 32 + (lane & 31)) * 16);
        return w;
    }
    template <int MT>
    __device__ static void mma(const W &w, const _Float16 *As, uint32_t pitch, uint32_t kl, int lane,
                               const float *Ss, uint32_t sub0, f16x (&acc)[MT]) {
        const int h = lane >> 5, r = lane & 31;
        const float d = h2f((uint16_t)(w.hdr.x & 0xffffu)), dmin = h2f((uint16_t)(w.hdr.x >> 16));
        const int j = (int)((kl / 64 + sub0 / 2) & 3);   // chunk index within the super-block
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float sc, mn;
            GQ4_K::scale_min(w.hdr, 2 * j + b, sc, mn);
            const float ds = d * sc, dm = dmin * mn;
            const h8 b0 = b == 0 ? unpack_nib8_q5<0>(w.q.x, w.fifth) : unpack_nib8_q5<2>(w.q.z, w.fifth);
            const h8 b1 = b == 0 ? unpack_nib8_q5<1>(w.q.y, w.fifth) : unpack_nib8_q5<3>(w.q.w, w.fifth);
            const uint32_t sub = kl / 32 + b;   // sub-block index within the pass
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const _Float16 *ap = As + (size_t)(mt * 32 + r) * pitch + kl + b * 32 + 8 * h;
                f16x t = mfma(lds_h8(ap), b0, (f16x){});
                t = mfma(lds_h8(ap + 16), b1, t);
                const float *sx = Ss + (size_t)sub * (MT * 32) + mt * 32 + 4 * h;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const jf4 s4 = *(const jf4 *)(sx + 8 * jj);
                    acc[mt][4 * jj + 0] = fmaf(-dm, s4.x, fmaf(ds, t[4 * jj + 0], acc[mt][4 * jj + 0]));
                    acc[mt][4 * jj + 1] = fmaf(-dm, s4.y, fmaf(ds, t[4 * jj + 1], acc[mt][4 * jj + 1]));
                    acc[mt][4 * jj + 2] = fmaf(-dm, s4.z, fmaf(ds, t[4 * jj + 2], acc[mt][4 * jj + 2]));
                    acc[mt][4 * jj + 3] = fmaf(-dm, s4.w, fmaf(ds, t[4 * jj + 3], acc[mt][4 * jj + 3]));
                }
            }
        }
    }
};

// formats whose block scales are applied one block late (mma_deferred)
template <class F, class = void> struct Defers { static constexpr bool value = false; };
template <class F> struct Defers<F, std::void_t<decltype(F::DEFER)>> { static constexpr bool value = F::DEFER; };

template <int MT>
__device__ __forceinline__ void flush_deferred(f16x (&acc)[MT], const Deferred<MT> &pend) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[mt][v] = fmaf(pend.d, pend.t[mt][v], acc[mt][v]);
}

// formats whose mins need the per-(row, sub-block) activation sums in LDS
template <class F> struct NeedsSums { static constexpr bool value = false; };
template <> struct NeedsSums<GQ4_K> { static constexpr bool value = true; };
template <> struct NeedsSums<GQ5_K> { static constexpr bool value = true; };

struct GF16 {
    static constexpr int CK = 16;
    struct W { uint4 q; };
    __device__ static W load(const GemmArgs &a, uint32_t g, uint32_t c, int lane) {
        const size_t ch = (size_t)g * a.chunks + c;
        W w;
        w.q = ld_stream(a.qs + (ch * 64 + lane) * 16);
        return w;
    }
    template <int MT>
    __device__ static void mma(const W &w, const _Float16 *As, uint32_t pitch, uint32_t kl, int lane,
                               const float *, uint32_t, f16x (&acc)[MT]) {
        const int h = lane >> 5, r = lane & 31;
        const h8 b = __builtin_bit_cast(h8, w.q);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma(lds_h8(As + (size_t)(mt * 32 + r) * pitch + kl + 8 * h), b, acc[mt]);
    }
};

// chunks per weight batch (two batches in flight per wavefront)
template <class F> struct Stage { static constexpr int PD = std::is_same<F, GQ4_0>::value ? 2 : (F::CK == 64 ? 4 : 8); };

// Output element (m, n) of wave-tile value v for lane (32x32 MFMA C layout):
// n = lane % 32, m = 8 * (v / 4) + 4 * (lane / 32) + v % 4.
__device__ __forceinline__ uint32_t out_row(int mt, int v, int lane) {
    return (uint32_t)(mt * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3));
}

template <int MT>
__device__ __forceinline__ void store_tile(const GemmArgs &a, uint32_t g, int lane, const f16x (&acc)[MT]) {
    const uint32_t n = g * 32 + (lane & 31);
    if (n >= a.n) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t m = out_row(mt, v, lane);
            if (m < a.rows) {
                float val = acc[mt][v];
                const size_t at = (size_t)m * a.n + n;
                if (a.resid) val += a.resid[at];
                if (a.c_f16) ((uint16_t *)a.c)[at] = f2h_bits(val);
                else ((float *)a.c)[at] = val;
            }
        }
}

// SwiGLU store of a finished tile: columns 2j, 2j+1 (lanes l, l^1) hold gate_j
// and up_j of the same rows; the even lane writes silu(gate) * up as binary16
// (the arithmetic of elementwise_kernel's SwiGLU).
template <int MT>
__device__ __forceinline__ void store_swiglu(const GemmArgs &a, uint32_t g, int lane, const f16x (&acc)[MT]) {
    const uint32_t n = g * 32 + (lane & 31);
    const uint32_t half = a.n / 2;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float mine = acc[mt][v];
            const float other = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mine), 0xb1, 0xf, 0xf, false));
            const uint32_t m = out_row(mt, v, lane);
            if (!(lane & 1) && m < a.rows && n + 1 < a.n) {
                const float act = mine * (1.0f / (1.0f + expf(-mine))) * other;
                ((uint16_t *)a.c)[(size_t)m * half + n / 2] = f2h_bits(act);
            }
        }
}

// KW wavefronts per row group, each on a K slice of the pass (4 where the
// format's registers fit 4 wavefronts per SIMD, else 2).
// SPT: 16-byte A segments per thread per pass, Mpad * kr / 8 / (256 * KW).
template <class F, int MT, int KW, int SPT, int PD = Stage<F>::PD>
__global__ __launch_bounds__(64 * WAVES * KW) void gemm_mfma_kernel(GemmArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr bool SUMS = NeedsSums<F>::value;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar chunk bases
    const int rgw = wave % WAVES, kw = wave / WAVES;   // row group in the tile, K slice of the pass
    const uint32_t G = (a.n + 31) / 32;
    const uint32_t tile = blockIdx.x, ks = blockIdx.y;
    const uint32_t g = tile * WAVES + rgw;
    const bool active = g < G;
    const uint32_t Mpad = MT * 32;
    _Float16 *As = (_Float16 *)smem;
    float *Ss = (float *)(smem + (size_t)Mpad * a.pitch * 2);

    f16x acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = (f16x){};
    Deferred<MT> pend;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) pend.t[mt] = (f16x){};
    pend.d = 0.0f;

    const uint32_t cpk = a.pass_chunks / KW;   // chunks per K slice
    const uint32_t p_begin = ks * a.passes_per_wg;
    const uint32_t p_end = min(a.total_passes, p_begin + a.passes_per_wg);
    for (uint32_t p = p_begin; p < p_end; ++p) {
        const uint32_t c0 = p * a.pass_chunks, c1 = min(a.chunks, c0 + a.pass_chunks);
        const uint32_t m0 = min(c1, c0 + kw * cpk), m1 = min(c1, m0 + cpk);   // this wave's chunks
        typename F::W wa[PD], wb[PD];
        auto load = [&](typename F::W (&w)[PD], uint32_t cs) {
#pragma unroll
            for (int i = 0; i < PD; ++i)
                if (cs + i < m1) w[i] = F::load(a, g, cs + i, lane);
        };
        if (active) load(wa, m0);   // in flight while A is staged

        // stage A[0..Mpad)[c0*CK .. c0*CK + kr) as binary16, zero outside rows / k:
        // segment s (8 halves) is row s >> seg_shift, column (s & mask) * 8 of the
        // full pass width (a power of two), so no division; every thread issues
        // all of its 16-byte loads before its LDS stores
        const uint32_t kbase = c0 * F::CK;
        const uint32_t smask = (1u << a.seg_shift) - 1u;
        uint4 sv[SPT];
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const uint32_t s = threadIdx.x + 64u * WAVES * KW * i;
            const uint32_t m = s >> a.seg_shift, col = kbase + (s & smask) * 8;
            sv[i] = make_uint4(0u, 0u, 0u, 0u);
            if (m < a.rows && col < a.k) sv[i] = *(const uint4 *)(a.a + (size_t)m * a.k + col);
        }
        __syncthreads();   // the previous pass is done with LDS
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const uint32_t s = threadIdx.x + 64u * WAVES * KW * i;
            if ((s >> a.seg_shift) < Mpad) *(uint4 *)(As + (size_t)(s >> a.seg_shift) * a.pitch + (s & smask) * 8) = sv[i];
        }
        if (SUMS) {
            __syncthreads();
            const uint32_t nsub = (c1 - c0) * F::CK / 32;
            for (uint32_t i = threadIdx.x; i < nsub * Mpad; i += 64u * WAVES * KW) {
                const uint32_t sub = i / Mpad, m = i % Mpad;
                const _Float16 *p8 = As + (size_t)m * a.pitch + sub * 32;
                float s = 0.0f;
#pragma unroll
                for (int t = 0; t < 32; ++t) s += (float)p8[t];
                Ss[i] = s;
            }
        }
        __syncthreads();
        if (!active) continue;

        auto compute = [&](typename F::W (&w)[PD], uint32_t cs) {
#pragma unroll
            for (int i = 0; i < PD; ++i)
                if (cs + i < m1) {
                    if constexpr (Defers<F>::value)
                        F::template mma_deferred<MT>(w[i], As, a.pitch, (cs + i - c0) * F::CK, lane, acc, pend);
                    else
                        F::template mma<MT>(w[i], As, a.pitch, (cs + i - c0) * F::CK, lane, Ss, 0, acc);
                }
        };
        uint32_t cs = m0;
        for (; cs + PD < m1; cs += 2 * PD) {
            load(wb, cs + PD);
            compute(wa, cs);
            if (cs + 2 * PD < m1) load(wa, cs + 2 * PD);
            compute(wb, cs + PD);
        }
        if (cs < m1) compute(wa, cs);
    }
    if constexpr (Defers<F>::value) flush_deferred<MT>(acc, pend);

    // add the K slices of each row group in slice order (LDS, reusing the A area)
    if (KW > 1) {
        float *red = (float *)smem;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            __syncthreads();
#pragma unroll
            for (int v = 0; v < 16; ++v) red[((size_t)wave * 16 + v) * 64 + lane] = acc[mt][v];
            __syncthreads();
            if (kw == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    float sum = red[((size_t)rgw * 16 + v) * 64 + lane];
                    for (int j = 1; j < KW; ++j) sum += red[((size_t)(j * WAVES + rgw) * 16 + v) * 64 + lane];
                    acc[mt][v] = sum;
                }
            }
        }
    }
    if (kw != 0 || !active) return;
    if (a.ksplit == 1 && !a.to_ws) {
        if (a.swiglu) store_swiglu<MT>(a, g, lane, acc);
        else store_tile<MT>(a, g, lane, acc);
        return;
    }
    // split-K: this split's tile goes to the workspace; gemm_reduce_kernel adds
    // the splits in order (the kernel boundary makes the partials visible)
    const uint32_t Npad = G * 32, n = g * 32 + (lane & 31);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v)
            __builtin_nontemporal_store(acc[mt][v], a.ws + ((size_t)ks * Mpad + out_row(mt, v, lane)) * Npad + n);
}

// Sums the split-K partials in split order and applies the epilogue.
// Cross-pass pipelined form of gemm_mfma_kernel (quantised and F16 weights),
// with the pass length KR fixed at compile time. A is double-buffered in LDS:
// the activations of pass p + 1 are requested while pass p computes and are
// stored at its end; each wavefront keeps one pass of weight chunks in
// registers and requests chunk i of the next pass as soon as chunk i of the
// current one is consumed, so a pass's weights are in flight during the
// previous pass and the barrier between them. One barrier per pass (two for
// Q4_K, whose activation sums are built from the staged pass). Products,
// scale rounding, slice order and outputs are those of gemm_mfma_kernel.
template <class F, int MT, int KW, int KR>
__global__ __launch_bounds__(64 * WAVES * KW) void gemm_pipe_kernel(GemmArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr bool SUMS = NeedsSums<F>::value;
    constexpr int NT = 64 * WAVES * KW;   // threads
    constexpr int PC = KR / F::CK;        // chunks per pass
    constexpr int CPW = PC / KW;          // chunks per wavefront per pass
    constexpr int MP = MT * 32;           // padded rows
    constexpr int PITCH = KR + 8;         // LDS row pitch in halves
    constexpr int SEGS = KR / 8;          // 16-byte segments per row of a pass
    constexpr int SPT = MP * SEGS / NT;   // segments per thread
    static_assert(CPW >= 1 && CPW * KW == PC && SPT >= 1 && SPT * NT == MP * SEGS, "pass shape");
    constexpr uint32_t ABYTES = (uint32_t)MP * PITCH * 2;
    constexpr uint32_t BUF = (ABYTES + (SUMS ? (uint32_t)(KR / 32) * MP * 4 : 0u) + 15u) / 16u * 16u;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar chunk bases
    const int rgw = wave % WAVES, kw = wave / WAVES;
    const uint32_t G = (a.n + 31) / 32;
    const uint32_t g = blockIdx.x * WAVES + rgw, ks = blockIdx.y;
    const bool active = g < G;
    const uint32_t p_begin = ks * a.passes_per_wg;
    const uint32_t p_end = min(a.total_passes, p_begin + a.passes_per_wg);

    f16x acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = (f16x){};
    Deferred<MT> pend;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) pend.t[mt] = (f16x){};
    pend.d = 0.0f;
    typename F::W w[CPW];
    uint4 sv[SPT];

    // Every wavefront issues the same sequence of loads whatever the shape
    // (addresses clamped into range, out-of-range A zeroed when stored,
    // inactive wavefronts stream a real row group and discard it), so the
    // compiler's load counters stay exact and no wait covers a later load.
    const uint32_t gl = active ? g : G - 1;
    auto load_a = [&](uint32_t p) {
        const uint32_t kbase = p * KR;
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const uint32_t s = threadIdx.x + NT * i;
            const uint32_t m = min(s / SEGS, a.rows - 1), col = min(kbase + (s % SEGS) * 8, a.k - 8);
            sv[i] = *(const uint4 *)(a.a + (size_t)m * a.k + col);
        }
    };
    auto store_a = [&](uint32_t p) {
        _Float16 *As = (_Float16 *)(smem + (p & 1) * BUF);
        const uint32_t kbase = p * KR;
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const uint32_t s = threadIdx.x + NT * i;
            const bool ok = s / SEGS < a.rows && kbase + (s % SEGS) * 8 < a.k;
            *(uint4 *)(As + (s / SEGS) * PITCH + (s % SEGS) * 8) = ok ? sv[i] : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    // Q4_K: per-(sub-block, row) sums of the staged activations, as gemm_mfma_kernel
    auto sums = [&](uint32_t p) {
        const _Float16 *As = (const _Float16 *)(smem + (p & 1) * BUF);
        float *Ss = (float *)(smem + (p & 1) * BUF + ABYTES);
        const uint32_t c0 = p * PC, c1 = min(a.chunks, c0 + PC);
        const uint32_t n = (c1 - c0) * F::CK / 32 * MP;
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const _Float16 *p8 = As + (i % MP) * PITCH + (i / MP) * 32;
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; ++j) t += (float)p8[j];
            Ss[i] = t;
        }
    };
    // chunk i of this wavefront's slice of pass p (K-tail slots repeat the
    // pass's last chunk and are not computed)
    auto chunk_of = [&](uint32_t p, int i) {
        return min(p * PC + kw * CPW + i, min(a.chunks, (p + 1) * PC) - 1);
    };
    // compute pass p from LDS buffer p & 1; with LOAD, request chunk i of pass
    // p + 1 into slot i as soon as slot i is consumed
    auto pass = [&](uint32_t p, auto load_next) {
        const _Float16 *As = (const _Float16 *)(smem + (p & 1) * BUF);
        const float *Ss = (const float *)(smem + (p & 1) * BUF + ABYTES);
        const uint32_t c1 = min(a.chunks, (p + 1) * PC), m0 = p * PC + kw * CPW;
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            if (m0 + i < c1) {
                if constexpr (Defers<F>::value)
                    F::template mma_deferred<MT>(w[i], As, PITCH, (uint32_t)(kw * CPW + i) * F::CK, lane, acc, pend);
                else
                    F::template mma<MT>(w[i], As, PITCH, (uint32_t)(kw * CPW + i) * F::CK, lane, Ss, 0, acc);
            }
            if (decltype(load_next)::value) w[i] = F::load(a, gl, chunk_of(p + 1, i), lane);
        }
    };

    if (p_begin < p_end) {
        const uint32_t last = p_end - 1;
        load_a(p_begin);
#pragma unroll
        for (int i = 0; i < CPW; ++i) w[i] = F::load(a, gl, chunk_of(p_begin, i), lane);
        store_a(p_begin);
        load_a(min(p_begin + 1, last));
        __syncthreads();
        if (SUMS) {
            sums(p_begin);
            __syncthreads();
        }
        for (uint32_t p = p_begin; p < last; ++p) {
            pass(p, std::true_type{});
            store_a(p + 1);   // that buffer was last read in pass p - 1
            load_a(min(p + 2, last));
            __syncthreads();
            if (SUMS) {
                sums(p + 1);
                __syncthreads();
            }
        }
        pass(last, std::false_type{});
    }
    if constexpr (Defers<F>::value) flush_deferred<MT>(acc, pend);

    if (KW > 1) {
        float *red = (float *)smem;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            __syncthreads();
#pragma unroll
            for (int v = 0; v < 16; ++v) red[((size_t)wave * 16 + v) * 64 + lane] = acc[mt][v];
            __syncthreads();
            if (kw == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    float sum = red[((size_t)rgw * 16 + v) * 64 + lane];
                    for (int j = 1; j < KW; ++j) sum += red[((size_t)(j * WAVES + rgw) * 16 + v) * 64 + lane];
                    acc[mt][v] = sum;
                }
            }
        }
    }
    if (kw != 0 || !active) return;
    if (a.ksplit == 1 && !a.to_ws) {
        if (a.swiglu) store_swiglu<MT>(a, g, lane, acc);
        else store_tile<MT>(a, g, lane, acc);
        return;
    }
    const uint32_t Npad = G * 32, n = g * 32 + (lane & 31);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v)
            __builtin_nontemporal_store(acc[mt][v], a.ws + ((size_t)ks * MP + out_row(mt, v, lane)) * Npad + n);
}

// LDS bytes of gemm_pipe_kernel: two A buffers (with Q4_K sums), at least the
// K-slice reduction area.
template <class F, int MT, int KW, int KR>
constexpr size_t pipe_lds() {
    constexpr size_t abytes = (size_t)MT * 32 * (KR + 8) * 2;
    constexpr size_t buf = (abytes + (NeedsSums<F>::value ? (size_t)(KR / 32) * MT * 32 * 4 : 0) + 15) / 16 * 16;
    constexpr size_t red = (size_t)WAVES * KW * 16 * 64 * 4;
    return 2 * buf > red ? 2 * buf : red;
}

template <class F, int MT, int KW, int KR>
void launch_pipe(janus_ctx *ctx, dim3 grid, const GemmArgs &a) {
    // thread-safe one-time set-up (a function-local static's initialiser)
    static const bool attr_set = [] {
        (void)hipFuncSetAttribute((const void *)gemm_pipe_kernel<F, MT, KW, KR>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        return true;
    }();
    (void)attr_set;
    constexpr size_t lds = pipe_lds<F, MT, KW, KR>();
    hipLaunchKernelGGL((gemm_pipe_kernel<F, MT, KW, KR>), grid, dim3(64 * WAVES * KW), lds, ctx->stream, a);
}

__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmArgs a, uint32_t Mpad) {
    const uint32_t Npad = (a.n + 31) / 32 * 32;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)a.rows * a.n) return;
    const uint32_t m = (uint32_t)(idx / a.n), n = (uint32_t)(idx % a.n);
    const float *p = a.ws + (size_t)m * Npad + n;
    const size_t stride = (size_t)Mpad * Npad;
    // split order; the loads of 8 splits are issued together
    float s = 0.0f;
    for (uint32_t j0 = 0; j0 < a.ksplit; j0 += 8) {
        float u[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) u[jj] = j0 + jj < a.ksplit ? p[(j0 + jj) * stride] : 0.0f;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            if (j0 + jj < a.ksplit) s += u[jj];
    }
    if (a.resid) s += a.resid[idx];
    if (a.c_f16) ((uint16_t *)a.c)[idx] = f2h_bits(s);
    else ((float *)a.c)[idx] = s;
}

// ---- T32 repack (one thread per lane of a chunk) -----------------------------

// Nibble slot of element j (0..7) within a T32 word.
__device__ __forceinline__ uint32_t nib_slot(int j) { return (uint32_t)((j >> 1) + 4 * (j & 1)); }

// Q4_0 / Q4_K word: nibbles nib(j), j = 0..7, in T32 slot order.
template <class GetNib>
__device__ __forceinline__ uint32_t pack_word(GetNib nib) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) w |= (nib(j) & 15u) << (4 * nib_slot(j));
    return w;
}

__global__ void t32_q4_0_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ sc, uint8_t *dq,
                                uint32_t *dside, uint32_t n, uint32_t k, uint32_t G, uint32_t C) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)G * C * 64) return;
    const int lane = (int)(t & 63), h = lane >> 5;
    const size_t ch = t >> 6;
    const uint32_t g = (uint32_t)(ch / C), c = (uint32_t)(ch % C);
    const uint32_t r = g * 32 + (lane & 31), nb = k / 32;
    uint32_t words[4] = {0u, 0u, 0u, 0u};
    uint16_t s[2] = {0, 0};
    for (int b = 0; b < 2; ++b) {
        const uint32_t blk = 2 * c + b;
        if (r >= n || blk >= nb) continue;
        const uint8_t *q = qs + ((size_t)r * nb + blk) * 16;
        words[2 * b] = pack_word([&](int j) { return (uint32_t)(q[8 * h + j] & 15); });
        words[2 * b + 1] = pack_word([&](int j) { return (uint32_t)(q[8 * h + j] >> 4); });
        s[b] = sc[(size_t)r * nb + blk];
    }
    *(uint4 *)(dq + t * 16) = make_uint4(words[0], words[1], words[2], words[3]);
    if (lane < 32) dside[ch * 32 + lane] = (uint32_t)s[0] | ((uint32_t)s[1] << 16);
}

__global__ void t32_q4_k_kernel(const uint8_t *__restrict__ blocks, uint8_t *dq, uint8_t *dside, uint32_t n,
                                uint32_t k, uint32_t G, uint32_t C) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)G * C * 64) return;
    const int lane = (int)(t & 63), h = lane >> 5;
    const size_t ch = t >> 6;
    const uint32_t g = (uint32_t)(ch / C), c = (uint32_t)(ch % C);
    const uint32_t r = g * 32 + (lane & 31), nsb = k / 256, sb = c / 4, j = c % 4;
    uint32_t words[4] = {0u, 0u, 0u, 0u};
    uint4 hdr = {0u, 0u, 0u, 0u};
    if (r < n) {
        const uint8_t *blk = blocks + ((size_t)r * nsb + sb) * 144;
        const uint8_t *q = blk + 16 + 32 * j;
        for (int b = 0; b < 2; ++b) {   // sub-block 2j + b: nibble b of bytes 32j + i
            const int sh = 4 * b;
            words[2 * b] = pack_word([&](int e) { return (uint32_t)(q[8 * h + e] >> sh); });
            words[2 * b + 1] = pack_word([&](int e) { return (uint32_t)(q[16 + 8 * h + e] >> sh); });
        }
        hdr = *(const uint4 *)blk;
    }
    *(uint4 *)(dq + t * 16) = make_uint4(words[0], words[1], words[2], words[3]);
    if (lane < 32 && j == 0) *(uint4 *)(dside + (((size_t)g * (C / 4) + sb) * 32 + lane) * 16) = hdr;
}

__global__ void t32_q5_k_kernel(const uint8_t *__restrict__ blocks, uint8_t *dq, uint8_t *dside, uint32_t *dfifth,
                                uint32_t n, uint32_t k, uint32_t G, uint32_t C) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)G * C * 64) return;
    const int lane = (int)(t & 63), h = lane >> 5;
    const size_t ch = t >> 6;
    const uint32_t g = (uint32_t)(ch / C), c = (uint32_t)(ch % C);
    const uint32_t r = g * 32 + (lane & 31), nsb = k / 256, sb = c / 4, j = c % 4;
    uint32_t words[4] = {0u, 0u, 0u, 0u}, fifth = 0u;
    uint4 hdr = {0u, 0u, 0u, 0u};
    if (r < n) {
        const uint8_t *blk = blocks + ((size_t)r * nsb + sb) * 176, *qs = blk + 48;
        // the upload's fifth-bit words: one per 16-byte quant chunk, bit
        // 8 (t % 4) + t / 4 (+ 4 for the high nibble) for quant byte t
        const uint32_t *qh = (const uint32_t *)(blk + 16);
        for (int b = 0; b < 2; ++b) {   // sub-block 2j + b: nibble b of bytes 32j + E
            for (int w = 0; w < 2; ++w) {
                const int i = 2 * b + w;
                words[i] = pack_word([&](int e) { return (uint32_t)(qs[32 * j + 16 * w + 8 * h + e] >> (4 * b)); });
                for (int e = 0; e < 8; ++e) {
                    const uint32_t tq = (uint32_t)(8 * h + e), pos = 8 * (tq % 4) + tq / 4 + 4 * (uint32_t)b;
                    const uint32_t bit = (qh[2 * j + w] >> pos) & 1u;
                    fifth |= bit << (4 * nib_slot(e) + (uint32_t)i);
                }
            }
        }
        hdr = *(const uint4 *)blk;
    }
    *(uint4 *)(dq + t * 16) = make_uint4(words[0], words[1], words[2], words[3]);
    dfifth[t] = fifth;
    if (lane < 32 && j == 0) *(uint4 *)(dside + (((size_t)g * (C / 4) + sb) * 32 + lane) * 16) = hdr;
}

__global__ void t32_q8_0_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ sc, uint8_t *dq,
                                uint16_t *dside, uint32_t n, uint32_t k, uint32_t G, uint32_t C) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)G * C * 64) return;
    const int lane = (int)(t & 63), h = lane >> 5;
    const size_t ch = t >> 6;
    const uint32_t g = (uint32_t)(ch / C), c = (uint32_t)(ch % C);
    const uint32_t r = g * 32 + (lane & 31), nb = k / 32;
    uint8_t out[16] = {0};
    uint16_t s = 0;
    if (r < n) {
        const uint8_t *q = qs + ((size_t)r * nb + c) * 32;
        for (int e = 0; e < 8; ++e) {
            out[e] = q[8 * h + e];
            out[8 + e] = q[16 + 8 * h + e];
        }
        s = sc[(size_t)r * nb + c];
    }
    uint4 v;
    std::memcpy(&v, out, 16);
    *(uint4 *)(dq + t * 16) = v;
    if (lane < 32) dside[ch * 32 + lane] = s;
}

__global__ void t32_f16_kernel(const uint16_t *__restrict__ src, uint8_t *dq, uint32_t n, uint32_t k, uint32_t G,
                               uint32_t C) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)G * C * 64) return;
    const int lane = (int)(t & 63), h = lane >> 5;
    const size_t ch = t >> 6;
    const uint32_t g = (uint32_t)(ch / C), c = (uint32_t)(ch % C);
    const uint32_t r = g * 32 + (lane & 31);
    uint16_t out[8] = {0};
    if (r < n)
        for (int e = 0; e < 8; ++e) {
            const uint32_t kk = c * 16 + 8 * h + e;
            if (kk < k) out[e] = src[(size_t)r * k + kk];
        }
    uint4 v;
    std::memcpy(&v, out, 16);
    *(uint4 *)(dq + t * 16) = v;
}

uint32_t chunk_k(int type) {
    switch (type) {
    case JANUS_DT_Q4_0: case JANUS_DT_Q4_K: case JANUS_DT_Q5_K: return 64;
    case JANUS_DT_Q8_0: return 32;
    default: return 16;
    }
}

// Builds the weight's T32 copy (device memory, kept with the weight).
int t32_ensure(janus_ctx *ctx, janus_weight *w) {
    if (w->t32) return JANUS_OK;
    const uint32_t G = (w->n + 31) / 32, ck = chunk_k(w->type);
    const uint32_t C = (w->k + ck - 1) / ck;
    const size_t qbytes = (size_t)G * C * 64 * 16;
    size_t side = 0;
    if (w->type == JANUS_DT_Q4_0) side = (size_t)G * C * 32 * 4;
    else if (w->type == JANUS_DT_Q8_0) side = (size_t)G * C * 32 * 2;
    else if (w->type == JANUS_DT_Q4_K || w->type == JANUS_DT_Q5_K) side = (size_t)G * (C / 4) * 32 * 16;
    const size_t fifth = w->type == JANUS_DT_Q5_K ? (size_t)G * C * 64 * 4 : 0;
    void *mem = nullptr;
    JANUS_HIP_CHECK(ctx, hipMalloc(&mem, qbytes + side + fifth + 256));
    uint8_t *dq = (uint8_t *)mem, *ds = (uint8_t *)mem + qbytes;
    uint32_t *df = (uint32_t *)((uint8_t *)mem + qbytes + side);
    const size_t threads = (size_t)G * C * 64;
    const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    switch (w->type) {
    case JANUS_DT_Q4_0:
        hipLaunchKernelGGL(t32_q4_0_kernel, grid, block, 0, ctx->stream, w->qs, w->sc, dq, (uint32_t *)ds, w->n,
                           w->k, G, C);
        break;
    case JANUS_DT_Q4_K:
        hipLaunchKernelGGL(t32_q4_k_kernel, grid, block, 0, ctx->stream, w->qs, dq, ds, w->n, w->k, G, C);
        break;
    case JANUS_DT_Q5_K:
        hipLaunchKernelGGL(t32_q5_k_kernel, grid, block, 0, ctx->stream, w->qs, dq, ds, df, w->n, w->k, G, C);
        break;
    case JANUS_DT_Q8_0:
        hipLaunchKernelGGL(t32_q8_0_kernel, grid, block, 0, ctx->stream, w->qs, w->sc, dq, (uint16_t *)ds, w->n,
                           w->k, G, C);
        break;
    default:
        hipLaunchKernelGGL(t32_f16_kernel, grid, block, 0, ctx->stream, (const uint16_t *)w->qs, dq, w->n, w->k, G,
                           C);
        break;
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(mem);   // already failing: the repack error is the one reported
        return hip_fail(ctx, e, "t32 repack");
    }
    w->t32 = mem;
    w->t32_qs = dq;
    w->t32_side = ds;
    w->t32_q5h = fifth ? df : nullptr;
    w->t32_chunks = C;
    return JANUS_OK;
}

template <class F, int MT>
constexpr int gemm_kw() {
    return (MT == 1 && std::is_same<F, GF16>::value) ? 4 : 2;
}

// kr_force / ks_force (0 = automatic) fix the pass length and the K split.
template <class F, int MT, int KW = gemm_kw<F, MT>(), int PD = Stage<F>::PD>
int launch_mfma(janus_ctx *ctx, GemmArgs a, const janus_weight *w, GemmPartials *parts, uint32_t kr_force = 0,
                uint32_t ks_force = 0) {
    constexpr int SPT1 = 16 / KW;   // kr = 1024 / MT
    if (!kr_force && !ks_force) {   // context-wide overrides (measurement)
        kr_force = ctx->gemm_kr;
        ks_force = ctx->gemm_ks;
    }
    const uint32_t G = (w->n + 31) / 32;
    const uint32_t tiles = (G + WAVES - 1) / WAVES;
    // K per LDS pass: 1024 (M <= 32) or 512 (M <= 64); products with too few
    // (tile, pass) pairs for two workgroups per CU use half-size passes
    const uint32_t want = 2u * (uint32_t)ctx->num_cus;
    uint32_t kr = MT == 1 ? 1024 : 512;
    if (tiles * ((w->t32_chunks * F::CK + kr - 1) / kr) < want && kr / F::CK >= 2 * KW) kr /= 2;
    uint32_t ks = 0;
    bool pipe = false;
    {
        // pipelined kernel (F16 LM head 128256x4096 at M = 32: 181.5 us
        // against 209.3 single-buffered; 512- / 1024-long passes 182.8 /
        // 188.4 us): 256-long passes, K split until
        // about 1.1 workgroups per CU, used when every workgroup then runs at
        // least 3 passes (fewer leave nothing to overlap)
        if (ctx->gemm_pipe && !kr_force && !ks_force) {
            const uint32_t pp = (w->t32_chunks * F::CK + 255) / 256;
            uint32_t pks = ((uint32_t)ctx->num_cus * 11 + 10 * tiles - 1) / (10 * tiles);
            if (pks > pp) pks = pp;
            if (pks < 1) pks = 1;
            if ((pp + pks - 1) / pks >= 3) {
                kr = 256;
                ks = pks;
                pipe = true;
            }
        } else if (ctx->gemm_pipe) {
            pipe = true;   // forced shapes use it wherever there are several passes per workgroup
        }
    }
    if (kr_force) kr = kr_force;
    if (kr % (F::CK * KW) || kr * MT > 2048) return fail(ctx, JANUS_E_INVALID_DIM, "gemm: bad pass length");
    a.pass_chunks = kr / F::CK;
    a.seg_shift = 0;
    while ((8u << a.seg_shift) < kr) ++a.seg_shift;
    if ((8u << a.seg_shift) != kr) return fail(ctx, JANUS_E_INVALID_DIM, "gemm: pass length must be a power of two");
    a.chunks = w->t32_chunks;
    a.total_passes = (a.chunks + a.pass_chunks - 1) / a.pass_chunks;
    // split K over workgroups until there are about two workgroups per CU
    if (!ks) ks = (want + tiles - 1) / tiles;
    if (ks_force) ks = ks_force;
    if (ks > a.total_passes) ks = a.total_passes;
    if (ks < 1) ks = 1;
    a.passes_per_wg = (a.total_passes + ks - 1) / ks;
    a.ksplit = (a.total_passes + a.passes_per_wg - 1) / a.passes_per_wg;
    a.pitch = a.pass_chunks * F::CK + 8;
    const bool sums = NeedsSums<F>::value;
    size_t lds = (size_t)MT * 32 * a.pitch * 2 + (sums ? (size_t)(kr / 32) * MT * 32 * 4 : 0);
    const size_t red = (size_t)WAVES * KW * 16 * 64 * 4;   // K-slice reduction, one M-tile at a time
    if (lds < red) lds = red;
    a.to_ws = parts != nullptr;
    size_t need = 0;
    if (a.ksplit > 1 || parts) {
        need = (size_t)a.ksplit * MT * 32 * G * 32 * 4;
        const size_t epi = parts ? (size_t)MT * 32 * kEpiSlices * 4 : 0;   // the epilogues' per-row area
        if (int e = ensure_gemm_ws(ctx, need + epi)) return e;
        a.ws = (float *)ctx->gemm_ws;
    }
    static const bool attr_set = [] {   // thread-safe one-time set-up
        (void)hipFuncSetAttribute((const void *)gemm_mfma_kernel<F, MT, KW, SPT1, PD>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void *)gemm_mfma_kernel<F, MT, KW, 2 * SPT1, PD>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        return true;
    }();
    (void)attr_set;
    const dim3 grid(tiles, a.ksplit), block(64 * WAVES * KW);
    // the cross-pass pipelined kernel for the usual pass lengths
    bool piped = false;
    {
        if (pipe && a.passes_per_wg > 1) {
            piped = true;
            if (kr == 256) launch_pipe<F, MT, KW, 256>(ctx, grid, a);
            else if (kr == 512) launch_pipe<F, MT, KW, 512>(ctx, grid, a);
            else if (MT == 1 && kr == 1024) launch_pipe<F, MT, KW, 1024 / MT>(ctx, grid, a);
            else piped = false;
        }
    }
    if (!piped && kr * MT <= 1024) hipLaunchKernelGGL((gemm_mfma_kernel<F, MT, KW, SPT1, PD>), grid, block, lds, ctx->stream, a);
    else if (!piped) hipLaunchKernelGGL((gemm_mfma_kernel<F, MT, KW, 2 * SPT1, PD>), grid, block, lds, ctx->stream, a);
    JANUS_LAUNCH_CHECK(ctx);
    if (parts) {
        parts->ws = a.ws;
        parts->ksplit = a.ksplit;
        parts->mpad = MT * 32;
        parts->npad = G * 32;
        parts->ss = a.ws + need / 4;
        return JANUS_OK;
    }
    if (a.ksplit > 1) {
        const size_t total = (size_t)a.rows * w->n;
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream, a,
                           (uint32_t)(MT * 32));
        JANUS_LAUNCH_CHECK(ctx);
    }
    return JANUS_OK;
}

template <int MT>
int launch_mt(janus_ctx *ctx, const GemmArgs &a, const janus_weight *w, GemmPartials *parts) {
    switch (w->type) {
    case JANUS_DT_Q4_0: return launch_mfma<GQ4_0, MT>(ctx, a, w, parts);
    case JANUS_DT_Q8_0: return launch_mfma<GQ8_0, MT>(ctx, a, w, parts);
    case JANUS_DT_Q4_K: return launch_mfma<GQ4_K, MT>(ctx, a, w, parts);
    case JANUS_DT_Q5_K: return launch_mfma<GQ5_K, MT>(ctx, a, w, parts);
    default: return launch_mfma<GF16, MT>(ctx, a, w, parts);
    }
}

GemmArgs make_args(const janus_weight *w, const void *a, void *c, int c_f16, uint32_t rows, const float *residual) {
    GemmArgs g;
    std::memset(&g, 0, sizeof(g));
    g.qs = w->t32_qs;
    g.side = w->t32_side;
    g.q5h = w->t32_q5h;
    g.a = (const _Float16 *)a;
    g.c = c;
    g.resid = residual;
    g.rows = rows;
    g.n = w->n;
    g.k = w->k;
    g.c_f16 = c_f16;
    return g;
}

// ---- batched epilogues over the split-K partials ------------------------------
// Each sums the splits of an element in split order, like gemm_reduce_kernel;
// the loads of up to 8 splits are issued together.

template <typename V>
__device__ __forceinline__ V sum_splits(const float *q, size_t stride, uint32_t ksplit) {
    V s = {};
    for (uint32_t k0 = 0; k0 < ksplit; k0 += 8) {
        V u[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            if (k0 + kk < ksplit) u[kk] = *(const V *)(q + (k0 + kk) * stride);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            if (k0 + kk < ksplit) s += u[kk];
    }
    return s;
}

__device__ __forceinline__ jf2 sum_pair(const GemmPartials &p, uint32_t m, uint32_t col) {
    return sum_splits<jf2>(p.ws + (size_t)m * p.npad + col, (size_t)p.mpad * p.npad, p.ksplit);
}

// Fused-QKV rows (RoPE pairs of q heads, of k heads, then v in order): rotate
// q into q_out [rows][heads * hd] (f32) and k, append k and v to the cache row
// rowbase[m] + pos[m] (m * max_seq + pos[m] without a table; the rotation of
// rope.wgsl:71-72, the row layout of kv_update_kernel).
template <typename KV>
__global__ __launch_bounds__(256) void epi_qkv_rope_kernel(GemmPartials p, QkvEpilogue e, uint32_t rows) {
    const uint32_t pairs = e.q_pairs + e.k_pairs + e.kv_row / 2;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)rows * pairs) return;
    const uint32_t m = (uint32_t)(idx / pairs), g = (uint32_t)(idx % pairs);
    const uint32_t pos = (uint32_t)e.pos[m];
    if (pos >= e.max_seq) return;   // host checks keep positions in range; never index past the tables
    const jf2 r = sum_pair(p, m, 2 * g);
    const size_t row = (e.rowbase ? (size_t)(uint32_t)e.rowbase[m] : (size_t)m * e.max_seq) + pos;
    if (g < e.q_pairs + e.k_pairs) {
        const bool isq = g < e.q_pairs;
        const uint32_t gg = isq ? g : g - e.q_pairs, h = gg / e.half_hd, i = gg % e.half_hd;
        const float2 cs = *(const float2 *)(e.rope + 2 * ((size_t)pos * e.half_hd + i));
        const float y0 = r.x * cs.x - r.y * cs.y;
        const float y1 = r.x * cs.y + r.y * cs.x;
        if (isq) {
            float *q = e.q + (size_t)m * e.q_pairs * 2 + (size_t)h * 2 * e.half_hd + i;
            q[0] = y0;
            q[e.half_hd] = y1;
        } else {
            KV *k = (KV *)e.kc + row * e.kv_row + (size_t)h * 2 * e.half_hd + i;
            k[0] = (KV)y0;
            k[e.half_hd] = (KV)y1;
        }
    } else {
        KV *v = (KV *)e.vc + row * e.kv_row + 2 * (size_t)(g - e.q_pairs - e.k_pairs);
        v[0] = (KV)r.x;
        v[1] = (KV)r.y;
    }
}

// Gate/up rows interleaved (gate_j, up_j): act[m][j] = silu(gate) * up as
// binary16 (the SwiGLU of elementwise_kernel).
__global__ __launch_bounds__(256) void epi_swiglu_kernel(GemmPartials p, _Float16 *act, uint32_t rows, uint32_t ffn) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)rows * ffn) return;
    const uint32_t m = (uint32_t)(idx / ffn), j = (uint32_t)(idx % ffn);
    const jf2 r = sum_pair(p, m, 2 * j);
    const float v = r.x * (1.0f / (1.0f + expf(-r.x))) * r.y;
    ((uint16_t *)act)[idx] = f2h_bits(v);
}

// One 1024-thread workgroup per row: out[m] = resid[m] + product (f32, may
// alias resid), then xn[m] = (out[m] / rms) * gamma as binary16 with
// rms = sqrt(mean(out^2) + eps) (the arithmetic of rmsnorm_kernel).
template <int NV>
__global__ __launch_bounds__(1024) void epi_resnorm_kernel(GemmPartials p, const float *resid, float *out,
                                                           const float *__restrict__ gamma, float eps, _Float16 *xn,
                                                           uint32_t hidden) {
    __shared__ float red[16];
    const uint32_t m = blockIdx.x;
    const float *q = p.ws + (size_t)m * p.npad;
    const size_t stride = (size_t)p.mpad * p.npad;
    jf4 v[NV], g[NV];
    float s = 0.0f;
    // gamma is requested with the partials: one memory round trip before the reduction
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = 4 * (threadIdx.x + 1024u * j);
        g[j] = i < hidden ? *(const jf4 *)(gamma + i) : jf4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = 4 * (threadIdx.x + 1024u * j);
        v[j] = jf4{0.0f, 0.0f, 0.0f, 0.0f};
        if (i < hidden) v[j] = sum_splits<jf4>(q + i, stride, p.ksplit) + *(const jf4 *)(resid + (size_t)m * hidden + i);
        s = fmaf(v[j].x, v[j].x, s);
        s = fmaf(v[j].y, v[j].y, s);
        s = fmaf(v[j].z, v[j].z, s);
        s = fmaf(v[j].w, v[j].w, s);
    }
    s = wave_sum_dpp(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; ++w) tot += red[w];
    // (x / rms) * gamma, the reference's formula (activations.wgsl:128), as in
    // the M = 1 kernels' fused norm
    const float rms = sqrtf(tot / (float)hidden + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = 4 * (threadIdx.x + 1024u * j);
        if (i < hidden) {
            *(jf4 *)(out + (size_t)m * hidden + i) = v[j];
            const uint32_t lo = (uint32_t)f2h_bits((v[j].x / rms) * g[j].x) | ((uint32_t)f2h_bits((v[j].y / rms) * g[j].y) << 16);
            const uint32_t hi = (uint32_t)f2h_bits((v[j].z / rms) * g[j].z) | ((uint32_t)f2h_bits((v[j].w / rms) * g[j].w) << 16);
            *(uint2 *)((uint16_t *)xn + (size_t)m * hidden + i) = make_uint2(lo, hi);
        }
    }
}

// Residual + RMSNorm spread over the GPU in two launches (a row's sum of
// squares spans workgroups): epi_ressum_kernel, one 128-thread workgroup per
// (512-column slice, row), writes out = resid + the summed partials and the
// slice's sum of squares (threads, then the wavefront by DPP, then the two
// wavefronts in order) to p.ss[row][slice]; epi_norm_kernel, the same grid,
// adds the row's slice sums in slice order and writes (x / rms) * gamma as
// binary16 (activations.wgsl:128, as the M = 1 kernels' fused norm).
constexpr uint32_t kEpiCols = 512;
__global__ __launch_bounds__(128) void epi_ressum_kernel(GemmPartials p, const float *resid, float *out,
                                                         uint32_t hidden) {
    __shared__ float red[2];
    const uint32_t m = blockIdx.y, slice = blockIdx.x;
    const uint32_t i = slice * kEpiCols + 4 * threadIdx.x;
    const float *q = p.ws + (size_t)m * p.npad;
    jf4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (i < hidden) {
        v = sum_splits<jf4>(q + i, (size_t)p.mpad * p.npad, p.ksplit) + *(const jf4 *)(resid + (size_t)m * hidden + i);
        *(jf4 *)(out + (size_t)m * hidden + i) = v;
    }
    float s = fmaf(v.x, v.x, 0.0f);
    s = fmaf(v.y, v.y, s);
    s = fmaf(v.z, v.z, s);
    s = fmaf(v.w, v.w, s);
    s = wave_sum_dpp(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) p.ss[(size_t)m * kEpiSlices + slice] = red[0] + red[1];
}

__global__ __launch_bounds__(128) void epi_norm_kernel(GemmPartials p, const float *out,
                                                       const float *__restrict__ gamma, float eps, _Float16 *xn,
                                                       uint32_t hidden) {
    const uint32_t m = blockIdx.y, slice = blockIdx.x;
    const uint32_t i = slice * kEpiCols + 4 * threadIdx.x;
    const uint32_t slices = (hidden + kEpiCols - 1) / kEpiCols;
    // the row and gamma are requested with the slice sums: one round trip
    jf4 v = {0.0f, 0.0f, 0.0f, 0.0f}, g = {0.0f, 0.0f, 0.0f, 0.0f};
    if (i < hidden) {
        v = *(const jf4 *)(out + (size_t)m * hidden + i);
        g = *(const jf4 *)(gamma + i);
    }
    float tot = 0.0f;
    for (uint32_t t = 0; t < slices; ++t) tot += p.ss[(size_t)m * kEpiSlices + t];
    const float rms = sqrtf(tot / (float)hidden + eps);
    if (i < hidden) {
        const uint32_t lo = (uint32_t)f2h_bits((v.x / rms) * g.x) | ((uint32_t)f2h_bits((v.y / rms) * g.y) << 16);
        const uint32_t hi = (uint32_t)f2h_bits((v.z / rms) * g.z) | ((uint32_t)f2h_bits((v.w / rms) * g.w) << 16);
        *(uint2 *)((uint16_t *)xn + (size_t)m * hidden + i) = make_uint2(lo, hi);
    }
}

int run_partials(janus_ctx *ctx, const void *a, const janus_weight *w, uint32_t rows, GemmPartials *parts) {
    if (!mfma_gemm_supported(JANUS_DT_F16, w))
        return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "batched epilogue: weight has no MFMA path");
    if (rows == 0 || rows > 64) return fail(ctx, JANUS_E_INVALID_DIM, "batched epilogue: rows must be 1..64");
    if (int e = mfma_gemm_prepare(ctx, w)) return e;
    const GemmArgs g = make_args(w, a, nullptr, 0, rows, nullptr);
    return rows <= 32 ? launch_mt<1>(ctx, g, w, parts) : launch_mt<2>(ctx, g, w, parts);
}

}  // namespace

bool mfma_gemm_supported(int a_dt, const janus_weight *w) {
    if (a_dt != JANUS_DT_F16 || w->k % 8) return false;
    return w->type == JANUS_DT_Q4_0 || w->type == JANUS_DT_Q8_0 || w->type == JANUS_DT_Q4_K ||
           w->type == JANUS_DT_Q5_K || w->type == JANUS_DT_F16;
}

int mfma_gemm_prepare(janus_ctx *ctx, const janus_weight *w) {
    return t32_ensure(ctx, const_cast<janus_weight *>(w));
}

int smallm_gemm_launch(janus_ctx *ctx, const void *a, int a_dt, const janus_weight *w, void *c, int c_dt,
                       uint32_t rows, const float *residual) {
    if (mfma_gemm_supported(a_dt, w)) {
        if (int e = mfma_gemm_prepare(ctx, w)) return e;
        const GemmArgs g = make_args(w, a, c, c_dt == JANUS_DT_F16, rows, residual);
        return rows <= 32 ? launch_mt<1>(ctx, g, w, nullptr) : launch_mt<2>(ctx, g, w, nullptr);
    }
    // f32 activations keep the reference's dtype: one GEMV launch per row
    const size_t as = act_bytes(a_dt) * w->k, cs = act_bytes(c_dt) * w->n;
    for (uint32_t r = 0; r < rows; ++r) {
        int e = gemv_dispatch(ctx, (const uint8_t *)a + r * as, a_dt, w, (uint8_t *)c + r * cs, c_dt,
                              residual ? residual + (size_t)r * w->n : nullptr);
        if (e) return e;
    }
    return JANUS_OK;
}

int gemm_qkv_rope(janus_ctx *ctx, const void *a16, const janus_weight *w, uint32_t rows, const QkvEpilogue &e,
                  int kv_f16) {
    if (w->n != 2 * (e.q_pairs + e.k_pairs) + e.kv_row || e.kv_row % 2)
        return fail(ctx, JANUS_E_INVALID_DIM, "qkv epilogue: row count does not match the head layout");
    GemmPartials p{};
    if (int r = run_partials(ctx, a16, w, rows, &p)) return r;
    const size_t total = (size_t)rows * (w->n / 2);
    const dim3 grid((unsigned)((total + 255) / 256));
    if (kv_f16) hipLaunchKernelGGL(epi_qkv_rope_kernel<_Float16>, grid, dim3(256), 0, ctx->stream, p, e, rows);
    else hipLaunchKernelGGL(epi_qkv_rope_kernel<float>, grid, dim3(256), 0, ctx->stream, p, e, rows);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

int gemm_swiglu(janus_ctx *ctx, const void *a16, const janus_weight *w, uint32_t rows, void *act16) {
    if (w->n % 2) return fail(ctx, JANUS_E_INVALID_DIM, "swiglu epilogue: odd row count");
    const uint32_t tiles = (w->n + 32 * WAVES - 1) / (32 * WAVES);
    if (w->type == JANUS_DT_Q4_0 && rows <= 32 && 4 * tiles >= 3 * (uint32_t)ctx->num_cus) {
        // enough row tiles for every CU without splitting K: 16-wavefront
        // workgroups over the whole K, SwiGLU applied to the finished tile
        if (int e = mfma_gemm_prepare(ctx, w)) return e;
        GemmArgs g = make_args(w, a16, act16, 1, rows, nullptr);
        g.swiglu = 1;
        return launch_mfma<GQ4_0, 1, 4, 2>(ctx, g, w, nullptr, ctx->gemm_pipe ? 512 : 1024, 1);
    }
    GemmPartials p{};
    if (int r = run_partials(ctx, a16, w, rows, &p)) return r;
    const size_t total = (size_t)rows * (w->n / 2);
    hipLaunchKernelGGL(epi_swiglu_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream, p,
                       (_Float16 *)act16, rows, w->n / 2);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

bool resnorm_supported(uint32_t hidden) { return hidden % 4 == 0 && hidden <= 8192; }

int gemm_residual_norm(janus_ctx *ctx, const void *a16, const janus_weight *w, uint32_t rows, const float *resid,
                       float *out, const float *gamma, float eps, void *xn16) {
    const uint32_t hidden = w->n;
    if (!resnorm_supported(hidden))
        return fail(ctx, JANUS_E_INVALID_DIM, "residual-norm epilogue: rows must be a multiple of 4, at most 8192");
    GemmPartials p{};
    if (int r = run_partials(ctx, a16, w, rows, &p)) return r;
    _Float16 *xn = (_Float16 *)xn16;
    if (ctx->epi_split) {
        const dim3 sgrid((hidden + kEpiCols - 1) / kEpiCols, rows), sblock(kEpiCols / 4);
        hipLaunchKernelGGL(epi_ressum_kernel, sgrid, sblock, 0, ctx->stream, p, resid, out, hidden);
        JANUS_LAUNCH_CHECK(ctx);
        hipLaunchKernelGGL(epi_norm_kernel, sgrid, sblock, 0, ctx->stream, p, out, gamma, eps, xn, hidden);
        JANUS_LAUNCH_CHECK(ctx);
        return JANUS_OK;
    }
    const dim3 grid(rows), block(1024);
    if (hidden <= 4096) hipLaunchKernelGGL(epi_resnorm_kernel<1>, grid, block, 0, ctx->stream, p, resid, out, gamma, eps, xn, hidden);
    else hipLaunchKernelGGL(epi_resnorm_kernel<2>, grid, block, 0, ctx->stream, p, resid, out, gamma, eps, xn, hidden);
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

}  // namespace janus
