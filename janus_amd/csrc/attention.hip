// attention.hip -- split-K GQA decode attention (one query token per sequence).
//
// Replaces compute_attention (crates/janus-engine/src/compute/ops/attention.rs:78-235:
// compute_qk_scores + softmax + apply_attention in attention.wgsl:62-186 and
// softmax.wgsl:18-51). Those three passes materialise scores/probabilities in
// HBM and run the softmax on one thread per head; here:
//  * One wavefront per (sequence, KV head, split of the context): it owns the
//    G = H / KVH query heads that share the KV head. Lanes are (position slot,
//    8-dimension slice), so every K/V load is a 128-bit load and a wavefront
//    step reads SLOTS whole cache rows; scores are reduced over the slice lanes
//    with DPP, and each slot runs an online (running max / running sum)
//    softmax with fp32 P.V accumulators in registers (exponentials in base 2
//    on log2(e)-scaled scores, one v_exp_f32 each). Batches of steps are
//    double-buffered; there is no LDS traffic and no barrier.
//  * Long contexts are split so the launch has ~8 wavefronts per CU; each split
//    writes (m, l, o[D]) partials and a merge kernel combines them with the
//    log-sum-exp rule. A sequence covered by one split writes its output
//    directly.
//  * Ragged batches: per-sequence row offsets and lengths are device tables,
//    so all sequences share one launch.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "internal.h"

namespace janus {

namespace {

constexpr int TP = 16;        // split granularity in positions
constexpr uint32_t kRowsMinBlocks = 8;   // row streaming: least 16-position blocks per workgroup

// Row streaming's split partials: [workgroup][2 slots][head][hd + 2] floats.
size_t rows_partial_bytes(const janus_ctx *ctx, uint32_t heads, uint32_t hd) {
    return (size_t)ctx->num_cus * 2 * heads * (hd + 2) * sizeof(float);
}

struct AttnArgs {
    const float *q;
    const void *kc, *vc;
    void *out;              // [B][H][D] f32, or binary16 when out_f16
    float *ws;              // [B][H][S][D + 2]
    const int32_t *row_base;
    const int32_t *seq_lens;
    uint32_t batch, heads, kv_heads;
    uint32_t seq_len, max_seq;
    uint32_t max_len;       // longest sequence the plan covers (row streaming clamps lengths to it)
    uint32_t chunk;         // positions per wavefront
    uint32_t nw;            // wavefronts per workgroup
    uint32_t splits;        // S: workgroup splits per sequence
    uint32_t qh_div;        // 0: grid.y = KV head (G query heads each); else grid.y = query head, KV head = y / qh_div
    uint32_t rows;          // 1: row-streaming kernel (chunk = least 16-position blocks per workgroup)
    float scale;
    float scale2;           // scale * log2(e): the softmax runs in the base-2 domain
    int out_f16;
};

__device__ __forceinline__ void put_out(const AttnArgs &a, size_t at, float v) {
    if (a.out_f16) ((uint16_t *)a.out)[at] = f2h_bits(v);
    else ((float *)a.out)[at] = v;
}

// 2^x with the native instruction. Scores are pre-multiplied by log2(e), so
// exp(s - m) = 2^(s*log2e - m*log2e); all running maxima (and the partials a
// split writes) are kept in that base-2 scale.
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// 8 head dimensions of one cached position, as loaded by one lane.
template <typename KV> struct KVRow;
template <> struct KVRow<_Float16> {
    uint4 r;
    __device__ void load(const _Float16 *p) { r = *(const uint4 *)p; }
    __device__ float get(int i) const {
        const uint32_t w = i < 2 ? r.x : i < 4 ? r.y : i < 6 ? r.z : r.w;
        return (float)__builtin_bit_cast(_Float16, (uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
    }
};
template <> struct KVRow<float> {
    jf4 a, b;
    __device__ void load(const float *p) { a = *(const jf4 *)p; b = *(const jf4 *)(p + 4); }
    __device__ float get(int i) const { return i < 4 ? a[i] : b[i - 4]; }
};

// Sum over the LPP lanes that share a position (every lane receives it).
template <int LPP> __device__ __forceinline__ float pos_sum(float v) {
    if (LPP == 16) {
        v += dpp_f<0x128>(v);   // row_ror:8
        v += dpp_f<0x124>(v);   // row_ror:4
        v += dpp_f<0x122>(v);   // row_ror:2
        v += dpp_f<0x121>(v);   // row_ror:1
    } else {                    // 8-lane groups
        v += dpp_f<0x141>(v);   // row_half_mirror: lane i of 8 adds lane 7 - i
        v += dpp_f<0x4e>(v);    // quad_perm [2,3,0,1]
        v += dpp_f<0xb1>(v);    // quad_perm [1,0,3,2]
    }
    return v;
}

// Value of lane ^ O for O = 8 (within a 16-lane row), 16 or 32.
template <int O> __device__ __forceinline__ float lane_xor(float v) {
    if (O == 8) return dpp_f<0x128>(v);   // row_ror:8 == xor 8 inside a row
    const uint32_t u = __float_as_uint(v);
    if (O == 16) {
        auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __uint_as_float((__lane_id() & 16) ? p[0] : p[1]);
    }
    auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float((__lane_id() & 32) ? p[0] : p[1]);
}

// Log-sum-exp merge of this lane's (m, l, acc) with lane ^ O's.
template <int O, int G>
__device__ __forceinline__ void merge_xor(float (&m)[G], float (&l)[G], float (&acc)[G][8]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float mo = lane_xor<O>(m[g]), lo = lane_xor<O>(l[g]);
        const float M = fmaxf(m[g], mo);
        const float fs = M == -INFINITY ? 0.0f : fexp2(m[g] - M);
        const float fo = M == -INFINITY ? 0.0f : fexp2(mo - M);
        l[g] = l[g] * fs + lo * fo;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = acc[g][i] * fs + lane_xor<O>(acc[g][i]) * fo;
        m[g] = M;
    }
}

// A workgroup of NW wavefronts owns (sequence, KV head, workgroup split); its
// span of NW * chunk positions is divided between the wavefronts. Lane =
// (position slot, 8-dim slice): a step reads SLOTS whole cache rows with
// 128-bit loads, scores are reduced over the slice lanes with DPP, and each
// slot runs an online (running max / running sum) softmax for the G query
// heads with fp32 P.V accumulators in registers; batches of U steps are
// double-buffered. Slots, then wavefronts (through LDS, in wavefront order),
// are merged with the log-sum-exp rule.
template <typename KV, int D, int G, int NW>
__global__ __launch_bounds__(64 * NW) void attn_decode_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float smem_f[];   // [NW][G][D + 2]
    constexpr int LPP = D / 8, SLOTS = 64 / LPP;
    constexpr int KB = sizeof(KV) == 2 ? 1 : 2;            // 16-byte loads per lane per row
    // steps per batch: sized to the registers a wavefront has at this workgroup size
    constexpr int U = NW == 16 ? 2 / KB : (G <= 2 ? 8 / KB : (G == 4 ? 4 / KB : 2));
    constexpr int BATCH = SLOTS * U;                  // positions per batch
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = NW;
    const int slot = lane / LPP, dl = lane % LPP;
    const uint32_t split = blockIdx.x, b = blockIdx.z;
    // per-query-head launch (short contexts): one head per workgroup, KV head y / qh_div
    const uint32_t kvh = a.qh_div ? blockIdx.y / a.qh_div : blockIdx.y;
    const uint32_t h0 = a.qh_div ? blockIdx.y : blockIdx.y * G;   // first query head of this workgroup
    // The sequence's length and row base are requested together, before
    // anything waits on either (one round trip, not one per value).
    const uint32_t len_raw = a.seq_lens ? (uint32_t)a.seq_lens[b] : a.seq_len;
    const uint32_t base_raw = a.row_base ? (uint32_t)a.row_base[b] : b * a.max_seq;
    float qr[G][8], acc[G][8], m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float *qp = a.q + ((size_t)b * a.heads + h0 + g) * D + 8 * dl;
        const jf4 q0 = *(const jf4 *)qp, q1 = *(const jf4 *)(qp + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) { qr[g][i] = q0[i]; qr[g][4 + i] = q1[i]; }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
        m[g] = -INFINITY;
        l[g] = 0.0f;
    }
    // lengths beyond the planned splits (or the capacity) are clamped, never read past
    const uint32_t span = (uint32_t)nw * a.chunk;
    const uint32_t len = min(min(len_raw, a.max_seq), a.splits * span);
    const uint32_t wg_start = split * span;
    if (wg_start >= len && !(split == 0 && len == 0)) return;   // whole workgroup; len 0: split 0 writes zeros
    const uint32_t wg_end = min(len, wg_start + span);
    const uint32_t start = wg_start + wave * a.chunk;
    const uint32_t end = min(wg_end, start + a.chunk);
    const size_t row0 = (size_t)base_raw;
    const uint32_t kvrow = a.kv_heads * D;
    const KV *kc = (const KV *)a.kc + row0 * kvrow + (size_t)kvh * D + 8 * dl;
    const KV *vc = (const KV *)a.vc + row0 * kvrow + (size_t)kvh * D + 8 * dl;

    KVRow<KV> ka[U], va[U], kb[U], vb[U];
    auto load = [&](KVRow<KV> (&k)[U], KVRow<KV> (&v)[U], uint32_t p0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint32_t p = p0 + u * SLOTS + slot;
            p = p < end ? p : end - 1;   // masked below; the address stays inside the sequence
            k[u].load(kc + (size_t)p * kvrow);
            v[u].load(vc + (size_t)p * kvrow);
        }
    };
    // MASK: the batch may run past `end` (only the last batch of a range);
    // full batches skip the per-position checks.
    auto consume = [&](const KVRow<KV> (&k)[U], const KVRow<KV> (&v)[U], uint32_t p0, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        float s[U][G];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool live = !MASK || p0 + u * SLOTS + slot < end;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    d0 = fmaf(qr[g][i], k[u].get(i), d0);
                    d1 = fmaf(qr[g][i + 1], k[u].get(i + 1), d1);
                }
                const float t = pos_sum<LPP>(d0 + d1);
                s[u][g] = live ? t * a.scale2 : -INFINITY;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mx = s[0][g];
#pragma unroll
            for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[u][g]);
            const float mn = fmaxf(m[g], mx);
            if (MASK && mn == -INFINITY) continue;   // nothing live in this slot yet
            const float alpha = fexp2(m[g] - mn);
            l[g] *= alpha;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] *= alpha;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float pu = fexp2(s[u][g] - mn);
                l[g] += pu;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(pu, v[u].get(i), acc[g][i]);
            }
            m[g] = mn;
        }
    };
    const std::true_type masked{};
    const std::false_type full{};
    if (start < end) {
        load(ka, va, start);
        uint32_t p0 = start;
        for (; p0 + BATCH < end; p0 += 2 * BATCH) {
            load(kb, vb, p0 + BATCH);
            consume(ka, va, p0, full);
            if (p0 + 2 * BATCH < end) load(ka, va, p0 + 2 * BATCH);
            if (p0 + 2 * BATCH <= end) consume(kb, vb, p0 + BATCH, full);
            else consume(kb, vb, p0 + BATCH, masked);
        }
        if (p0 < end) {
            if (p0 + BATCH <= end) consume(ka, va, p0, full);
            else consume(ka, va, p0, masked);
        }
    }

    // merge the slots (lanes lane ^ (LPP * 2^j) hold the same dims of other slots)
    if (LPP == 8) merge_xor<8, G>(m, l, acc);
    merge_xor<16, G>(m, l, acc);
    merge_xor<32, G>(m, l, acc);
    // merge the wavefronts through LDS, in wavefront order
    if (slot == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float *r = smem_f + ((size_t)wave * G + g) * (D + 2);
            if (dl == 0) { r[0] = m[g]; r[1] = l[g]; }
#pragma unroll
            for (int i = 0; i < 8; ++i) r[2 + 8 * dl + i] = acc[g][i];
        }
    }
    __syncthreads();
    if (wave != 0 || slot != 0) return;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float M = -INFINITY;
        for (int w = 0; w < nw; ++w) M = fmaxf(M, smem_f[((size_t)w * G + g) * (D + 2)]);
        float L = 0.0f, o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = 0.0f;
        if (M != -INFINITY) {
            for (int w = 0; w < nw; ++w) {
                const float *r = smem_f + ((size_t)w * G + g) * (D + 2);
                const float f = fexp2(r[0] - M);
                L = fmaf(r[1], f, L);
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = fmaf(r[2 + 8 * dl + i], f, o[i]);
            }
        }
        const uint32_t h = h0 + g;
        if (a.splits == 1 || len <= span) {
            const float inv = 1.0f / fmaxf(L, 1e-20f);
            const size_t at = ((size_t)b * a.heads + h) * D + 8 * dl;
#pragma unroll
            for (int i = 0; i < 8; ++i) put_out(a, at + i, o[i] * inv);
        } else {
            float *w = a.ws + (((size_t)b * a.heads + h) * a.splits + split) * (D + 2);
            if (dl == 0) { w[0] = M; w[1] = L; }
#pragma unroll
            for (int i = 0; i < 8; ++i) w[2 + 8 * dl + i] = o[i];
        }
    }
}

typedef _Float16 ah8 __attribute__((ext_vector_type(8)));
typedef _Float16 ah4 __attribute__((ext_vector_type(4)));
typedef float af4 __attribute__((ext_vector_type(4)));

// Binary16 caches: one wavefront attends G query heads of one KV head over a
// position range. The scores of 16 positions x the G heads come from
// v_mfma_f32_16x16x32_f16 (positions as rows, heads as columns, head dims as
// K), with q split into binary16 hi + mid + lo parts so the scores keep fp32
// accuracy (f16 x f16 products are exact; the three parts carry 33
// significant bits of q, after a power-of-two prescale that keeps them in
// range). The softmax runs on
// the MFMA output layout (lane = head column, 4 positions), publishes P and the
// rescale factors through a small per-wavefront LDS area, and P.V runs on the
// VALU in the (position slot, 8-dim slice) layout, so K is read as MFMA
// operands and V as 128-bit rows. All slots share one running maximum per head,
// so they merge by plain sums. On return every lane holds (m, l) of head
// `lane & 15` and the slot-0 lanes hold acc for dims 8 * (lane % (D / 8)).
template <int D, int G>
struct MfmaAttn {
    static constexpr int KS = D / 32;                  // MFMA K steps over the head dims
    static constexpr int LPP = D / 8, SLOTS = 64 / LPP;
    static constexpr int BP = 16;                      // positions per MFMA block
    static constexpr int STEPS = BP / SLOTS;           // P.V steps per block
    static constexpr int PW = BP * G + G;              // floats of a wavefront's P area
    static_assert(G <= 16 && (D == 64 || D == 128), "MfmaAttn: G <= 16, D in {64, 128}");

    __device__ static void run(const AttnArgs &a, uint32_t b, uint32_t kvh, uint32_t start, uint32_t end, float *Pw,
                               float &m, float &l, float (&acc)[G][8]) {
        const int lane = __lane_id();
        const int slot = lane / LPP, dl = lane % LPP;   // P.V layout
        const int col = lane & 15, grp = lane >> 4;     // MFMA layout
        const uint32_t h0 = kvh * G;
        const size_t row0 = (size_t)(a.row_base ? (uint32_t)a.row_base[b] : b * a.max_seq);
        const uint32_t kvrow = a.kv_heads * D;
        const _Float16 *kc = (const _Float16 *)a.kc + row0 * kvrow + (size_t)kvh * D + 8 * grp;
        const _Float16 *vc = (const _Float16 *)a.vc + row0 * kvrow + (size_t)kvh * D + 8 * dl;

        uint4 ka[KS], kb[KS], va[STEPS], vb[STEPS];
        auto load = [&](uint4 (&k)[KS], uint4 (&v)[STEPS], uint32_t p0) {
            uint32_t kp = p0 + col;
            kp = kp < end ? kp : end - 1;   // masked below; the address stays inside the sequence
#pragma unroll
            for (int t = 0; t < KS; ++t) k[t] = ld_stream(kc + (size_t)kp * kvrow + 32 * t);
#pragma unroll
            for (int u = 0; u < STEPS; ++u) {
                uint32_t vp = p0 + u * SLOTS + slot;
                vp = vp < end ? vp : end - 1;
                v[u] = ld_stream(vc + (size_t)vp * kvrow);
            }
        };
        // the first batch is requested before q is read and split: its latency
        // overlaps the q loads
        if (start < end) load(ka, va, start);

        // q of head `col` (zero for col >= G), dims 8*grp + 32t + i
        float qv[KS][8];
        float qmax = 0.0f;
#pragma unroll
        for (int t = 0; t < KS; ++t) {
            if (col < G) {
                const float *qp = a.q + ((size_t)b * a.heads + h0 + col) * D + 8 * grp + 32 * t;
                const jf4 q0 = *(const jf4 *)qp, q1 = *(const jf4 *)(qp + 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) { qv[t][i] = q0[i]; qv[t][4 + i] = q1[i]; }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) qv[t][i] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) qmax = fmaxf(qmax, fabsf(qv[t][i]));
        }
        qmax = fmaxf(qmax, lane_xor<16>(qmax));
        qmax = fmaxf(qmax, lane_xor<32>(qmax));
        int qe = 0;
        (void)frexpf(qmax, &qe);                  // qmax < 2^qe
        const int sh = qe > 15 ? qe - 15 : 0;     // |q| * 2^-sh < 2^15
        const float qs = ldexpf(1.0f, -sh);
        const float sc2 = a.scale2 * ldexpf(1.0f, sh);
        ah8 qh[KS], qm[KS], ql[KS];   // x = hi + mid + lo: 33 significant bits, more than fp32's 24
#pragma unroll
        for (int t = 0; t < KS; ++t)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x = qv[t][i] * qs;
                const _Float16 hi = (_Float16)x;
                const float r = x - (float)hi;
                const _Float16 mid = (_Float16)r;
                qh[t][i] = hi;
                qm[t][i] = mid;
                ql[t][i] = (_Float16)(r - (float)mid);
            }

#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
        m = -INFINITY;
        l = 0.0f;

        auto consume = [&](const uint4 (&k)[KS], const uint4 (&v)[STEPS], uint32_t p0) {
            af4 S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < KS; ++t) {
                const ah8 kk = __builtin_bit_cast(ah8, k[t]);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, ql[t], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, qm[t], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, qh[t], S, 0, 0, 0);
            }
            // S[r]: head col, position p0 + 4*grp + r
            float sv[4];
            float bm = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool live = p0 + 4 * grp + r < end;
                sv[r] = live ? S[r] * sc2 : -INFINITY;
                bm = fmaxf(bm, sv[r]);
            }
            bm = fmaxf(bm, lane_xor<16>(bm));
            bm = fmaxf(bm, lane_xor<32>(bm));
            const float mn = fmaxf(m, bm);
            const float alpha = mn == -INFINITY ? 1.0f : fexp2(m - mn);
            float ps[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ps[r] = mn == -INFINITY ? 0.0f : fexp2(sv[r] - mn);
            l = l * alpha + ((ps[0] + ps[1]) + (ps[2] + ps[3]));
            m = mn;
            if (col < G) {
#pragma unroll
                for (int r = 0; r < 4; ++r) Pw[(4 * grp + r) * G + col] = ps[r];
                if (grp == 0) Pw[BP * G + col] = alpha;
            }
            // the area is read by other lanes of this wavefront only: LDS
            // operations of one wavefront complete in order
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float al = Pw[BP * G + g];
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[g][i] *= al;
            }
#pragma unroll
            for (int u = 0; u < STEPS; ++u) {
                const float *pr = Pw + (u * SLOTS + slot) * G;
                KVRow<_Float16> vrow;
                vrow.r = v[u];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float pg = pr[g];
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(pg, vrow.get(i), acc[g][i]);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        };
        if (start < end) {
            uint32_t p0 = start;
            for (; p0 + BP < end; p0 += 2 * BP) {
                load(kb, vb, p0 + BP);
                consume(ka, va, p0);
                if (p0 + 2 * BP < end) load(ka, va, p0 + 2 * BP);
                consume(kb, vb, p0 + BP);
            }
            if (p0 < end) consume(ka, va, p0);
        }
        // slots share the running maximum: sum acc over slots, l over the 4 position groups
        l += lane_xor<16>(l);
        l += lane_xor<32>(l);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float x = acc[g][i];
                if (LPP == 8) x += lane_xor<8>(x);
                x += lane_xor<16>(x);
                x += lane_xor<32>(x);
                acc[g][i] = x;
            }
    }
};

// Work list of (sequence, context piece) x KV head tasks of at most `chunk`
// positions, enumerated on the device from the length table (ragged batches
// balance across wavefronts whatever the lengths); a persistent grid of
// wavefronts walks it. A sequence held by one piece writes its output; the
// others write (m, l, o) partials for attn_merge_kernel. Requires batch <= 64.
template <int D, int G>
__global__ __launch_bounds__(256) void attn_task_kernel(AttnArgs a) {
    using A = MfmaAttn<D, G>;
    __shared__ float parea[4 * A::PW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float *Pw = parea + wave * A::PW;
    const uint32_t C = a.chunk;
    const uint32_t cap = a.splits * C;
    // lane b: pieces of sequence b (at least one, so an empty sequence writes zeros)
    uint32_t lenb = 0, nb = 0;
    if ((uint32_t)lane < a.batch) {
        lenb = min(min(a.seq_lens ? (uint32_t)a.seq_lens[lane] : a.seq_len, a.max_seq), cap);
        nb = lenb == 0 ? 1u : (lenb + C - 1) / C;
    }
    uint32_t incl = nb;   // inclusive prefix over lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t up = (uint32_t)__shfl_up((int)incl, o, 64);
        if (lane >= o) incl += up;
    }
    const uint32_t pieces = (uint32_t)__shfl((int)incl, 63, 64);
    const uint32_t ntask = pieces * a.kv_heads;
    const uint32_t nwave = gridDim.x * 4;
    for (uint32_t t = blockIdx.x * 4 + wave; t < ntask; t += nwave) {
        const uint32_t q = t / a.kv_heads, kvh = t % a.kv_heads;
        // sequence: the number of lanes whose inclusive prefix is <= q
        const uint64_t le = __ballot(incl <= q);
        const uint32_t b = (uint32_t)__popcll(le);
        const uint32_t excl = (uint32_t)__shfl((int)(incl - nb), (int)b, 64);
        const uint32_t len = (uint32_t)__shfl((int)lenb, (int)b, 64);
        const uint32_t nseq = (uint32_t)__shfl((int)nb, (int)b, 64);
        const uint32_t j = q - excl;
        const uint32_t start = j * C, end = min(len, start + C);
        float m, l, acc[G][8];
        A::run(a, b, kvh, start, end, Pw, m, l, acc);
        // every lane: (m, l) of head lane & 15; slot-0 lanes: acc of dims 8 * dl
        const int dl = lane % A::LPP;
        const bool writer = lane < A::LPP;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mg = __shfl(m, g, 64), lg = __shfl(l, g, 64);
            const uint32_t h = kvh * G + g;
            if (!writer) continue;
            if (nseq == 1) {
                const float inv = 1.0f / fmaxf(lg, 1e-20f);
                const size_t at = ((size_t)b * a.heads + h) * D + 8 * dl;
#pragma unroll
                for (int i = 0; i < 8; ++i) put_out(a, at + i, acc[g][i] * inv);
            } else {
                float *w = a.ws + (((size_t)b * a.heads + h) * a.splits + j) * (D + 2);
                if (dl == 0) { w[0] = mg; w[1] = lg; }
#pragma unroll
                for (int i = 0; i < 8; ++i) w[2 + 8 * dl + i] = acc[g][i];
            }
        }
    }
}

// Row-streaming attention for ragged batches (binary16 caches, D = 128, 4 or
// 8 KV heads): one workgroup of KVH wavefronts (wavefront w = KV head w) per
// CU. A cache row holds every KV head of a position (the reference layout
// [position][kv_head][dim]), so a workgroup that serves all KV heads reads
// whole contiguous rows: per 16-position block its wavefronts copy 16 K rows
// and 16 V rows straight into LDS (LDS-DMA loads, 1 KB each, rows padded by 16
// bytes so the MFMA operand reads hit every bank), double buffered across
// blocks and sequences, and each wavefront runs the block step for its KV
// head from LDS: scores on MFMA as in MfmaAttn, online softmax, and P.V on
// MFMA as o^T += V^T P^T. Work split: the blocks of all sequences, in order,
// are divided into equal contiguous ranges, one per active workgroup (at least
// a.chunk blocks each); a sequence spread over several ranges writes one
// (m, l, o) partial per range, in the range's two slots (the segment holding
// its first block, the one running past its end), for attn_merge_rows_kernel.
// Lengths are clamped to max_len. batch <= 64.
constexpr int RBP = 16;   // positions per block

struct RowsPlan {
    uint32_t lenb, nbk, incl, rowb;   // lane b: length, blocks, inclusive block prefix, first cache row
    uint32_t T, nwg;                  // blocks in the launch, active workgroups
};

__device__ __forceinline__ RowsPlan rows_plan(const AttnArgs &a, int lane, uint32_t nwg_grid) {
    RowsPlan f;
    f.lenb = 0;
    f.nbk = 0;
    f.rowb = 0;
    if ((uint32_t)lane < a.batch) {
        f.lenb = min(min(a.seq_lens ? (uint32_t)a.seq_lens[lane] : a.seq_len, a.max_seq), a.max_len);
        f.nbk = f.lenb == 0 ? 1u : (f.lenb + RBP - 1) / RBP;   // an empty sequence still writes zeros
        f.rowb = a.row_base ? (uint32_t)a.row_base[lane] : (uint32_t)lane * a.max_seq;
    }
    f.incl = f.nbk;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t up = (uint32_t)__shfl_up((int)f.incl, o, 64);
        if (lane >= o) f.incl += up;
    }
    f.T = (uint32_t)__shfl((int)f.incl, 63, 64);
    const uint32_t cap = f.T / a.chunk;
    f.nwg = min(nwg_grid, cap ? cap : 1u);
    return f;
}
// floor(T * w / nwg) and the workgroup that holds block i. The products are
// below 2^53 and the divisors below 2^32, so correctly rounded double
// division followed by truncation is the exact integer quotient (a quotient
// that is not an integer is at least 1 / divisor away from one).
__device__ __forceinline__ uint32_t rows_begin(const RowsPlan &f, uint32_t w) {
    return (uint32_t)((double)((uint64_t)f.T * w) / (double)f.nwg);
}
__device__ __forceinline__ uint32_t rows_owner(const RowsPlan &f, uint32_t i) {
    return (uint32_t)((double)(((uint64_t)i + 1) * f.nwg - 1) / (double)f.T);
}

template <int D, int G, int KVH>
struct RowsLds {
    static constexpr uint32_t RB = KVH * D * 2;       // bytes of a cache row
    static constexpr uint32_t RP = RB + 16;           // LDS row pitch
    static constexpr uint32_t TILE = RBP * RP;        // 16 rows
    static constexpr uint32_t BUF = 2 * TILE;         // K and V tiles of a block
    static constexpr uint32_t NDMA = RBP / KVH * (RB / 1024) * 2;   // 1 KB requests per wavefront per block
    static constexpr uint32_t QW = G * D * 4;         // q of a wavefront's G heads (fp32)
    static constexpr uint32_t NQ = (QW + 1023) / 1024;   // requests for it
    static constexpr uint32_t BYTES = 2 * BUF + KVH * QW;
};

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (non-temporal; lds is wavefront-uniform and goes to M0). Issued as inline
// assembly so that the compiler tracks none of these requests: every wait for
// them is an explicit vmcnt wait below. M0 is named as clobbered, so the
// statement defines M0 for the compiler and no value of its own is assumed to
// survive it (clang warns that M0 is a reserved register; that is the point).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// s_waitcnt vmcnt(N), other counters unconstrained (gfx9 encoding)
template <uint32_t N> __device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int D, int G, int KVH>
__global__ __launch_bounds__(64 * KVH) void attn_rows_kernel(AttnArgs a) {
    using L = RowsLds<D, G, KVH>;
    constexpr int KS = D / 32, NT = D / 16;
    static_assert(D == 128 && (KVH == 4 || KVH == 8) && L::NDMA == 8 && G <= 8, "row streaming: D 128, 4 or 8 KV heads");
    static_assert(L::BYTES <= 160 * 1024, "row streaming: LDS");
    __shared__ __align__(16) unsigned char lds[L::BYTES];
    const int lane = threadIdx.x & 63;
    const uint32_t kvh = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    unsigned char *qw = lds + 2 * L::BUF + kvh * L::QW;   // this wavefront's q
    const int col = lane & 15, grp = lane >> 4;           // MFMA layout
    const RowsPlan f = rows_plan(a, lane, gridDim.x);
    const uint32_t w = blockIdx.x;
    if (w >= f.nwg) return;
    const uint32_t i0 = rows_begin(f, w), i1 = rows_begin(f, w + 1);
    const uint32_t kvrow = KVH * D;

    struct Blk { uint32_t b, j, nb, len, first; };
    auto locate = [&](uint32_t i) {
        Blk k;
        const uint64_t le = __ballot(f.incl <= i);   // sequences that end before block i
        k.b = (uint32_t)__popcll(le);
        k.nb = (uint32_t)__shfl((int)f.nbk, (int)k.b, 64);
        k.first = (uint32_t)__shfl((int)(f.incl - f.nbk), (int)k.b, 64);
        k.len = (uint32_t)__shfl((int)f.lenb, (int)k.b, 64);
        k.j = i - k.first;
        return k;
    };
    // This wavefront's share of block k's rows (RBP / KVH rows of K and of V)
    // into buffer buf; returns the number of requests (0 or NDMA).
    auto issue_rows = [&](int buf, const Blk &k) -> uint32_t {
        if (!k.len) return 0;
        const uint32_t rowb = (uint32_t)__shfl((int)f.rowb, (int)k.b, 64);
        const uint32_t kt = lds_addr(lds) + buf * L::BUF, vt = kt + L::TILE;
#pragma unroll
        for (int r = 0; r < RBP / KVH; ++r) {
            const uint32_t row = kvh * (RBP / KVH) + r;
            const uint32_t p = min(k.j * RBP + row, k.len - 1);   // rows past the end: masked, stay in the sequence
            const size_t e = ((size_t)rowb + p) * kvrow + lane * 8;
#pragma unroll
            for (uint32_t h = 0; h < L::RB / 1024; ++h) {
                lds_dma16((const _Float16 *)a.kc + e + h * 512, kt + row * L::RP + h * 1024);
                lds_dma16((const _Float16 *)a.vc + e + h * 512, vt + row * L::RP + h * 1024);
            }
        }
        return L::NDMA;
    };
    // q of the G heads of KV head kvh of sequence b (G * D contiguous floats)
    // into this wavefront's q area: NQ requests
    auto issue_q = [&](uint32_t b) {
        const float *src = a.q + ((size_t)b * a.heads + kvh * G) * D;
#pragma unroll
        for (uint32_t c = 0; c < L::NQ; ++c)
            if (L::QW >= 1024 * (c + 1) || lane * 16 < L::QW - 1024 * c)
                lds_dma16(src + c * 256 + lane * 4, lds_addr(qw) + c * 1024);
    };

    ah8 qh[KS], qm[KS], ql[KS];
    float sc2 = 0.0f;
    // acc[t]: o^T for dims 16t + 4*grp + e (e = 0..3) of head `col`, scaled by 2^14
    float m = -INFINITY, l = 0.0f;
    af4 acc[NT];

    Blk cur = locate(i0);
    bool cur_start = true;
    (void)issue_rows(0, cur);
    issue_q(cur.b);
    // q requests were made after the current block's rows: the wait for the
    // rows may leave them pending unless the block starts a segment
    bool q_newer = true;
    uint32_t i = i0;
    // One block: request block i + 1 into the other buffer, wait for block i,
    // run it. BUF is the buffer of block i.
    auto step = [&](auto BUF) {
        constexpr int buf = decltype(BUF)::value;
        const bool cur_end = i + 1 == i1 || cur.j + 1 == cur.nb;
        Blk nxt = cur;
        bool nxt_start = false;
        uint32_t nn = 0;
        if (i + 1 < i1) {
            nxt = locate(i + 1);
            nxt_start = cur_end;
            nn = issue_rows(buf ^ 1, nxt);
        }
        // requests complete in order: block i's rows (and q when the block
        // starts a segment) are older than the newest nn (+ NQ) requests
        const bool qp = q_newer && !cur_start;
        if (nn && qp) wait_vm<L::NDMA + L::NQ>();
        else if (nn) wait_vm<L::NDMA>();
        else if (qp) wait_vm<L::NQ>();
        else wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        q_newer = false;

        if (cur_start) {
            // q of head `col` (zero for col >= G), dims 8*grp + 32t + e
            float qv[KS][8];
            float qmax = 0.0f;
            const float *qs_lds = (const float *)qw + (col < G ? col : 0) * D + 8 * grp;
#pragma unroll
            for (int t = 0; t < KS; ++t) {
                const jf4 q0 = *(const jf4 *)(qs_lds + 32 * t), q1 = *(const jf4 *)(qs_lds + 32 * t + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    qv[t][e] = col < G ? q0[e] : 0.0f;
                    qv[t][4 + e] = col < G ? q1[e] : 0.0f;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) qmax = fmaxf(qmax, fabsf(qv[t][e]));
            }
            qmax = fmaxf(qmax, lane_xor<16>(qmax));
            qmax = fmaxf(qmax, lane_xor<32>(qmax));
            int qe = 0;
            (void)frexpf(qmax, &qe);                  // qmax < 2^qe
            const int sh = qe > 15 ? qe - 15 : 0;     // |q| * 2^-sh < 2^15
            const float qs = ldexpf(1.0f, -sh);
            sc2 = a.scale2 * ldexpf(1.0f, sh);
#pragma unroll
            for (int t = 0; t < KS; ++t)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = qv[t][e] * qs;
                    const _Float16 hi = (_Float16)x;
                    const float r = x - (float)hi;
                    const _Float16 mid = (_Float16)r;
                    qh[t][e] = hi;
                    qm[t][e] = mid;
                    ql[t][e] = (_Float16)(r - (float)mid);
                }
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = af4{0.0f, 0.0f, 0.0f, 0.0f};
            m = -INFINITY;
            l = 0.0f;
            // q of the next sequence, when its first block is in this range;
            // the q area is rewritten only after this wavefront's reads of it
            if (cur.first + cur.nb < i1) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                issue_q(cur.b + 1);
                q_newer = true;
            }
        }

        // ---- the block step for KV head kvh, K and V from LDS ----
        const unsigned char *kt = lds + buf * L::BUF, *vt = kt + L::TILE;
        const uint32_t p0 = cur.j * RBP, end = cur.len;
        if (p0 < end) {
            af4 S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < KS; ++t) {
                const ah8 kk = __builtin_bit_cast(
                    ah8, *(const uint4 *)(kt + col * L::RP + kvh * D * 2 + (8 * grp + 32 * t) * 2));
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, ql[t], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, qm[t], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(kk, qh[t], S, 0, 0, 0);
            }
            // S[r]: head col, position p0 + 4*grp + r
            float sv[4];
            float bm = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool live = p0 + 4 * grp + r < end;
                sv[r] = live ? S[r] * sc2 : -INFINITY;
                bm = fmaxf(bm, sv[r]);
            }
            bm = fmaxf(bm, lane_xor<16>(bm));
            bm = fmaxf(bm, lane_xor<32>(bm));
            const float mn = fmaxf(m, bm);
            const float alpha = mn == -INFINITY ? 1.0f : fexp2(m - mn);
            float ps[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ps[r] = mn == -INFINITY ? 0.0f : fexp2(sv[r] - mn);
            l = l * alpha + ((ps[0] + ps[1]) + (ps[2] + ps[3]));
            m = mn;
            // o^T += V^T P^T on v_mfma_f32_16x16x16_f16: A = V^T (dims x the
            // block's 16 positions, gathered from the LDS rows), B = P^T
            // straight from the softmax layout (lane = head col, positions
            // 4*grp + e) as binary16 hi + lo parts of 2^14 p (22 significant
            // bits; p below 2^-38 of the running maximum flushes to zero).
            // The rescale is per lane: every lane's column is its own head.
            ah4 ph, pl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = ps[r] * 16384.0f;
                const _Float16 hi = (_Float16)x;
                ph[r] = hi;
                pl[r] = (_Float16)(x - (float)hi);
            }
            const unsigned char *vcol = vt + (4 * grp) * L::RP + kvh * D * 2 + col * 2;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                ah4 va;
#pragma unroll
                for (int e = 0; e < 4; ++e) va[e] = *(const _Float16 *)(vcol + e * L::RP + 32 * t);
                acc[t] *= alpha;
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, acc[t], 0, 0, 0);
            }
        }

        if (cur_end) {
            // l over the 4 position groups; o^T is complete in every lane
            float lt = l + lane_xor<16>(l);
            lt += lane_xor<32>(lt);
            // the sequence's blocks all lie in this workgroup's range: write
            // the output; else a partial in slot 0 (the segment that holds the
            // range's first block) or slot 1 (the one that runs past its end)
            const bool whole = rows_owner(f, cur.first) == w && rows_owner(f, cur.first + cur.nb - 1) == w;
            const uint32_t slot2 = cur.first <= i0 ? 0u : 1u;
            if (col < G) {
                const uint32_t h = kvh * G + col;
                if (whole) {
                    const float inv = (1.0f / 16384.0f) / fmaxf(lt, 1e-20f);
                    const size_t at0 = ((size_t)cur.b * a.heads + h) * D + 4 * grp;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int e = 0; e < 4; ++e) put_out(a, at0 + 16 * t + e, acc[t][e] * inv);
                } else {
                    float *ws = a.ws + (((size_t)w * 2 + slot2) * a.heads + h) * (D + 2);
                    if (grp == 0) { ws[0] = m; ws[1] = lt; }
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int e = 0; e < 4; ++e) ws[2 + 16 * t + 4 * grp + e] = acc[t][e] * (1.0f / 16384.0f);
                }
            }
        }
        // every wavefront is done with this buffer before it is refilled
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        cur = nxt;
        cur_start = nxt_start;
        ++i;
    };
    while (i < i1) {
        step(std::integral_constant<int, 0>{});
        if (i >= i1) break;
        step(std::integral_constant<int, 1>{});
    }
}

// Merge of the row-streaming split: sequence b's segments are the partials
// of the workgroups whose ranges meet its blocks ([w][slot][head][D + 2]:
// slot 0 when the sequence holds the range's first block, else slot 1); a
// sequence inside one range was written directly. Per chunk of 32 segments,
// lane j finds segment j's partial; the o loads of every segment of the
// chunk are issued with the (m, l) loads (their addresses do not depend on
// the loaded values), so a chunk costs one memory round trip after the
// length table.
template <int D>
__global__ __launch_bounds__(D) void attn_merge_rows_kernel(AttnArgs a, uint32_t nwg_grid) {
    constexpr int CH = 32;
    const uint32_t h = blockIdx.x, b = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const RowsPlan f = rows_plan(a, lane, nwg_grid);
    const uint32_t nb = (uint32_t)__shfl((int)f.nbk, (int)b, 64);
    const uint32_t first = (uint32_t)__shfl((int)(f.incl - f.nbk), (int)b, 64);
    const uint32_t w0 = rows_owner(f, first), ns = rows_owner(f, first + nb - 1) - w0 + 1;
    if (ns <= 1) return;
    __shared__ uint32_t off_s[D / 64][CH];
    __shared__ float e_s[D / 64][CH];
    const int wv = threadIdx.x >> 6;
    float M = -INFINITY, L = 0.0f, o = 0.0f;
    // Idle lanes read the sequence's first segment (workgroup w0 always writes
    // it, since ns >= 2), so the zero weight they apply multiplies a partial of
    // this launch, never stale workspace bits (0 * inf would be NaN).
    const uint32_t off0 = ((w0 * 2 + (first <= rows_begin(f, w0) ? 0u : 1u)) * a.heads + h) * (D + 2);
    for (uint32_t j0 = 0; j0 < ns; j0 += CH) {
        const uint32_t j = j0 + lane;
        const bool mine = lane < CH && j < ns;
        uint32_t offj = off0;
        if (mine) {
            const uint32_t wj = w0 + j;
            const uint32_t slot = first <= rows_begin(f, wj) ? 0u : 1u;
            offj = ((wj * 2 + slot) * a.heads + h) * (D + 2);
        }
        if (lane < CH) off_s[wv][lane] = offj;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float ov[CH];
#pragma unroll
        for (int k = 0; k < CH; ++k) ov[k] = a.ws[off_s[wv][k] + 2 + threadIdx.x];
        const float mj = mine ? a.ws[offj] : -INFINITY;
        const float lj = mine ? a.ws[offj + 1] : 0.0f;
        float Mc = mj;
#pragma unroll
        for (int s2 = 32; s2 >= 1; s2 >>= 1) Mc = fmaxf(Mc, __shfl_xor(Mc, s2, 64));
        const float Mn = fmaxf(M, Mc);
        if (Mn != -INFINITY) {           // else no live segment yet
            const float r = fexp2(M - Mn);   // 0 while M = -inf
            const float ej = fexp2(mj - Mn); // 0 for dead segments and idle lanes
            float ls = lj * ej;
#pragma unroll
            for (int s2 = 32; s2 >= 1; s2 >>= 1) ls += __shfl_xor(ls, s2, 64);
            L = L * r + ls;
            o *= r;
            if (lane < CH) e_s[wv][lane] = ej;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int k = 0; k < CH; ++k) o = fmaf(e_s[wv][k], ov[k], o);
            M = Mn;
        }
        // the slots are rewritten by the next chunk
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    put_out(a, ((size_t)b * a.heads + h) * D + threadIdx.x, o / fmaxf(L, 1e-20f));
}

// Merge: o = sum_s o_s e^{m_s - M} / sum_s l_s e^{m_s - M}, in one pass over
// the splits with a running maximum. The partials of the first SB planned
// splits (8 or 16, the launch's choice) are requested together with the
// sequence length, which decides how many of them are live (the others hold
// earlier calls' values and are masked by selects), so a merge of up to SB
// splits costs one dependent round trip; further splits follow SB at a time. The first batch is folded
// whatever the length, so its loads stay ahead of the length's use; m and l
// are read by lanes 0 and 1 (vector loads, issued with the o loads) and
// broadcast.
template <int D, uint32_t SB>
__global__ __launch_bounds__(D) void attn_merge_kernel(AttnArgs a) {
    const uint32_t h = blockIdx.x, b = blockIdx.y;
    const float *w = a.ws + ((size_t)b * a.heads + h) * a.splits * (D + 2);
    const uint32_t len_raw = a.seq_lens ? (uint32_t)a.seq_lens[b] : a.seq_len;
    float ml[SB], os[SB];
    // splits s0 .. s0 + SB - 1 below lim; the rest re-read split s0 (in bounds)
    auto load = [&](uint32_t s0, uint32_t lim) {
#pragma unroll
        for (uint32_t j = 0; j < SB; ++j) {
            const float *ws = w + (size_t)(s0 + j < lim ? s0 + j : s0) * (D + 2);
            ml[j] = ws[threadIdx.x & 1u];
            os[j] = ws[2 + threadIdx.x];
        }
    };
    load(0, a.splits);
    __builtin_amdgcn_sched_barrier(0);   // the loads above issue before the length is waited for
    // lengths beyond the planned splits (or the capacity) are clamped, never read past
    const uint32_t span = a.nw * a.chunk;
    const uint32_t len = min(min(len_raw, a.max_seq), a.splits * span);
    // ns = 0: a single split, whose output the partial kernel wrote directly
    const uint32_t nsr = (len + span - 1) / span;   // division first: no branch ahead of the loads' uses
    const uint32_t ns = len > span ? nsr : 0;
    float M = -INFINITY, L = 0.0f, o = 0.0f;
    for (uint32_t s0 = 0;;) {
        float ms[SB];
#pragma unroll
        for (uint32_t j = 0; j < SB; ++j) {
            const bool live = s0 + j < ns;
            ms[j] = live ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml[j]), 0)) : -INFINITY;
            ml[j] = live ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ml[j]), 1)) : 0.0f;
            os[j] = live ? os[j] : 0.0f;
        }
        float Mn = M;
#pragma unroll
        for (uint32_t j = 0; j < SB; ++j) Mn = fmaxf(Mn, ms[j]);
        if (Mn != -INFINITY) {   // else no live split yet
            const float r = fexp2(M - Mn);
            L *= r;
            o *= r;
#pragma unroll
            for (uint32_t j = 0; j < SB; ++j) {
                const float f = fexp2(ms[j] - Mn);   // 0 for masked splits (m = -inf)
                L = fmaf(ml[j], f, L);
                o = fmaf(os[j], f, o);
            }
            M = Mn;
        }
        s0 += SB;
        if (s0 >= ns) break;
        load(s0, ns);
    }
    if (ns) put_out(a, ((size_t)b * a.heads + h) * D + threadIdx.x, o / fmaxf(L, 1e-20f));
}

template <int D>
void merge_launch(janus_ctx *ctx, const AttnArgs &a) {
    if (a.splits <= 8) hipLaunchKernelGGL((attn_merge_kernel<D, 8>), dim3(a.heads, a.batch), dim3(D), 0, ctx->stream, a);
    else hipLaunchKernelGGL((attn_merge_kernel<D, 16>), dim3(a.heads, a.batch), dim3(D), 0, ctx->stream, a);
}

template <typename KV, int D>
int launch_d(janus_ctx *ctx, const AttnArgs &a, uint32_t G) {
    if (a.qh_div) {   // one query head per workgroup
        dim3 grid(a.splits, a.heads, a.batch), block(64 * a.nw);
        const size_t lds = (size_t)a.nw * (D + 2) * 4;
        if (a.nw == 4) hipLaunchKernelGGL((attn_decode_kernel<KV, D, 1, 4>), grid, block, lds, ctx->stream, a);
        else if (a.nw == 8) hipLaunchKernelGGL((attn_decode_kernel<KV, D, 1, 8>), grid, block, lds, ctx->stream, a);
        else hipLaunchKernelGGL((attn_decode_kernel<KV, D, 1, 16>), grid, block, lds, ctx->stream, a);
        JANUS_LAUNCH_CHECK(ctx);
        if (a.splits > 1) {
            merge_launch<D>(ctx, a);
            JANUS_LAUNCH_CHECK(ctx);
        }
        return JANUS_OK;
    }
    if constexpr (D == 128 && std::is_same<KV, _Float16>::value) {
        if (a.rows) {   // row streaming: one workgroup of kv_heads wavefronts per CU
            const dim3 rgrid(ctx->num_cus);
#define JANUS_ROWS_CASE(GG, KK)                                                                               \
    if (G == GG && a.kv_heads == KK) {                                                                        \
        hipLaunchKernelGGL((attn_rows_kernel<D, GG, KK>), rgrid, dim3(64 * KK), 0, ctx->stream, a);           \
        found = true;                                                                                         \
    }
            bool found = false;
            JANUS_ROWS_CASE(1, 4) JANUS_ROWS_CASE(2, 4) JANUS_ROWS_CASE(4, 4) JANUS_ROWS_CASE(8, 4)
            JANUS_ROWS_CASE(1, 8) JANUS_ROWS_CASE(2, 8) JANUS_ROWS_CASE(4, 8)
#undef JANUS_ROWS_CASE
            if (!found) return fail(ctx, JANUS_E_INVALID_DIM, "attention: row streaming needs 4 or 8 KV heads, at most 32 heads");
            JANUS_LAUNCH_CHECK(ctx);
            if (a.splits > 1) {
                hipLaunchKernelGGL((attn_merge_rows_kernel<D>), dim3(a.heads, a.batch), dim3(D), 0, ctx->stream, a,
                                   (uint32_t)ctx->num_cus);
                JANUS_LAUNCH_CHECK(ctx);
            }
            return JANUS_OK;
        }
    }
    dim3 grid(a.splits, a.kv_heads, a.batch), block(64 * a.nw);
    const size_t lds = (size_t)a.nw * G * (D + 2) * 4;
    if (std::is_same<KV, _Float16>::value && a.nw == 1) {   // task mode (binary16 caches)
        const dim3 tgrid(ctx->num_cus * ctx->attn_wpc / 4);
        switch (G) {
        case 1: hipLaunchKernelGGL((attn_task_kernel<D, 1>), tgrid, dim3(256), 0, ctx->stream, a); break;
        case 2: hipLaunchKernelGGL((attn_task_kernel<D, 2>), tgrid, dim3(256), 0, ctx->stream, a); break;
        case 4: hipLaunchKernelGGL((attn_task_kernel<D, 4>), tgrid, dim3(256), 0, ctx->stream, a); break;
        case 8: hipLaunchKernelGGL((attn_task_kernel<D, 8>), tgrid, dim3(256), 0, ctx->stream, a); break;
        default: return fail(ctx, JANUS_E_INVALID_DIM, "attention: heads / kv_heads must be 1, 2, 4 or 8");
        }
        JANUS_LAUNCH_CHECK(ctx);
        if (a.splits > 1) {
            merge_launch<D>(ctx, a);
            JANUS_LAUNCH_CHECK(ctx);
        }
        return JANUS_OK;
    }
    const bool big = a.nw == 16;
    switch (G) {
    case 1:
        if (big) hipLaunchKernelGGL((attn_decode_kernel<KV, D, 1, 16>), grid, block, lds, ctx->stream, a);
        else hipLaunchKernelGGL((attn_decode_kernel<KV, D, 1, 4>), grid, block, lds, ctx->stream, a);
        break;
    case 2:
        if (big) hipLaunchKernelGGL((attn_decode_kernel<KV, D, 2, 16>), grid, block, lds, ctx->stream, a);
        else hipLaunchKernelGGL((attn_decode_kernel<KV, D, 2, 4>), grid, block, lds, ctx->stream, a);
        break;
    case 4:
        if (a.nw == 8) hipLaunchKernelGGL((attn_decode_kernel<KV, D, 4, 8>), grid, block, lds, ctx->stream, a);
        else hipLaunchKernelGGL((attn_decode_kernel<KV, D, 4, 4>), grid, block, lds, ctx->stream, a);
        break;
    case 8: hipLaunchKernelGGL((attn_decode_kernel<KV, D, 8, 4>), grid, block, lds, ctx->stream, a); break;
    default: return fail(ctx, JANUS_E_INVALID_DIM, "attention: heads / kv_heads must be 1, 2, 4 or 8");
    }
    JANUS_LAUNCH_CHECK(ctx);
    if (a.splits > 1) {
        merge_launch<D>(ctx, a);
        JANUS_LAUNCH_CHECK(ctx);
    }
    return JANUS_OK;
}

}  // namespace

// Splits each sequence's context over wavefronts so the launch has roughly 8
// wavefronts per CU (at least TP positions each). One workgroup per (sequence,
// head group), its wavefronts merged in LDS and no merge launch, for contexts
// of up to 512 positions, or up to 1024 when those workgroups fill at least
// half the CUs; otherwise the context splits over workgroups, with a merge
// kernel across the splits. Single-sequence attention per call (graph
// replays, 32 query heads of 128 dims, fp16 cache, plan for the length's
// bucket): 8 KV heads at 800 / 1500 / 3000 / 6000 positions 7.3 / 7.5 / 10.0 /
// 13.8 us with per-query-head splits against 9.6 / 11.0 / 15.5 / 18.3 us with
// one workgroup per head up to 1024 and KV-head splits beyond; 32 KV heads at
// 640-1024 positions 9.4-10.1 against 11.6-15.5 us with one workgroup per
// head. Four or eight sequences at 800 positions: 12.5 / 17.0 us with one
// workgroup per head against 13.8 / 17.9 split.
void attention_plan(const janus_ctx *ctx, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                    uint32_t max_len, int kv_f16, uint32_t *chunk_out, uint32_t *nw_out, uint32_t *splits_out,
                    uint32_t *qh_div_out, uint32_t *rows_out) {
    if (max_len == 0) max_len = 1;
    const uint32_t G = heads / kv_heads;
    *rows_out = 0;
    // Short contexts with few sequences: one workgroup per query head (the G
    // heads of a KV head re-read its rows from L2) so the launch spreads over
    // G times more CUs and each wavefront does 1/G of the arithmetic.
    // Beyond 1024 positions only while batch * heads is at most an eighth of
    // the CUs (4 sequences of 32 heads at 6000 positions: 70 us per query head
    // against 29 us per KV head; 1 sequence: 13.8 against 18.3 us).
    const uint64_t bh = (uint64_t)batch * heads;
    const bool qh = G > 1 && bh <= (uint64_t)ctx->num_cus && (max_len <= 1024 || 8 * bh <= (uint64_t)ctx->num_cus);
    *qh_div_out = qh ? G : 0;
    const uint64_t waves = (uint64_t)ctx->num_cus * (uint64_t)ctx->attn_wpc;
    // Row streaming (one workgroup per CU over ranges of 16-position blocks):
    // ragged batches that give every CU's range at least kRowsMinBlocks
    // blocks when all sequences are max_len long. Partials are kept per
    // workgroup (two slots), so their size depends on neither batch nor length.
    const uint64_t nbmax = (max_len + 15) / 16;
    const bool rows_ok = kv_f16 && !qh && !ctx->attn_valu && batch >= 2 && batch <= 64 && hd == 128 &&
                         (kv_heads == 4 || kv_heads == 8) && (G == 1 || G == 2 || G == 4 || G == 8) &&
                         heads == G * kv_heads && heads <= 32 && ctx->num_cus > 0 &&
                         rows_partial_bytes(ctx, heads, hd) <= kAttnScratchBytes;
    if (rows_ok && (ctx->attn_rows == 1 ||
                    (ctx->attn_rows < 0 && batch * nbmax >= (uint64_t)kRowsMinBlocks * ctx->num_cus))) {
        *rows_out = 1;
        *chunk_out = kRowsMinBlocks;
        *nw_out = kv_heads;
        *splits_out = 2;   // partial slots per workgroup
        return;
    }
    if (kv_f16 && !qh && !ctx->attn_valu && batch >= 2 && batch <= 64) {
        // task mode for ragged batches (nw = 1): pieces of `chunk` positions,
        // about two per wavefront when every sequence is max_len long (three
        // measured 77 against 74 us on config 4 and no better on config 5)
        uint64_t c = ctx->attn_task ? ctx->attn_task
                                    : ((uint64_t)max_len * batch * kv_heads + 2 * waves - 1) / (2 * waves);
        c = (c + TP - 1) / TP * TP;
        c = c < 64 ? 64 : (c > 1024 ? 1024 : c);
        *chunk_out = (uint32_t)c;
        *nw_out = 1;
        *splits_out = (uint32_t)((max_len + c - 1) / c);
        return;
    }
    const uint64_t groups = (uint64_t)batch * (qh ? heads : kv_heads);
    // one MHA sequence over 513-1024 positions: half the wavefronts per CU
    // (longer pieces, half the splits to merge): 7.8-9.0 us per call against
    // 8.6-9.7 at 520-1024 positions, 32 heads of 128 dims; at other lengths
    // and with GQA the full count is as fast or faster
    const uint64_t wv = (!qh && G == 1 && batch == 1 && max_len > 512 && max_len <= 1024 && waves >= 2 * ctx->num_cus)
                            ? waves / 2
                            : waves;
    uint64_t chunk = (max_len * groups + wv - 1) / wv;
    chunk = (chunk + TP - 1) / TP * TP;
    const bool single = max_len <= 512 || (max_len <= 1024 && 2 * groups >= (uint64_t)ctx->num_cus);
    // per-query-head launches: 8 wavefronts (bs=1 decode step at contexts
    // 148-348: 1.458 ms/token against 1.480 with 4 and with 16; split
    // contexts of 520-1024 positions 7.3-7.7 us against 8.0-8.4 with 4), 16
    // for one workgroup over 513-1024 positions. MHA (G = 1): 4 wavefronts
    // beyond 256 positions (300-500 positions in one workgroup 6.2-7.1 us
    // against 6.5-7.7 with 16).
    uint32_t nw;
    if (qh) nw = ctx->attn_qh_nw ? ctx->attn_qh_nw : (single && max_len > 512 ? 16u : 8u);
    else if (max_len > 1024 || !single || (G == 1 && max_len > 256)) nw = 4;
    else nw = G <= 2 ? 16 : (G == 4 ? 8 : 4);
    if (single && chunk * nw < max_len) chunk = (max_len + nw * TP - 1) / (nw * TP) * TP;
    *chunk_out = (uint32_t)chunk;
    *nw_out = nw;
    *splits_out = (uint32_t)((max_len + chunk * nw - 1) / (chunk * nw));
}

size_t attention_ws_bytes(const janus_ctx *ctx, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                          uint32_t max_len, int kv_f16) {
    uint32_t chunk, nw, splits, qh, rows;
    attention_plan(ctx, batch, heads, kv_heads, hd, max_len, kv_f16, &chunk, &nw, &splits, &qh, &rows);
    if (rows) return rows_partial_bytes(ctx, heads, hd);
    if (splits <= 1) return 0;
    return (size_t)batch * heads * splits * (hd + 2) * sizeof(float);
}

int attention_reserve(janus_ctx *ctx, uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd,
                      uint32_t max_len, int kv_f16) {
    const size_t bytes = attention_ws_bytes(ctx, batch, heads, kv_heads, hd, max_len, kv_f16);
    return bytes ? ensure_attn_ws(ctx, bytes) : JANUS_OK;
}

// ---- fixed scratch for the allocation-free entry point -------------------------
// The split partials of janus_attention_noalloc live in this array, one copy
// per device for the life of the process. Host code never passes the array's
// name to a kernel or a copy: it uses the device address that
// attention_scratch_init obtains per device with hipGetSymbolAddress.
static __device__ __align__(256) float scratch[kAttnScratchBytes / sizeof(float)];

namespace {
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

int attention_scratch_init(janus_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxScratchDevices) return JANUS_OK;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[ctx->device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(attention scratch)");
        g_scratch_ptr[ctx->device] = (float *)p;
    }
    ctx->attn_scratch = g_scratch_ptr[ctx->device];
    return JANUS_OK;
}

int attention_launch(janus_ctx *ctx, const float *q, const void *kc, const void *vc, int kv_dt, void *out,
                     uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t seq_len,
                     uint32_t max_seq, const int32_t *row_base, const int32_t *seq_lens, uint32_t max_len,
                     float scale, int out_f16, float *fixed_ws, size_t fixed_ws_bytes) {
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
    a.max_len = max_len;
    a.scale = scale;
    a.scale2 = scale * 1.4426950408889634f;
    a.out_f16 = out_f16;
    uint32_t chunk, nw, splits, qh, rows;
    attention_plan(ctx, batch, heads, kv_heads, hd, max_len, kv_dt == JANUS_DT_F16, &chunk, &nw, &splits, &qh,
                   &rows);
    a.chunk = chunk;
    a.nw = nw;
    a.qh_div = qh;
    a.rows = rows;
    a.splits = splits;
    a.ws = nullptr;
    if (splits > 1) {
        const size_t bytes = rows ? rows_partial_bytes(ctx, heads, hd)
                                  : (size_t)batch * heads * splits * (hd + 2) * sizeof(float);
        if (fixed_ws) {
            if (bytes > fixed_ws_bytes)
                return fail(ctx, JANUS_E_INVALID_DIM,
                            "attention: split partials need " + std::to_string(bytes) + " bytes, above the " +
                                std::to_string(fixed_ws_bytes) + "-byte fixed scratch");
            a.ws = fixed_ws;
        } else {
            if (int e = ensure_attn_ws(ctx, bytes)) return e;
            a.ws = (float *)ctx->attn_ws;
        }
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
