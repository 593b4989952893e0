// runtime.hip -- context, buffers, error reporting and weight upload/repack.
//
// Stands in for ComputeEngine (crates/janus-engine/src/compute/engine.rs):
// device init (:27-83), allocate_tensors' per-dtype layout choice
// (:424-858) and the f16 packing helpers (:112-136).
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <new>
#include <vector>

#include "internal.h"

namespace janus {

int fail(janus_ctx *ctx, int code, const std::string &msg) {
    if (ctx) ctx->last_error = msg;
    return code;
}

int hip_fail(janus_ctx *ctx, hipError_t e, const char *what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    int code = (e == hipErrorOutOfMemory) ? JANUS_E_OOM : JANUS_E_HIP;
    return fail(ctx, code, m);
}

namespace {

// Grows a context workspace to at least `bytes`. The old buffer is retired,
// not freed: a HIP graph captured earlier may still write it, so it lives
// until janus_destroy. Growth at least doubles the size, which bounds the
// retired memory by the final size. Growing while the stream is being
// captured is refused: the capture would record the new buffer, but
// allocating inside a capture is not allowed, so the caller must reserve
// first.
int grow_workspace(janus_ctx *ctx, void **buf, size_t *have, size_t bytes, size_t floor_bytes, const char *what) {
    if (*have >= bytes) return JANUS_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(ctx, JANUS_E_INVALID_ARG, std::string(what) + " workspace must grow to " + std::to_string(bytes) +
                                                  " bytes during graph capture; reserve it before capturing");
    size_t sz = bytes < floor_bytes ? floor_bytes : bytes;
    if (*buf && sz < 2 * *have) sz = 2 * *have;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess && sz > bytes && bytes >= floor_bytes) {
        sz = bytes;   // the doubling failed; the exact size may still fit
        e = hipMalloc(&p, sz);
    }
    if (e != hipSuccess) return hip_fail(ctx, e, what);
    if (*buf) ctx->retired.push_back(*buf);
    *buf = p;
    *have = sz;
    return JANUS_OK;
}

}  // namespace

int ensure_attn_ws(janus_ctx *ctx, size_t bytes) {
    return grow_workspace(ctx, &ctx->attn_ws, &ctx->attn_ws_bytes, bytes, 1u << 20, "hipMalloc(attention workspace)");
}

int ensure_gemm_ws(janus_ctx *ctx, size_t bytes) {
    return grow_workspace(ctx, &ctx->gemm_ws, &ctx->gemm_ws_bytes, bytes, 4u << 20, "hipMalloc(gemm workspace)");
}

int need_device(janus_ctx *ctx) {
    if (ctx->device < 0) return fail(ctx, JANUS_E_NO_DEVICE, "validation-only context has no device");
    return JANUS_OK;
}

size_t weight_qs_row_bytes(int type, uint32_t k) {
    switch (type) {
    case JANUS_DT_Q4_0: return (size_t)k / 32 * 16;
    case JANUS_DT_Q8_0: return (size_t)k / 32 * 32;
    case JANUS_DT_Q4_K: return (size_t)k / 256 * 144;
    case JANUS_DT_Q5_K: return (size_t)k / 256 * 176;
    case JANUS_DT_F16: return (size_t)k * 2;
    default: return 0;
    }
}

size_t weight_sc_row_elems(int type, uint32_t k) {
    return (type == JANUS_DT_Q4_0 || type == JANUS_DT_Q8_0) ? k / 32 : 0;
}

int weight_alloc(janus_ctx *ctx, int type, uint32_t n, uint32_t k, uint32_t flags, janus_weight **out) {
    const size_t qs_used = weight_qs_row_bytes(type, k) * n;
    const size_t sc_used = weight_sc_row_elems(type, k) * n * 2;
    const size_t qs_bytes = (qs_used + 255) & ~(size_t)255;
    const size_t total = qs_bytes + sc_used + 256;
    janus_weight *w = new (std::nothrow) janus_weight();
    if (!w) return fail(ctx, JANUS_E_OOM, "host allocation failed");
    hipError_t e = hipMalloc(&w->base, total);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(ctx, e, "hipMalloc(weight)");
    }
    w->type = type;
    w->n = n;
    w->k = k;
    w->flags = flags;
    w->bytes = total;
    w->qs = (const uint8_t *)w->base;
    w->sc = sc_used ? (const uint16_t *)((uint8_t *)w->base + qs_bytes) : nullptr;
    *out = w;
    return JANUS_OK;
}

}  // namespace janus

using namespace janus;

namespace {

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) (void)hipSetDevice(dev);
        else prev = -1;
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

inline uint16_t ftz16(uint16_t h) { return ((h & 0x7c00u) == 0) ? (uint16_t)(h & 0x8000u) : h; }

inline uint16_t f32_to_f16_host(float f) {
    _Float16 h = (_Float16)f;  // IEEE round-to-nearest-even
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// Q5_K in HBM: the GGML block with its 32 qh bytes rewritten as one 32-bit
// word per 16-byte quant chunk c = 2j + h (bytes 16 + 4c): for t = 0..15,
// bit 8 (t % 4) + t / 4 is the fifth bit of the low-nibble element of qs
// byte 32j + 16h + t (bit 2j of qh[16h + t]) and bit 8 (t % 4) + 4 + t / 4
// that of its high-nibble element (bit 2j + 1). A kernel then holds one
// register of high bits per chunk, and (w >> i) & 0x01010101 puts the bits
// of quant word i under its four bytes.
void q5k_pack_high_bits(uint8_t *blk) {
    uint8_t qh[32];
    std::memcpy(qh, blk + 16, 32);
    for (int c = 0; c < 8; ++c) {
        const int j = c / 2, h = c % 2;
        uint32_t w = 0;
        for (int t = 0; t < 16; ++t) {
            const uint32_t b = qh[16 * h + t];
            const int pos = 8 * (t % 4) + t / 4;
            w |= ((b >> (2 * j)) & 1u) << pos;
            w |= ((b >> (2 * j + 1)) & 1u) << (pos + 4);
        }
        for (int i = 0; i < 4; ++i) blk[16 + 4 * c + i] = (uint8_t)(w >> (8 * i));
    }
}

// The 12 GGML scale bytes of a Q4_K / Q5_K super-block (6-bit sc and m of
// the 8 sub-blocks, get_scale_min_k4's packing) rewritten in place as the
// chunk-pair fields of kq_group: field j (bits 24j .. 24j + 23 of bytes
// 4..15, little-endian) = sc(2j) | sc(2j+1) << 6 | m(2j) << 12 | m(2j+1) << 18.
void kquant_pack_scales(uint8_t *blk) {
    uint8_t s[12];
    std::memcpy(s, blk + 4, 12);
    uint32_t sc[8], mn[8];
    for (int i = 0; i < 8; ++i) {
        if (i < 4) {
            sc[i] = s[i] & 63u;
            mn[i] = s[i + 4] & 63u;
        } else {
            sc[i] = (s[i + 4] & 15u) | ((uint32_t)(s[i - 4] >> 6) << 4);
            mn[i] = (uint32_t)(s[i + 4] >> 4) | ((uint32_t)(s[i] >> 6) << 4);
        }
    }
    uint32_t w[3] = {0u, 0u, 0u};
    for (int j = 0; j < 4; ++j) {
        const uint32_t f = sc[2 * j] | (sc[2 * j + 1] << 6) | (mn[2 * j] << 12) | (mn[2 * j + 1] << 18);
        const int bit = 24 * j, wi = bit / 32, sh = bit % 32;
        w[wi] |= f << sh;
        if (sh + 24 > 32) w[wi + 1] |= f >> (32 - sh);
    }
    for (int i = 0; i < 12; ++i) blk[4 + i] = (uint8_t)(w[i / 4] >> (8 * (i % 4)));
}

// ---- dequantisation kernels (debug/bit-exactness entry) --------------------

__global__ void dequant_q4_0_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ sc,
                                    float *__restrict__ out, size_t nblocks) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    float d = h2f(sc[b]);
    const uint8_t *q = qs + b * 16;
    for (int j = 0; j < 16; ++j) {
        out[b * 32 + j] = d * (float)((int)(q[j] & 15) - 8);
        out[b * 32 + j + 16] = d * (float)((int)(q[j] >> 4) - 8);
    }
}

__global__ void dequant_q8_0_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ sc,
                                    float *__restrict__ out, size_t nblocks) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    float d = h2f_q8(sc[b]);
    const int8_t *q = (const int8_t *)(qs + b * 32);
    for (int j = 0; j < 32; ++j) out[b * 32 + j] = d * (float)q[j];
}

// sc and m of sub-block i from the packed scale words at blk + 4.
__device__ __forceinline__ void q4k_scale_min(const uint8_t *s, int i, int &sc, int &mn) {
    const uint32_t *w = (const uint32_t *)s;
    const uint32_t g = kq_group(w[0], w[1], w[2], (uint32_t)i >> 1), o = 6u * (uint32_t)(i & 1);
    sc = (int)((g >> o) & 63u);
    mn = (int)((g >> (12u + o)) & 63u);
}

__global__ void dequant_q4_k_kernel(const uint8_t *__restrict__ blocks, float *__restrict__ out,
                                    size_t nblocks) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t *blk = blocks + b * 144;
    float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    float dmin = h2f((uint16_t)(blk[2] | (blk[3] << 8)));
    for (int j = 0; j < 4; ++j) {
        int sl, ml, sh, mh;
        q4k_scale_min(blk + 4, 2 * j, sl, ml);
        q4k_scale_min(blk + 4, 2 * j + 1, sh, mh);
        float scale_lo = d * (float)sl, min_lo = dmin * (float)ml;
        float scale_hi = d * (float)sh, min_hi = dmin * (float)mh;
        for (int t = 0; t < 32; ++t) {
            uint8_t byte = blk[16 + 32 * j + t];
            out[b * 256 + 64 * j + t] = scale_lo * (float)(byte & 15) - min_lo;
            out[b * 256 + 64 * j + 32 + t] = scale_hi * (float)(byte >> 4) - min_hi;
        }
    }
}

// Q5_K (GGML block_q5_K, high bits packed per chunk by q5k_pack_high_bits):
// the Q4_K form with a fifth bit per element. (d*sc)*q is exact in binary32
// (11 + 6 + 5 bits), so the one rounding is the difference.
__global__ void dequant_q5_k_kernel(const uint8_t *__restrict__ blocks, float *__restrict__ out,
                                    size_t nblocks) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t *blk = blocks + b * 176;
    float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    float dmin = h2f((uint16_t)(blk[2] | (blk[3] << 8)));
    const uint32_t *qh = (const uint32_t *)(blk + 16);
    const uint8_t *qs = blk + 48;
    for (int j = 0; j < 4; ++j) {
        int sl, ml, sh, mh;
        q4k_scale_min(blk + 4, 2 * j, sl, ml);
        q4k_scale_min(blk + 4, 2 * j + 1, sh, mh);
        float scale_lo = d * (float)sl, min_lo = dmin * (float)ml;
        float scale_hi = d * (float)sh, min_hi = dmin * (float)mh;
        for (int t = 0; t < 32; ++t) {
            const uint8_t byte = qs[32 * j + t];
            const uint32_t w = qh[2 * j + t / 16];
            const int pos = 8 * (t % 4) + (t % 16) / 4;
            const int lo = (byte & 15) | (int)(((w >> pos) & 1u) << 4);
            const int hi = (byte >> 4) | (int)(((w >> (pos + 4)) & 1u) << 4);
            out[b * 256 + 64 * j + t] = scale_lo * (float)lo - min_lo;
            out[b * 256 + 64 * j + 32 + t] = scale_hi * (float)hi - min_hi;
        }
    }
}

__global__ void dequant_f16_kernel(const uint16_t *__restrict__ in, float *__restrict__ out, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = h2f(in[i]);
}

}  // namespace

extern "C" {

int janus_abi_version(void) { return JANUS_ABI_VERSION; }

const char *janus_status_string(int s) {
    switch (s) {
    case JANUS_OK: return "ok";
    case JANUS_E_INVALID_ARG: return "invalid argument";
    case JANUS_E_INVALID_DIM: return "invalid dimensions";
    case JANUS_E_UNSUPPORTED_DTYPE: return "unsupported dtype";
    case JANUS_E_KV_OVERFLOW: return "kv cache overflow";
    case JANUS_E_TOKEN_RANGE: return "token id out of range";
    case JANUS_E_HIP: return "hip error";
    case JANUS_E_OOM: return "out of device memory";
    case JANUS_E_NO_DEVICE: return "no device";
    case JANUS_E_NAN_LOGITS: return "NaN logits";
    default: return "unknown status";
    }
}

int janus_device_count(int *count) {
    if (!count) return JANUS_E_INVALID_ARG;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return JANUS_OK;
}

int janus_create(int hip_device, janus_ctx **out) {
    if (!out) return JANUS_E_INVALID_ARG;
    *out = nullptr;
    if (hip_device == -1) {   // validation-only context: host-side checks, no device work
        janus_ctx *v = new (std::nothrow) janus_ctx();
        if (!v) return JANUS_E_OOM;
        v->device = -1;
        *out = v;
        return JANUS_OK;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return JANUS_E_NO_DEVICE;
    if (hip_device < 0 || hip_device >= n) return JANUS_E_INVALID_ARG;
    janus_ctx *ctx = new (std::nothrow) janus_ctx();
    if (!ctx) return JANUS_E_OOM;
    ctx->device = hip_device;
    if (hipSetDevice(hip_device) != hipSuccess) {
        delete ctx;
        return JANUS_E_HIP;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, hip_device) == hipSuccess) ctx->num_cus = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return JANUS_E_HIP;
    }
    ctx->stream = ctx->own_stream;
    // the allocation-free attention entry point's scratch: its device address
    // on this device (a failure is reported by that entry point)
    if (attention_scratch_init(ctx) != JANUS_OK) {
        ctx->attn_scratch_error = ctx->last_error;
        ctx->last_error.clear();
    }
    if (const char *k = std::getenv("JANUS_GEMV_KERNEL")) ctx->gemv_lds = std::strcmp(k, "reg") != 0;
    if (const char *k = std::getenv("JANUS_ATTN_KERNEL")) ctx->attn_valu = std::strcmp(k, "valu") == 0;
    if (const char *k = std::getenv("JANUS_ATTN_WPC")) {
        const long v = std::strtol(k, nullptr, 10);
        if (v >= 1 && v <= 32) ctx->attn_wpc = (uint32_t)v;
    }
    if (const char *k = std::getenv("JANUS_GEMV_WPC")) {
        const long v = std::strtol(k, nullptr, 10);
        if (v >= 4 && v <= 64) ctx->gemv_wpc = (uint32_t)v;
    }
    if (const char *k = std::getenv("JANUS_GEMV_LDS_WPC")) {
        const long v = std::strtol(k, nullptr, 10);
        if (v >= 8 && v <= 64) ctx->gemv_lds_wpc = (uint32_t)v;
    }
    if (const char *k = std::getenv("JANUS_GEMV_LDS_THREADS")) {
        const int v = std::atoi(k);
        if (v >= 256 && v <= 1024 && v % 64 == 0) ctx->gemv_lds_threads = (uint32_t)v;
    }
    if (const char *k = std::getenv("JANUS_GEMV_F16_ROWS")) ctx->gemv_f16_rows2 = std::strcmp(k, "1") != 0;
    if (const char *k = std::getenv("JANUS_GEMM_PIPE")) ctx->gemm_pipe = std::strcmp(k, "0") != 0;
    if (const char *k = std::getenv("JANUS_EPI_SPLIT")) ctx->epi_split = std::strcmp(k, "0") != 0;
    if (const char *k = std::getenv("JANUS_GRAPH_BUCKETS")) ctx->graph_buckets = std::strcmp(k, "0") != 0;
    if (const char *k = std::getenv("JANUS_GEMM_KR")) {
        const long v = std::strtol(k, nullptr, 10);
        if (v == 256 || v == 512 || v == 1024) ctx->gemm_kr = (uint32_t)v;
    }
    if (const char *k = std::getenv("JANUS_GEMM_KS")) {
        const long v = std::strtol(k, nullptr, 10);
        if (v >= 1 && v <= 64) ctx->gemm_ks = (uint32_t)v;
    }
    if (const char *k = std::getenv("JANUS_ATTN_QH_NW")) {
        const long v = std::strtol(k, nullptr, 10);
        if (v == 4 || v == 8 || v == 16) ctx->attn_qh_nw = (uint32_t)v;
    }
    if (const char *k = std::getenv("JANUS_ATTN_ROWS")) {
        if (!std::strcmp(k, "0")) ctx->attn_rows = 0;
        else if (!std::strcmp(k, "1")) ctx->attn_rows = 1;
    }
    if (const char *k = std::getenv("JANUS_FUSED")) ctx->fused_step = std::strcmp(k, "0") != 0;
    if (const char *k = std::getenv("JANUS_ATTN_TASK")) {
        const long v = std::strtol(k, nullptr, 10);
        if (v >= 16 && v <= 4096) ctx->attn_task = (uint32_t)v;
    }
    *out = ctx;
    return JANUS_OK;
}

void janus_destroy(janus_ctx *ctx) {
    if (!ctx) return;
    if (ctx->device < 0) {
        delete ctx;
        return;
    }
    DeviceGuard g(ctx->device);
    if (ctx->own_stream) (void)hipStreamSynchronize(ctx->own_stream);
    if (ctx->stream && ctx->stream != ctx->own_stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->attn_ws) (void)hipFree(ctx->attn_ws);
    if (ctx->gemm_ws) (void)hipFree(ctx->gemm_ws);
    for (void *p : ctx->retired) (void)hipFree(p);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

const char *janus_last_error(const janus_ctx *ctx) { return ctx ? ctx->last_error.c_str() : ""; }

int janus_set_stream(janus_ctx *ctx, void *s) {
    if (!ctx) return JANUS_E_INVALID_ARG;
    if (int e = need_device(ctx)) return e;
    ctx->stream = (hipStream_t)s;   // NULL is the device's legacy default stream
    return JANUS_OK;
}

void *janus_get_stream(janus_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int janus_workspace_bytes(const janus_ctx *ctx, size_t *attn_bytes, size_t *gemm_bytes) {
    if (!ctx) return JANUS_E_INVALID_ARG;
    if (attn_bytes) *attn_bytes = ctx->attn_ws_bytes;
    if (gemm_bytes) *gemm_bytes = ctx->gemm_ws_bytes;
    return JANUS_OK;
}

int janus_sync(janus_ctx *ctx) {
    if (!ctx) return JANUS_E_INVALID_ARG;
    if (int e = need_device(ctx)) return e;
    DeviceGuard g(ctx->device);
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
    return JANUS_OK;
}

int janus_alloc(janus_ctx *ctx, size_t bytes, void **d_ptr) {
    if (!ctx || !d_ptr || bytes == 0) return fail(ctx, JANUS_E_INVALID_ARG, "janus_alloc: bad argument");
    if (int e = need_device(ctx)) return e;
    DeviceGuard g(ctx->device);
    JANUS_HIP_CHECK(ctx, hipMalloc(d_ptr, bytes));
    return JANUS_OK;
}

int janus_free(janus_ctx *ctx, void *d_ptr) {
    if (!ctx) return JANUS_E_INVALID_ARG;
    if (!d_ptr) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    DeviceGuard g(ctx->device);
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
    JANUS_HIP_CHECK(ctx, hipFree(d_ptr));
    return JANUS_OK;
}

int janus_h2d(janus_ctx *ctx, void *d, const void *h, size_t bytes) {
    if (!ctx || (!d && bytes) || (!h && bytes)) return fail(ctx, JANUS_E_INVALID_ARG, "janus_h2d: null pointer");
    if (!bytes) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    DeviceGuard g(ctx->device);
    JANUS_HIP_CHECK(ctx, hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, ctx->stream));
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
    return JANUS_OK;
}

int janus_d2h(janus_ctx *ctx, void *h, const void *d, size_t bytes) {
    if (!ctx || (!d && bytes) || (!h && bytes)) return fail(ctx, JANUS_E_INVALID_ARG, "janus_d2h: null pointer");
    if (!bytes) return JANUS_OK;
    if (int e = need_device(ctx)) return e;
    DeviceGuard g(ctx->device);
    JANUS_HIP_CHECK(ctx, hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, ctx->stream));
    JANUS_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
    return JANUS_OK;
}

int janus_weight_upload(janus_ctx *ctx, int type, uint32_t n, uint32_t k, const void *bytes,
                        size_t nbytes, uint32_t flags, janus_weight **out) {
    if (!ctx || !out || !bytes) return fail(ctx, JANUS_E_INVALID_ARG, "janus_weight_upload: null argument");
    *out = nullptr;
    if (n == 0 || k == 0) return fail(ctx, JANUS_E_INVALID_DIM, "janus_weight_upload: empty tensor");
    const uint8_t *src = (const uint8_t *)bytes;
    size_t elems = (size_t)n * k;
    std::vector<uint8_t> qs;
    std::vector<uint16_t> sc;
    bool ftz = (flags & JANUS_WEIGHT_FTZ_F16) != 0;
    switch (type) {
    case JANUS_DT_F32: {
        if (nbytes != elems * 4) return fail(ctx, JANUS_E_INVALID_DIM, "F32 tensor byte size mismatch");
        qs.resize(elems * 2);
        uint16_t *dst = (uint16_t *)qs.data();
        for (size_t i = 0; i < elems; ++i) {
            float f;
            std::memcpy(&f, src + 4 * i, 4);
            uint16_t h = f32_to_f16_host(f);
            dst[i] = ftz ? ftz16(h) : h;
        }
        type = JANUS_DT_F16;
        break;
    }
    case JANUS_DT_F16: {
        if (nbytes != elems * 2) return fail(ctx, JANUS_E_INVALID_DIM, "F16 tensor byte size mismatch");
        qs.resize(elems * 2);
        uint16_t *dst = (uint16_t *)qs.data();
        for (size_t i = 0; i < elems; ++i) {
            uint16_t h = rd16(src + 2 * i);
            dst[i] = ftz ? ftz16(h) : h;
        }
        break;
    }
    case JANUS_DT_Q4_0:
    case JANUS_DT_Q8_0: {
        if (k % 32) return fail(ctx, JANUS_E_INVALID_DIM,
                                "quantized gemm requires cols to be multiple of 32, got " + std::to_string(k));
        size_t nblk = elems / 32, bb = (type == JANUS_DT_Q4_0) ? 18 : 34, qb = bb - 2;
        if (nbytes != nblk * bb) return fail(ctx, JANUS_E_INVALID_DIM, "quantized tensor byte size mismatch");
        qs.resize(nblk * qb);
        sc.resize(nblk);
        for (size_t b = 0; b < nblk; ++b) {
            sc[b] = rd16(src + b * bb);
            std::memcpy(qs.data() + b * qb, src + b * bb + 2, qb);
        }
        break;
    }
    case JANUS_DT_Q4_K:
    case JANUS_DT_Q5_K: {
        const bool q5 = type == JANUS_DT_Q5_K;
        const size_t bb = q5 ? 176 : 144;
        if (k % 256) return fail(ctx, JANUS_E_INVALID_DIM,
                                 std::string(q5 ? "Q5_K" : "Q4_K") +
                                     " gemm requires cols to be multiple of 256, got " + std::to_string(k));
        size_t nblk = elems / 256;
        if (nbytes != nblk * bb) return fail(ctx, JANUS_E_INVALID_DIM, "K-quant tensor byte size mismatch");
        qs.assign(src, src + nbytes);
        for (size_t b = 0; b < nblk; ++b) {
            kquant_pack_scales(qs.data() + b * bb);
            if (q5) q5k_pack_high_bits(qs.data() + b * bb);
        }
        if (ftz)
            for (size_t b = 0; b < nblk; ++b) {
                uint8_t *blk = qs.data() + b * bb;
                for (int o = 0; o < 4; o += 2) {
                    uint16_t h = ftz16(rd16(blk + o));
                    blk[o] = (uint8_t)(h & 0xff);
                    blk[o + 1] = (uint8_t)(h >> 8);
                }
            }
        break;
    }
    case JANUS_DT_Q6_K: {
        // The reference dequantises Q6_K on the host and keeps binary16
        // weights (engine.rs:800-831); so does this upload, in GGML element
        // order or, with JANUS_WEIGHT_Q6K_REF_ORDER, in q6_k_to_f32's
        // (engine.rs:198-248). Both form (d * scale) * (q - 32) in binary32
        // and round to binary16 to nearest even.
        if (k % 256) return fail(ctx, JANUS_E_INVALID_DIM,
                                 "Q6_K requires cols to be multiple of 256, got " + std::to_string(k));
        size_t nblk = elems / 256;
        if (nbytes != nblk * 210)
            return fail(ctx, JANUS_E_INVALID_DIM,
                        "Q6_K tensor byte size " + std::to_string(nbytes) + " is not " + std::to_string(nblk) +
                            " blocks of 210");
        const bool ref_order = (flags & JANUS_WEIGHT_Q6K_REF_ORDER) != 0;
        qs.resize(elems * 2);
        uint16_t *dst = (uint16_t *)qs.data();
        for (size_t b = 0; b < nblk; ++b) {
            const uint8_t *blk = src + b * 210, *ql = blk, *qh = blk + 128;
            const int8_t *sc = (const int8_t *)(blk + 192);
            _Float16 dh;
            uint16_t dbits = rd16(blk + 208);
            std::memcpy(&dh, &dbits, 2);
            const float d = (float)dh;
            uint16_t *o = dst + b * 256;
            for (int i = 0; i < 256; ++i) {
                int q, s;
                if (ref_order) {
                    const unsigned lo = (i & 1) ? (ql[i / 2] >> 4) : (ql[i / 2] & 15u);
                    const unsigned hi = (qh[i / 4] >> (2 * (i % 4))) & 3u;
                    q = (int)((hi << 4) | lo) - 32;
                    s = sc[i / 16];
                } else {
                    // element i = 128 h + 32 p + l: ql byte 64 h + l (+ 32 for p odd),
                    // nibble p / 2, qh byte 32 h + l bits 2 p, scale 8 h + l / 16 + 2 p
                    const int h = i >> 7, p = (i >> 5) & 3, l = i & 31;
                    const uint8_t qlb = ql[64 * h + l + ((p & 1) ? 32 : 0)];
                    const unsigned lo = (p & 2) ? (qlb >> 4) : (qlb & 15u);
                    const unsigned hi = (qh[32 * h + l] >> (2 * p)) & 3u;
                    q = (int)((hi << 4) | lo) - 32;
                    s = sc[8 * h + l / 16 + 2 * p];
                }
                const float v = d * (float)s * (float)q;
                const uint16_t hb = f32_to_f16_host(v);
                o[i] = ftz ? ftz16(hb) : hb;
            }
        }
        type = JANUS_DT_F16;
        break;
    }
    default:
        return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "unsupported tensor dtype " + std::to_string(type));
    }
    if (int e = need_device(ctx)) return e;
    DeviceGuard g(ctx->device);
    janus_weight *w = nullptr;
    if (int st = weight_alloc(ctx, type, n, k, flags, &w)) return st;
    hipError_t e = hipMemcpy(w->base, qs.data(), qs.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && !sc.empty())
        e = hipMemcpy((void *)w->sc, sc.data(), sc.size() * 2, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(w->base);
        delete w;
        return hip_fail(ctx, e, "hipMemcpy(weight)");
    }
    *out = w;
    return JANUS_OK;
}

int janus_weight_free(janus_ctx *ctx, janus_weight *w) {
    if (!w) return JANUS_OK;
    if (ctx && ctx->device >= 0) {
        DeviceGuard g(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
    }
    if (w->base) (void)hipFree(w->base);
    if (w->t32) (void)hipFree(w->t32);
    delete w;
    return JANUS_OK;
}

int janus_weight_info(const janus_weight *w, int *type, uint32_t *n, uint32_t *k, size_t *bytes) {
    if (!w) return JANUS_E_INVALID_ARG;
    if (type) *type = w->type;
    if (n) *n = w->n;
    if (k) *k = w->k;
    if (bytes) *bytes = w->bytes;
    return JANUS_OK;
}

int janus_weight_dequant(janus_ctx *ctx, const janus_weight *w, float *d_out) {
    if (!ctx || !w || !d_out) return fail(ctx, JANUS_E_INVALID_ARG, "janus_weight_dequant: null argument");
    if (int e = need_device(ctx)) return e;
    DeviceGuard g(ctx->device);
    size_t elems = (size_t)w->n * w->k;
    const int T = 256;
    switch (w->type) {
    case JANUS_DT_Q4_0: {
        size_t nb = elems / 32;
        dequant_q4_0_kernel<<<(unsigned)((nb + T - 1) / T), T, 0, ctx->stream>>>(w->qs, w->sc, d_out, nb);
        break;
    }
    case JANUS_DT_Q8_0: {
        size_t nb = elems / 32;
        dequant_q8_0_kernel<<<(unsigned)((nb + T - 1) / T), T, 0, ctx->stream>>>(w->qs, w->sc, d_out, nb);
        break;
    }
    case JANUS_DT_Q4_K: {
        size_t nb = elems / 256;
        dequant_q4_k_kernel<<<(unsigned)((nb + T - 1) / T), T, 0, ctx->stream>>>(w->qs, d_out, nb);
        break;
    }
    case JANUS_DT_Q5_K: {
        size_t nb = elems / 256;
        dequant_q5_k_kernel<<<(unsigned)((nb + T - 1) / T), T, 0, ctx->stream>>>(w->qs, d_out, nb);
        break;
    }
    case JANUS_DT_F16:
        dequant_f16_kernel<<<(unsigned)((elems + T - 1) / T), T, 0, ctx->stream>>>((const uint16_t *)w->qs,
                                                                                   d_out, elems);
        break;
    default:
        return fail(ctx, JANUS_E_UNSUPPORTED_DTYPE, "dequant: unsupported dtype");
    }
    JANUS_LAUNCH_CHECK(ctx);
    return JANUS_OK;
}

}  // extern "C"
