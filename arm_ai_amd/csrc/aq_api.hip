// aq_api.hip -- the extern "C" boundary (include/aq.h) of libarm_ai_amd.so.
//
// Host-side replacement for candle-core 0.8.4's QMatMul / QTensor on the
// CPU (reached from native/arm_ai_nif/src/llama_candle.rs:42 at load and
// :93 / :119 at prefill / decode).  Weights are uploaded once, repacked into
// the HBM row-block tile layout (aq_internal.h), and every matmul runs on the context's
// stream as either one matvec kernel that quantises the f32 activation itself
// (m <= 8), or the activation quantizer kernel (Q8_K, or Q8_0 for Q8_0
// weights) followed by the MFMA GEMM (m > 8).  Errors are status codes plus
// a thread-local message;
// nothing here aborts (the reference crate builds with panic = "abort",
// Cargo.toml:33, which this library must not inherit).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "../../include/aq.h"
#include "aq_internal.h"

using namespace aq;

struct aq_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    void *scratch = nullptr;  // device, grow-only
    size_t scratch_bytes = 0;
    void *pinned = nullptr;  // host staging, grow-only
    size_t pinned_bytes = 0;
    void *fixed_scratch = nullptr;  // this device's copy of g_fixed_scratch (its device address)
    // decode attention's per-slice partial records: allocated with the
    // context, so a captured decode step never allocates
    float *attn_part = nullptr;
    // the output head's per-workgroup (largest logit, row) pairs
    int2 *head_part = nullptr;
};
constexpr size_t ATTN_PART_BYTES = (size_t)2 << 20;
constexpr int HEAD_PARTS = 4096;

// Scratch of aq_qmatmul_f32_device_noalloc: a fixed array in the library's
// device image, one copy per GPU (held until the process ends).  Its name is
// only a host-side handle: device code receives the address that
// hipGetSymbolAddress returns for the current device (fixed_scratch_of).
constexpr size_t FIXED_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) uint8_t g_fixed_scratch[FIXED_SCRATCH_BYTES];

struct aq_qweight {
    int type = 0;
    int device = 0;
    int64_t n = 0, k = 0;
    void *base = nullptr;
    size_t bytes = 0;
    WLayout layout{};
    // the layout the prefill GEMM reads: the same tiles, except for Q4_0,
    // whose GEMM runs on an expanded copy in the Q8_0 tile layout (values
    // q - 8 as int8), kept after the decode tiles in the same allocation
    WLayout glayout{};
};

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(call)                                                                      \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess) return fail(AQ_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

int block_elems(int type) {
    switch (type) {
    case AQ_TYPE_Q2_K:
    case AQ_TYPE_Q3_K:
    case AQ_TYPE_Q4_K:
    case AQ_TYPE_Q5_K:
    case AQ_TYPE_Q6_K: return QK_K;
    case AQ_TYPE_Q8_0:
    case AQ_TYPE_Q4_0:
    case AQ_TYPE_Q5_0: return QK8_0;
    default: return 0;
    }
}
int block_bytes(int type) {
    switch (type) {
    case AQ_TYPE_Q2_K: return 84;
    case AQ_TYPE_Q3_K: return 110;
    case AQ_TYPE_Q4_K: return 144;
    case AQ_TYPE_Q5_K: return 176;
    case AQ_TYPE_Q6_K: return 210;
    case AQ_TYPE_Q8_0: return 34;
    case AQ_TYPE_Q4_0: return 18;
    case AQ_TYPE_Q5_0: return 22;
    default: return 0;
    }
}

int use_device(int device) {
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur == device) return AQ_OK;
    HIP_TRY(hipSetDevice(device));
    return AQ_OK;
}

// The device address of g_fixed_scratch on `device`, looked up once per
// device with that device current (aq_ctx_create makes it current).
constexpr int MAX_DEVICES = 64;
std::mutex g_fixed_mu;
void *g_fixed_ptr[MAX_DEVICES] = {};
int fixed_scratch_of(int device, void **out) {
    if (device < 0 || device >= MAX_DEVICES) return fail(AQ_ERR_NO_DEVICE, "device %d beyond the fixed-scratch table", device);
    std::lock_guard<std::mutex> lk(g_fixed_mu);
    if (!g_fixed_ptr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_fixed_scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return fail(AQ_ERR_HIP, "hipGetSymbolAddress of the fixed scratch failed: %s", hipGetErrorString(e));
        }
        g_fixed_ptr[device] = p;
    }
    *out = g_fixed_ptr[device];
    return AQ_OK;
}

int ensure_scratch(aq_ctx *c, size_t bytes) {
    if (bytes <= c->scratch_bytes) return AQ_OK;
    size_t want = align_up(bytes + bytes / 4, 1 << 20);
    if (c->scratch) {
        HIP_TRY(hipStreamSynchronize(c->stream));
        HIP_TRY(hipFree(c->scratch));
        c->scratch = nullptr;
        c->scratch_bytes = 0;
    }
    void *p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        return fail(AQ_ERR_OOM, "hipMalloc of %zu bytes of scratch failed", want);
    }
    c->scratch = p;
    c->scratch_bytes = want;
    return AQ_OK;
}

int ensure_pinned(aq_ctx *c, size_t bytes) {
    if (bytes <= c->pinned_bytes) return AQ_OK;
    size_t want = align_up(bytes + bytes / 4, 1 << 20);
    if (c->pinned) {
        HIP_TRY(hipStreamSynchronize(c->stream));
        HIP_TRY(hipHostFree(c->pinned));
        c->pinned = nullptr;
        c->pinned_bytes = 0;
    }
    void *p = nullptr;
    if (hipHostMalloc(&p, want, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return fail(AQ_ERR_OOM, "hipHostMalloc of %zu bytes failed", want);
    }
    c->pinned = p;
    c->pinned_bytes = want;
    return AQ_OK;
}

bool use_mmv(const aq_qweight *w, int64_t m);

// Scratch layout for one matmul call: [activation planes | x f32 | y f32 | S | Smin | gemm or
// batched-matvec workspace]
struct CallLayout {
    size_t act, x, y, s, smin, ws, total;
};
CallLayout call_layout(const aq_qweight *w, int64_t m, bool host_io, bool dump, bool gemm) {
    CallLayout L;
    size_t off = 0;
    L.act = off;
    off += align_up(act_sizes(m, w->k).total, 256);
    L.x = off;
    if (host_io) off += align_up((size_t)m * w->k * 4, 256);
    L.y = off;
    if (host_io) off += align_up((size_t)m * w->n * 4, 256);
    const size_t nblk = (size_t)(w->k / block_elems(w->type));
    L.s = off;
    if (dump) off += align_up((size_t)m * w->n * nblk * 4, 256);
    L.smin = off;
    if (dump) off += align_up((size_t)m * w->n * nblk * 4, 256);
    L.ws = off;
    // (a GEMM that declines the shape falls back to the batched matvec: room for either)
    size_t ws = gemm ? gemm_workspace_bytes(w->glayout.type, m, w->n, w->k) : 0;
    if (use_mmv(w, m)) ws = std::max(ws, mmv_workspace_bytes(w->layout.type, w->n, w->k));
    off += align_up(ws, 256);
    L.total = off;
    return L;
}

bool use_gemm(const aq_qweight *w, int64_t m) {
    return m > 8 && gemm_workspace_bytes(w->glayout.type, m, w->n, w->k) != (size_t)-1;
}
// 2 or more rows of Q4_K / Q6_K without a GEMM: quantizer kernel, then the
// matrix-core matvec
bool use_mmv(const aq_qweight *w, int64_t m) {
    return m >= 2 && (w->type == AQ_TYPE_Q4_K || w->type == AQ_TYPE_Q6_K) && w->k <= mmv_max_k();
}

int check_mm(aq_ctx *ctx, const aq_qweight *w, int64_t m, int64_t k) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (!w) return fail(AQ_ERR_INVALID_ARG, "null weight");
    if (m < 0) return fail(AQ_ERR_INVALID_ARG, "negative m (%lld)", (long long)m);
    if (k != w->k) return fail(AQ_ERR_SHAPE, "lhs last dim %lld != weight k %lld", (long long)k, (long long)w->k);
    if (w->device != ctx->device) return fail(AQ_ERR_INVALID_ARG, "weight is on device %d, context on %d", w->device, ctx->device);
    return AQ_OK;
}

// The matmul of d_x [m][k] into d_y on ctx->stream.  m > 8 with a GEMM for
// the shape: the quantizer kernel writes the activation planes at `act`, then
// the GEMM.  Other m >= 2 of Q4_K / Q6_K: the quantizer, then the
// matrix-core matvec (passes of 8 rows).  Otherwise (m = 1, Q8_0): one matvec
// launch that quantises d_x itself.
int run_matmul(aq_ctx *ctx, const aq_qweight *w, const float *d_x, int64_t m, float *d_y, void *act, int32_t *dS,
               int32_t *dSmin, void *ws, size_t ws_bytes) {
    hipError_t e;
    if (use_gemm(w, m)) {
        ActPlanes a = act_planes(act, m, w->k);
        if (w->glayout.type != TYPE_Q6_K && w->glayout.type != TYPE_Q5_K) a.q16 = nullptr;  // f16-MFMA GEMMs only
        e = act_q80(w->type) ? launch_quantize_q8_0(d_x, m, w->k, a, ctx->stream)
                                    : launch_quantize_q8k(d_x, m, w->k, a, ctx->stream);
        if (e != hipSuccess) return fail(AQ_ERR_HIP, "activation quantizer: %s", hipGetErrorString(e));
        e = launch_gemm(w->glayout, w->n, w->k, a, m, d_y, dS, dSmin, ws, ws_bytes, ctx->stream);
        if (e == hipSuccess) return AQ_OK;
        if (e != hipErrorNotSupported) return fail(AQ_ERR_HIP, "gemm: %s", hipGetErrorString(e));
        e = launch_matvec(w->layout, w->n, w->k, nullptr, &a, m, d_y, dS, dSmin, ctx->stream);
    } else if (use_mmv(w, m)) {
        ActPlanes a = act_planes(act, m, w->k);
        a.q16 = nullptr;
        e = launch_quantize_q8k(d_x, m, w->k, a, ctx->stream);
        if (e != hipSuccess) return fail(AQ_ERR_HIP, "activation quantizer: %s", hipGetErrorString(e));
        e = launch_mmv(w->layout, w->n, w->k, a, m, d_y, dS, dSmin, ws, ws_bytes, ctx->stream);
        if (e == hipErrorNotSupported) e = launch_matvec(w->layout, w->n, w->k, nullptr, &a, m, d_y, dS, dSmin, ctx->stream);
    } else if (((uintptr_t)d_x & 15) == 0) {
        e = launch_matvec(w->layout, w->n, w->k, d_x, nullptr, m, d_y, dS, dSmin, ctx->stream);
    } else {
        // the fused prologue reads float4; quantise separately instead
        ActPlanes a = act_planes(act, m, w->k);
        a.q16 = nullptr;
        e = act_q80(w->type) ? launch_quantize_q8_0(d_x, m, w->k, a, ctx->stream)
                                    : launch_quantize_q8k(d_x, m, w->k, a, ctx->stream);
        if (e != hipSuccess) return fail(AQ_ERR_HIP, "activation quantizer: %s", hipGetErrorString(e));
        e = launch_matvec(w->layout, w->n, w->k, nullptr, &a, m, d_y, dS, dSmin, ctx->stream);
    }
    if (e == hipErrorNotSupported) return fail(AQ_ERR_SHAPE, "k=%lld is larger than the matvec supports", (long long)w->k);
    if (e != hipSuccess) return fail(AQ_ERR_HIP, "matvec: %s", hipGetErrorString(e));
    return AQ_OK;
}

}  // namespace

extern "C" {

int aq_abi_version(void) { return 1; }

const char *aq_last_error(void) { return g_err.c_str(); }

int aq_device_count(int *count) {
    if (!count) return fail(AQ_ERR_INVALID_ARG, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        n = 0;
    }
    *count = n;
    return AQ_OK;
}

int aq_ctx_create(int device, aq_ctx **out) {
    if (!out) return fail(AQ_ERR_INVALID_ARG, "null out");
    *out = nullptr;
    int n = 0;
    aq_device_count(&n);
    if (n == 0) return fail(AQ_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= n) return fail(AQ_ERR_NO_DEVICE, "device %d out of range (%d visible)", device, n);
    int rc = use_device(device);
    if (rc) return rc;
    void *fixed = nullptr;
    if ((rc = fixed_scratch_of(device, &fixed))) return rc;
    aq_ctx *c = new (std::nothrow) aq_ctx();
    if (!c) return fail(AQ_ERR_OOM, "out of host memory");
    c->device = device;
    c->fixed_scratch = fixed;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return fail(AQ_ERR_HIP, "hipStreamCreateWithFlags failed");
    }
    if (hipMalloc(&c->attn_part, ATTN_PART_BYTES) != hipSuccess ||
        hipMalloc(&c->head_part, HEAD_PARTS * sizeof(int2)) != hipSuccess) {
        (void)hipGetLastError();
        aq_ctx_destroy(c);
        return fail(AQ_ERR_OOM, "allocation of the decode workspaces failed");
    }
    *out = c;
    return AQ_OK;
}

int aq_ctx_destroy(aq_ctx *c) {
    if (!c) return AQ_OK;
    use_device(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->scratch) (void)hipFree(c->scratch);
    if (c->pinned) (void)hipHostFree(c->pinned);
    if (c->attn_part) (void)hipFree(c->attn_part);
    if (c->head_part) (void)hipFree(c->head_part);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return AQ_OK;
}

int aq_ctx_synchronize(aq_ctx *c) {
    if (!c) return fail(AQ_ERR_INVALID_ARG, "null context");
    int rc = use_device(c->device);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    return AQ_OK;
}

int aq_ctx_stream(aq_ctx *c, void **stream) {
    if (!c || !stream) return fail(AQ_ERR_INVALID_ARG, "null argument");
    *stream = (void *)c->stream;
    return AQ_OK;
}

static int upload_impl(aq_ctx *ctx, int type, const void *blocks, size_t nbytes, int64_t n, int64_t k,
                       bool src_on_device, aq_qweight **out) {
    if (!out) return fail(AQ_ERR_INVALID_ARG, "null out");
    *out = nullptr;
    if (!ctx || !blocks) return fail(AQ_ERR_INVALID_ARG, "null argument");
    const int be = block_elems(type);
    if (!be) return fail(AQ_ERR_UNSUPPORTED_TYPE, "unsupported weight type %d", type);
    if (n <= 0 || k <= 0) return fail(AQ_ERR_SHAPE, "bad weight shape (%lld, %lld)", (long long)n, (long long)k);
    if (k % be) return fail(AQ_ERR_SHAPE, "k=%lld is not a multiple of the block size %d", (long long)k, be);
    if (n > 0x7fffffff || k > 0x7fffffff) return fail(AQ_ERR_SHAPE, "weight dimension too large");
    const size_t nb = (size_t)(k / be);
    const size_t row_bytes = nb * block_bytes(type);
    if (nbytes != row_bytes * (size_t)n)
        return fail(AQ_ERR_SHAPE, "nbytes=%zu != n*k/%d*%d = %zu", nbytes, be, block_bytes(type), row_bytes * (size_t)n);
    int rc = use_device(ctx->device);
    if (rc) return rc;
    // row-block tile layout (aq_internal.h): rows padded to a multiple of 8,
    // plus, for Q6_K, the d plane [n/8][ng][8]
    const int ng = groups_of(type, k);
    const int64_t nrb = (n + RB - 1) / RB;
    const int64_t rb_stride = (int64_t)slabs_of(type) * ng * 128;
    const size_t slab_bytes = align_up((size_t)rb_stride * (size_t)nrb, 256);
    const size_t d_bytes = type == AQ_TYPE_Q6_K   ? align_up((size_t)nrb * ng * RB * 2, 256)
                           : type == AQ_TYPE_Q2_K ? align_up((size_t)nrb * ng * RB * 4, 256)
                                                  : 0;
    // Q4_0, Q5_0: the GEMM's expanded copy in the Q8_0 tile layout
    const int64_t g_stride = type == AQ_TYPE_Q4_0 || type == AQ_TYPE_Q5_0 ? (int64_t)slabs_of(TYPE_Q8_0) * ng * 128 : 0;
    const size_t g_bytes = align_up((size_t)g_stride * (size_t)nrb, 256);
    const size_t d_u16 = type == AQ_TYPE_Q2_K ? 2 : 1;  // 16-bit units per d-plane entry
    const size_t total = slab_bytes + d_bytes + g_bytes;
    aq_qweight *w = new (std::nothrow) aq_qweight();
    if (!w) return fail(AQ_ERR_OOM, "out of host memory");
    if (hipMalloc(&w->base, total) != hipSuccess) {
        (void)hipGetLastError();
        delete w;
        return fail(AQ_ERR_OOM, "hipMalloc of %zu weight bytes failed", total);
    }
    w->type = type;
    w->device = ctx->device;
    w->n = n;
    w->k = k;
    w->bytes = total;
    uint8_t *base = (uint8_t *)w->base;
    w->layout.slab = base;
    w->layout.d = d_bytes ? (const uint16_t *)(base + slab_bytes) : nullptr;
    w->layout.type = type;
    w->layout.ng = ng;
    w->layout.rb_stride = rb_stride;
    w->glayout = w->layout;
    uint8_t *gslab = base + slab_bytes + d_bytes;
    if (g_bytes) {
        w->glayout.slab = gslab;
        w->glayout.d = nullptr;
        w->glayout.type = TYPE_Q8_0;
        w->glayout.rb_stride = g_stride;
    }

    int status = AQ_OK;
    // padding rows (n not a multiple of 8) and Q8_0 padding blocks must read as
    // zeros; Q3_K's two padding bytes per group are cleared too
    if ((n % RB != 0 || (act_q80(type) && (k / QK8_0) % 8 != 0) || type == AQ_TYPE_Q3_K) &&
        hipMemsetAsync(base, 0, total, ctx->stream) != hipSuccess)
        status = fail(AQ_ERR_HIP, "hipMemsetAsync of the weight padding failed");

    // Stage whole rows through a bounded device buffer (256 MiB; the
    // environment variable ARM_AI_AMD_UPLOAD_STAGE_BYTES lowers it, which the
    // tests use to force uploads of many chunks) unless the blocks are
    // already on the device.
    size_t stage_cap = (size_t)256 << 20;
    if (const char *env = getenv("ARM_AI_AMD_UPLOAD_STAGE_BYTES")) {
        const long long v = atoll(env);
        if (v > 0 && (size_t)v < stage_cap) stage_cap = (size_t)v;
    }
    int64_t rows_per = (int64_t)(stage_cap / row_bytes) / RB * RB;  // chunks start on a row block
    if (rows_per < RB) rows_per = RB;
    if (rows_per > n) rows_per = n;
    void *stage = nullptr;
    if (!src_on_device && status == AQ_OK) {
        if (hipMalloc(&stage, (size_t)rows_per * row_bytes) != hipSuccess) {
            (void)hipGetLastError();
            status = fail(AQ_ERR_OOM, "hipMalloc of the upload staging buffer failed");
        }
    }
    for (int64_t r0 = 0; r0 < n && status == AQ_OK; r0 += rows_per) {
        const int64_t rows = (n - r0) < rows_per ? (n - r0) : rows_per;
        const uint8_t *src = (const uint8_t *)blocks + (size_t)r0 * row_bytes;
        if (!src_on_device) {
            if (hipMemcpyAsync(stage, src, (size_t)rows * row_bytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess) {
                status = fail(AQ_ERR_HIP, "weight upload copy failed");
                break;
            }
            src = (const uint8_t *)stage;
        }
        hipError_t e = launch_repack(type, src, rows, k, base + (size_t)(r0 / RB) * rb_stride,
                                     d_bytes ? (uint16_t *)(base + slab_bytes) + (size_t)(r0 / RB) * ng * RB * d_u16 : nullptr,
                                     ctx->stream);
        if (e != hipSuccess) status = fail(AQ_ERR_HIP, "repack: %s", hipGetErrorString(e));
        if (status == AQ_OK && g_bytes &&
            (e = launch_expand_q80(type, src, rows, k, gslab + (size_t)(r0 / RB) * g_stride, ctx->stream)) != hipSuccess)
            status = fail(AQ_ERR_HIP, "expansion to the Q8_0 layout: %s", hipGetErrorString(e));
        // the staging buffer is reused by the next chunk
        if (status == AQ_OK && hipStreamSynchronize(ctx->stream) != hipSuccess) status = fail(AQ_ERR_HIP, "upload sync failed");
    }
    if (stage) (void)hipFree(stage);
    if (status != AQ_OK) {
        (void)hipFree(w->base);
        delete w;
        return status;
    }
    *out = w;
    return AQ_OK;
}

int aq_qweight_upload(aq_ctx *ctx, int type, const void *blocks, size_t nbytes, int64_t n, int64_t k, aq_qweight **out) {
    return upload_impl(ctx, type, blocks, nbytes, n, k, false, out);
}

int aq_qweight_upload_device(aq_ctx *ctx, int type, const void *d_blocks, size_t nbytes, int64_t n, int64_t k,
                             aq_qweight **out) {
    return upload_impl(ctx, type, d_blocks, nbytes, n, k, true, out);
}

int aq_qweight_free(aq_qweight *w) {
    if (!w) return AQ_OK;
    use_device(w->device);
    if (w->base) (void)hipFree(w->base);
    delete w;
    return AQ_OK;
}

int aq_qweight_info(const aq_qweight *w, int *type, int64_t *n, int64_t *k, size_t *device_bytes) {
    if (!w) return fail(AQ_ERR_INVALID_ARG, "null weight");
    if (type) *type = w->type;
    if (n) *n = w->n;
    if (k) *k = w->k;
    if (device_bytes) *device_bytes = w->bytes;
    return AQ_OK;
}

int aq_qmatmul_f32(aq_ctx *ctx, const aq_qweight *w, const float *lhs, int64_t m, int64_t k, float *dst) {
    int rc = check_mm(ctx, w, m, k);
    if (rc) return rc;
    if (m == 0) return AQ_OK;
    if (!lhs || !dst) return fail(AQ_ERR_INVALID_ARG, "null lhs or dst");
    if ((rc = use_device(ctx->device))) return rc;
    const bool gemm = use_gemm(w, m);
    CallLayout L = call_layout(w, m, true, false, gemm);
    if ((rc = ensure_scratch(ctx, L.total))) return rc;
    const size_t xin = (size_t)m * k * 4, yout = (size_t)m * w->n * 4;
    if ((rc = ensure_pinned(ctx, xin > yout ? xin : yout))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    float *d_x = (float *)(S + L.x), *d_y = (float *)(S + L.y);
    memcpy(ctx->pinned, lhs, xin);
    HIP_TRY(hipMemcpyAsync(d_x, ctx->pinned, xin, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = run_matmul(ctx, w, d_x, m, d_y, S + L.act, nullptr, nullptr, S + L.ws, L.total - L.ws))) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->pinned, d_y, yout, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    memcpy(dst, ctx->pinned, yout);
    return AQ_OK;
}

int aq_qmatmul_f32_device(aq_ctx *ctx, const aq_qweight *w, const float *d_lhs, int64_t m, int64_t k, float *d_dst) {
    int rc = check_mm(ctx, w, m, k);
    if (rc) return rc;
    if (m == 0) return AQ_OK;
    if (!d_lhs || !d_dst) return fail(AQ_ERR_INVALID_ARG, "null lhs or dst");
    if ((rc = use_device(ctx->device))) return rc;
    const bool gemm = use_gemm(w, m);
    CallLayout L = call_layout(w, m, false, false, gemm);
    if ((rc = ensure_scratch(ctx, L.total))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    return run_matmul(ctx, w, d_lhs, m, d_dst, S + L.act, nullptr, nullptr, S + L.ws, L.total - L.ws);
}

int aq_qmatmul_f32_device_noalloc(aq_ctx *ctx, const aq_qweight *w, const float *d_lhs, int64_t m, int64_t k,
                                  float *d_dst) {
    int rc = check_mm(ctx, w, m, k);
    if (rc) return rc;
    if (m == 0) return AQ_OK;
    if (!d_lhs || !d_dst) return fail(AQ_ERR_INVALID_ARG, "null lhs or dst");
    if (!ctx->fixed_scratch) return fail(AQ_ERR_INVALID_ARG, "context has no fixed scratch");
    if ((rc = use_device(ctx->device))) return rc;
    const bool gemm = use_gemm(w, m);
    CallLayout L = call_layout(w, m, false, false, gemm);
    if (L.total > FIXED_SCRATCH_BYTES)
        return fail(AQ_ERR_SHAPE, "m=%lld needs %zu bytes of scratch, more than the fixed %zu; use aq_qmatmul_f32_device",
                    (long long)m, L.total, FIXED_SCRATCH_BYTES);
    uint8_t *S = (uint8_t *)ctx->fixed_scratch;
    return run_matmul(ctx, w, d_lhs, m, d_dst, S + L.act, nullptr, nullptr, S + L.ws, L.total - L.ws);
}

size_t aq_fixed_scratch_bytes(void) { return FIXED_SCRATCH_BYTES; }

size_t aq_act_bytes(int act_type, int64_t m, int64_t k) {
    if ((act_type != AQ_TYPE_Q8_K && act_type != AQ_TYPE_Q8_0) || m < 0 || k <= 0) return 0;
    return align_up(act_sizes(m, k).total, 256);
}

int aq_quantize_act_device(aq_ctx *ctx, int act_type, const float *d_x, int64_t m, int64_t k, void *d_act) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (act_type != AQ_TYPE_Q8_K && act_type != AQ_TYPE_Q8_0)
        return fail(AQ_ERR_UNSUPPORTED_TYPE, "activation type %d is not Q8_K or Q8_0", act_type);
    const int blk = act_type == AQ_TYPE_Q8_K ? QK_K : QK8_0;
    if (m < 0 || k <= 0 || k % blk) return fail(AQ_ERR_SHAPE, "bad activation shape (%lld, %lld)", (long long)m, (long long)k);
    if (m == 0) return AQ_OK;
    if (!d_x || !d_act) return fail(AQ_ERR_INVALID_ARG, "null argument");
    if ((uintptr_t)d_act & 255) return fail(AQ_ERR_INVALID_ARG, "activation buffer must be 256-byte aligned");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    ActPlanes a = act_planes(d_act, m, k);
    hipError_t e = act_type == AQ_TYPE_Q8_K ? launch_quantize_q8k(d_x, m, k, a, ctx->stream)
                                            : launch_quantize_q8_0(d_x, m, k, a, ctx->stream);
    if (e != hipSuccess) return fail(AQ_ERR_HIP, "quantizer: %s", hipGetErrorString(e));
    return AQ_OK;
}

int aq_qmatmul_preq_device(aq_ctx *ctx, const aq_qweight *w, const void *d_act, int64_t m, int64_t k, float *d_dst) {
    int rc = check_mm(ctx, w, m, k);
    if (rc) return rc;
    if (m == 0) return AQ_OK;
    if (!d_act || !d_dst) return fail(AQ_ERR_INVALID_ARG, "null activation or dst");
    if ((uintptr_t)d_act & 255) return fail(AQ_ERR_INVALID_ARG, "activation buffer must be 256-byte aligned");
    if ((rc = use_device(ctx->device))) return rc;
    ActPlanes a = act_planes((void *)d_act, m, k);
    hipError_t e = hipErrorNotSupported;
    const bool gemm = use_gemm(w, m);
    CallLayout L = call_layout(w, m, false, false, gemm);
    if ((gemm || use_mmv(w, m)) && (rc = ensure_scratch(ctx, L.total))) return rc;
    if (gemm) {
        e = launch_gemm(w->glayout, w->n, w->k, a, m, d_dst, nullptr, nullptr, (uint8_t *)ctx->scratch + L.ws,
                        L.total - L.ws, ctx->stream);
        if (e != hipSuccess && e != hipErrorNotSupported) return fail(AQ_ERR_HIP, "gemm: %s", hipGetErrorString(e));
    }
    if (e == hipErrorNotSupported && use_mmv(w, m))
        e = launch_mmv(w->layout, w->n, w->k, a, m, d_dst, nullptr, nullptr, (uint8_t *)ctx->scratch + L.ws,
                       L.total - L.ws, ctx->stream);
    if (e == hipErrorNotSupported) e = launch_matvec(w->layout, w->n, w->k, nullptr, &a, m, d_dst, nullptr, nullptr, ctx->stream);
    if (e == hipErrorNotSupported) return fail(AQ_ERR_SHAPE, "k=%lld is larger than the matvec supports", (long long)w->k);
    if (e != hipSuccess) return fail(AQ_ERR_HIP, "matvec: %s", hipGetErrorString(e));
    return AQ_OK;
}

int aq_qmatmul2_preq_device(aq_ctx *ctx, const aq_qweight *w1, const aq_qweight *w2, const void *d_act, int64_t m,
                            int64_t k, float *d_y1, float *d_y2) {
    int rc = check_mm(ctx, w1, m, k);
    if (rc) return rc;
    if ((rc = check_mm(ctx, w2, m, k))) return rc;
    if (m == 0) return AQ_OK;
    if (!d_act || !d_y1 || !d_y2) return fail(AQ_ERR_INVALID_ARG, "null activation or output");
    if ((uintptr_t)d_act & 255) return fail(AQ_ERR_INVALID_ARG, "activation buffer must be 256-byte aligned");
    if ((rc = use_device(ctx->device))) return rc;
    hipError_t e = hipErrorNotSupported;
    if (use_gemm(w1, m) && use_gemm(w2, m)) {
        CallLayout L = call_layout(w2, m, false, false, true);  // the second GEMM's split-K partials
        if ((rc = ensure_scratch(ctx, L.total))) return rc;
        e = launch_gemm_pair(w1->glayout, w1->n, d_y1, w2->glayout, w2->n, d_y2, k, act_planes((void *)d_act, m, k), m,
                             (uint8_t *)ctx->scratch + L.ws, L.total - L.ws, ctx->stream);
    }
    if (e == hipSuccess) return AQ_OK;
    if (e != hipErrorNotSupported) return fail(AQ_ERR_HIP, "paired gemm: %s", hipGetErrorString(e));
    if ((rc = aq_qmatmul_preq_device(ctx, w1, d_act, m, k, d_y1))) return rc;
    return aq_qmatmul_preq_device(ctx, w2, d_act, m, k, d_y2);
}

static int quantize_host(aq_ctx *ctx, int atype, const float *x, int64_t m, int64_t k, void *out_blocks) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    const int blk = atype == AQ_TYPE_Q8_K ? QK_K : QK8_0;
    if (m < 0 || k <= 0) return fail(AQ_ERR_SHAPE, "bad shape (%lld, %lld)", (long long)m, (long long)k);
    if (k % blk) return fail(AQ_ERR_SHAPE, "k=%lld is not a multiple of %d", (long long)k, blk);
    if (m == 0) return AQ_OK;
    if (!x || !out_blocks) return fail(AQ_ERR_INVALID_ARG, "null argument");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    const size_t act = align_up(act_sizes(m, k).total, 256), xin = (size_t)m * k * 4;
    if ((rc = ensure_scratch(ctx, act + xin))) return rc;
    if ((rc = ensure_pinned(ctx, act > xin ? act : xin))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    float *d_x = (float *)(S + act);
    memcpy(ctx->pinned, x, xin);
    HIP_TRY(hipMemcpyAsync(d_x, ctx->pinned, xin, hipMemcpyHostToDevice, ctx->stream));
    ActPlanes a = act_planes(S, m, k);
    a.q16 = nullptr;
    hipError_t e = atype == AQ_TYPE_Q8_K ? launch_quantize_q8k(d_x, m, k, a, ctx->stream)
                                         : launch_quantize_q8_0(d_x, m, k, a, ctx->stream);
    if (e != hipSuccess) return fail(AQ_ERR_HIP, "quantizer: %s", hipGetErrorString(e));
    HIP_TRY(hipMemcpyAsync(ctx->pinned, S, act, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    // planes -> GGUF blocks
    ActPlanes h = act_planes(ctx->pinned, m, k);
    uint8_t *o = (uint8_t *)out_blocks;
    if (atype == AQ_TYPE_Q8_K) {
        const int64_t nb = k / QK_K;
        for (int64_t r = 0; r < m; r++)
            for (int64_t b = 0; b < nb; b++) {
                uint8_t *blkp = o + (size_t)(r * nb + b) * 292;
                memcpy(blkp, &h.d[r * nb + b], 4);
                memcpy(blkp + 4, h.qs + r * k + b * QK_K, 256);
                memcpy(blkp + 260, h.bsums + r * (k / 16) + b * 16, 32);
            }
    } else {
        const int64_t nb = k / QK8_0;
        for (int64_t r = 0; r < m; r++)
            for (int64_t b = 0; b < nb; b++) {
                uint8_t *blkp = o + (size_t)(r * nb + b) * 34;
                memcpy(blkp, &h.d16[r * nb + b], 2);
                memcpy(blkp + 2, h.qs + r * k + b * QK8_0, 32);
            }
    }
    return AQ_OK;
}

int aq_quantize_q8k(aq_ctx *ctx, const float *x, int64_t m, int64_t k, void *out_blocks) {
    return quantize_host(ctx, AQ_TYPE_Q8_K, x, m, k, out_blocks);
}

int aq_quantize_q8_0(aq_ctx *ctx, const float *x, int64_t m, int64_t k, void *out_blocks) {
    return quantize_host(ctx, AQ_TYPE_Q8_0, x, m, k, out_blocks);
}

int aq_qmatmul_block_sums(aq_ctx *ctx, const aq_qweight *w, const float *lhs, int64_t m, int64_t k, int32_t *S,
                          int32_t *Smin) {
    int rc = check_mm(ctx, w, m, k);
    if (rc) return rc;
    if (m == 0) return AQ_OK;
    if (!lhs || !S || !Smin) return fail(AQ_ERR_INVALID_ARG, "null argument");
    if ((rc = use_device(ctx->device))) return rc;
    const bool gemm = use_gemm(w, m);
    CallLayout L = call_layout(w, m, true, true, gemm);
    if ((rc = ensure_scratch(ctx, L.total))) return rc;
    const size_t nblk = (size_t)(w->k / block_elems(w->type));
    const size_t xin = (size_t)m * k * 4, sbytes = (size_t)m * w->n * nblk * 4;
    if ((rc = ensure_pinned(ctx, xin > sbytes ? xin : sbytes))) return rc;
    uint8_t *B = (uint8_t *)ctx->scratch;
    float *d_x = (float *)(B + L.x), *d_y = (float *)(B + L.y);
    int32_t *dS = (int32_t *)(B + L.s), *dSm = (int32_t *)(B + L.smin);
    memcpy(ctx->pinned, lhs, xin);
    HIP_TRY(hipMemcpyAsync(d_x, ctx->pinned, xin, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = run_matmul(ctx, w, d_x, m, d_y, B + L.act, dS, dSm, B + L.ws, L.total - L.ws))) return rc;
    HIP_TRY(hipMemcpyAsync(ctx->pinned, dS, sbytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    memcpy(S, ctx->pinned, sbytes);
    HIP_TRY(hipMemcpyAsync(ctx->pinned, dSm, sbytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    memcpy(Smin, ctx->pinned, sbytes);
    return AQ_OK;
}

}  // extern "C"

// ===========================================================================
// The NIF crate's own int8 / int4 kernels (shape_ops.rs; include/aq.h,
// "crate kernels").  Each host-buffer entry copies its inputs into the
// context's device scratch, runs the kernel on the context's stream and
// copies the outputs back before returning; each _device entry takes device
// pointers and returns with the work queued on the stream.
// ===========================================================================
namespace {

struct ScratchPlan {
    size_t total = 0;
    size_t add(size_t bytes) {
        const size_t o = total;
        total += align_up(bytes ? bytes : 1, 256);
        return o;
    }
};

bool mul_ok(int64_t a, int64_t b, int64_t lim = ((int64_t)1 << 40)) { return a >= 0 && b >= 0 && (b == 0 || a <= lim / b); }

int crate_prologue(aq_ctx *ctx, int64_t m, int64_t n, int64_t k) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x7fffffff || !mul_ok(m, k) || !mul_ok(n, k) || !mul_ok(m, n))
        return fail(AQ_ERR_SHAPE, "bad shape (m=%lld, n=%lld, k=%lld)", (long long)m, (long long)n, (long long)k);
    return use_device(ctx->device);
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return AQ_OK;
    if (e == hipErrorInvalidValue) return fail(AQ_ERR_SHAPE, "%s: invalid shape or argument", what);
    return fail(AQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int h2d(aq_ctx *c, void *dst, const void *src, size_t bytes) {
    if (bytes) HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    return AQ_OK;
}

int d2h_sync(aq_ctx *c, void *dst, const void *src, size_t bytes) {
    if (bytes) HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return AQ_OK;
}

int int8_matmul_host(aq_ctx *ctx, const int8_t *a, const int8_t *w, const float *act_scales, float act_scale,
                     const float *w_scales, int64_t m, int64_t n, int64_t k, float *out) {
    int rc = crate_prologue(ctx, m, n, k);
    if (rc) return rc;
    if (m == 0) return AQ_OK;
    if (!a || !w || !w_scales || !out) return fail(AQ_ERR_INVALID_ARG, "null argument");
    ScratchPlan P;
    const size_t oa = P.add(m * k), ow = P.add(n * k), osa = P.add(act_scales ? m * 4 : 0), osw = P.add(n * 4),
                 oo = P.add(m * n * 4);
    if ((rc = ensure_scratch(ctx, P.total))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    if ((rc = h2d(ctx, S + oa, a, m * k)) || (rc = h2d(ctx, S + ow, w, n * k)) ||
        (rc = h2d(ctx, S + osw, w_scales, n * 4)) || (act_scales && (rc = h2d(ctx, S + osa, act_scales, m * 4))))
        return rc;
    if ((rc = hip_status(launch_int8_matmul((int8_t *)(S + oa), (int8_t *)(S + ow), act_scales ? (float *)(S + osa) : nullptr,
                                            act_scale, (float *)(S + osw), m, n, k, (float *)(S + oo), ctx->stream),
                         "int8 matmul")))
        return rc;
    return d2h_sync(ctx, out, S + oo, m * n * 4);
}

int weight_only_host(aq_ctx *ctx, int wt, const float *act, const void *w, size_t w_bytes, const float *scales,
                     size_t s_bytes, int64_t m, int64_t n, int64_t k, float *out) {
    int rc = crate_prologue(ctx, m, n, k);
    if (rc) return rc;
    if (m == 0) return AQ_OK;
    if (!act || !w || !out || (s_bytes && !scales)) return fail(AQ_ERR_INVALID_ARG, "null argument");
    ScratchPlan P;
    const size_t oa = P.add(m * k * 4), ow = P.add(w_bytes), os = P.add(s_bytes), oo = P.add(m * n * 4);
    if ((rc = ensure_scratch(ctx, P.total))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    if ((rc = h2d(ctx, S + oa, act, m * k * 4)) || (rc = h2d(ctx, S + ow, w, w_bytes)) ||
        (rc = h2d(ctx, S + os, scales, s_bytes)))
        return rc;
    if ((rc = hip_status(launch_weight_only_matmul(wt, (float *)(S + oa), S + ow, s_bytes ? (float *)(S + os) : nullptr,
                                                   m, n, k, (float *)(S + oo), ctx->stream),
                         "weight-only matmul")))
        return rc;
    return d2h_sync(ctx, out, S + oo, m * n * 4);
}

}  // namespace

int aq_int8_matmul_f32(aq_ctx *ctx, const int8_t *a, const int8_t *w, const float *w_scales, float act_scale, int64_t m,
                       int64_t n, int64_t k, float *out) {
    return int8_matmul_host(ctx, a, w, nullptr, act_scale, w_scales, m, n, k, out);
}

int aq_int8_matmul_f32_per_token(aq_ctx *ctx, const int8_t *a, const int8_t *w, const float *act_scales,
                                 const float *w_scales, int64_t m, int64_t n, int64_t k, float *out) {
    if (m > 0 && !act_scales) return fail(AQ_ERR_INVALID_ARG, "null act_scales");
    return int8_matmul_host(ctx, a, w, act_scales, 0.0f, w_scales, m, n, k, out);
}

int aq_int8_matmul_f32_device(aq_ctx *ctx, const int8_t *d_a, const int8_t *d_w, const float *d_act_scales,
                              float act_scale, const float *d_w_scales, int64_t m, int64_t n, int64_t k, float *d_out) {
    int rc = crate_prologue(ctx, m, n, k);
    if (rc) return rc;
    return hip_status(launch_int8_matmul(d_a, d_w, d_act_scales, act_scale, d_w_scales, m, n, k, d_out, ctx->stream),
                      "int8 matmul");
}

int aq_quantize_int8_per_token(aq_ctx *ctx, const float *a, int64_t m, int64_t k, int8_t *q, float *scales) {
    int rc = crate_prologue(ctx, m, 1, k);
    if (rc) return rc;
    if (m == 0) return AQ_OK;
    if (!a || !q || !scales) return fail(AQ_ERR_INVALID_ARG, "null argument");
    ScratchPlan P;
    const size_t oa = P.add(m * k * 4), oq = P.add(m * k), os = P.add(m * 4);
    if ((rc = ensure_scratch(ctx, P.total))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    if ((rc = h2d(ctx, S + oa, a, m * k * 4))) return rc;
    if ((rc = hip_status(launch_quantize_int8_per_token((float *)(S + oa), m, k, (int8_t *)(S + oq), (float *)(S + os),
                                                        ctx->stream),
                         "quantize_int8_per_token")))
        return rc;
    HIP_TRY(hipMemcpyAsync(q, S + oq, m * k, hipMemcpyDeviceToHost, ctx->stream));
    return d2h_sync(ctx, scales, S + os, m * 4);
}

int aq_quantize_int8_per_token_device(aq_ctx *ctx, const float *d_a, int64_t m, int64_t k, int8_t *d_q, float *d_scales) {
    int rc = crate_prologue(ctx, m, 1, k);
    if (rc) return rc;
    return hip_status(launch_quantize_int8_per_token(d_a, m, k, d_q, d_scales, ctx->stream), "quantize_int8_per_token");
}

int aq_dequant_matmul_int8_f32(aq_ctx *ctx, const float *act, const int8_t *w, const float *scales, int64_t b, int64_t m,
                               int64_t n, int64_t k, float *out) {
    if (b < 0 || !mul_ok(b, m)) return fail(AQ_ERR_SHAPE, "bad batch");
    return weight_only_host(ctx, CRATE_W_I8, act, w, (size_t)(n * k), scales, (size_t)n * 4, b * m, n, k, out);
}

int aq_dequant_matmul_f16_f32(aq_ctx *ctx, const float *act, const uint16_t *w, int64_t b, int64_t m, int64_t n,
                              int64_t k, float *out) {
    if (b < 0 || !mul_ok(b, m)) return fail(AQ_ERR_SHAPE, "bad batch");
    return weight_only_host(ctx, CRATE_W_F16, act, w, (size_t)(n * k) * 2, nullptr, 0, b * m, n, k, out);
}

int aq_int4_matmul_f32(aq_ctx *ctx, const float *a, const uint8_t *w_packed, const float *w_scales, int64_t m, int64_t n,
                       int64_t k, float *out) {
    if (k <= 0 || k % 32) return fail(AQ_ERR_SHAPE, "int4_matmul: K=%lld must be a multiple of 32", (long long)k);
    return weight_only_host(ctx, CRATE_W_Q4_0, a, w_packed, (size_t)(n * (k / 2)), w_scales, (size_t)(n * (k / 32)) * 4, m,
                            n, k, out);
}

int aq_int4_matmul_gemv(aq_ctx *ctx, const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n, int64_t k,
                        float *out) {
    return aq_int4_matmul_f32(ctx, a, w_packed, w_scales, 1, n, k, out);
}

int aq_weight_only_matmul_device(aq_ctx *ctx, int weight_format, const float *d_act, const void *d_w,
                                 const float *d_scales, int64_t m, int64_t n, int64_t k, float *d_out) {
    int rc = crate_prologue(ctx, m, n, k);
    if (rc) return rc;
    if (weight_format != AQ_CRATE_W_Q4_0 && weight_format != AQ_CRATE_W_I8 && weight_format != AQ_CRATE_W_F16)
        return fail(AQ_ERR_UNSUPPORTED_TYPE, "unknown weight format %d", weight_format);
    if (weight_format == AQ_CRATE_W_Q4_0 && k % 32)
        return fail(AQ_ERR_SHAPE, "int4_matmul: K=%lld must be a multiple of 32", (long long)k);
    const int wt = weight_format == AQ_CRATE_W_Q4_0 ? CRATE_W_Q4_0 : weight_format == AQ_CRATE_W_I8 ? CRATE_W_I8 : CRATE_W_F16;
    return hip_status(launch_weight_only_matmul(wt, d_act, d_w, d_scales, m, n, k, d_out, ctx->stream),
                      "weight-only matmul");
}

int aq_int4_matmul_gemv_q4_x_q8(aq_ctx *ctx, const float *a, const uint8_t *w_packed, const float *w_scales, int64_t n,
                                int64_t k, float *out) {
    int rc = crate_prologue(ctx, 1, n, k);
    if (rc) return rc;
    if (k % 32) return fail(AQ_ERR_SHAPE, "K=%lld must be a multiple of 32", (long long)k);
    if (!a || !w_packed || !w_scales || !out) return fail(AQ_ERR_INVALID_ARG, "null argument");
    ScratchPlan P;
    const size_t oa = P.add(k * 4), ow = P.add(n * (k / 2)), os = P.add(n * (k / 32) * 4), oo = P.add(n * 4),
                 orec = P.add(q4_x_q8_act_bytes(k));
    if ((rc = ensure_scratch(ctx, P.total))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    if ((rc = h2d(ctx, S + oa, a, k * 4)) || (rc = h2d(ctx, S + ow, w_packed, n * (k / 2))) ||
        (rc = h2d(ctx, S + os, w_scales, n * (k / 32) * 4)))
        return rc;
    if ((rc = hip_status(launch_q4_x_q8_gemv((float *)(S + oa), S + ow, (float *)(S + os), n, k, (float *)(S + oo), S + orec,
                                             nullptr, nullptr, ctx->stream),
                         "q4 x q8 gemv")))
        return rc;
    return d2h_sync(ctx, out, S + oo, n * 4);
}

size_t aq_q4_x_q8_act_bytes(int64_t k) { return k > 0 && k % 32 == 0 ? q4_x_q8_act_bytes(k) : 0; }

int aq_int4_matmul_gemv_q4_x_q8_device(aq_ctx *ctx, const float *d_a, const uint8_t *d_w_packed, const float *d_w_scales,
                                       int64_t n, int64_t k, float *d_out, void *d_act, int8_t *d_q, float *d_qscales) {
    int rc = crate_prologue(ctx, 1, n, k);
    if (rc) return rc;
    if (k % 32) return fail(AQ_ERR_SHAPE, "K=%lld must be a multiple of 32", (long long)k);
    return hip_status(launch_q4_x_q8_gemv(d_a, d_w_packed, d_w_scales, n, k, d_out, d_act, d_q, d_qscales, ctx->stream),
                      "q4 x q8 gemv");
}

int aq_quantize_int4_q4_0(aq_ctx *ctx, const float *w, int64_t n, int64_t k, uint8_t *packed, float *scales) {
    int rc = crate_prologue(ctx, 1, n, k);
    if (rc) return rc;
    if (k % 32) return fail(AQ_ERR_SHAPE, "quantize_int4: K=%lld must be a multiple of 32", (long long)k);
    if (!w || !packed || !scales) return fail(AQ_ERR_INVALID_ARG, "null argument");
    ScratchPlan P;
    const size_t ow = P.add(n * k * 4), op = P.add(n * (k / 2)), os = P.add(n * (k / 32) * 4);
    if ((rc = ensure_scratch(ctx, P.total))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    if ((rc = h2d(ctx, S + ow, w, n * k * 4))) return rc;
    if ((rc = hip_status(launch_quantize_int4_q4_0((float *)(S + ow), n, k, S + op, (float *)(S + os), ctx->stream),
                         "quantize_int4_q4_0")))
        return rc;
    HIP_TRY(hipMemcpyAsync(packed, S + op, n * (k / 2), hipMemcpyDeviceToHost, ctx->stream));
    return d2h_sync(ctx, scales, S + os, n * (k / 32) * 4);
}

int aq_dequantize_q6_k(aq_ctx *ctx, const void *blocks, size_t nbytes, int64_t n_elements, float *out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (n_elements <= 0 || n_elements % 256 || nbytes != (size_t)(n_elements / 256) * 210)
        return fail(AQ_ERR_SHAPE, "dequantize_q6_k: %zu bytes for %lld elements", nbytes, (long long)n_elements);
    if (!blocks || !out) return fail(AQ_ERR_INVALID_ARG, "null argument");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    ScratchPlan P;
    const size_t ob = P.add(nbytes), oo = P.add(n_elements * 4);
    if ((rc = ensure_scratch(ctx, P.total))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    if ((rc = h2d(ctx, S + ob, blocks, nbytes))) return rc;
    if ((rc = hip_status(launch_dequantize_q6_k_crate(S + ob, n_elements, (float *)(S + oo), ctx->stream), "dequantize_q6_k")))
        return rc;
    return d2h_sync(ctx, out, S + oo, n_elements * 4);
}

int aq_dequantize_q6_k_device(aq_ctx *ctx, const void *d_blocks, int64_t n_elements, float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_dequantize_q6_k_crate((const uint8_t *)d_blocks, n_elements, d_out, ctx->stream),
                      "dequantize_q6_k");
}

static int dequant_row_host(aq_ctx *ctx, int wt, const void *table, const float *scales, int64_t n_rows, int64_t row,
                            int64_t k, float *out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (k <= 0 || k % 32) return fail(AQ_ERR_SHAPE, "K=%lld must be a multiple of 32", (long long)k);
    if (row < 0 || row >= n_rows) return fail(AQ_ERR_SHAPE, "row %lld outside 0..%lld", (long long)row, (long long)n_rows);
    if (!table || !scales || !out) return fail(AQ_ERR_INVALID_ARG, "null argument");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    const size_t rb = wt == CRATE_W_Q4_0 ? (size_t)k / 2 : (size_t)k, sb = (size_t)(k / 32) * 4;
    ScratchPlan P;
    const size_t ot = P.add(rb), os = P.add(sb), orow = P.add(8), oo = P.add(k * 4);
    if ((rc = ensure_scratch(ctx, P.total))) return rc;
    uint8_t *S = (uint8_t *)ctx->scratch;
    const int64_t zero = 0;
    // only the requested row travels: it becomes row 0 of a one-row table
    if ((rc = h2d(ctx, S + ot, (const uint8_t *)table + (size_t)row * rb, rb)) ||
        (rc = h2d(ctx, S + os, (const uint8_t *)scales + (size_t)row * sb, sb)) || (rc = h2d(ctx, S + orow, &zero, 8)))
        return rc;
    if ((rc = hip_status(launch_dequant_rows(wt, S + ot, (float *)(S + os), 1, (int64_t *)(S + orow), 1, k, (float *)(S + oo),
                                             ctx->stream),
                         "dequant row")))
        return rc;
    return d2h_sync(ctx, out, S + oo, k * 4);
}

int aq_q4_0_dequant_row(aq_ctx *ctx, const uint8_t *packed, const float *scales, int64_t n_rows, int64_t row, int64_t k,
                        float *out) {
    return dequant_row_host(ctx, CRATE_W_Q4_0, packed, scales, n_rows, row, k, out);
}

int aq_q8_0_dequant_row(aq_ctx *ctx, const int8_t *w, const float *scales, int64_t n_rows, int64_t row, int64_t k,
                        float *out) {
    return dequant_row_host(ctx, CRATE_W_I8, w, scales, n_rows, row, k, out);
}

int aq_dequant_rows_device(aq_ctx *ctx, int weight_format, const void *d_table, const float *d_scales, int64_t n_rows,
                           const int64_t *d_rows, int64_t n_out, int64_t k, float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (weight_format != AQ_CRATE_W_Q4_0 && weight_format != AQ_CRATE_W_I8)
        return fail(AQ_ERR_UNSUPPORTED_TYPE, "row tables are Q4_0-style or int8");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_dequant_rows(weight_format == AQ_CRATE_W_Q4_0 ? CRATE_W_Q4_0 : CRATE_W_I8, d_table, d_scales,
                                          n_rows, d_rows, n_out, k, d_out, ctx->stream),
                      "dequant rows");
}

// ---------------------------------------------------------------- decode-step glue
int aq_llama_embed(aq_ctx *ctx, const float *d_table, int64_t vocab, const int64_t *d_tok, int64_t hidden,
                   float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_embed(d_table, vocab, d_tok, 1, hidden, d_out, ctx->stream), "embed");
}

int aq_llama_embed_rows(aq_ctx *ctx, const float *d_table, int64_t vocab, const int64_t *d_tok, int64_t m,
                        int64_t hidden, float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (m == 0) return AQ_OK;
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_embed(d_table, vocab, d_tok, m, hidden, d_out, ctx->stream), "embed rows");
}

int aq_llama_rmsnorm(aq_ctx *ctx, float *d_x, const float *d_delta, const float *d_w, int64_t m, int64_t n, float eps,
                     float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (m == 0) return AQ_OK;
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_rmsnorm(d_x, d_delta, d_w, m, n, eps, d_out, ctx->stream), "rmsnorm");
}

int aq_llama_silu_mul(aq_ctx *ctx, const float *d_gu, int64_t n, float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    if (!d_gu) return fail(AQ_ERR_INVALID_ARG, "null gu");
    return hip_status(launch_silu_mul(d_gu, d_gu + n, 2 * n, 1, n, d_out, ctx->stream), "silu_mul");
}

int aq_llama_silu_mul_rows(aq_ctx *ctx, const float *d_g, const float *d_u, int64_t ld, int64_t m, int64_t n,
                           float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (m == 0) return AQ_OK;
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_silu_mul(d_g, d_u, ld, m, n, d_out, ctx->stream), "silu_mul rows");
}

int aq_llama_attn_decode(aq_ctx *ctx, const float *d_qk, const float *d_v, const float *d_cos, const float *d_sin,
                         const int64_t *d_pos, float *d_kcache, float *d_vcache, int64_t n_head, int64_t n_kv,
                         int64_t head_dim, int64_t max_seq, float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    if (!d_qk || !d_v || !d_cos || !d_sin || !d_pos || !d_kcache || !d_vcache || !d_out)
        return fail(AQ_ERR_INVALID_ARG, "null pointer");
    if (max_seq <= 0 || max_seq > 8192) return fail(AQ_ERR_INVALID_ARG, "max_seq %lld outside 1..8192", (long long)max_seq);
    if (((uintptr_t)d_kcache | (uintptr_t)d_vcache | (uintptr_t)d_out) & 15)
        return fail(AQ_ERR_INVALID_ARG, "caches and output must be 16-byte aligned");
    // the query heads of a kv head together, the context split over workgroups;
    // other head shapes: one workgroup per query head
    hipError_t e = launch_attn_split(d_qk, d_v, d_cos, d_sin, d_pos, d_kcache, d_vcache, n_head, n_kv, head_dim,
                                     max_seq, d_out, ctx->attn_part, ATTN_PART_BYTES, ctx->stream);
    if (e == hipErrorNotSupported)
        e = launch_attn_decode(d_qk, d_v, d_cos, d_sin, d_pos, d_kcache, d_vcache, n_head, n_kv, head_dim, max_seq,
                               d_out, ctx->stream);
    return hip_status(e, "attn_decode");
}

int aq_llama_attn_prefill(aq_ctx *ctx, const float *d_q, int64_t ldq, const float *d_k, int64_t ldk, const float *d_v,
                          int64_t ldv, const float *d_cos, const float *d_sin, int64_t index_pos, int64_t m,
                          float *d_kcache, float *d_vcache, int64_t n_head, int64_t n_kv, int64_t head_dim,
                          int64_t max_seq, float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (m == 0) return AQ_OK;
    int rc = use_device(ctx->device);
    if (rc) return rc;
    const hipError_t e = launch_attn_prefill(d_q, ldq, d_k, ldk, d_v, ldv, d_cos, d_sin, index_pos, m, d_kcache,
                                             d_vcache, n_head, n_kv, head_dim, max_seq, d_out, ctx->stream);
    if (e == hipErrorNotSupported) return fail(AQ_ERR_SHAPE, "head_dim %lld: the prompt attention takes 64 or 128", (long long)head_dim);
    return hip_status(e, "attn_prefill");
}


int aq_llama_argmax(aq_ctx *ctx, const float *d_x, int64_t n, int64_t *d_tok, int64_t *d_pos, int64_t *d_hist,
                    int64_t hist_len) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_argmax(d_x, n, d_tok, d_pos, d_hist, hist_len, ctx->stream), "argmax");
}

int aq_qmatmul_rmsnorm_f32_device(aq_ctx *ctx, const aq_qweight *w, const float *d_x, const float *d_delta,
                                  const float *d_norm_w, float eps, int64_t k, float *d_h_out, float *d_dst) {
    int rc = check_mm(ctx, w, 1, k);
    if (rc) return rc;
    if (!d_x || !d_norm_w || !d_dst) return fail(AQ_ERR_INVALID_ARG, "null pointer");
    if (d_h_out && (d_h_out == d_x || d_h_out == d_delta)) return fail(AQ_ERR_INVALID_ARG, "d_h_out aliases an input");
    if ((rc = use_device(ctx->device))) return rc;
    const hipError_t e = launch_matvec_rmsnorm(w->layout, w->n, w->k, d_x, d_delta, d_norm_w, eps, d_h_out, d_dst,
                                               ctx->stream);
    if (e == hipErrorNotSupported) return fail(AQ_ERR_SHAPE, "k=%lld is too long for the fused norm", (long long)k);
    return hip_status(e, "matvec rmsnorm");
}

int aq_llama_swiglu_pairs(aq_ctx *ctx, const float *d_y, int64_t ld, int64_t m, int64_t ffn, float *d_out) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (m == 0) return AQ_OK;
    if (ffn <= 0 || ffn % 4) return fail(AQ_ERR_SHAPE, "ffn=%lld is not a positive multiple of 4", (long long)ffn);
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_swiglu_pairs(d_y, ld, m, ffn, d_out, ctx->stream), "swiglu pairs");
}

int aq_llama_rmsnorm_act(aq_ctx *ctx, float *d_x, const float *d_delta, const float *d_w, int64_t m, int64_t n,
                         float eps, float *d_out, void *d_act) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (m < 0 || n <= 0 || n % QK_K) return fail(AQ_ERR_SHAPE, "n=%lld is not a positive multiple of 256", (long long)n);
    if (m == 0) return AQ_OK;
    if (!d_x || !d_w || !d_act) return fail(AQ_ERR_INVALID_ARG, "null argument");
    if ((uintptr_t)d_act & 255) return fail(AQ_ERR_INVALID_ARG, "activation buffer must be 256-byte aligned");
    if (((uintptr_t)d_x | (uintptr_t)d_delta | (uintptr_t)d_w | (uintptr_t)d_out) & 15)
        return fail(AQ_ERR_INVALID_ARG, "x, delta, w and out must be 16-byte aligned");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_rmsnorm_act(d_x, d_delta, d_w, m, n, eps, d_out, act_planes(d_act, m, n), ctx->stream),
                      "rmsnorm + quantize");
}

int aq_llama_swiglu_pairs_act(aq_ctx *ctx, const float *d_y, int64_t ld, int64_t m, int64_t ffn, float *d_out,
                              void *d_act) {
    if (!ctx) return fail(AQ_ERR_INVALID_ARG, "null context");
    if (m < 0 || ffn <= 0 || ffn % QK_K)
        return fail(AQ_ERR_SHAPE, "ffn=%lld is not a positive multiple of 256", (long long)ffn);
    if (m == 0) return AQ_OK;
    if (!d_y || !d_act) return fail(AQ_ERR_INVALID_ARG, "null argument");
    if ((uintptr_t)d_act & 255) return fail(AQ_ERR_INVALID_ARG, "activation buffer must be 256-byte aligned");
    if ((((uintptr_t)d_y | (uintptr_t)d_out) & 15) || ld % 4)
        return fail(AQ_ERR_INVALID_ARG, "y and out must be 16-byte aligned, ld a multiple of 4");
    int rc = use_device(ctx->device);
    if (rc) return rc;
    return hip_status(launch_swiglu_pairs_act(d_y, ld, m, ffn, d_out, act_planes(d_act, m, ffn), ctx->stream),
                      "swiglu pairs + quantize");
}

int aq_llama_head_argmax_embed(aq_ctx *ctx, const aq_qweight *w, const float *d_x, const float *d_delta,
                               const float *d_norm_w, float eps, int64_t k, float *d_logits, int64_t *d_tok,
                               int64_t *d_pos, int64_t *d_hist, int64_t hist_len, const float *d_table,
                               int64_t hidden, float *d_x_next) {
    int rc = check_mm(ctx, w, 1, k);
    if (rc) return rc;
    if (!d_x || !d_norm_w || !d_logits || !d_tok || !d_pos || !d_table || !d_x_next)
        return fail(AQ_ERR_INVALID_ARG, "null pointer");
    if (hidden <= 0 || hidden % 4 || (((uintptr_t)d_table | (uintptr_t)d_x_next | (uintptr_t)d_logits) & 15))
        return fail(AQ_ERR_INVALID_ARG, "hidden must be a positive multiple of 4, table / output / logits 16-byte aligned");
    if ((rc = use_device(ctx->device))) return rc;
    int nparts = 0;
    hipError_t e = launch_matvec_rmsnorm_argmax(w->layout, w->n, w->k, d_x, d_delta, d_norm_w, eps, d_logits,
                                                ctx->head_part, HEAD_PARTS, &nparts, ctx->stream);
    if (e == hipSuccess)
        return hip_status(launch_argmax_parts_embed(ctx->head_part, nparts, d_tok, d_pos, d_hist, hist_len, d_table,
                                                    w->n, hidden, d_x_next, ctx->stream),
                          "argmax parts embed");
    if (e != hipErrorNotSupported) return hip_status(e, "matvec rmsnorm argmax");
    // other heads: the fused-norm matvec, first maxima of the logits per
    // workgroup, then the pick and the embedding as above
    e = launch_matvec_rmsnorm(w->layout, w->n, w->k, d_x, d_delta, d_norm_w, eps, nullptr, d_logits, ctx->stream);
    if (e == hipErrorNotSupported) return fail(AQ_ERR_SHAPE, "k=%lld is too long for the fused norm", (long long)k);
    if (e != hipSuccess) return hip_status(e, "matvec rmsnorm");
    e = launch_argmax_parts(d_logits, w->n, ctx->head_part, HEAD_PARTS, &nparts, ctx->stream);
    if (e == hipSuccess)
        return hip_status(launch_argmax_parts_embed(ctx->head_part, nparts, d_tok, d_pos, d_hist, hist_len, d_table,
                                                    w->n, hidden, d_x_next, ctx->stream),
                          "argmax parts embed");
    if (e != hipErrorNotSupported) return hip_status(e, "argmax parts");
    if ((e = launch_argmax(d_logits, w->n, d_tok, d_pos, d_hist, hist_len, ctx->stream)) != hipSuccess)
        return hip_status(e, "argmax");
    return hip_status(launch_embed(d_table, w->n, d_tok, 1, hidden, d_x_next, ctx->stream), "embed");
}

int aq_swiglu_fused(int type, int64_t n, int64_t k) {
    return n > 0 && k > 0 && n % 8 == 0 && rowlane_xf_applies(type, n, k, RL_XF_NORM) ? 1 : 0;
}

int aq_qmatmul_rmsnorm_swiglu_f32_device(aq_ctx *ctx, const aq_qweight *w, const float *d_x, const float *d_delta,
                                         const float *d_norm_w, float eps, int64_t k, float *d_h_out, float *d_dst) {
    int rc = check_mm(ctx, w, 1, k);
    if (rc) return rc;
    if (!d_x || !d_norm_w || !d_dst) return fail(AQ_ERR_INVALID_ARG, "null pointer");
    if (d_h_out && (d_h_out == d_x || d_h_out == d_delta)) return fail(AQ_ERR_INVALID_ARG, "d_h_out aliases an input");
    if (w->n % 8) return fail(AQ_ERR_SHAPE, "n=%lld: a paired gate|up weight has whole 8-row blocks", (long long)w->n);
    if ((rc = use_device(ctx->device))) return rc;
    hipError_t e = launch_matvec_rmsnorm_swiglu(w->layout, w->n, w->k, d_x, d_delta, d_norm_w, eps, d_h_out, d_dst,
                                                ctx->stream);
    if (e != hipErrorNotSupported) return hip_status(e, "matvec rmsnorm swiglu");
    // the fused-norm matmul into scratch, then the pairs
    if ((rc = ensure_scratch(ctx, (size_t)w->n * sizeof(float)))) return rc;
    float *y = (float *)ctx->scratch;
    e = launch_matvec_rmsnorm(w->layout, w->n, w->k, d_x, d_delta, d_norm_w, eps, d_h_out, y, ctx->stream);
    if (e == hipErrorNotSupported) return fail(AQ_ERR_SHAPE, "k=%lld is too long for the fused norm", (long long)k);
    if (e != hipSuccess) return hip_status(e, "matvec rmsnorm");
    return hip_status(launch_swiglu_pairs(y, w->n, 1, w->n / 2, d_dst, ctx->stream), "swiglu pairs");
}

int aq_qmatmul_silu_mul_f32_device(aq_ctx *ctx, const aq_qweight *w, const float *d_gu, int64_t k, float *d_dst) {
    int rc = check_mm(ctx, w, 1, k);
    if (rc) return rc;
    if (!d_gu || !d_dst) return fail(AQ_ERR_INVALID_ARG, "null pointer");
    if ((rc = use_device(ctx->device))) return rc;
    const hipError_t e = launch_matvec_silu(w->layout, w->n, w->k, d_gu, d_dst, ctx->stream);
    if (e == hipErrorNotSupported) return fail(AQ_ERR_SHAPE, "k=%lld is larger than the matvec supports", (long long)k);
    return hip_status(e, "matvec silu");
}

int aq_qmatmul2_rmsnorm_f32_device(aq_ctx *ctx, const aq_qweight *w1, const aq_qweight *w2, const float *d_x,
                                   const float *d_delta, const float *d_norm_w, float eps, int64_t k, float *d_h_out,
                                   float *d_dst1, float *d_dst2) {
    int rc = check_mm(ctx, w1, 1, k);
    if (rc) return rc;
    if ((rc = check_mm(ctx, w2, 1, k))) return rc;
    if (!d_x || !d_norm_w || !d_dst1 || !d_dst2) return fail(AQ_ERR_INVALID_ARG, "null pointer");
    if (d_h_out && (d_h_out == d_x || d_h_out == d_delta)) return fail(AQ_ERR_INVALID_ARG, "d_h_out aliases an input");
    if ((rc = use_device(ctx->device))) return rc;
    const hipError_t e = launch_matvec2_rmsnorm(w1->layout, w1->n, d_dst1, w2->layout, w2->n, d_dst2, k, d_x, d_delta,
                                                d_norm_w, eps, d_h_out, ctx->stream);
    if (e == hipErrorNotSupported)
        return fail(AQ_ERR_SHAPE, "k=%lld is too long for the fused norm", (long long)k);
    return hip_status(e, "matvec2 rmsnorm");
}
