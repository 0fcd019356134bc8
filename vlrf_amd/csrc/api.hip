// api.hip - C ABI of the gfx950 decode backend: context, device memory,
// resident quantized weights, the Q8_0 KV cache and the standalone ops.
// Declarations and the reference interface each entry replaces are in
// include/vlrf_hip.h.
#include "internal.hpp"
#include "runtime.hpp"

#include <cmath>
#include <cstdarg>
#include <cstring>
#include <new>
#include <vector>

namespace vlrf_hip {

namespace {
thread_local std::string g_error;
thread_local LaunchTimer* g_launch_timer = nullptr;
}

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
}

LaunchTimer*& launch_timer() { return g_launch_timer; }

size_t weight_device_bytes(int dtype, int N, int K) {
    const size_t n = (size_t)N * K;
    switch (dtype) {
        case VLRF_HIP_DT_Q8_0: return n + (n / 32) * 2;
        case VLRF_HIP_DT_Q4_0: return n / 2 + (n / 32) * 2;
        default: return n * 4;
    }
}

int weight_alloc(DevWeight& w, int dtype, int N, int K) {
    VH_ARG(N > 0 && K > 0, "weight: empty shape %dx%d", N, K);
    VH_ARG(dtype == VLRF_HIP_DT_F32 || dtype == VLRF_HIP_DT_Q8_0 || dtype == VLRF_HIP_DT_Q4_0,
           "weight: unsupported dtype %d", dtype);
    VH_ARG(dtype == VLRF_HIP_DT_F32 || K % 32 == 0, "weight: K=%d not a multiple of 32", K);
    w.dtype = dtype;
    w.N = N;
    w.K = K;
    const size_t n = (size_t)N * K;
    if (dtype == VLRF_HIP_DT_F32) {
        if (hipMalloc(&w.f, n * 4) != hipSuccess) {
            set_error("weight: hipMalloc(%zu) failed", n * 4);
            return VLRF_HIP_ERR_NOMEM;
        }
        return VLRF_HIP_OK;
    }
    const size_t qbytes = dtype == VLRF_HIP_DT_Q8_0 ? n : n / 2;
    if (hipMalloc(&w.q, qbytes) != hipSuccess || hipMalloc(&w.d, (n / 32) * 2) != hipSuccess) {
        weight_release(w);
        set_error("weight: hipMalloc failed for %dx%d", N, K);
        return VLRF_HIP_ERR_NOMEM;
    }
    return VLRF_HIP_OK;
}

void weight_release(DevWeight& w) {
    if (w.q) (void)hipFree(w.q);
    if (w.d) (void)hipFree(w.d);
    if (w.f) (void)hipFree(w.f);
    if (w.bf) (void)hipFree(w.bf);
    w.q = nullptr;
    w.d = nullptr;
    w.f = nullptr;
    w.bf = nullptr;
}

int weight_upload_rows(hipStream_t s, DevWeight& w, const void* host, int row0, int nrows) {
    VH_ARG(host != nullptr, "weight upload: null host pointer");
    VH_ARG(row0 >= 0 && nrows >= 0 && row0 + nrows <= w.N, "weight upload: rows out of range");
    if (w.bf) {   // the expansion no longer matches the codes: made again when next needed
        VH_CHECK(hipStreamSynchronize(s));
        (void)hipFree(w.bf);
        w.bf = nullptr;
    }
    const int K = w.K;
    const size_t nel = (size_t)nrows * K;
    if (w.dtype == VLRF_HIP_DT_F32) {
        VH_CHECK(hipMemcpyAsync(w.f + (size_t)row0 * K, host, nel * 4, hipMemcpyHostToDevice, s));
        VH_CHECK(hipStreamSynchronize(s));
        return VLRF_HIP_OK;
    }
    const int bpr = K / 32;                       // blocks per row
    const size_t nb = (size_t)nrows * bpr;
    const uint8_t* in = static_cast<const uint8_t*>(host);
    const bool q8 = w.dtype == VLRF_HIP_DT_Q8_0;
    const size_t bsz = q8 ? 34 : 18, qpb = q8 ? 32 : 16;
    std::vector<uint8_t> q(nb * qpb);
    std::vector<uint16_t> d(nb);
    for (size_t b = 0; b < nb; ++b) {
        std::memcpy(&d[b], in + b * bsz, 2);
        std::memcpy(&q[b * qpb], in + b * bsz + 2, qpb);
    }
    VH_CHECK(hipMemcpyAsync(w.q + (size_t)row0 * bpr * qpb, q.data(), q.size(), hipMemcpyHostToDevice, s));
    VH_CHECK(hipMemcpyAsync(w.d + (size_t)row0 * bpr, d.data(), d.size() * 2, hipMemcpyHostToDevice, s));
    VH_CHECK(hipStreamSynchronize(s));
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip

using namespace vlrf_hip;

int vlrf_hip_ctx::rope_tables(int max_seq, int d_head, float theta, const float** c, const float** s) {
    for (auto& t : ropes)
        if (t.max_seq == max_seq && t.d_head == d_head && t.theta == theta) {
            *c = t.cos_t;
            *s = t.sin_t;
            return VLRF_HIP_OK;
        }
    // RopeCache::init (rope.hpp:49-71): same formula, in float, on the host.
    const int half = d_head / 2;
    std::vector<float> hc((size_t)max_seq * half), hs((size_t)max_seq * half);
    for (int pos = 0; pos < max_seq; ++pos)
        for (int i = 0; i < half; ++i) {
            const float freq = 1.f / std::pow(theta, (float)(2 * i) / (float)d_head);
            const float angle = (float)pos * freq;
            hc[(size_t)pos * half + i] = std::cos(angle);
            hs[(size_t)pos * half + i] = std::sin(angle);
        }
    RopeTab t;
    t.max_seq = max_seq;
    t.d_head = d_head;
    t.theta = theta;
    const size_t bytes = hc.size() * sizeof(float);
    if (hipMalloc(&t.cos_t, bytes) != hipSuccess || hipMalloc(&t.sin_t, bytes) != hipSuccess) {
        if (t.cos_t) (void)hipFree(t.cos_t);
        set_error("rope: hipMalloc failed");
        return VLRF_HIP_ERR_NOMEM;
    }
    VH_CHECK(hipMemcpyAsync(t.cos_t, hc.data(), bytes, hipMemcpyHostToDevice, stream));
    VH_CHECK(hipMemcpyAsync(t.sin_t, hs.data(), bytes, hipMemcpyHostToDevice, stream));
    VH_CHECK(hipStreamSynchronize(stream));
    ropes.push_back(t);
    *c = t.cos_t;
    *s = t.sin_t;
    return VLRF_HIP_OK;
}

int vlrf_hip_ctx::scratch(size_t bytes, float** out) {
    if (bytes > scratch_bytes) {
        // Growing synchronises and allocates, which a stream under graph
        // capture must not record.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
            (void)hipGetLastError();
            set_error("scratch: the call needs %zu bytes of context scratch (%zu held) while the stream is being "
                      "captured; make the same call once before capturing", bytes, scratch_bytes);
            return VLRF_HIP_ERR_ARG;
        }
        if (scratch_buf) {
            VH_CHECK(hipStreamSynchronize(stream));
            (void)hipFree(scratch_buf);
            scratch_buf = nullptr;
            scratch_bytes = 0;
        }
        if (hipMalloc(&scratch_buf, bytes) != hipSuccess) {
            set_error("scratch: hipMalloc(%zu) failed", bytes);
            return VLRF_HIP_ERR_NOMEM;
        }
        scratch_bytes = bytes;
    }
    *out = static_cast<float*>(scratch_buf);
    return VLRF_HIP_OK;
}

vlrf_hip_ctx::~vlrf_hip_ctx() {
    (void)hipSetDevice(device);
    (void)hipStreamSynchronize(stream);
    for (auto& t : ropes) {
        (void)hipFree(t.cos_t);
        (void)hipFree(t.sin_t);
    }
    if (scratch_buf) (void)hipFree(scratch_buf);
    if (small_tile_ctr) (void)hipFree(small_tile_ctr);
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (stream) (void)hipStreamDestroy(stream);
}


struct vlrf_hip_weight {
    Ctx* ctx = nullptr;
    DevWeight w;
};

struct vlrf_hip_kv {
    Ctx* ctx = nullptr;
    int n_layers = 0, max_seq = 0, n_kv = 0, d_head = 0;
    std::vector<KVLayer> layers;
    std::vector<int> used;
};

#define VH_CTX(c)                                                  \
    do {                                                           \
        if (!(c)) {                                                \
            set_error("null context");                             \
            return VLRF_HIP_ERR_ARG;                               \
        }                                                          \
        VH_CHECK(hipSetDevice((c)->device));                       \
    } while (0)

namespace vlrf_hip {
// Rows [row0, row0+n) of a head-major cache layer to host, token-major, as
// the cache's own elements (int8 codes, f16 bits or f32); scales for Q8_0.
int kv_rows_to_host(hipStream_t s, const KVLayer& L, int G, int D, int max_seq, int row0, int n,
                    int8_t* k_q, int8_t* v_q, float* k_s, float* v_s) {
    const size_t eb = (size_t)kv_elem_bytes(L.dtype), hd = (size_t)D * eb, row = (size_t)G * hd;
    std::vector<int8_t> hk((size_t)G * n * hd), hv((size_t)G * n * hd);
    for (int g = 0; g < G; ++g) {
        const size_t off = ((size_t)g * max_seq + row0) * hd;
        VH_CHECK(hipMemcpyAsync(hk.data() + (size_t)g * n * hd, L.k + off, n * hd, hipMemcpyDeviceToHost, s));
        VH_CHECK(hipMemcpyAsync(hv.data() + (size_t)g * n * hd, L.v + off, n * hd, hipMemcpyDeviceToHost, s));
    }
    const bool q8 = L.dtype == VLRF_HIP_KV_Q8_0;
    if (k_s && q8) VH_CHECK(hipMemcpyAsync(k_s, L.ks + row0, n * sizeof(float), hipMemcpyDeviceToHost, s));
    if (v_s && q8) VH_CHECK(hipMemcpyAsync(v_s, L.vs + row0, n * sizeof(float), hipMemcpyDeviceToHost, s));
    VH_CHECK(hipStreamSynchronize(s));
    for (int t = 0; t < n; ++t)
        for (int g = 0; g < G; ++g) {
            const size_t src = ((size_t)g * n + t) * hd, dst = (size_t)t * row + g * hd;
            if (k_q) std::memcpy(k_q + dst, hk.data() + src, hd);
            if (v_q) std::memcpy(v_q + dst, hv.data() + src, hd);
        }
    return VLRF_HIP_OK;
}
}  // namespace vlrf_hip

extern "C" {

const char* vlrf_hip_last_error(void) { return g_error.c_str(); }

int vlrf_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

// Split-K partials of vlrf_hip_attn_decode_noalloc: one fixed array per GPU,
// held until the process ends, so that call allocates nothing.  Host code uses
// the device address hipGetSymbolAddress returns for the context's GPU
// (vlrf_hip_ctx::noalloc_scratch), never the symbol itself.  Every call on one
// GPU shares the array: calls that overlap on one GPU race.
namespace noalloc {
constexpr size_t kScratchFloats = size_t(1) << 19;   // 2 MiB
static __device__ __align__(256) float scratch[kScratchFloats];
}  // namespace noalloc

int vlrf_hip_init(int device, vlrf_hip_ctx_t* out) {
    VH_ARG(out != nullptr, "init: null output handle");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        set_error("init: no HIP device visible");
        return VLRF_HIP_ERR_NODEV;
    }
    VH_ARG(device >= 0 && device < n, "init: device %d outside [0,%d)", device, n);
    hipDeviceProp_t prop;
    VH_CHECK(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error("init: device %d is %s, this build targets gfx950 only", device, prop.gcnArchName);
        return VLRF_HIP_ERR_NODEV;
    }
    VH_CHECK(hipSetDevice(device));
    auto* c = new (std::nothrow) vlrf_hip_ctx();
    if (!c) return VLRF_HIP_ERR_NOMEM;
    c->device = device;
    c->num_cus = prop.multiProcessorCount;
    std::snprintf(c->name, sizeof(c->name), "HIP: %s (%s, %d CUs, %.1f GiB)", prop.name,
                  prop.gcnArchName, prop.multiProcessorCount,
                  (double)prop.totalGlobalMem / (1024.0 * 1024.0 * 1024.0));
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&c->ev0) != hipSuccess || hipEventCreate(&c->ev1) != hipSuccess) {
        set_error("init: stream/event creation failed");
        delete c;
        return VLRF_HIP_ERR_RUNTIME;
    }
    void* fixed = nullptr;   // this device's copy of the fixed scratch array (device is current)
    const hipError_t se = hipGetSymbolAddress(&fixed, HIP_SYMBOL(noalloc::scratch));
    if (se != hipSuccess || !fixed) {
        set_error("init: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(se));
        delete c;
        return VLRF_HIP_ERR_RUNTIME;
    }
    c->noalloc_scratch = static_cast<float*>(fixed);
    const size_t ctr_bytes = (size_t)kSmallMaxTiles * kSmallTileCtrStride * sizeof(int);
    if (hipMalloc((void**)&c->small_tile_ctr, ctr_bytes) != hipSuccess ||
        hipMemset(c->small_tile_ctr, 0, ctr_bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        set_error("init: the small-M tile counters could not be allocated");
        delete c;
        return VLRF_HIP_ERR_NOMEM;
    }
    *out = c;
    return VLRF_HIP_OK;
}

void vlrf_hip_shutdown(vlrf_hip_ctx_t ctx) { delete ctx; }

int vlrf_hip_device_info(vlrf_hip_ctx_t ctx, char* buf, size_t len) {
    VH_ARG(ctx && buf && len > 0, "device_info: bad arguments");
    std::snprintf(buf, len, "%s", ctx->name);
    return VLRF_HIP_OK;
}

int vlrf_hip_sync(vlrf_hip_ctx_t ctx) {
    VH_CTX(ctx);
    VH_CHECK(hipStreamSynchronize(ctx->stream));
    return VLRF_HIP_OK;
}

void* vlrf_hip_stream(vlrf_hip_ctx_t ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int vlrf_hip_malloc(vlrf_hip_ctx_t ctx, size_t bytes, void** dptr) {
    VH_CTX(ctx);
    VH_ARG(dptr != nullptr, "malloc: null output");
    *dptr = nullptr;
    if (bytes == 0) return VLRF_HIP_OK;
    if (hipMalloc(dptr, bytes) != hipSuccess) {
        set_error("malloc: hipMalloc(%zu) failed", bytes);
        return VLRF_HIP_ERR_NOMEM;
    }
    return VLRF_HIP_OK;
}

int vlrf_hip_free(vlrf_hip_ctx_t ctx, void* dptr) {
    VH_CTX(ctx);
    if (dptr) {
        VH_CHECK(hipStreamSynchronize(ctx->stream));
        VH_CHECK(hipFree(dptr));
    }
    return VLRF_HIP_OK;
}

int vlrf_hip_h2d(vlrf_hip_ctx_t ctx, void* dst, const void* src, size_t bytes) {
    VH_CTX(ctx);
    if (!bytes) return VLRF_HIP_OK;
    VH_ARG(dst && src, "h2d: null pointer");
    VH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    VH_CHECK(hipStreamSynchronize(ctx->stream));
    return VLRF_HIP_OK;
}

int vlrf_hip_d2h(vlrf_hip_ctx_t ctx, void* dst, const void* src, size_t bytes) {
    VH_CTX(ctx);
    if (!bytes) return VLRF_HIP_OK;
    VH_ARG(dst && src, "d2h: null pointer");
    VH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    VH_CHECK(hipStreamSynchronize(ctx->stream));
    return VLRF_HIP_OK;
}

int vlrf_hip_d2d(vlrf_hip_ctx_t ctx, void* dst, const void* src, size_t bytes) {
    VH_CTX(ctx);
    if (!bytes) return VLRF_HIP_OK;
    VH_ARG(dst && src, "d2d: null pointer");
    VH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return VLRF_HIP_OK;
}

int vlrf_hip_memset(vlrf_hip_ctx_t ctx, void* dst, int value, size_t bytes) {
    VH_CTX(ctx);
    if (!bytes) return VLRF_HIP_OK;
    VH_ARG(dst != nullptr, "memset: null pointer");
    VH_CHECK(hipMemsetAsync(dst, value, bytes, ctx->stream));
    return VLRF_HIP_OK;
}

int vlrf_hip_timer_start(vlrf_hip_ctx_t ctx) {
    VH_CTX(ctx);
    VH_CHECK(hipEventRecord(ctx->ev0, ctx->stream));
    return VLRF_HIP_OK;
}

int vlrf_hip_timer_stop(vlrf_hip_ctx_t ctx, float* ms) {
    VH_CTX(ctx);
    VH_ARG(ms != nullptr, "timer_stop: null output");
    VH_CHECK(hipEventRecord(ctx->ev1, ctx->stream));
    VH_CHECK(hipEventSynchronize(ctx->ev1));
    VH_CHECK(hipEventElapsedTime(ms, ctx->ev0, ctx->ev1));
    return VLRF_HIP_OK;
}

// ---- attention -----------------------------------------------------------------
int vlrf_hip_attn_f32(vlrf_hip_ctx_t ctx, const float* Q, const float* K, const float* V, float* O,
                      int n_h, int T, int ctx_len, int d_h, float scale, int causal) {
    VH_CTX(ctx);
    VH_ARG(Q && K && V && O, "attn_f32: null pointer");
    VH_ARG(n_h >= 1 && T >= 1 && ctx_len >= 1 && d_h >= 1, "attn_f32: empty shape");
    if (T == 1 && !causal && (d_h == 64 || d_h == 128)) {
        // Decode shape: split-K over the context, K/V heads = query heads.
        const int splits = attn_decode_splits(ctx_len);
        float* part = nullptr;
        int rc = ctx->scratch((size_t)n_h * splits * (d_h + 2) * sizeof(float), &part);
        if (rc) return rc;
        return launch_attn_decode(ctx->stream, Q, K, V, nullptr, nullptr, VLRF_HIP_KV_F32, (long)ctx_len * d_h, n_h,
                                  n_h, d_h, ctx_len, nullptr, splits, scale, part, O, nullptr, ctx->small_tile_ctr);
    }
    return launch_attn_f32_tiled(ctx->stream, Q, K, V, O, n_h, T, ctx_len, d_h, scale, causal);
}

// ---- KV cache ---------------------------------------------------------------------
int vlrf_hip_kv_create(vlrf_hip_ctx_t ctx, int n_layers, int max_seq, int n_kv_heads, int d_head,
                       int dtype, vlrf_hip_kv_t* out) {
    VH_CTX(ctx);
    VH_ARG(out != nullptr, "kv_create: null output");
    *out = nullptr;
    VH_ARG(dtype == VLRF_HIP_KV_Q8_0 || dtype == VLRF_HIP_KV_F16 || dtype == VLRF_HIP_KV_F32,
           "kv_create: cache dtype %d is not F32, F16 or Q8_0", dtype);
    VH_ARG(n_layers >= 1 && max_seq >= 1 && n_kv_heads >= 1 && d_head >= 2 && d_head % 16 == 0,
           "kv_create: bad shape layers=%d max_seq=%d n_kv=%d d_head=%d", n_layers, max_seq,
           n_kv_heads, d_head);
    auto* kv = new (std::nothrow) vlrf_hip_kv();
    if (!kv) return VLRF_HIP_ERR_NOMEM;
    kv->ctx = ctx;
    kv->n_layers = n_layers;
    kv->max_seq = max_seq;
    kv->n_kv = n_kv_heads;
    kv->d_head = d_head;
    kv->layers.resize(n_layers);
    kv->used.assign(n_layers, 0);
    const size_t data = (size_t)n_kv_heads * max_seq * d_head * kv_elem_bytes(dtype);
    for (auto& L : kv->layers) {
        L.dtype = dtype;
        const bool q8 = dtype == VLRF_HIP_KV_Q8_0;
        if (hipMalloc(&L.k, data) != hipSuccess || hipMalloc(&L.v, data) != hipSuccess ||
            (q8 && hipMalloc(&L.ks, max_seq * sizeof(float)) != hipSuccess) ||
            (q8 && hipMalloc(&L.vs, max_seq * sizeof(float)) != hipSuccess)) {
            vlrf_hip_kv_destroy(kv);
            set_error("kv_create: hipMalloc failed");
            return VLRF_HIP_ERR_NOMEM;
        }
    }
    int rc = vlrf_hip_kv_reset(kv);
    if (rc) {
        vlrf_hip_kv_destroy(kv);
        return rc;
    }
    *out = kv;
    return VLRF_HIP_OK;
}

void vlrf_hip_kv_destroy(vlrf_hip_kv_t kv) {
    if (!kv) return;
    (void)hipSetDevice(kv->ctx->device);
    (void)hipStreamSynchronize(kv->ctx->stream);
    for (auto& L : kv->layers) {
        if (L.k) (void)hipFree(L.k);
        if (L.v) (void)hipFree(L.v);
        if (L.ks) (void)hipFree(L.ks);
        if (L.vs) (void)hipFree(L.vs);
    }
    delete kv;
}

int vlrf_hip_kv_reset(vlrf_hip_kv_t kv) {
    VH_ARG(kv != nullptr, "kv_reset: null cache");
    VH_CTX(kv->ctx);
    for (auto& L : kv->layers) {
        const size_t data = (size_t)kv->n_kv * kv->max_seq * kv->d_head * kv_elem_bytes(L.dtype);
        VH_CHECK(hipMemsetAsync(L.k, 0, data, kv->ctx->stream));
        VH_CHECK(hipMemsetAsync(L.v, 0, data, kv->ctx->stream));
        if (L.ks) VH_CHECK(hipMemsetAsync(L.ks, 0, kv->max_seq * sizeof(float), kv->ctx->stream));
        if (L.vs) VH_CHECK(hipMemsetAsync(L.vs, 0, kv->max_seq * sizeof(float), kv->ctx->stream));
    }
    VH_CHECK(hipStreamSynchronize(kv->ctx->stream));
    kv->used.assign(kv->n_layers, 0);
    return VLRF_HIP_OK;
}

int vlrf_hip_kv_used(vlrf_hip_kv_t kv, int layer) {
    if (!kv || layer < 0 || layer >= kv->n_layers) return -1;
    return kv->used[layer];
}

int vlrf_hip_kv_append(vlrf_hip_kv_t kv, int layer, const float* k, const float* v, int T) {
    VH_ARG(kv != nullptr, "kv_append: null cache");
    VH_CTX(kv->ctx);
    VH_ARG(layer >= 0 && layer < kv->n_layers, "kv_append: layer %d out of range", layer);
    VH_ARG(k && v && T >= 1, "kv_append: bad arguments");
    if (kv->used[layer] + T > kv->max_seq) {
        set_error("KVCache::append: exceeds max_seq_len (%d + %d > %d)", kv->used[layer], T, kv->max_seq);
        return VLRF_HIP_ERR_OVERFLOW;
    }
    int rc = launch_kv_append(kv->ctx->stream, kv->layers[layer], kv->n_kv, kv->d_head, kv->max_seq,
                              k, v, T, kv->used[layer], nullptr);
    if (rc) return rc;
    kv->used[layer] += T;
    return VLRF_HIP_OK;
}


int vlrf_hip_kv_read(vlrf_hip_kv_t kv, int layer, int row0, int n, int8_t* k_q, int8_t* v_q,
                     float* k_s, float* v_s) {
    VH_ARG(kv != nullptr, "kv_read: null cache");
    VH_CTX(kv->ctx);
    VH_ARG(layer >= 0 && layer < kv->n_layers, "kv_read: layer %d out of range", layer);
    VH_ARG(row0 >= 0 && n >= 0 && row0 + n <= kv->max_seq, "kv_read: rows out of range");
    return kv_rows_to_host(kv->ctx->stream, kv->layers[layer], kv->n_kv, kv->d_head, kv->max_seq, row0, n,
                           k_q, v_q, k_s, v_s);
}

int vlrf_hip_kv_dequant(vlrf_hip_kv_t kv, int layer, int ctx_len, float* K_out, float* V_out) {
    VH_ARG(kv != nullptr, "kv_dequant: null cache");
    VH_CTX(kv->ctx);
    VH_ARG(layer >= 0 && layer < kv->n_layers, "kv_dequant: layer %d out of range", layer);
    VH_ARG(K_out && V_out, "kv_dequant: null output");
    return launch_kv_dequant(kv->ctx->stream, kv->layers[layer], kv->n_kv, kv->d_head, kv->max_seq,
                             ctx_len, K_out, V_out);
}

int vlrf_hip_attn_decode(vlrf_hip_kv_t kv, int layer, const float* q, float* out, int n_heads,
                         int ctx_len, float scale) {
    VH_ARG(kv != nullptr, "attn_decode: null cache");
    VH_CTX(kv->ctx);
    VH_ARG(layer >= 0 && layer < kv->n_layers, "attn_decode: layer %d out of range", layer);
    VH_ARG(q && out, "attn_decode: null pointer");
    VH_ARG(ctx_len >= 1 && ctx_len <= kv->max_seq, "attn_decode: ctx_len %d outside [1,%d]", ctx_len,
           kv->max_seq);
    const int splits = attn_decode_splits(ctx_len);
    float* part = nullptr;
    int rc = kv->ctx->scratch((size_t)n_heads * splits * (kv->d_head + 2) * sizeof(float), &part);
    if (rc) return rc;
    const KVLayer& L = kv->layers[layer];
    return launch_attn_decode(kv->ctx->stream, q, L.k, L.v, L.ks, L.vs, L.dtype, (long)kv->max_seq * kv->d_head,
                              n_heads, kv->n_kv, kv->d_head, ctx_len, nullptr, splits, scale, part, out, nullptr,
                              kv->ctx->small_tile_ctr);
}

int vlrf_hip_attn_decode_noalloc(vlrf_hip_kv_t kv, int layer, const float* q, float* out, int n_heads,
                                 int ctx_len, float scale) {
    VH_ARG(kv != nullptr, "attn_decode_noalloc: null cache");
    VH_CTX(kv->ctx);
    VH_ARG(layer >= 0 && layer < kv->n_layers, "attn_decode_noalloc: layer %d out of range", layer);
    VH_ARG(q && out, "attn_decode_noalloc: null pointer");
    VH_ARG(ctx_len >= 1 && ctx_len <= kv->max_seq, "attn_decode_noalloc: ctx_len %d outside [1,%d]", ctx_len,
           kv->max_seq);
    VH_ARG(n_heads >= 1, "attn_decode_noalloc: n_heads %d", n_heads);
    VH_ARG(kv->ctx->noalloc_scratch != nullptr, "attn_decode_noalloc: context has no fixed scratch");
    const int splits = attn_decode_splits(ctx_len);
    const size_t need = (size_t)n_heads * splits * (kv->d_head + 2);
    VH_ARG(need <= noalloc::kScratchFloats,
           "attn_decode_noalloc: %zu partial floats (n_heads %d x %d splits x %d) exceed the fixed scratch of %zu",
           need, n_heads, splits, kv->d_head + 2, noalloc::kScratchFloats);
    const KVLayer& L = kv->layers[layer];
    return launch_attn_decode(kv->ctx->stream, q, L.k, L.v, L.ks, L.vs, L.dtype, (long)kv->max_seq * kv->d_head,
                              n_heads, kv->n_kv, kv->d_head, ctx_len, nullptr, splits, scale,
                              kv->ctx->noalloc_scratch, out, nullptr, kv->ctx->small_tile_ctr);
}

// ---- quantized linear ----------------------------------------------------------
int vlrf_hip_weight_upload(vlrf_hip_ctx_t ctx, const void* host, int dtype, int N, int K,
                           vlrf_hip_weight_t* out) {
    VH_CTX(ctx);
    VH_ARG(out != nullptr && host != nullptr, "weight_upload: null pointer");
    *out = nullptr;
    auto* w = new (std::nothrow) vlrf_hip_weight();
    if (!w) return VLRF_HIP_ERR_NOMEM;
    w->ctx = ctx;
    int rc = weight_alloc(w->w, dtype, N, K);
    if (!rc) rc = weight_upload_rows(ctx->stream, w->w, host, 0, N);
    if (rc) {
        weight_release(w->w);
        delete w;
        return rc;
    }
    *out = w;
    return VLRF_HIP_OK;
}

void vlrf_hip_weight_free(vlrf_hip_weight_t w) {
    if (!w) return;
    (void)hipSetDevice(w->ctx->device);
    (void)hipStreamSynchronize(w->ctx->stream);
    weight_release(w->w);
    delete w;
}

size_t vlrf_hip_weight_bytes(vlrf_hip_weight_t w) {
    if (!w) return 0;
    return weight_device_bytes(w->w.dtype, w->w.N, w->w.K) + (w->w.bf ? (size_t)w->w.N * w->w.K * 2 : 0);
}

// M <= 16 runs the f32 GEMV / small-M kernels; larger M (prefill) runs the
// MFMA GEMM on bf16 operands (x, optionally RMS-normalised, is rounded to bf16
// in the context's scratch buffer first).
int vlrf_hip_qlinear(vlrf_hip_ctx_t ctx, vlrf_hip_weight_t w, const float* x, float* y, int M,
                     const float* norm_w, float eps, const float* residual) {
    VH_CTX(ctx);
    VH_ARG(w != nullptr, "qlinear: null weight");
    VH_ARG(x != y, "qlinear: x must not alias y");
    if (M >= 2 && M <= 16 && qlinear_small_supported(w->w)) {
        float* scratch = nullptr;
        int rc = ctx->scratch(qlinear_small_scratch(w->w.N, w->w.K, false), &scratch);
        if (rc) return rc;
        return launch_qlinear_small(ctx->stream, w->w, nullptr, x, M, norm_w, eps, residual, scratch,
                                    ctx->small_tile_ctr, kSmallMaxTiles, y);
    }
    if (M <= 16) return launch_qlinear(ctx->stream, w->w, x, y, M, norm_w, eps, residual);
    VH_ARG(x && y, "qlinear: null activation pointer");
    // Scratch: the bf16 rows, then the K-split partial sums (17 <= M <= 128).
    const size_t a_bytes = ((size_t)M * w->w.K * sizeof(uint16_t) + 255) & ~(size_t)255;
    const size_t p_bytes = qgemm_part_bytes(w->w, M, false);
    float* scratch = nullptr;
    int rc = ctx->scratch(a_bytes + p_bytes, &scratch);
    if (rc) return rc;
    uint16_t* a = reinterpret_cast<uint16_t*>(scratch);
    float* part = p_bytes ? reinterpret_cast<float*>(reinterpret_cast<char*>(scratch) + a_bytes) : nullptr;
    rc = launch_rows_to_bf16(ctx->stream, x, norm_w, a, M, w->w.K, eps);
    if (rc) return rc;
    return launch_qgemm(ctx->stream, w->w, a, M, residual, y, part);
}

int vlrf_hip_qlinear_swiglu(vlrf_hip_ctx_t ctx, vlrf_hip_weight_t wg, vlrf_hip_weight_t wu,
                            const float* x, float* h, int M, const float* norm_w, float eps) {
    VH_CTX(ctx);
    VH_ARG(wg && wu, "swiglu: null weight");
    VH_ARG(x != h, "swiglu: x must not alias h");
    if (M >= 2 && M <= 16 && qlinear_small_supported(wg->w)) {
        float* scratch = nullptr;
        int rc = ctx->scratch(qlinear_small_scratch(wg->w.N, wg->w.K, true), &scratch);
        if (rc) return rc;
        return launch_qlinear_small(ctx->stream, wg->w, &wu->w, x, M, norm_w, eps, nullptr, scratch,
                                    ctx->small_tile_ctr, kSmallMaxTiles, h);
    }
    if (M <= 16) return launch_qlinear_swiglu(ctx->stream, wg->w, wu->w, x, h, M, norm_w, eps);
    VH_ARG(x && h, "swiglu: null activation pointer");
    const size_t a_bytes = ((size_t)M * wg->w.K * sizeof(uint16_t) + 255) & ~(size_t)255;
    const size_t p_bytes = qgemm_part_bytes(wg->w, M, true);
    float* scratch = nullptr;
    int rc = ctx->scratch(a_bytes + p_bytes, &scratch);
    if (rc) return rc;
    uint16_t* a = reinterpret_cast<uint16_t*>(scratch);
    float* part = p_bytes ? reinterpret_cast<float*>(reinterpret_cast<char*>(scratch) + a_bytes) : nullptr;
    rc = launch_rows_to_bf16(ctx->stream, x, norm_w, a, M, wg->w.K, eps);
    if (rc) return rc;
    return launch_qgemm_swiglu(ctx->stream, wg->w, wu->w, a, M, h, false, part);
}

// ---- the engine's remaining per-op backend calls --------------------------------------
int vlrf_hip_gemm_f32(vlrf_hip_ctx_t ctx, const float* A, const float* B, float* C, int M, int N, int K,
                      int lda, int ldb, int ldc, float alpha, float beta, int transA, int transB) {
    VH_CTX(ctx);
    return launch_gemm_f32(ctx->stream, A, B, C, M, N, K, lda, ldb, ldc, alpha, beta, transA != 0, transB != 0);
}

int vlrf_hip_layer_norm(vlrf_hip_ctx_t ctx, const float* x, const float* w, const float* b, float* out,
                        int rows, int D, float eps) {
    VH_CTX(ctx);
    return launch_layer_norm(ctx->stream, x, w, b, out, rows, D, eps);
}

int vlrf_hip_softmax(vlrf_hip_ctx_t ctx, float* x, int rows, int D) {
    VH_CTX(ctx);
    return launch_softmax(ctx->stream, x, rows, D);
}

int vlrf_hip_gelu(vlrf_hip_ctx_t ctx, float* x, int64_t n) {
    VH_CTX(ctx);
    return launch_gelu(ctx->stream, x, n);
}

int vlrf_hip_add(vlrf_hip_ctx_t ctx, float* dst, const float* src, int64_t n) {
    VH_CTX(ctx);
    return launch_add(ctx->stream, dst, src, n);
}

// ---- edge ops ----------------------------------------------------------------------
int vlrf_hip_rmsnorm(vlrf_hip_ctx_t ctx, const float* x, const float* w, float* out, int rows, int D,
                     float eps) {
    VH_CTX(ctx);
    VH_ARG(x && w && out, "rmsnorm: null pointer");
    return launch_rmsnorm(ctx->stream, x, w, out, rows, D, eps);
}

int vlrf_hip_rope(vlrf_hip_ctx_t ctx, float* x, int T, int n_heads, int d_head, int pos_offset,
                  int max_seq, float theta) {
    VH_CTX(ctx);
    VH_ARG(x != nullptr, "rope: null pointer");
    VH_ARG(max_seq >= 1 && d_head >= 2 && d_head % 2 == 0, "rope: bad table shape");
    const float *c = nullptr, *s = nullptr;
    int rc = ctx->rope_tables(max_seq, d_head, theta, &c, &s);
    if (rc) return rc;
    return launch_rope(ctx->stream, x, T, n_heads, d_head, pos_offset, max_seq, c, s);
}

}  // extern "C"
