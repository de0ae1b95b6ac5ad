// Context, errors, device memory helpers and the prefix K/V cache.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <new>

#include <math.h>

#include <vector>

#include "internal.h"

namespace qimm_host {

int set_err(qimm_ctx *ctx, int status, const std::string &msg) {
    if (ctx) ctx->err = msg;
    return status;
}

int hip_err(qimm_ctx *ctx, hipError_t e, const char *what) {
    char buf[512];
    snprintf(buf, sizeof(buf), "HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
    return set_err(ctx, e == hipErrorOutOfMemory ? QIMM_ERR_OOM : QIMM_ERR_HIP, buf);
}

int ensure_workspace(qimm_ctx *ctx, size_t bytes) {
    if (bytes <= ctx->ws_bytes) return QIMM_OK;
    if (ctx->ws) {
        QIMM_HIP(ctx, hipDeviceSynchronize());
        QIMM_HIP(ctx, hipFree(ctx->ws));
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    bytes = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    QIMM_HIP(ctx, hipMalloc(&ctx->ws, bytes));
    ctx->ws_bytes = bytes;
    return QIMM_OK;
}

int ensure_part_workspace(qimm_ctx *ctx, size_t bytes) {
    if (bytes <= ctx->ws_part_bytes) return QIMM_OK;
    if (ctx->ws_part) {
        QIMM_HIP(ctx, hipDeviceSynchronize());
        QIMM_HIP(ctx, hipFree(ctx->ws_part));
        ctx->ws_part = nullptr;
        ctx->ws_part_bytes = 0;
    }
    bytes = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    QIMM_HIP(ctx, hipMalloc(&ctx->ws_part, bytes));
    ctx->ws_part_bytes = bytes;
    // the arrival counters at the front of the short-M GEMM scratch start at
    // zero; the kernels leave them zero after every call. The fill runs on the
    // null stream, so wait for it: the GEMM that reads the counters may be
    // launched on a non-blocking stream, which the null stream does not order.
    QIMM_HIP(ctx, hipMemset(ctx->ws_part, 0, std::min(bytes, qimm::STREAM_COUNTER_BYTES)));
    QIMM_HIP(ctx, hipDeviceSynchronize());
    return QIMM_OK;
}

}  // namespace qimm_host

using namespace qimm_host;

extern "C" {

int qimm_abi_version(void) { return QIMM_ABI_VERSION; }

const char *qimm_status_string(int status) {
    switch (status) {
    case QIMM_OK: return "ok";
    case QIMM_ERR_ARG: return "invalid argument";
    case QIMM_ERR_SHAPE: return "unsupported or inconsistent shape";
    case QIMM_ERR_TYPE: return "unsupported GGML type";
    case QIMM_ERR_OOM: return "out of memory";
    case QIMM_ERR_HIP: return "HIP runtime error";
    case QIMM_ERR_STATE: return "invalid state";
    case QIMM_ERR_NOT_FOUND: return "not found";
    case QIMM_ERR_FORMAT: return "malformed file";
    default: return "unknown status";
    }
}

int qimm_ctx_create(int device, qimm_ctx **out) {
    if (!out) return QIMM_ERR_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return QIMM_ERR_ARG;
    if (hipSetDevice(device) != hipSuccess) return QIMM_ERR_HIP;
    // once per device: the static scratch of qimm_qmatmul_noalloc
    if (qimm::noalloc_scratch_setup(device) != hipSuccess) return QIMM_ERR_HIP;
    qimm_ctx *c = new (std::nothrow) qimm_ctx();
    if (!c) return QIMM_ERR_OOM;
    c->device = device;
    *out = c;
    return QIMM_OK;
}

int qimm_ctx_destroy(qimm_ctx *ctx) {
    if (!ctx) return QIMM_ERR_ARG;
    if (ctx->ws || ctx->ws_part) {
        (void)hipSetDevice(ctx->device);
        (void)hipDeviceSynchronize();
        if (ctx->ws) (void)hipFree(ctx->ws);
        if (ctx->ws_part) (void)hipFree(ctx->ws_part);
    }
    delete ctx;
    return QIMM_OK;
}

const char *qimm_last_error(const qimm_ctx *ctx) {
    if (!ctx) return "null context";
    return ctx->err.c_str();
}

int qimm_malloc(qimm_ctx *ctx, size_t bytes, void **dptr) {
    if (!ctx || !dptr) return QIMM_ERR_ARG;
    QIMM_HIP(ctx, hipSetDevice(ctx->device));
    QIMM_HIP(ctx, hipMalloc(dptr, bytes ? bytes : 1));
    return QIMM_OK;
}

int qimm_free(qimm_ctx *ctx, void *dptr) {
    if (!ctx) return QIMM_ERR_ARG;
    if (!dptr) return QIMM_OK;
    QIMM_HIP(ctx, hipFree(dptr));
    return QIMM_OK;
}

int qimm_memcpy_h2d(qimm_ctx *ctx, void *dst, const void *src, size_t bytes, void *stream) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return QIMM_ERR_ARG;
    QIMM_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
    return QIMM_OK;
}

int qimm_memcpy_d2h(qimm_ctx *ctx, void *dst, const void *src, size_t bytes, void *stream) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return QIMM_ERR_ARG;
    QIMM_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
    QIMM_HIP(ctx, hipStreamSynchronize((hipStream_t)stream));
    return QIMM_OK;
}

int qimm_stream_synchronize(qimm_ctx *ctx, void *stream) {
    if (!ctx) return QIMM_ERR_ARG;
    QIMM_HIP(ctx, hipStreamSynchronize((hipStream_t)stream));
    return QIMM_OK;
}

}  // extern "C"

/* ---- prefix K/V cache (TextKvCache, src/transformer.rs:14-45) ---- */

namespace {

int kv_new(qimm_ctx *ctx, int64_t layers, int64_t batch, int64_t heads, int64_t prefix_len, int64_t head_dim,
           qimm_kv **kv_out) {
    if (layers <= 0 || batch <= 0 || heads <= 0 || prefix_len < 0)
        return set_err(ctx, QIMM_ERR_SHAPE, "kv cache: layers, batch and heads must be positive");
    if (head_dim != 128) return set_err(ctx, QIMM_ERR_SHAPE, "kv cache: head_dim must be 128");
    qimm_kv *kv = new (std::nothrow) qimm_kv();
    if (!kv) return QIMM_ERR_OOM;
    kv->ctx = ctx;
    kv->layers = layers;
    kv->batch = batch;
    kv->heads = heads;
    kv->prefix = prefix_len;
    kv->head_dim = head_dim;
    *kv_out = kv;
    return QIMM_OK;
}

// The per-layer key-norm bounds, +inf (no bound) until a layer is stored.
hipError_t kv_alloc_norms(qimm_kv *kv) {
    hipError_t e = hipMalloc((void **)&kv->knorm, (size_t)kv->layers * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&kv->knorm_part, (size_t)kv->layers * qimm::QK_NORM_PARTS * 4);
    if (e == hipSuccess) {
        std::vector<float> inf((size_t)kv->layers, INFINITY);
        e = hipMemcpy(kv->knorm, inf.data(), inf.size() * 4, hipMemcpyHostToDevice);
    }
    return e;
}

void kv_free(qimm_kv *kv) {
    if (kv->knorm) (void)hipFree(kv->knorm);
    if (kv->knorm_part) (void)hipFree(kv->knorm_part);
    if (kv->host) {
        if (kv->k) (void)hipHostFree(kv->k);
        if (kv->vt) (void)hipHostFree(kv->vt);
        for (auto &sl : kv->slot) {
            if (sl.k) (void)hipFree(sl.k);
            if (sl.vt) (void)hipFree(sl.vt);
            if (sl.ready) (void)hipEventDestroy(sl.ready);
            if (sl.released) (void)hipEventDestroy(sl.released);
        }
        if (kv->written) (void)hipEventDestroy(kv->written);
    } else {
        if (kv->k) (void)hipFree(kv->k);
        if (kv->vt) (void)hipFree(kv->vt);
    }
    delete kv;
}

// Claims the slot to stage `layer` on stream s: waits (on s) until the slot's
// last copy and last reader are done and every store into host memory landed.
qimm_kv::Slot *kv_claim(const qimm_kv *kv, int64_t layer, hipStream_t s, int &rc) {
    qimm_ctx *ctx = kv->ctx;
    qimm_kv::Slot *sl = &kv->slot[kv->next];
    kv->next ^= 1;
    hipError_t e = hipStreamWaitEvent(s, sl->ready, 0);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, sl->released, 0);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, kv->written, 0);
    if (e != hipSuccess) {
        rc = hip_err(ctx, e, "hipStreamWaitEvent(kv slot)");
        return nullptr;
    }
    sl->layer = layer;
    rc = QIMM_OK;
    return sl;
}

// Copies host layer `layer` into slot sl on s and records its ready event.
int kv_stage(const qimm_kv *kv, qimm_kv::Slot *sl, int64_t layer, hipStream_t s) {
    qimm_ctx *ctx = kv->ctx;
    const size_t bytes = (size_t)kv->layer_elems() * 2;
    QIMM_HIP(ctx, hipMemcpyAsync(sl->k, kv->k + layer * kv->layer_elems(), bytes, hipMemcpyHostToDevice, s));
    QIMM_HIP(ctx, hipMemcpyAsync(sl->vt, kv->vt + layer * kv->layer_elems(), bytes, hipMemcpyHostToDevice, s));
    QIMM_HIP(ctx, hipEventRecord(sl->ready, s));
    return QIMM_OK;
}

}  // namespace

namespace qimm_host {

int kv_layer(const qimm_kv *kv, int64_t layer, hipStream_t s, const uint16_t **k, const uint16_t **vt) {
    if (!kv->host) {
        *k = kv->k + layer * kv->layer_elems();
        *vt = kv->vt + layer * kv->layer_elems();
        return QIMM_OK;
    }
    if (!kv->layer_elems()) {
        *k = *vt = nullptr;
        return QIMM_OK;
    }
    qimm_kv::Slot *sl = nullptr;
    for (auto &x : kv->slot)
        if (x.layer == layer) sl = &x;
    if (sl) {  // staged by a prefetch (possibly on another stream)
        QIMM_HIP(kv->ctx, hipStreamWaitEvent(s, sl->ready, 0));
    } else {
        int rc;
        sl = kv_claim(kv, layer, s, rc);
        if (!sl) return rc;
        if ((rc = kv_stage(kv, sl, layer, s))) return rc;
    }
    *k = sl->k;
    *vt = sl->vt;
    return QIMM_OK;
}

int kv_release(const qimm_kv *kv, int64_t layer, hipStream_t s) {
    if (!kv->host) return QIMM_OK;
    for (auto &x : kv->slot)
        if (x.layer == layer) QIMM_HIP(kv->ctx, hipEventRecord(x.released, s));
    return QIMM_OK;
}

}  // namespace qimm_host

extern "C" {

int qimm_kv_create(qimm_ctx *ctx, int64_t layers, int64_t batch, int64_t heads, int64_t prefix_len,
                   int64_t head_dim, qimm_kv **out) {
    if (!ctx || !out) return QIMM_ERR_ARG;
    *out = nullptr;
    qimm_kv *kv;
    int rc = kv_new(ctx, layers, batch, heads, prefix_len, head_dim, &kv);
    if (rc) return rc;
    const size_t bytes = (size_t)(layers * kv->layer_elems()) * 2;
    if (bytes) {
        hipError_t e = hipSetDevice(ctx->device);
        if (e == hipSuccess) e = hipMalloc((void **)&kv->k, bytes);
        if (e == hipSuccess) e = hipMalloc((void **)&kv->vt, bytes);
        if (e == hipSuccess) e = kv_alloc_norms(kv);
        if (e != hipSuccess) {
            kv_free(kv);
            return hip_err(ctx, e, "hipMalloc(kv cache)");
        }
    }
    *out = kv;
    return QIMM_OK;
}

int qimm_kv_create_host(qimm_ctx *ctx, int64_t layers, int64_t batch, int64_t heads, int64_t prefix_len,
                        int64_t head_dim, qimm_kv **out) {
    if (!ctx || !out) return QIMM_ERR_ARG;
    *out = nullptr;
    qimm_kv *kv;
    int rc = kv_new(ctx, layers, batch, heads, prefix_len, head_dim, &kv);
    if (rc) return rc;
    kv->host = true;
    const size_t lbytes = (size_t)kv->layer_elems() * 2, bytes = lbytes * (size_t)layers;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess && bytes) e = hipHostMalloc((void **)&kv->k, bytes, hipHostMallocDefault);
    if (e == hipSuccess && bytes) e = hipHostMalloc((void **)&kv->vt, bytes, hipHostMallocDefault);
    for (auto &sl : kv->slot) {
        if (e == hipSuccess && lbytes) e = hipMalloc((void **)&sl.k, lbytes);
        if (e == hipSuccess && lbytes) e = hipMalloc((void **)&sl.vt, lbytes);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&sl.ready, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&sl.released, hipEventDisableTiming);
    }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&kv->written, hipEventDisableTiming);
    if (e == hipSuccess) e = kv_alloc_norms(kv);
    if (e != hipSuccess) {
        kv_free(kv);
        return hip_err(ctx, e, "kv host cache allocation");
    }
    *out = kv;
    return QIMM_OK;
}

int qimm_kv_destroy(qimm_kv *kv) {
    if (!kv) return QIMM_ERR_ARG;
    if (kv->host) (void)hipDeviceSynchronize();  // no copy may still read or write the buffers
    kv_free(kv);
    return QIMM_OK;
}

int64_t qimm_kv_prefix_len(const qimm_kv *kv) { return kv ? kv->prefix : -1; }

int qimm_kv_is_host(const qimm_kv *kv) { return kv && kv->host ? 1 : 0; }

int qimm_kv_store_layer(qimm_kv *kv, int64_t layer, const uint16_t *k_bhpd, const uint16_t *v_bhpd,
                        void *stream) {
    if (!kv || !k_bhpd || !v_bhpd) return QIMM_ERR_ARG;
    qimm_ctx *ctx = kv->ctx;
    if (layer < 0 || layer >= kv->layers) return set_err(ctx, QIMM_ERR_SHAPE, "kv store: layer out of range");
    const int64_t n = kv->layer_elems();
    if (!n) return QIMM_OK;
    hipStream_t s = (hipStream_t)stream;
    // the layer's largest key norm: the attention's score bound
    QIMM_HIP(ctx, qimm::launch_row_norm_max(k_bhpd, n / 128, kv->knorm_part + layer * qimm::QK_NORM_PARTS,
                                            kv->knorm + layer, s));
    if (!kv->host) {
        QIMM_HIP(ctx, hipMemcpyAsync(kv->k + layer * n, k_bhpd, (size_t)n * 2, hipMemcpyDeviceToDevice, s));
        QIMM_HIP(ctx, qimm::launch_transpose_sd(v_bhpd, kv->batch * kv->heads, kv->prefix, kv->vt + layer * n, 0, s));
        return QIMM_OK;
    }
    // transpose V into a slot, then both halves down to host memory; the slot
    // then holds this layer (K copied device-to-device beside it)
    int rc;
    for (auto &x : kv->slot) {
        if (x.layer == layer) x.layer = -1;  // a staged copy of the old contents is stale
        // no staging copy may still be reading the host memory this store overwrites
        QIMM_HIP(ctx, hipStreamWaitEvent(s, x.ready, 0));
    }
    qimm_kv::Slot *sl = kv_claim(kv, layer, s, rc);
    if (!sl) return rc;
    QIMM_HIP(ctx, hipMemcpyAsync(sl->k, k_bhpd, (size_t)n * 2, hipMemcpyDeviceToDevice, s));
    QIMM_HIP(ctx, qimm::launch_transpose_sd(v_bhpd, kv->batch * kv->heads, kv->prefix, sl->vt, 0, s));
    QIMM_HIP(ctx, hipMemcpyAsync(kv->k + layer * n, sl->k, (size_t)n * 2, hipMemcpyDeviceToHost, s));
    QIMM_HIP(ctx, hipMemcpyAsync(kv->vt + layer * n, sl->vt, (size_t)n * 2, hipMemcpyDeviceToHost, s));
    QIMM_HIP(ctx, hipEventRecord(sl->ready, s));
    QIMM_HIP(ctx, hipEventRecord(kv->written, s));
    return QIMM_OK;
}

int qimm_kv_load_layer(const qimm_kv *kv, int64_t layer, uint16_t *k_bhpd, uint16_t *v_bhpd, void *stream) {
    if (!kv || !k_bhpd || !v_bhpd) return QIMM_ERR_ARG;
    qimm_ctx *ctx = kv->ctx;
    if (layer < 0 || layer >= kv->layers) return set_err(ctx, QIMM_ERR_SHAPE, "kv load: layer out of range");
    const int64_t n = kv->layer_elems();
    if (!n) return QIMM_OK;
    hipStream_t s = (hipStream_t)stream;
    const uint16_t *k, *vt;
    int rc = kv_layer(kv, layer, s, &k, &vt);
    if (rc) return rc;
    QIMM_HIP(ctx, hipMemcpyAsync(k_bhpd, k, (size_t)n * 2, hipMemcpyDeviceToDevice, s));
    QIMM_HIP(ctx, qimm::launch_transpose_sd(vt, kv->batch * kv->heads, kv->prefix, v_bhpd, 1, s));
    return kv_release(kv, layer, s);
}

int qimm_kv_prefetch(qimm_kv *kv, int64_t layer, void *stream) {
    if (!kv) return QIMM_ERR_ARG;
    qimm_ctx *ctx = kv->ctx;
    if (layer < 0 || layer >= kv->layers) return set_err(ctx, QIMM_ERR_SHAPE, "kv prefetch: layer out of range");
    if (!kv->host || !kv->layer_elems()) return QIMM_OK;
    for (auto &x : kv->slot)
        if (x.layer == layer) return QIMM_OK;
    hipStream_t s = (hipStream_t)stream;
    int rc;
    qimm_kv::Slot *sl = kv_claim(kv, layer, s, rc);
    if (!sl) return rc;
    return kv_stage(kv, sl, layer, s);
}

}  // extern "C"
