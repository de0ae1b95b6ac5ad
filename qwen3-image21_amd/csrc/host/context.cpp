// Context, errors, device memory helpers and the prefix K/V cache.
#include <stdio.h>
#include <string.h>

#include <new>

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
    default: return "unknown status";
    }
}

int qimm_ctx_create(int device, qimm_ctx **out) {
    if (!out) return QIMM_ERR_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return QIMM_ERR_ARG;
    if (hipSetDevice(device) != hipSuccess) return QIMM_ERR_HIP;
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

/* ---- prefix K/V cache (TextKvCache, src/transformer.rs:14-45) ---- */

int qimm_kv_create(qimm_ctx *ctx, int64_t layers, int64_t batch, int64_t heads, int64_t prefix_len,
                   int64_t head_dim, qimm_kv **out) {
    if (!ctx || !out) return QIMM_ERR_ARG;
    *out = nullptr;
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
    const size_t bytes = (size_t)(layers * kv->layer_elems()) * 2;
    if (bytes) {
        hipError_t e = hipSetDevice(ctx->device);
        if (e == hipSuccess) e = hipMalloc((void **)&kv->k, bytes);
        if (e == hipSuccess) e = hipMalloc((void **)&kv->vt, bytes);
        if (e != hipSuccess) {
            if (kv->k) (void)hipFree(kv->k);
            delete kv;
            return hip_err(ctx, e, "hipMalloc(kv cache)");
        }
    }
    *out = kv;
    return QIMM_OK;
}

int qimm_kv_destroy(qimm_kv *kv) {
    if (!kv) return QIMM_ERR_ARG;
    if (kv->k) (void)hipFree(kv->k);
    if (kv->vt) (void)hipFree(kv->vt);
    delete kv;
    return QIMM_OK;
}

int64_t qimm_kv_prefix_len(const qimm_kv *kv) { return kv ? kv->prefix : -1; }

int qimm_kv_store_layer(qimm_kv *kv, int64_t layer, const uint16_t *k_bhpd, const uint16_t *v_bhpd,
                        void *stream) {
    if (!kv || !k_bhpd || !v_bhpd) return QIMM_ERR_ARG;
    qimm_ctx *ctx = kv->ctx;
    if (layer < 0 || layer >= kv->layers) return set_err(ctx, QIMM_ERR_SHAPE, "kv store: layer out of range");
    const int64_t n = kv->layer_elems();
    if (!n) return QIMM_OK;
    hipStream_t s = (hipStream_t)stream;
    QIMM_HIP(ctx, hipMemcpyAsync(kv->k + layer * n, k_bhpd, (size_t)n * 2, hipMemcpyDeviceToDevice, s));
    QIMM_HIP(ctx, qimm::launch_transpose_sd(v_bhpd, kv->batch * kv->heads, kv->prefix, kv->vt + layer * n, 0, s));
    return QIMM_OK;
}

int qimm_kv_load_layer(const qimm_kv *kv, int64_t layer, uint16_t *k_bhpd, uint16_t *v_bhpd, void *stream) {
    if (!kv || !k_bhpd || !v_bhpd) return QIMM_ERR_ARG;
    qimm_ctx *ctx = kv->ctx;
    if (layer < 0 || layer >= kv->layers) return set_err(ctx, QIMM_ERR_SHAPE, "kv load: layer out of range");
    const int64_t n = kv->layer_elems();
    if (!n) return QIMM_OK;
    hipStream_t s = (hipStream_t)stream;
    QIMM_HIP(ctx, hipMemcpyAsync(k_bhpd, kv->k + layer * n, (size_t)n * 2, hipMemcpyDeviceToDevice, s));
    QIMM_HIP(ctx, qimm::launch_transpose_sd(kv->vt + layer * n, kv->batch * kv->heads, kv->prefix, v_bhpd, 1, s));
    return QIMM_OK;
}

}  // extern "C"
