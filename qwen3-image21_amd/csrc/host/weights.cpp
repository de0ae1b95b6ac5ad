// GGUF weight upload and re-striding, exact dequant and the plain quantized
// matmul entry point.
#include <string.h>

#include <new>
#include <vector>

#include "internal.h"

namespace qimm_host {

int block_values(int type) {
    switch (type) {
    case QIMM_TYPE_F32: case QIMM_TYPE_F16: case QIMM_TYPE_BF16: return 1;
    case QIMM_TYPE_Q8_0: return 32;
    case QIMM_TYPE_Q4_K: case QIMM_TYPE_Q6_K: return 256;
    default: return 0;
    }
}

static int block_bytes(int type) {
    switch (type) {
    case QIMM_TYPE_F32: return 4;
    case QIMM_TYPE_F16: case QIMM_TYPE_BF16: return 2;
    case QIMM_TYPE_Q8_0: return 34;
    case QIMM_TYPE_Q4_K: return 144;
    case QIMM_TYPE_Q6_K: return 210;
    default: return 0;
    }
}

int64_t row_bytes(int type, int64_t cols) {
    const int bv = block_values(type);
    if (!bv || cols % bv) return -1;
    return cols / bv * block_bytes(type);
}

static inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

static inline float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// Re-lay one tensor (rows of GGUF blocks) into the device format the GEMM
// reads with 128-bit loads, then upload.
int upload_weight_rows(qimm_ctx *ctx, int type, int64_t rows, int64_t cols, const uint8_t *src,
                       qimm_weight **out) {
    *out = nullptr;
    if (!block_values(type)) return set_err(ctx, QIMM_ERR_TYPE, "weight: unsupported GGML type");
    const int64_t rb = row_bytes(type, cols);
    if (rb < 0) return set_err(ctx, QIMM_ERR_SHAPE, "weight: cols is not a multiple of the block size");
    if (rows <= 0 || cols <= 0) return set_err(ctx, QIMM_ERR_SHAPE, "weight: empty tensor");
    qimm_weight *w = new (std::nothrow) qimm_weight();
    if (!w) return QIMM_ERR_OOM;
    w->ctx = ctx;
    w->ggml_type = type;
    w->rows = rows;
    w->cols = cols;
    std::vector<uint8_t> main_bytes, scale_bytes;
    int fmt;
    try {
        if (type == QIMM_TYPE_Q8_0) {
            fmt = qimm::WF_Q8_0;
            main_bytes.resize((size_t)(rows * cols));
            scale_bytes.resize((size_t)(rows * (cols / 32)) * 2);
            for (int64_t r = 0; r < rows; r++)
                for (int64_t b = 0; b < cols / 32; b++) {
                    const uint8_t *blk = src + r * rb + b * 34;
                    memcpy(&scale_bytes[(size_t)(r * (cols / 32) + b) * 2], blk, 2);
                    memcpy(&main_bytes[(size_t)(r * cols + b * 32)], blk + 2, 32);
                }
        } else if (type == QIMM_TYPE_Q4_K) {
            // 16-row groups, interleaved per super-block (the byte order the
            // short-M kernel streams; every kernel addresses blocks the same way)
            fmt = qimm::WF_Q4_K;
            if (rows % 16) {
                delete w;
                return set_err(ctx, QIMM_ERR_SHAPE, "weight: Q4_K tensors need rows % 16 == 0");
            }
            const int64_t sbs = cols / 256;
            main_bytes.resize((size_t)(rows * rb));
            for (int64_t r = 0; r < rows; r++)
                for (int64_t sb = 0; sb < sbs; sb++)
                    memcpy(&main_bytes[(size_t)((((r / 16) * sbs + sb) * 16 + r % 16) * 144)], src + r * rb + sb * 144,
                           144);
        } else if (type == QIMM_TYPE_Q6_K) {
            // 210 B blocks padded to 224 B (16 B aligned), 16-row groups
            // interleaved per super-block like Q4_K, so a wave's rows load from
            // one contiguous run
            fmt = qimm::WF_Q6_K;
            if (rows % 16) {
                delete w;
                return set_err(ctx, QIMM_ERR_SHAPE, "weight: Q6_K tensors need rows % 16 == 0");
            }
            const int64_t sbs = cols / 256;
            main_bytes.assign((size_t)(rows * sbs) * 224, 0);
            for (int64_t r = 0; r < rows; r++)
                for (int64_t sb = 0; sb < sbs; sb++)
                    memcpy(&main_bytes[(size_t)((((r / 16) * sbs + sb) * 16 + r % 16) * 224)], src + r * rb + sb * 210,
                           210);
        } else {
            // Float-stored weights feed the bf16 MFMA path: BF16 as is, F16 and
            // F32 rounded to bf16 (nearest even).
            fmt = qimm::WF_BF16;
            main_bytes.resize((size_t)(rows * cols) * 2);
            uint16_t *dst = (uint16_t *)main_bytes.data();
            for (int64_t i = 0; i < rows * cols; i++) {
                if (type == QIMM_TYPE_BF16) memcpy(&dst[i], src + 2 * i, 2);
                else if (type == QIMM_TYPE_F16) {
                    uint16_t h;
                    memcpy(&h, src + 2 * i, 2);
                    dst[i] = f32_to_bf16_rne(f16_to_f32(h));
                } else {
                    float f;
                    memcpy(&f, src + 4 * i, 4);
                    dst[i] = f32_to_bf16_rne(f);
                }
            }
        }
    } catch (const std::bad_alloc &) {
        delete w;
        return set_err(ctx, QIMM_ERR_OOM, "weight: host staging allocation failed");
    }
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMalloc(&w->dev, main_bytes.size());
    if (e == hipSuccess) e = hipMemcpy(w->dev, main_bytes.data(), main_bytes.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && !scale_bytes.empty()) {
        e = hipMalloc(&w->dev_scales, scale_bytes.size());
        if (e == hipSuccess)
            e = hipMemcpy(w->dev_scales, scale_bytes.data(), scale_bytes.size(), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        if (w->dev) (void)hipFree(w->dev);
        if (w->dev_scales) (void)hipFree(w->dev_scales);
        delete w;
        return hip_err(ctx, e, "weight upload");
    }
    w->dev_bytes = main_bytes.size() + scale_bytes.size();
    w->gw.fmt = fmt;
    w->gw.n = rows;
    w->gw.k = cols;
    w->gw.q = (const uint8_t *)w->dev;
    w->gw.scales = (const uint16_t *)w->dev_scales;
    *out = w;
    return QIMM_OK;
}

}  // namespace qimm_host

using namespace qimm_host;

extern "C" {

int qimm_weight_upload(qimm_ctx *ctx, int ggml_type, int64_t rows, int64_t cols, const void *host_bytes,
                       size_t nbytes, qimm_weight **out) {
    if (!ctx || !host_bytes || !out) return QIMM_ERR_ARG;
    if (!block_values(ggml_type)) return set_err(ctx, QIMM_ERR_TYPE, "weight: unsupported GGML type");
    const int64_t rb = row_bytes(ggml_type, cols);
    if (rb < 0) return set_err(ctx, QIMM_ERR_SHAPE, "weight: cols is not a multiple of the block size");
    if (rows <= 0 || (size_t)(rb * rows) != nbytes)
        return set_err(ctx, QIMM_ERR_SHAPE, "weight: byte count does not match rows x cols");
    return upload_weight_rows(ctx, ggml_type, rows, cols, (const uint8_t *)host_bytes, out);
}

int qimm_weight_free(qimm_weight *w) {
    if (!w) return QIMM_ERR_ARG;
    if (w->dev) (void)hipFree(w->dev);
    if (w->dev_scales) (void)hipFree(w->dev_scales);
    delete w;
    return QIMM_OK;
}

int64_t qimm_weight_device_bytes(const qimm_weight *w) { return w ? (int64_t)w->dev_bytes : -1; }

int qimm_dequant(qimm_ctx *ctx, int ggml_type, const void *dev_bytes, int64_t n, float *dev_out, void *stream) {
    if (!ctx || !dev_bytes || !dev_out || n < 0) return QIMM_ERR_ARG;
    const int bv = block_values(ggml_type);
    if (!bv) return set_err(ctx, QIMM_ERR_TYPE, "dequant: unsupported GGML type");
    if (n % 32 || n % bv) return set_err(ctx, QIMM_ERR_SHAPE, "dequant: n must be a multiple of 32 and of the block size");
    QIMM_HIP(ctx, qimm::launch_dequant(ggml_type, (const uint8_t *)dev_bytes, n, dev_out, (hipStream_t)stream));
    return QIMM_OK;
}

namespace {

static_assert(qimm::NOALLOC_SCRATCH_BYTES == QIMM_NOALLOC_SCRATCH_BYTES, "static scratch size of qimm.h");

int qmatmul_check(qimm_ctx *ctx, const qimm_weight *w, const void *x_bf16, int64_t m, int64_t lda, void *y,
                  int out_type) {
    if (!ctx || !w || !x_bf16 || !y || m < 0) return QIMM_ERR_ARG;
    if (out_type != QIMM_TYPE_F32 && out_type != QIMM_TYPE_BF16)
        return set_err(ctx, QIMM_ERR_TYPE, "qmatmul: output must be F32 or BF16");
    if (w->rows % 128 || w->cols % 64 || lda < w->cols || lda % 8)
        return set_err(ctx, QIMM_ERR_SHAPE, "qmatmul: needs N % 128 == 0, K % 64 == 0, lda >= K, lda % 8 == 0");
    if (((uintptr_t)x_bf16 | (uintptr_t)y) & 15)
        return set_err(ctx, QIMM_ERR_ARG, "qmatmul: x and y must be 16-byte aligned");
    return QIMM_OK;
}

}  // namespace

int qimm_qmatmul(qimm_ctx *ctx, const qimm_weight *w, const void *x_bf16, int64_t m, int64_t lda, void *y,
                 int out_type, void *stream) {
    if (const int rc = qmatmul_check(ctx, w, x_bf16, m, lda, y, out_type)) return rc;
    QIMM_HIP(ctx, hipSetDevice(ctx->device));
    qimm::EpiParams ep{};
    ep.out = y;
    ep.ldo = w->rows;
    if (const size_t need = qimm::qgemm_workspace(w->gw, m)) {
        const int rc = qimm_host::ensure_part_workspace(ctx, need);
        if (rc) return rc;
        ep.part_ws = (float *)ctx->ws_part;
        ep.part_ws_bytes = ctx->ws_part_bytes;
    }
    QIMM_HIP(ctx, qimm::launch_qgemm(w->gw, (const uint16_t *)x_bf16, m, lda,
                                     out_type == QIMM_TYPE_F32 ? qimm::EPI_F32 : qimm::EPI_BF16, ep,
                                     (hipStream_t)stream));
    return QIMM_OK;
}

int qimm_qmatmul_noalloc(qimm_ctx *ctx, const qimm_weight *w, const void *x_bf16, int64_t m, int64_t lda, void *y,
                         int out_type, void *stream) {
    if (const int rc = qmatmul_check(ctx, w, x_bf16, m, lda, y, out_type)) return rc;
    QIMM_HIP(ctx, hipSetDevice(ctx->device));
    qimm::EpiParams ep{};
    ep.out = y;
    ep.ldo = w->rows;
    if (const size_t need = qimm::qgemm_workspace(w->gw, m)) {
        if (need > qimm::NOALLOC_SCRATCH_BYTES)
            return set_err(ctx, QIMM_ERR_SHAPE,
                           "qmatmul_noalloc: this product needs " + std::to_string(need) +
                               " bytes of scratch, more than the static " +
                               std::to_string(qimm::NOALLOC_SCRATCH_BYTES) + "; use qimm_qmatmul");
        void *p = qimm::noalloc_scratch(ctx->device);
        if (!p) return set_err(ctx, QIMM_ERR_STATE, "qmatmul_noalloc: static scratch not set up on this device");
        ep.part_ws = (float *)p;
        ep.part_ws_bytes = qimm::NOALLOC_SCRATCH_BYTES;
    }
    QIMM_HIP(ctx, qimm::launch_qgemm(w->gw, (const uint16_t *)x_bf16, m, lda,
                                     out_type == QIMM_TYPE_F32 ? qimm::EPI_F32 : qimm::EPI_BF16, ep,
                                     (hipStream_t)stream));
    return QIMM_OK;
}

int64_t qimm_qmatmul_scratch_bytes(const qimm_weight *w, int64_t m) {
    if (!w || m < 0) return -1;
    if (hipSetDevice(w->ctx->device) != hipSuccess) return -1;
    return (int64_t)qimm::qgemm_workspace(w->gw, m);
}

}  // extern "C"
