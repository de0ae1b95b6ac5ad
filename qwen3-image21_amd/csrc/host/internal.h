// Host-side objects behind the C ABI of include/qimm.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../kernels/kernels.h"
#include "qimm.h"

struct qimm_ctx {
    int device = 0;
    std::string err;
    // Growable scratch for block intermediates, reused across calls on this
    // context (calls on one context are serialized by the caller).
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // Growable f32 scratch for the split-K partial sums of the short-M GEMM.
    void *ws_part = nullptr;
    size_t ws_part_bytes = 0;
};

struct qimm_weight {
    qimm_ctx *ctx = nullptr;
    int ggml_type = 0;
    int64_t rows = 0, cols = 0;
    void *dev = nullptr;        // codes / blocks
    void *dev_scales = nullptr; // Q8_0 f16 scales
    size_t dev_bytes = 0;
    qimm::GemmWeight gw{};
};

struct qimm_kv {
    qimm_ctx *ctx = nullptr;
    int64_t layers = 0, batch = 0, heads = 0, prefix = 0, head_dim = 0;
    // device cache: k [L][B][H][P][128], vt [L][B][H][128][P]; host cache: the
    // same layout in pinned host memory, staged one layer at a time into slots
    uint16_t *k = nullptr;
    uint16_t *vt = nullptr;
    bool host = false;
    // device [layers]: the largest key norm of each stored layer (+inf until
    // stored), the attention's score bound; [layers][QK_NORM_PARTS] scratch of
    // its reduction
    float *knorm = nullptr;
    float *knorm_part = nullptr;
    // Host cache: two device slots of one layer each. `ready` is recorded after
    // the copy into the slot, `released` after the last kernel reading it; a
    // copy into a slot waits for both, a reader waits for `ready`. `written` is
    // recorded after each store into host memory; every staging copy waits on it.
    struct Slot {
        uint16_t *k = nullptr, *vt = nullptr;
        int64_t layer = -1;
        hipEvent_t ready = nullptr, released = nullptr;
    };
    mutable Slot slot[2];
    mutable int next = 0;
    hipEvent_t written = nullptr;
    int64_t layer_elems() const { return batch * heads * prefix * head_dim; }
};

struct qimm_block {
    qimm_ctx *ctx = nullptr;
    qimm_block_config cfg{};
    bool qkv_fused = false;
    qimm_weight *qkv = nullptr;          // fused [3*hidden, hidden] when types match
    qimm_weight *q = nullptr, *k = nullptr, *v = nullptr;
    qimm_weight *out = nullptr;
    qimm_weight *gate_up = nullptr;      // rows interleaved per 64: gate | up
    qimm_weight *down = nullptr;
    float *norm_q = nullptr, *norm_k = nullptr;  // device [128]
    // bounds of the q (softmax scale and log2 e folded in) and k norms after the
    // q/k RmsNorm: sqrt(128) max|w| times those factors, with slack for RoPE
    // and the bf16 rounding
    float q_norm_bound = 0.f, k_norm_bound = 0.f;
    int act = QIMM_ACT_CANDLE;           // arithmetic at the quantized matmul inputs
    // stage timing (qimm_block_profile): events around the stages of a forward
    bool profiling = false;
    bool profiled_once = false;
    hipEvent_t ev[QIMM_BLOCK_STAGES + 1] = {};
};

namespace qimm_host {

int set_err(qimm_ctx *ctx, int status, const std::string &msg);
int hip_err(qimm_ctx *ctx, hipError_t e, const char *what);
int ensure_workspace(qimm_ctx *ctx, size_t bytes);
int ensure_part_workspace(qimm_ctx *ctx, size_t bytes);
int upload_weight_rows(qimm_ctx *ctx, int type, int64_t rows, int64_t cols, const uint8_t *bytes,
                       qimm_weight **out);
int64_t row_bytes(int type, int64_t cols);
int block_values(int type);

// Device pointers of cache layer `layer` for kernels launched on stream s. A
// host cache stages the layer into a slot first (or waits for a prefetch);
// kv_release must follow the last kernel that reads the pointers.
int kv_layer(const qimm_kv *kv, int64_t layer, hipStream_t s, const uint16_t **k, const uint16_t **vt);
int kv_release(const qimm_kv *kv, int64_t layer, hipStream_t s);

}  // namespace qimm_host

#define QIMM_HIP(ctx, call)                                         \
    do {                                                            \
        hipError_t e_ = (call);                                     \
        if (e_ != hipSuccess) return qimm_host::hip_err((ctx), e_, #call); \
    } while (0)
