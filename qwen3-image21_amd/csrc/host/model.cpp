// The denoising step around the blocks: the transformer's global layers
// (QwenImageTransformerQuantized, src/quantized_transformer.rs:311-551), the
// prefix fill (prefix_kv, :359-392), the t = 0 modulation (:334-343), the
// sigma schedule and Euler update (src/scheduler.rs:24-66), the CFG combine
// (src/pipeline.rs:180-186) and the joint layout's pieces
// (src/joint_layout.rs:52-126).
#include <math.h>
#include <string.h>

#include <new>
#include <vector>

#include "internal.h"

struct qimm_model {
    qimm_ctx *ctx = nullptr;
    qimm_model_config cfg{};
    std::vector<qimm_block *> blocks;
    // global weights, f32 [out][in] on the device
    float *img_in = nullptr, *t1 = nullptr, *t2 = nullptr, *mod = nullptr, *norm_out = nullptr,
          *proj_out = nullptr, *txt_norm = nullptr, *txt_in = nullptr, *txt_out = nullptr;
    // grow-only workspace
    void *ws = nullptr;
    size_t ws_bytes = 0;
};

namespace {

using namespace qimm_host;

constexpr float kEps = 1e-6f;  // LayerNorm and RmsNorm eps (src/quantized_transformer.rs:65-68, 231-237)
constexpr int kTimeDim = 256;  // timestep_embedding width (src/pipeline.rs:176)

// Dequantizes one global tensor (rows x cols, any supported type) to f32 on the device.
int upload_f32(qimm_ctx *ctx, const qimm_tensor &t, int64_t rows, int64_t cols, const char *what, float **out) {
    *out = nullptr;
    if (!t.data) return set_err(ctx, QIMM_ERR_ARG, std::string("model: missing ") + what);
    // a vector (rows == 1) may come as [1, n] or [n, 1]
    if (t.rows * t.cols != rows * cols || (rows > 1 && (t.rows != rows || t.cols != cols)))
        return set_err(ctx, QIMM_ERR_SHAPE, std::string("model: ") + what + " has the wrong shape");
    const int64_t rb = row_bytes(t.ggml_type, cols);
    if (rb < 0) return set_err(ctx, QIMM_ERR_TYPE, std::string("model: ") + what + ": unsupported type or row length");
    const size_t nbytes = (size_t)(rb * rows);
    if (t.nbytes != nbytes) return set_err(ctx, QIMM_ERR_SHAPE, std::string("model: ") + what + " has the wrong byte count");
    const int64_t n = rows * cols;
    if (n % 32) return set_err(ctx, QIMM_ERR_SHAPE, std::string("model: ") + what + " size must be a multiple of 32");
    void *raw = nullptr;
    float *dst = nullptr;
    hipError_t e = hipMalloc(&raw, nbytes);
    if (e == hipSuccess) e = hipMalloc((void **)&dst, (size_t)n * 4);
    if (e == hipSuccess) e = hipMemcpy(raw, t.data, nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = qimm::launch_dequant(t.ggml_type, (const uint8_t *)raw, n, dst, 0);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (raw) (void)hipFree(raw);
    if (e != hipSuccess) {
        if (dst) (void)hipFree(dst);
        return hip_err(ctx, e, what);
    }
    *out = dst;
    return QIMM_OK;
}

int ensure_ws(qimm_model *m, size_t bytes) {
    if (bytes <= m->ws_bytes) return QIMM_OK;
    qimm_ctx *ctx = m->ctx;
    if (m->ws) {
        QIMM_HIP(ctx, hipDeviceSynchronize());
        QIMM_HIP(ctx, hipFree(m->ws));
        m->ws = nullptr;
        m->ws_bytes = 0;
    }
    bytes = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    QIMM_HIP(ctx, hipMalloc(&m->ws, bytes));
    m->ws_bytes = bytes;
    return QIMM_OK;
}

// Carves 256-byte aligned f32 / byte regions out of one workspace.
struct Carver {
    char *base;
    size_t off = 0;
    template <class T>
    T *take(int64_t n) {
        T *p = (T *)(base + off);
        off += ((size_t)n * sizeof(T) + 255) & ~(size_t)255;
        return p;
    }
};

// t_emb = linear_2(silu(linear_1(t_sin))) and the three consumers' inputs
int time_embed(qimm_model *m, const float *t_sin, int64_t batch, float *tmp, float *temb, hipStream_t s) {
    const int64_t hid = m->cfg.hidden;
    QIMM_HIP(m->ctx, qimm::launch_linear_f32(t_sin, kTimeDim, m->t1, batch, hid, kTimeDim, qimm::ACT_NONE, tmp, hid, s));
    QIMM_HIP(m->ctx, qimm::launch_linear_f32(tmp, hid, m->t2, batch, hid, hid, qimm::ACT_SILU, temb, hid, s));
    return QIMM_OK;
}

void free_model(qimm_model *m) {
    for (float *p : {m->img_in, m->t1, m->t2, m->mod, m->norm_out, m->proj_out, m->txt_norm, m->txt_in, m->txt_out})
        if (p) (void)hipFree(p);
    if (m->ws) (void)hipFree(m->ws);
    delete m;
}

}  // namespace

extern "C" {

int qimm_model_create(qimm_ctx *ctx, const qimm_model_config *cfg, const qimm_model_tensors *t,
                      qimm_block *const *blocks, qimm_model **out) {
    if (!ctx || !cfg || !t || !out || (cfg->layers > 0 && !blocks)) return QIMM_ERR_ARG;
    *out = nullptr;
    if (cfg->in_channels <= 0 || cfg->hidden <= 0 || cfg->layers < 0 || cfg->joint_dim < 0)
        return set_err(ctx, QIMM_ERR_SHAPE, "model: sizes must be positive");
    for (int64_t i = 0; i < cfg->layers; i++)
        if (!blocks[i] || blocks[i]->cfg.hidden != cfg->hidden)
            return set_err(ctx, QIMM_ERR_SHAPE, "model: every block must exist and share the model's hidden size");
    qimm_model *m = new (std::nothrow) qimm_model();
    if (!m) return QIMM_ERR_OOM;
    m->ctx = ctx;
    m->cfg = *cfg;
    m->blocks.assign(blocks, blocks + cfg->layers);
    const int64_t hid = cfg->hidden, ch = cfg->in_channels, jd = cfg->joint_dim;
    int rc = hipSetDevice(ctx->device) == hipSuccess ? QIMM_OK : set_err(ctx, QIMM_ERR_HIP, "hipSetDevice");
    if (!rc) rc = upload_f32(ctx, t->img_in, hid, ch, "img_in", &m->img_in);
    if (!rc) rc = upload_f32(ctx, t->t_linear_1, hid, kTimeDim, "timestep_embedder.linear_1", &m->t1);
    if (!rc) rc = upload_f32(ctx, t->t_linear_2, hid, hid, "timestep_embedder.linear_2", &m->t2);
    if (!rc) rc = upload_f32(ctx, t->modulation, 4 * hid, hid, "modulation.1", &m->mod);
    if (!rc) rc = upload_f32(ctx, t->norm_out, hid, hid, "norm_out.linear", &m->norm_out);
    if (!rc) rc = upload_f32(ctx, t->proj_out, ch, hid, "proj_out", &m->proj_out);
    if (!rc && jd > 0) {
        rc = upload_f32(ctx, t->txt_norm, 1, jd, "txt_in.text_norm", &m->txt_norm);
        if (!rc) rc = upload_f32(ctx, t->txt_in, hid, jd, "txt_in.in_layer", &m->txt_in);
        if (!rc) rc = upload_f32(ctx, t->txt_out, hid, hid, "txt_in.out_layer", &m->txt_out);
        if (!rc) {  // ZeroCenterRMSNorm: the checkpoint stores scale - 1
            std::vector<float> w((size_t)jd);
            hipError_t e = hipMemcpy(w.data(), m->txt_norm, (size_t)jd * 4, hipMemcpyDeviceToHost);
            for (float &v : w) v += 1.0f;
            if (e == hipSuccess) e = hipMemcpy(m->txt_norm, w.data(), (size_t)jd * 4, hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = hip_err(ctx, e, "txt_in.text_norm");
        }
    }
    if (rc) {
        free_model(m);
        return rc;
    }
    *out = m;
    return QIMM_OK;
}

int qimm_model_destroy(qimm_model *m) {
    if (!m) return QIMM_ERR_ARG;
    (void)hipSetDevice(m->ctx->device);
    (void)hipDeviceSynchronize();
    free_model(m);
    return QIMM_OK;
}

int qimm_timestep_embedding(qimm_ctx *ctx, const float *t, int64_t batch, float *out, void *stream) {
    if (!ctx || !t || !out || batch <= 0) return QIMM_ERR_ARG;
    // exponent_i = exp(-ln(1e4) * (i / 128)) and emb = (t * 1000) * exponent_i, in f32 as the reference
    std::vector<float> h((size_t)batch * kTimeDim);
    const float log_theta = logf(10000.0f);
    for (int64_t b = 0; b < batch; b++) {
        const float tt = t[b] * 1000.0f;
        for (int i = 0; i < kTimeDim / 2; i++) {
            const float ex = expf(-log_theta * ((float)i / (float)(kTimeDim / 2)));
            const float a = tt * ex;
            h[(size_t)b * kTimeDim + i] = (float)cos((double)a);
            h[(size_t)b * kTimeDim + kTimeDim / 2 + i] = (float)sin((double)a);
        }
    }
    hipStream_t s = (hipStream_t)stream;
    QIMM_HIP(ctx, hipMemcpyAsync(out, h.data(), h.size() * 4, hipMemcpyHostToDevice, s));
    QIMM_HIP(ctx, hipStreamSynchronize(s));  // the host buffer is released on return
    return QIMM_OK;
}

int qimm_model_forward(qimm_model *m, const float *latents, int64_t batch, int64_t seq, const float *t_sin,
                       const float *pe, const qimm_kv *kv, const uint8_t *key_valid, float *pred, void *stream) {
    if (!m || !latents || !t_sin || !pe || !pred || batch <= 0 || seq <= 0) return QIMM_ERR_ARG;
    qimm_ctx *ctx = m->ctx;
    if (kv && (int64_t)kv->layers < m->cfg.layers) return set_err(ctx, QIMM_ERR_SHAPE, "model forward: cache has too few layers");
    const int64_t hid = m->cfg.hidden, ch = m->cfg.in_channels, rows = batch * seq;
    hipStream_t s = (hipStream_t)stream;
    QIMM_HIP(ctx, hipSetDevice(ctx->device));
    int rc = ensure_ws(m, (size_t)(rows * hid * 4) + (size_t)batch * (7 * hid) * 4 + 4096);
    if (rc) return rc;
    Carver c{(char *)m->ws};
    float *h = c.take<float>(rows * hid);
    float *tmp = c.take<float>(batch * hid), *temb = c.take<float>(batch * hid);
    float *modv = c.take<float>(batch * 4 * hid), *scale = c.take<float>(batch * hid);
    // time embedding and modulation (:537-539)
    if ((rc = time_embed(m, t_sin, batch, tmp, temb, s))) return rc;
    QIMM_HIP(ctx, qimm::launch_linear_f32(temb, hid, m->mod, batch, 4 * hid, hid, qimm::ACT_SILU, modv, 4 * hid, s));
    // target = img_in(latents) (:483)
    QIMM_HIP(ctx, qimm::launch_linear_f32(latents, ch, m->img_in, rows, hid, ch, qimm::ACT_NONE, h, hid, s));
    // the blocks, in place (:538-543)
    qimm_attn_mask mask{nullptr, key_valid};
    for (int64_t i = 0; i < m->cfg.layers; i++) {
        rc = key_valid ? qimm_block_forward_masked(m->blocks[(size_t)i], h, h, batch, seq, modv, 1, pe, &mask, kv, i,
                                                   nullptr, nullptr, stream)
                       : qimm_block_forward(m->blocks[(size_t)i], h, h, batch, seq, modv, pe, kv, i, nullptr, nullptr,
                                            stream);
        if (rc) return rc;
    }
    // norm_out and proj_out (:545, 300-309)
    QIMM_HIP(ctx, qimm::launch_linear_f32(temb, hid, m->norm_out, batch, hid, hid, qimm::ACT_SILU, scale, hid, s));
    QIMM_HIP(ctx, qimm::launch_rows_ln_scale(h, scale, rows, hid, seq, kEps, h, s));
    QIMM_HIP(ctx, qimm::launch_linear_f32(h, hid, m->proj_out, rows, ch, hid, qimm::ACT_NONE, pred, ch, s));
    return QIMM_OK;
}

int qimm_model_prefix_fill(qimm_model *m, const float *txt, int64_t text_len, const float *cond, int64_t cond_len,
                           int64_t batch, const int64_t *pieces, int64_t npieces, const int32_t *image_ids,
                           const uint8_t *key_valid, const float *pe, qimm_kv *kv, void *stream) {
    if (!m || !kv || !pe || batch <= 0 || text_len < 0 || cond_len < 0 || npieces < 0 || (npieces && !pieces) ||
        (text_len && !txt) || (cond_len && !cond))
        return QIMM_ERR_ARG;
    qimm_ctx *ctx = m->ctx;
    const int64_t hid = m->cfg.hidden, ch = m->cfg.in_channels, jd = m->cfg.joint_dim, P = kv->prefix;
    if (kv->batch != batch || kv->layers < m->cfg.layers)
        return set_err(ctx, QIMM_ERR_SHAPE, "prefix fill: cache batch or layer count differs");
    // without txt_in the prompt rows are used as they are (:368-371), so they are hidden wide
    const int64_t tw = jd ? jd : hid;  // prompt row width before txt_in
    int64_t total = 0;
    for (int64_t p = 0; p < npieces; p++) {
        const int64_t kind = pieces[3 * p], st = pieces[3 * p + 1], len = pieces[3 * p + 2];
        const int64_t lim = kind == 0 ? text_len : cond_len;
        if ((kind != 0 && kind != 1) || st < 0 || len < 0 || st + len > lim)
            return set_err(ctx, QIMM_ERR_SHAPE, "prefix fill: a piece lies outside its source rows");
        total += len;
    }
    if (total != P) return set_err(ctx, QIMM_ERR_SHAPE, "prefix fill: pieces do not cover the cache's prefix length");
    if (!P) return QIMM_OK;
    hipStream_t s = (hipStream_t)stream;
    QIMM_HIP(ctx, hipSetDevice(ctx->device));
    const int64_t H = kv->heads, trows = batch * text_len, crows = batch * cond_len;
    const size_t need = (size_t)(trows * (tw + 2 * hid) + crows * hid + batch * P * hid) * 4 +
                        (size_t)(2 * batch * H * P * 128) * 2 + (size_t)batch * (kTimeDim + 6 * hid) * 4 + 16 * 256;
    int rc = ensure_ws(m, need);
    if (rc) return rc;
    Carver c{(char *)m->ws};
    float *tn = c.take<float>(trows * tw), *tmid = c.take<float>(trows * hid), *tx = c.take<float>(trows * hid);
    float *cx = c.take<float>(crows * hid), *x = c.take<float>(batch * P * hid);
    uint16_t *kl = c.take<uint16_t>(batch * H * P * 128), *vl = c.take<uint16_t>(batch * H * P * 128);
    float *tsin = c.take<float>(batch * kTimeDim), *tmp = c.take<float>(batch * hid), *temb = c.take<float>(batch * hid);
    float *modv = c.take<float>(batch * 4 * hid);
    // txt_in: text_norm -> in_layer -> GELU(tanh) -> out_layer (:56-81)
    const float *txt_h = txt;
    if (text_len) {
        if (jd) {
            QIMM_HIP(ctx, qimm::launch_rows_rmsnorm(txt, m->txt_norm, trows, jd, kEps, tn, s));
            QIMM_HIP(ctx, qimm::launch_linear_f32(tn, jd, m->txt_in, trows, hid, jd, qimm::ACT_NONE, tmid, hid, s));
            QIMM_HIP(ctx, qimm::launch_linear_f32(tmid, hid, m->txt_out, trows, hid, hid, qimm::ACT_GELU_TANH, tx, hid, s));
            txt_h = tx;
        }
    }
    // condition latents through img_in (:373)
    if (cond_len)
        QIMM_HIP(ctx, qimm::launch_linear_f32(cond, ch, m->img_in, crows, hid, ch, qimm::ACT_NONE, cx, hid, s));
    // assemble the prefix rows in layout order (JointLayout::assemble narrowed to the prefix, :374)
    int64_t at = 0;
    for (int64_t p = 0; p < npieces; p++) {
        const int64_t kind = pieces[3 * p], st = pieces[3 * p + 1], len = pieces[3 * p + 2];
        if (!len) continue;
        const float *src = kind == 0 ? txt_h : cx;
        const int64_t src_rows = kind == 0 ? text_len : cond_len;
        QIMM_HIP(ctx, hipMemcpy2DAsync(x + at * hid, (size_t)(P * hid * 4), src + st * hid, (size_t)(src_rows * hid * 4),
                                       (size_t)(len * hid * 4), (size_t)batch, hipMemcpyDeviceToDevice, s));
        at += len;
    }
    // zero_modulation: the t = 0 sinusoid [1 .. 1, 0 .. 0] through the embedder (:334-343)
    {
        std::vector<float> z((size_t)batch * kTimeDim, 0.f);
        for (int64_t b = 0; b < batch; b++)
            for (int i = 0; i < kTimeDim / 2; i++) z[(size_t)b * kTimeDim + i] = 1.0f;
        QIMM_HIP(ctx, hipMemcpyAsync(tsin, z.data(), z.size() * 4, hipMemcpyHostToDevice, s));
        QIMM_HIP(ctx, hipStreamSynchronize(s));
    }
    if ((rc = time_embed(m, tsin, batch, tmp, temb, s))) return rc;
    QIMM_HIP(ctx, qimm::launch_linear_f32(temb, hid, m->mod, batch, 4 * hid, hid, qimm::ACT_SILU, modv, 4 * hid, s));
    // every block under the block-causal mask, keeping its k, v (:383-391)
    qimm_attn_mask mask{image_ids, key_valid};
    for (int64_t i = 0; i < m->cfg.layers; i++) {
        rc = qimm_block_forward_masked(m->blocks[(size_t)i], x, x, batch, P, modv, 1, pe, image_ids || key_valid ? &mask : nullptr,
                                       nullptr, 0, kl, vl, stream);
        if (rc) return rc;
        if ((rc = qimm_kv_store_layer(kv, i, kl, vl, stream))) return rc;
    }
    return QIMM_OK;
}

int qimm_joint_layout_pieces(int64_t text_len, const uint8_t *text_image_mask, const int64_t *cond_shapes,
                             int64_t ncond, int64_t *pieces, int64_t cap, int64_t *npieces) {
    if (text_len < 0 || ncond < 0 || !npieces || (ncond > 0 && !cond_shapes) || (cap > 0 && !pieces))
        return QIMM_ERR_ARG;
    constexpr int64_t kTokensPerSlot = 4;  // src/joint_layout.rs:10
    std::vector<int64_t> out;
    auto slot = [&](int64_t j) { return text_image_mask && text_image_mask[j] != 0; };
    int64_t i = 0, next_image = 0, cond_tokens = 0;
    while (i < text_len) {
        if (!slot(i)) {
            int64_t len = 0;
            while (i + len < text_len && !slot(i + len)) len++;
            out.insert(out.end(), {0, i, len});
            i += len;
            continue;
        }
        if (next_image >= ncond) return QIMM_ERR_SHAPE;
        const int64_t h = cond_shapes[2 * next_image], w = cond_shapes[2 * next_image + 1];
        const int64_t needed = h * w / kTokensPerSlot;
        int64_t have = 0;
        for (int64_t j = i; j < text_len && j < i + needed; j++) have += slot(j);
        if ((h * w) % kTokensPerSlot || have != needed) return QIMM_ERR_SHAPE;
        out.insert(out.end(), {1, cond_tokens, h * w});
        cond_tokens += h * w;
        next_image++;
        i += needed;
    }
    if (next_image != ncond) return QIMM_ERR_SHAPE;
    *npieces = (int64_t)out.size() / 3;
    if (cap < *npieces) return QIMM_ERR_ARG;
    if (!out.empty()) memcpy(pieces, out.data(), out.size() * sizeof(int64_t));
    return QIMM_OK;
}

int qimm_flow_match_sigmas(int64_t steps, int64_t image_seq_len, float *sigmas) {
    if (steps <= 0 || image_seq_len < 0 || !sigmas) return QIMM_ERR_ARG;
    // scheduler_config.json constants (src/scheduler.rs:16-20)
    const float base_shift = 0.5f, max_shift = 0.9f, shift_terminal = 0.02f;
    const int64_t base_len = 256, max_len = 8192;
    // calculate_shift (:70-74)
    const float mslope = (max_shift - base_shift) / ((float)max_len - (float)base_len);
    const float b = base_shift - mslope * (float)base_len;
    const float mu = (float)image_seq_len * mslope + b;
    // linspace(1, 1/steps, steps) (:96-101), then time_shift_exponential with exponent 1 (:77-80)
    const float start = 1.0f, end = 1.0f / (float)steps;
    const float e_mu = expf(mu);
    for (int64_t i = 0; i < steps; i++) {
        const float t = steps <= 1 ? start : start + (end - start) * (float)i / (float)(steps - 1);
        sigmas[i] = e_mu / (e_mu + powf(1.0f / t - 1.0f, 1.0f));
    }
    // stretch_shift_to_terminal (:84-91)
    const float scale = (1.0f - sigmas[steps - 1]) / (1.0f - shift_terminal);
    for (int64_t i = 0; i < steps; i++) sigmas[i] = 1.0f - (1.0f - sigmas[i]) / scale;
    return QIMM_OK;
}

int qimm_euler_step(qimm_ctx *ctx, float *latents, const float *pred, int64_t n, float dt, void *stream) {
    if (!ctx || !latents || !pred || n < 0) return QIMM_ERR_ARG;
    QIMM_HIP(ctx, qimm::launch_euler(latents, pred, n, dt, (hipStream_t)stream));
    return QIMM_OK;
}

int qimm_cfg_combine(qimm_ctx *ctx, const float *cond, const float *neg, int64_t n, float scale, float *out,
                     void *stream) {
    if (!ctx || !cond || !neg || !out || n < 0) return QIMM_ERR_ARG;
    QIMM_HIP(ctx, qimm::launch_cfg(cond, neg, n, scale, out, (hipStream_t)stream));
    return QIMM_OK;
}

}  // extern "C"
