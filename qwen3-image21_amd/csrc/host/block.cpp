// The single-stream MMDiT block on the cached step, and the standalone
// attention entry points.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <vector>

#include "internal.h"

using namespace qimm_host;

namespace {

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Norm weights are GGUF tensors too (usually F32); dequantize on the host like
// vb.get(d_head, "norm_q.weight")?.dequantize() (src/quantized_transformer.rs:108-110).
int tensor_to_f32(qimm_ctx *ctx, const qimm_tensor &t, int64_t n, std::vector<float> &out) {
    if (!t.data) return set_err(ctx, QIMM_ERR_ARG, "block: missing norm weight");
    if (t.rows * t.cols != n && !(t.rows == n && t.cols == 1) && !(t.rows == 1 && t.cols == n))
        return set_err(ctx, QIMM_ERR_SHAPE, "block: norm weight must have head_dim values");
    out.resize((size_t)n);
    const uint8_t *p = (const uint8_t *)t.data;
    if (t.ggml_type == QIMM_TYPE_F32 && t.nbytes == (size_t)n * 4) {
        memcpy(out.data(), p, (size_t)n * 4);
    } else if ((t.ggml_type == QIMM_TYPE_F16 || t.ggml_type == QIMM_TYPE_BF16) && t.nbytes == (size_t)n * 2) {
        for (int64_t i = 0; i < n; i++) {
            uint16_t h;
            memcpy(&h, p + 2 * i, 2);
            uint32_t bits;
            if (t.ggml_type == QIMM_TYPE_BF16) {
                bits = (uint32_t)h << 16;
            } else {
                uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
                if (e == 0) {
                    float v = (float)m * 5.9604644775390625e-08f;
                    memcpy(&bits, &v, 4);
                    bits |= sign;
                } else if (e == 31) {
                    bits = sign | 0x7f800000u | (m << 13);
                } else {
                    bits = sign | ((e + 112u) << 23) | (m << 13);
                }
            }
            memcpy(&out[(size_t)i], &bits, 4);
        }
    } else {
        return set_err(ctx, QIMM_ERR_TYPE, "block: norm weights must be F32, F16 or BF16");
    }
    return QIMM_OK;
}

bool tensor_ok(const qimm_tensor &t, int64_t rows, int64_t cols) {
    if (!t.data || t.rows != rows || t.cols != cols) return false;
    const int64_t rb = row_bytes(t.ggml_type, cols);
    return rb > 0 && (size_t)(rb * rows) == t.nbytes;
}

void free_block(qimm_block *b) {
    if (!b) return;
    for (qimm_weight *w : {b->qkv, b->q, b->k, b->v, b->out, b->gate_up, b->down})
        if (w) qimm_weight_free(w);
    if (b->norm_q) (void)hipFree(b->norm_q);
    if (b->norm_k) (void)hipFree(b->norm_k);
    for (hipEvent_t e : b->ev)
        if (e) (void)hipEventDestroy(e);
    delete b;
}

}  // namespace

extern "C" {

int qimm_block_create(qimm_ctx *ctx, const qimm_block_config *cfg, const qimm_block_tensors *t,
                      qimm_block **out) {
    if (!ctx || !cfg || !t || !out) return QIMM_ERR_ARG;
    *out = nullptr;
    const int64_t hid = cfg->hidden, H = cfg->heads, D = cfg->head_dim, F = cfg->mlp;
    if (D != 128 || H <= 0 || H * D != hid || F <= 0 || F % 64 || hid % 256)
        return set_err(ctx, QIMM_ERR_SHAPE, "block: needs head_dim 128, hidden = heads*128 (multiple of 256), mlp % 64 == 0");
    // the LayerNorm kernel holds one row in registers: 256 threads x 8 float4
    if (hid > qimm::LN_MAX_HIDDEN)
        return set_err(ctx, QIMM_ERR_SHAPE, "block: hidden must be at most " + std::to_string(qimm::LN_MAX_HIDDEN));
    if (!tensor_ok(t->to_q, hid, hid) || !tensor_ok(t->to_k, hid, hid) || !tensor_ok(t->to_v, hid, hid) ||
        !tensor_ok(t->to_out, hid, hid) || !tensor_ok(t->mlp_out, hid, F))
        return set_err(ctx, QIMM_ERR_SHAPE, "block: attention / mlp_out tensors missing or mis-shaped");
    const bool fused_gu = t->gate_up.data != nullptr;
    if (fused_gu ? !tensor_ok(t->gate_up, 2 * F, hid)
                 : (!tensor_ok(t->proj, F, hid) || !tensor_ok(t->gate_layer, F, hid)))
        return set_err(ctx, QIMM_ERR_SHAPE, "block: gate_up (or proj + gate_layer) missing or mis-shaped");
    if (!fused_gu && t->proj.ggml_type != t->gate_layer.ggml_type)
        return set_err(ctx, QIMM_ERR_TYPE, "block: proj and gate_layer must share a GGML type");
    if (hipSetDevice(ctx->device) != hipSuccess) return set_err(ctx, QIMM_ERR_HIP, "hipSetDevice failed");

    qimm_block *b = new (std::nothrow) qimm_block();
    if (!b) return QIMM_ERR_OOM;
    b->ctx = ctx;
    b->cfg = *cfg;
    int rc = QIMM_OK;
    try {
        // q | k | v fused along N when the types match (GGML blocks run along K,
        // so stacking rows keeps every block intact).
        const int tq = t->to_q.ggml_type;
        if (t->to_k.ggml_type == tq && t->to_v.ggml_type == tq) {
            const int64_t rb = row_bytes(tq, hid);
            std::vector<uint8_t> cat((size_t)(3 * hid * rb));
            memcpy(cat.data(), t->to_q.data, (size_t)(hid * rb));
            memcpy(cat.data() + hid * rb, t->to_k.data, (size_t)(hid * rb));
            memcpy(cat.data() + 2 * hid * rb, t->to_v.data, (size_t)(hid * rb));
            rc = upload_weight_rows(ctx, tq, 3 * hid, hid, cat.data(), &b->qkv);
            b->qkv_fused = true;
        } else {
            rc = upload_weight_rows(ctx, t->to_q.ggml_type, hid, hid, (const uint8_t *)t->to_q.data, &b->q);
            if (!rc) rc = upload_weight_rows(ctx, t->to_k.ggml_type, hid, hid, (const uint8_t *)t->to_k.data, &b->k);
            if (!rc) rc = upload_weight_rows(ctx, t->to_v.ggml_type, hid, hid, (const uint8_t *)t->to_v.data, &b->v);
        }
        if (!rc)
            rc = upload_weight_rows(ctx, t->to_out.ggml_type, hid, hid, (const uint8_t *)t->to_out.data, &b->out);
        if (!rc) {
            // [gate ; up] -> per 64 output columns: 64 gate rows then 64 up rows,
            // so one 128-wide GEMM tile holds both halves of its SwiGLU outputs.
            const int tg = fused_gu ? t->gate_up.ggml_type : t->gate_layer.ggml_type;
            const int64_t rb = row_bytes(tg, hid);
            const uint8_t *gate = fused_gu ? (const uint8_t *)t->gate_up.data : (const uint8_t *)t->gate_layer.data;
            const uint8_t *up = fused_gu ? gate + F * rb : (const uint8_t *)t->proj.data;
            std::vector<uint8_t> il((size_t)(2 * F * rb));
            for (int64_t tile = 0; tile < F / 64; tile++) {
                memcpy(il.data() + (2 * tile) * 64 * rb, gate + tile * 64 * rb, (size_t)(64 * rb));
                memcpy(il.data() + (2 * tile + 1) * 64 * rb, up + tile * 64 * rb, (size_t)(64 * rb));
            }
            rc = upload_weight_rows(ctx, tg, 2 * F, hid, il.data(), &b->gate_up);
        }
        if (!rc)
            rc = upload_weight_rows(ctx, t->mlp_out.ggml_type, hid, F, (const uint8_t *)t->mlp_out.data, &b->down);
        std::vector<float> nq, nk;
        if (!rc) rc = tensor_to_f32(ctx, t->norm_q, D, nq);
        if (!rc) rc = tensor_to_f32(ctx, t->norm_k, D, nk);
        if (!rc) {
            // ||RmsNorm(x) w|| <= sqrt(128) max|w|; q also carries 128^-1/2 log2 e
            // (its epilogue scale); 2% covers RoPE's f32 rotation and bf16 rounding
            float wq = 0.f, wk = 0.f;
            for (float v : nq) wq = fmaxf(wq, fabsf(v));
            for (float v : nk) wk = fmaxf(wk, fabsf(v));
            b->q_norm_bound = wq * 1.4426950408889634f * 1.02f;
            b->k_norm_bound = wk * sqrtf(128.0f) * 1.02f;
            if (!(b->q_norm_bound < INFINITY) || !(b->k_norm_bound < INFINITY)) b->q_norm_bound = 0.f;
        }
        if (!rc) {
            hipError_t e = hipMalloc((void **)&b->norm_q, (size_t)D * 4);
            if (e == hipSuccess) e = hipMalloc((void **)&b->norm_k, (size_t)D * 4);
            if (e == hipSuccess) e = hipMemcpy(b->norm_q, nq.data(), (size_t)D * 4, hipMemcpyHostToDevice);
            if (e == hipSuccess) e = hipMemcpy(b->norm_k, nk.data(), (size_t)D * 4, hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = hip_err(ctx, e, "block norm weights");
        }
    } catch (const std::bad_alloc &) {
        rc = set_err(ctx, QIMM_ERR_OOM, "block: host staging allocation failed");
    }
    if (rc) {
        free_block(b);
        return rc;
    }
    *out = b;
    return QIMM_OK;
}

int qimm_block_destroy(qimm_block *blk) {
    if (!blk) return QIMM_ERR_ARG;
    free_block(blk);
    return QIMM_OK;
}

}  // extern "C"

namespace {

// Workspace of one forward: modp [B*mod_rows,4h] f32 | xn [M,h] | q | k | vt |
// attn [M,h] | hmid [M,F] (bf16) | lim | f32 staging of the attention output
// [M,h] and then of the SwiGLU hidden state [M,F] ahead of their activation
// rounding (candle mode only), and the split-K scratch of the short- and mid-M
// GEMM paths, sized for the largest projection.
struct WsLayout {
    size_t modp, xn, q, k, vt, att, h, lim, f32, total, part;
};

// The activation block of candle's vec-dot type for weight w under the
// block's mode (0: bf16 operands, no int8 rounding).
int act_qblk(const qimm_block *blk, const qimm_weight *w) {
    return blk->act == QIMM_ACT_CANDLE ? qimm::act_block(w->gw.fmt) : 0;
}

// QIMM_SEPARATE_ROUNDING=1 in the environment (read at every forward) rounds
// the hidden state and the attention output in their own passes even where
// their producers would round them in their epilogues (the gate_up kernels
// for Q8_K blocks at large M and for Q8_0 blocks at large M or in the
// undivided 128x128 kernel, the attention kernels for Q8_0 and, paired over
// two heads, for Q8_K): the reference form the fused ones are checked against
// bit for bit.
bool separate_rounding() {
    const char *e = getenv("QIMM_SEPARATE_ROUNDING");
    return e && e[0] == '1';
}

WsLayout ws_layout(const qimm_block *blk, int64_t batch, int64_t seq, int64_t mod_rows) {
    const int64_t hid = blk->cfg.hidden, F = blk->cfg.mlp, M = batch * seq;
    WsLayout L{};
    size_t off = 0;
    L.modp = off; off += align_up((size_t)(batch * mod_rows * 4 * hid) * 4);
    L.xn = off; off += align_up((size_t)(M * hid) * 2);
    L.q = off; off += align_up((size_t)(M * hid) * 2);
    L.k = off; off += align_up((size_t)(M * hid) * 2);
    L.vt = off; off += align_up((size_t)(M * hid) * 2);
    L.att = off; off += align_up((size_t)(M * hid) * 2);
    L.h = off; off += align_up((size_t)(M * F) * 2);
    L.lim = off; off += align_up((size_t)seq * 4);  // per-query key limits of the block-causal mask
    L.f32 = off;
    if (act_qblk(blk, blk->out) || act_qblk(blk, blk->down))
        off += align_up((size_t)(M * std::max(hid, F)) * 4);
    L.total = off;
    L.part = 0;
    const qimm_weight *ws_list[] = {blk->qkv, blk->q, blk->k, blk->v, blk->out, blk->gate_up, blk->down};
    for (const qimm_weight *wt : ws_list)
        if (wt) L.part = std::max(L.part, qimm::qgemm_workspace(wt->gw, M));
    return L;
}

// TransformerBlock::forward (src/quantized_transformer.rs:258-285) with
// modulation rows [B, mod_rows, 4 hidden] (mod_rows 1 broadcasts over the
// tokens, mod_rows == seq gives one row per token) and an optional attention
// mask; kv supplies the prefix K/V of the cached step.
int block_forward_impl(qimm_block *blk, const float *x, float *x_out, int64_t batch, int64_t seq, const float *mod,
                       int64_t mod_rows, const float *pe, const qimm_attn_mask *mask, const qimm_kv *kv,
                       int64_t layer, uint16_t *k_out, uint16_t *v_out, void *stream) {
    if (!blk || !x || !x_out || !mod || !pe) return QIMM_ERR_ARG;
    qimm_ctx *ctx = blk->ctx;
    const int64_t hid = blk->cfg.hidden, H = blk->cfg.heads, F = blk->cfg.mlp;
    if (batch <= 0 || seq <= 0) return set_err(ctx, QIMM_ERR_SHAPE, "block forward: batch and seq must be positive");
    if (mod_rows != 1 && mod_rows != seq)
        return set_err(ctx, QIMM_ERR_SHAPE, "block forward: modulation needs 1 or seq rows per batch entry");
    const int32_t *img = mask ? mask->image_ids : nullptr;
    const uint8_t *kvalid = mask ? mask->key_valid : nullptr;
    if (img && kv) return set_err(ctx, QIMM_ERR_SHAPE, "block forward: the block-causal mask has no prefix cache");
    if (!aligned16(x) || !aligned16(x_out) || !aligned16(mod) || !aligned16(pe) ||
        (k_out && !aligned16(k_out)) || (v_out && !aligned16(v_out)))
        return set_err(ctx, QIMM_ERR_ARG, "block forward: device pointers must be 16-byte aligned");
    int64_t P = 0;
    if (kv) {
        if (kv->batch != batch || kv->heads != H)
            return set_err(ctx, QIMM_ERR_SHAPE, "block forward: cache batch/heads differ from the block call");
        if (layer < 0 || layer >= kv->layers) return set_err(ctx, QIMM_ERR_SHAPE, "block forward: cache layer out of range");
        P = kv->prefix;
    }
    const int64_t M = batch * seq;
    hipStream_t s = (hipStream_t)stream;

    // the workspace grows (a device-wide sync, free and allocation) only when
    // this call needs more than any earlier call or qimm_block_reserve
    const WsLayout L = ws_layout(blk, batch, seq, mod_rows);
    QIMM_HIP(ctx, hipSetDevice(ctx->device));
    int rc = ensure_workspace(ctx, L.total);
    if (rc) return rc;
    char *ws = (char *)ctx->ws;
    float *modp = (float *)(ws + L.modp);
    uint16_t *xn = (uint16_t *)(ws + L.xn), *qb = (uint16_t *)(ws + L.q);
    uint16_t *kb = k_out ? k_out : (uint16_t *)(ws + L.k);
    uint16_t *vt = (uint16_t *)(ws + L.vt), *att = (uint16_t *)(ws + L.att), *hm = (uint16_t *)(ws + L.h);
    const size_t part_need = L.part;
    if (part_need) {
        rc = ensure_part_workspace(ctx, part_need);
        if (rc) return rc;
    }
    float *part_ws = part_need ? (float *)ctx->ws_part : nullptr;
    const size_t part_bytes = part_need ? ctx->ws_part_bytes : 0;

#define STAGE_MARK(i) \
    if (blk->profiling) QIMM_HIP(ctx, hipEventRecord(blk->ev[i], s))
    STAGE_MARK(0);
    const int64_t rows_per = seq / mod_rows;  // tokens sharing one modulation row
    // norm1(x) * (1 + scale1)                                  (:267-269)
    // In candle mode the output is already the q/k/v matmuls' quantized input
    // (Linear::forward -> QMatMul::forward rounds its f32 input rows, :19-29).
    // The same launch prepares modulation.chunk(4) -> (1 + scale1, tanh gate1,
    // 1 + scale2, tanh gate2) into modp for the later stages.
    const qimm_weight *qkv0 = blk->qkv_fused ? blk->qkv : blk->q;
    int qb_norm1 = act_qblk(blk, qkv0);
    QIMM_HIP(ctx, qimm::launch_ln_mod(x, M, hid, mod, 4 * hid, rows_per, xn, s, qb_norm1, modp, batch * mod_rows));
    STAGE_MARK(1);
    // to_q/to_k/to_v + per-head RmsNorm + RoPE                 (:133-142)
    qimm::EpiParams ep{};
    ep.part_ws = part_ws;
    ep.part_ws_bytes = part_bytes;
    ep.q = qb;
    ep.k = kb;
    ep.vt = vt;
    ep.v_bhsd = v_out;
    ep.norm_q = blk->norm_q;
    ep.norm_k = blk->norm_k;
    ep.pe = pe;
    ep.seq = seq;
    ep.heads = H;
    ep.hidden = hid;
    // q leaves the epilogue multiplied by the softmax scale and log2(e): the
    // attention then works on scores in log2 units (transformer.rs:275 scales
    // q by D^-1/2 before the product as well)
    ep.q_scale = (1.0f / sqrtf(128.0f)) * 1.4426950408889634f;
    if (blk->qkv_fused) {
        ep.n_offset = 0;
        QIMM_HIP(ctx, qimm::launch_qgemm(blk->qkv->gw, xn, M, hid, qimm::EPI_QKV, ep, s));
    } else {
        const qimm_weight *parts[3] = {blk->q, blk->k, blk->v};
        for (int i = 0; i < 3; i++) {
            ep.n_offset = i * hid;
            // q, k, v of different vec-dot types round the same norm1 output
            // to their own blocks: norm1 again, in place of xn (stream order)
            if (const int qb = act_qblk(blk, parts[i]); qb != qb_norm1) {
                QIMM_HIP(ctx, qimm::launch_ln_mod(x, M, hid, modp, 4 * hid, rows_per, xn, s, qb));
                qb_norm1 = qb;
            }
            QIMM_HIP(ctx, qimm::launch_qgemm(parts[i]->gw, xn, M, hid, qimm::EPI_QKV, ep, s));
        }
    }
    STAGE_MARK(2);
    // attention over [prefix ; own]                            (:143-148)
    const uint16_t *pk = nullptr, *pvt = nullptr;
    if (kv) {
        const int rc = kv_layer(kv, layer, s, &pk, &pvt);
        if (rc) return rc;
    }
    // candle mode: to_out's activation rounding, done by the attention launch
    // (in its kernels' epilogue where they can; the f32 staging is its scratch)
    const int qb_out = act_qblk(blk, blk->out);
    float *stage_f32 = (float *)(ws + L.f32);
    const bool round_sep = separate_rounding();
    const int att_q = round_sep ? 0 : qb_out;
    float *att_f32 = qb_out ? stage_f32 : nullptr;
    // score bound: q and own k from the RmsNorm weights, prefix k from the cache
    const float *kpn = kv ? kv->knorm + layer : nullptr;
    if (img || kvalid)
        QIMM_HIP(ctx, qimm::launch_attention_masked(qb, pk, pvt, P, kb, vt, seq, batch, H, seq, 1.0f, img, kvalid,
                                                    (int32_t *)(ws + L.lim), att, s, att_f32, kpn,
                                                    blk->q_norm_bound, blk->k_norm_bound, att_q));
    else
        QIMM_HIP(ctx, qimm::launch_attention_log2(qb, pk, pvt, P, kb, vt, seq, batch, H, seq, att, s, att_f32, kpn,
                                                  blk->q_norm_bound, blk->k_norm_bound, att_q));
    if (kv) {
        const int rc = kv_release(kv, layer, s);
        if (rc) return rc;
    }
    STAGE_MARK(3);
    if (round_sep && qb_out) QIMM_HIP(ctx, qimm::launch_quant_rows(att_f32, hid, M, hid, qb_out, att, hid, s));
    STAGE_MARK(4);
    // x1 = x + tanh(gate1) * to_out(attn)                       (:150-151, 271-273)
    qimm::EpiParams er{};
    er.part_ws = part_ws;
    er.part_ws_bytes = part_bytes;
    er.x_in = x;
    er.x_out = x_out;
    er.gvec = modp + hid;
    er.g_stride = 4 * hid;
    er.g_rows_per = rows_per;
    QIMM_HIP(ctx, qimm::launch_qgemm(blk->out->gw, att, M, hid, qimm::EPI_RESID, er, s));
    STAGE_MARK(5);
    // norm2(x1) * (1 + scale2)                                 (:276-278)
    QIMM_HIP(ctx, qimm::launch_ln_mod(x_out, M, hid, modp + 2 * hid, 4 * hid, rows_per, xn, s,
                                      act_qblk(blk, blk->gate_up)));
    STAGE_MARK(6);
    // silu(gate) * up                                          (:191-201)
    qimm::EpiParams eg{};
    eg.part_ws = part_ws;
    eg.part_ws_bytes = part_bytes;
    eg.hmid = hm;
    eg.ldh = F;
    // candle mode: the hidden state leaves in f32 for the down matmul's rounding
    const int qb_down = act_qblk(blk, blk->down);
    if (qb_down) eg.hmid_f32 = stage_f32;
    // the gate_up launch rounds them itself: Q8_K blocks (K-quant down
    // weights), Q8_0 blocks (Q8_0 down weights)
    const bool round_in_gemm = (qb_down == 32 || (qb_down == 256 && F % 256 == 0)) && !separate_rounding();
    eg.hmid_q8k = round_in_gemm && qb_down == 256;
    eg.hmid_q8_0 = round_in_gemm && qb_down == 32;
    QIMM_HIP(ctx, qimm::launch_qgemm(blk->gate_up->gw, xn, M, hid, qimm::EPI_SWIGLU, eg, s));
    STAGE_MARK(7);
    if (qb_down && !round_in_gemm) QIMM_HIP(ctx, qimm::launch_quant_rows(stage_f32, F, M, F, qb_down, hm, F, s));
    STAGE_MARK(8);
    // x2 = x1 + tanh(gate2) * out(hidden)                       (:202, 280-282)
    qimm::EpiParams ed{};
    ed.part_ws = part_ws;
    ed.part_ws_bytes = part_bytes;
    ed.x_in = x_out;
    ed.x_out = x_out;
    ed.gvec = modp + 3 * hid;
    ed.g_stride = 4 * hid;
    ed.g_rows_per = rows_per;
    QIMM_HIP(ctx, qimm::launch_qgemm(blk->down->gw, hm, M, F, qimm::EPI_RESID, ed, s));
    STAGE_MARK(9);
#undef STAGE_MARK
    if (blk->profiling) blk->profiled_once = true;
    return QIMM_OK;
}

}  // namespace

extern "C" {

int qimm_block_reserve(qimm_block *blk, int64_t batch, int64_t seq, int64_t mod_rows) {
    if (!blk) return QIMM_ERR_ARG;
    qimm_ctx *ctx = blk->ctx;
    if (batch <= 0 || seq <= 0 || (mod_rows != 1 && mod_rows != seq))
        return set_err(ctx, QIMM_ERR_SHAPE, "block reserve: batch, seq > 0 and mod_rows 1 or seq");
    const WsLayout L = ws_layout(blk, batch, seq, mod_rows);
    QIMM_HIP(ctx, hipSetDevice(ctx->device));
    int rc = ensure_workspace(ctx, L.total);
    if (rc) return rc;
    return L.part ? ensure_part_workspace(ctx, L.part) : QIMM_OK;
}

int qimm_block_set_act_mode(qimm_block *blk, int mode) {
    if (!blk) return QIMM_ERR_ARG;
    if (mode != QIMM_ACT_CANDLE && mode != QIMM_ACT_BF16)
        return set_err(blk->ctx, QIMM_ERR_ARG, "block act mode: QIMM_ACT_CANDLE or QIMM_ACT_BF16");
    blk->act = mode;
    return QIMM_OK;
}

int qimm_block_act_mode(const qimm_block *blk) { return blk ? blk->act : -1; }

int qimm_block_forward(qimm_block *blk, const float *x, float *x_out, int64_t batch, int64_t seq,
                       const float *mod, const float *pe, const qimm_kv *kv, int64_t layer, uint16_t *k_out,
                       uint16_t *v_out, void *stream) {
    return block_forward_impl(blk, x, x_out, batch, seq, mod, 1, pe, nullptr, kv, layer, k_out, v_out, stream);
}

int qimm_block_forward_masked(qimm_block *blk, const float *x, float *x_out, int64_t batch, int64_t seq,
                              const float *mod, int64_t mod_rows, const float *pe, const qimm_attn_mask *mask,
                              const qimm_kv *kv, int64_t layer, uint16_t *k_out, uint16_t *v_out, void *stream) {
    return block_forward_impl(blk, x, x_out, batch, seq, mod, mod_rows, pe, mask, kv, layer, k_out, v_out, stream);
}

int qimm_block_profile(qimm_block *blk, int enable) {
    if (!blk) return QIMM_ERR_ARG;
    qimm_ctx *ctx = blk->ctx;
    if (enable && !blk->ev[0]) {
        QIMM_HIP(ctx, hipSetDevice(ctx->device));
        for (int i = 0; i <= QIMM_BLOCK_STAGES; i++) QIMM_HIP(ctx, hipEventCreate(&blk->ev[i]));
    }
    blk->profiling = enable != 0;
    blk->profiled_once = false;
    return QIMM_OK;
}

int qimm_block_stage_times(qimm_block *blk, float *ms_out, int n) {
    if (!blk || !ms_out || n < QIMM_BLOCK_STAGES) return QIMM_ERR_ARG;
    qimm_ctx *ctx = blk->ctx;
    if (!blk->profiled_once) return set_err(ctx, QIMM_ERR_STATE, "stage times: no profiled forward since enabling");
    QIMM_HIP(ctx, hipEventSynchronize(blk->ev[QIMM_BLOCK_STAGES]));
    for (int i = 0; i < QIMM_BLOCK_STAGES; i++)
        QIMM_HIP(ctx, hipEventElapsedTime(&ms_out[i], blk->ev[i], blk->ev[i + 1]));
    return QIMM_OK;
}

int qimm_qk_norm_rope(qimm_ctx *ctx, const float *x, int64_t batch, int64_t seq, int64_t heads,
                      const float *norm_w, const float *pe, uint16_t *out, void *stream) {
    if (!ctx || !x || !norm_w || !pe || !out) return QIMM_ERR_ARG;
    if (batch < 0 || seq < 0 || heads < 0) return set_err(ctx, QIMM_ERR_SHAPE, "qk_norm_rope: negative size");
    if (!aligned16(out)) return set_err(ctx, QIMM_ERR_ARG, "qk_norm_rope: out must be 16-byte aligned");
    QIMM_HIP(ctx, qimm::launch_qk_prep(x, batch, seq, heads, norm_w, pe, 0, out, (hipStream_t)stream));
    return QIMM_OK;
}

int qimm_v_transpose(qimm_ctx *ctx, const float *x, int64_t batch, int64_t seq, int64_t heads, uint16_t *vt_out,
                     void *stream) {
    if (!ctx || !x || !vt_out) return QIMM_ERR_ARG;
    if (batch < 0 || seq < 0 || heads < 0) return set_err(ctx, QIMM_ERR_SHAPE, "v_transpose: negative size");
    QIMM_HIP(ctx, qimm::launch_qk_prep(x, batch, seq, heads, nullptr, nullptr, 1, vt_out, (hipStream_t)stream));
    return QIMM_OK;
}

int qimm_quantize_act(qimm_ctx *ctx, int weight_type, const float *x, int64_t m, int64_t k, int64_t ldx,
                      uint16_t *out, int64_t ldo, void *stream) {
    if (!ctx || !x || !out) return QIMM_ERR_ARG;
    const int qblk = weight_type == QIMM_TYPE_Q8_0 ? 32
                     : (weight_type == QIMM_TYPE_Q4_K || weight_type == QIMM_TYPE_Q6_K) ? 256 : 0;
    if (!qblk) return set_err(ctx, QIMM_ERR_TYPE, "quantize_act: weight type must be Q8_0, Q4_K or Q6_K");
    if (m < 0 || k <= 0 || k % qblk || ldx < k || ldo < k || ldx % 4 || ldo % 4)
        return set_err(ctx, QIMM_ERR_SHAPE, "quantize_act: k must be a positive multiple of the block (32 or 256), "
                                            "ldx, ldo >= k and multiples of 4");
    if (((uintptr_t)x | (uintptr_t)out) & 15)
        return set_err(ctx, QIMM_ERR_ARG, "quantize_act: x and out must be 16-byte aligned");
    if (m == 0) return QIMM_OK;
    QIMM_HIP(ctx, hipSetDevice(ctx->device));
    QIMM_HIP(ctx, qimm::launch_quant_rows(x, ldx, m, k, qblk, out, ldo, (hipStream_t)stream));
    return QIMM_OK;
}

int qimm_attention(qimm_ctx *ctx, const uint16_t *q, int64_t batch, int64_t heads, int64_t sq, const qimm_kv *kv,
                   int64_t layer, const uint16_t *k_own, const uint16_t *vt_own, int64_t so, float scale,
                   uint16_t *out, void *stream) {
    if (!ctx || !q || !out || (so > 0 && (!k_own || !vt_own))) return QIMM_ERR_ARG;
    if (batch <= 0 || heads <= 0 || sq < 0 || so < 0) return set_err(ctx, QIMM_ERR_SHAPE, "attention: bad sizes");
    if (!aligned16(q) || !aligned16(out) || (k_own && !aligned16(k_own)) || (vt_own && !aligned16(vt_own)))
        return set_err(ctx, QIMM_ERR_ARG, "attention: q, k, vt and out must be 16-byte aligned");
    int64_t P = 0;
    if (kv) {
        if (kv->batch != batch || kv->heads != heads)
            return set_err(ctx, QIMM_ERR_SHAPE, "attention: cache batch/heads differ");
        if (layer < 0 || layer >= kv->layers) return set_err(ctx, QIMM_ERR_SHAPE, "attention: cache layer out of range");
        P = kv->prefix;
    }
    if (P + so == 0) return set_err(ctx, QIMM_ERR_SHAPE, "attention: no keys");
    const hipStream_t s = (hipStream_t)stream;
    const uint16_t *pk = nullptr, *pvt = nullptr;
    if (kv) {
        const int rc = kv_layer(kv, layer, s, &pk, &pvt);
        if (rc) return rc;
    }
    QIMM_HIP(ctx, qimm::launch_attention(q, pk, pvt, P, k_own, vt_own, so, batch, heads, sq, scale, out, s));
    return kv ? kv_release(kv, layer, s) : QIMM_OK;
}

int qimm_attention_masked(qimm_ctx *ctx, const uint16_t *q, int64_t batch, int64_t heads, int64_t sq,
                          const qimm_kv *kv, int64_t layer, const uint16_t *k_own, const uint16_t *vt_own,
                          int64_t so, float scale, const qimm_attn_mask *mask, uint16_t *out, void *stream) {
    if (!mask || (!mask->image_ids && !mask->key_valid))
        return qimm_attention(ctx, q, batch, heads, sq, kv, layer, k_own, vt_own, so, scale, out, stream);
    if (!ctx || !q || !out || (so > 0 && (!k_own || !vt_own))) return QIMM_ERR_ARG;
    if (batch <= 0 || heads <= 0 || sq < 0 || so < 0) return set_err(ctx, QIMM_ERR_SHAPE, "attention: bad sizes");
    if (!aligned16(q) || !aligned16(out) || (k_own && !aligned16(k_own)) || (vt_own && !aligned16(vt_own)))
        return set_err(ctx, QIMM_ERR_ARG, "attention: q, k, vt and out must be 16-byte aligned");
    int64_t P = 0;
    if (kv) {
        if (kv->batch != batch || kv->heads != heads)
            return set_err(ctx, QIMM_ERR_SHAPE, "attention: cache batch/heads differ");
        if (layer < 0 || layer >= kv->layers) return set_err(ctx, QIMM_ERR_SHAPE, "attention: cache layer out of range");
        P = kv->prefix;
    }
    if (P + so == 0) return set_err(ctx, QIMM_ERR_SHAPE, "attention: no keys");
    if (mask->image_ids && (P != 0 || so != sq))
        return set_err(ctx, QIMM_ERR_SHAPE, "attention: the block-causal mask needs no prefix and so == sq");
    const hipStream_t s = (hipStream_t)stream;
    int32_t *lim = nullptr;
    if (mask->image_ids) {
        QIMM_HIP(ctx, hipSetDevice(ctx->device));
        const int rc = ensure_workspace(ctx, (size_t)sq * 4);
        if (rc) return rc;
        lim = (int32_t *)ctx->ws;
    }
    const uint16_t *pk = nullptr, *pvt = nullptr;
    if (kv) {
        const int rc = kv_layer(kv, layer, s, &pk, &pvt);
        if (rc) return rc;
    }
    QIMM_HIP(ctx, qimm::launch_attention_masked(q, pk, pvt, P, k_own, vt_own, so, batch, heads, sq,
                                                scale * 1.4426950408889634f, mask->image_ids, mask->key_valid, lim,
                                                out, s));
    return kv ? kv_release(kv, layer, s) : QIMM_OK;
}

}  // extern "C"
