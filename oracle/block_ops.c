/*
 * CPU oracle, part 2: row norms, 3-axis RoPE, joint layout, block-causal mask,
 * chunked attention and the single-stream MMDiT block.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* norms                                                               */
/* ------------------------------------------------------------------ */

/* LayerNorm with weight 1 and bias 0, eps 1e-6, then the adaLN scale:
 * src/quantized_transformer.rs:231-237 (layer_norm_no_bias), 267-269 and
 * 276-278 (normed * (scale + 1)). Mean and variance in f64. */
void oq_layernorm_mod(const float *x, int64_t rows, int64_t cols,
                      const float *scale, int64_t scale_row_stride,
                      int64_t rows_per_scale_row, float eps, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * cols;
        double mean = 0.0;
        for (int64_t c = 0; c < cols; c++) mean += xr[c];
        mean /= (double)cols;
        double var = 0.0;
        for (int64_t c = 0; c < cols; c++) {
            double t = xr[c] - mean;
            var += t * t;
        }
        var /= (double)cols;
        float rstd = (float)(1.0 / sqrt(var + (double)eps));
        const float *sc = scale ? scale + (r / rows_per_scale_row) * scale_row_stride : NULL;
        for (int64_t c = 0; c < cols; c++) {
            float nrm = (float)((xr[c] - mean)) * rstd;
            float s1 = sc ? sc[c] + 1.0f : 1.0f;
            out[r * cols + c] = nrm * s1;
        }
    }
}

/* RmsNorm over the last dim: src/quantized_transformer.rs:108-111,137-138
 * (candle_nn::RmsNorm, eps 1e-6): x / sqrt(mean(x^2) + eps) * w. */
void oq_rmsnorm(float *x, int64_t rows, int64_t d, const float *w, float eps) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        float *xr = x + r * d;
        double ss = 0.0;
        for (int64_t c = 0; c < d; c++) ss += (double)xr[c] * xr[c];
        float rs = (float)(1.0 / sqrt(ss / (double)d + (double)eps));
        for (int64_t c = 0; c < d; c++) xr[c] = xr[c] * rs * w[c];
    }
}

/* ------------------------------------------------------------------ */
/* RoPE                                                                */
/* ------------------------------------------------------------------ */

#define ROPE_NEG 1024
#define ROPE_POS 8192

/* EmbedNd::new_with_mode (src/rope.rs:37-88) builds per-axis tables over
 * positions -1024..8191 with inv_freq_i = exp(i * (-2 ln(theta)/dim)) in f32
 * and angle = position * inv_freq; EmbedNd::forward (src/rope.rs:104-211)
 * assigns (frame, height, width) positions per token and gathers the tables
 * at position + 1024. Output row: (cos, sin) interleaved over
 * [frame pairs | height pairs | width pairs]. */
int oq_rope_table(const int64_t *shapes, int nshapes, const uint8_t *image_mask,
                  int64_t seq, const int64_t *axes, double theta, float *pe) {
    int64_t *pos[3];
    for (int a = 0; a < 3; a++) {
        pos[a] = (int64_t *)malloc(sizeof(int64_t) * (size_t)(seq > 0 ? seq : 1));
        if (!pos[a]) return -2;
    }
    int64_t n[3] = {0, 0, 0};
    int64_t cursor = 0, position = 0;
    for (int bi = 0; bi < nshapes; bi++) {
        int64_t frame = shapes[3 * bi], height = shapes[3 * bi + 1], width = shapes[3 * bi + 2];
        int64_t block_tokens = frame * height * width;
        int64_t block_start = seq;
        for (int64_t i = cursor; i < seq; i++)
            if (image_mask[i]) { block_start = i; break; }
        for (int64_t t = cursor; t < block_start; t++) {
            if (n[0] >= seq) goto overflow;
            pos[0][n[0]++] = position; pos[1][n[1]++] = position; pos[2][n[2]++] = position;
            position++;
        }
        cursor = block_start;
        for (int64_t t = 0; t < block_tokens; t++) {
            if (n[0] >= seq) goto overflow;
            pos[0][n[0]++] = position;
        }
        position += height > width ? height : width;
        int64_t h0 = -(height - height / 2), w0 = -(width - width / 2);
        for (int64_t hh = 0; hh < height; hh++)
            for (int64_t ww = 0; ww < width; ww++) {
                if (n[1] >= seq) goto overflow;
                pos[1][n[1]++] = h0 + hh;
                pos[2][n[2]++] = w0 + ww;
            }
        cursor += block_tokens;
    }
    for (int64_t t = cursor; t < seq; t++) {
        if (n[0] >= seq) goto overflow;
        pos[0][n[0]++] = position; pos[1][n[1]++] = position; pos[2][n[2]++] = position;
        position++;
    }
    if (n[0] != seq || n[1] != seq || n[2] != seq) goto overflow;
    {
        int64_t dim_total = axes[0] + axes[1] + axes[2];
        double ln_theta = log((double)(float)theta);
        for (int64_t t = 0; t < seq; t++) {
            int64_t col = 0;
            for (int a = 0; a < 3; a++) {
                int64_t p = pos[a][t];
                if (p < -ROPE_NEG || p >= ROPE_POS) goto overflow;
                int64_t half = axes[a] / 2;
                float mul = (float)(-2.0 * ln_theta / (double)axes[a]);
                for (int64_t i = 0; i < half; i++) {
                    float inv_freq = expf((float)i * mul);
                    float ang = (float)p * inv_freq;
                    pe[t * dim_total + 2 * col] = cosf(ang);
                    pe[t * dim_total + 2 * col + 1] = sinf(ang);
                    col++;
                }
            }
        }
    }
    for (int a = 0; a < 3; a++) free(pos[a]);
    return 0;
overflow:
    for (int a = 0; a < 3; a++) free(pos[a]);
    return -1;
}

/* rope_i on interleaved pairs (src/rope.rs:222-228):
 * (x0, x1) -> (x0 cos - x1 sin, x0 sin + x1 cos). */
void oq_apply_rope(float *x, int64_t bh, int64_t s, int64_t d, const float *pe) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < bh; b++)
        for (int64_t t = 0; t < s; t++) {
            float *xr = x + (b * s + t) * d;
            const float *pr = pe + t * d;
            for (int64_t i = 0; i < d / 2; i++) {
                float c = pr[2 * i], sn = pr[2 * i + 1];
                float x0 = xr[2 * i], x1 = xr[2 * i + 1];
                xr[2 * i] = x0 * c - x1 * sn;
                xr[2 * i + 1] = x0 * sn + x1 * c;
            }
        }
}

/* ------------------------------------------------------------------ */
/* joint layout + mask                                                 */
/* ------------------------------------------------------------------ */

#define TOKENS_PER_SLOT 4

/* JointLayout::new (src/joint_layout.rs:52-103): text runs stay in place,
 * each condition image replaces h*w/4 consecutive image slots, the target is
 * appended; image_ids = -1 for text, else the image block index. Returns 0,
 * or -1 for the reference's bail! cases, -2 if cap is too small. */
int oq_joint_layout(int64_t text_len, const uint8_t *text_image_mask,
                    const int64_t *cond_shapes, int ncond, int64_t th, int64_t tw,
                    int64_t *image_ids, int64_t cap, int64_t *prefix_len,
                    int64_t *target_len, int64_t *total_len) {
    int64_t len = 0;
    int64_t i = 0;
    int next_image = 0;
#define PUSH(v) do { if (len >= cap) return -2; image_ids[len++] = (v); } while (0)
    while (i < text_len) {
        int slot = text_image_mask ? text_image_mask[i] != 0 : 0;
        if (!slot) {
            while (i < text_len && !(text_image_mask && text_image_mask[i])) { PUSH(-1); i++; }
            continue;
        }
        if (next_image >= ncond) return -1;
        int64_t h = cond_shapes[2 * next_image], w = cond_shapes[2 * next_image + 1];
        int64_t needed = h * w / TOKENS_PER_SLOT;
        if ((h * w) % TOKENS_PER_SLOT) return -1;
        int64_t have = 0;
        for (int64_t j = i; j < text_len && j < i + needed; j++) have += text_image_mask[j] != 0;
        if (have != needed) return -1;
        for (int64_t t = 0; t < h * w; t++) PUSH(next_image);
        next_image++;
        i += needed;
    }
    if (next_image != ncond) return -1;
    for (int64_t t = 0; t < th * tw; t++) PUSH(ncond);
#undef PUSH
    *target_len = th * tw;
    *prefix_len = len - th * tw;
    *total_len = len;
    return 0;
}

/* build_block_causal_mask (src/attention_mask.rs:18-66):
 * allowed(q, k) = (q >= k) || (id[q] == id[k] && id[q] >= 0). */
void oq_block_causal_mask(const int64_t *image_ids, int64_t s, uint8_t *mask) {
#pragma omp parallel for schedule(static)
    for (int64_t q = 0; q < s; q++)
        for (int64_t k = 0; k < s; k++)
            mask[q * s + k] = (uint8_t)((q >= k) || (image_ids[q] == image_ids[k] && image_ids[q] >= 0));
}

/* ------------------------------------------------------------------ */
/* attention                                                           */
/* ------------------------------------------------------------------ */

/* chunked_attention (src/transformer.rs:259-296): q is scaled first (275),
 * scores q.k, additive -inf mask, f32 softmax over keys (292), then p.v.
 * Keys are [prefix ; own] as in Attention::forward (src/quantized_transformer.rs:143-146).
 * Candle mode computes in f32; exact mode in f64. A row with every key masked
 * yields NaN, as softmax over all -inf does in the reference. */
int oq_attention(const float *q, const float *kp, const float *vp, int64_t p,
                 const float *ko, const float *vo, int64_t so,
                 int64_t b, int64_t h, int64_t sq, int64_t d, double scale,
                 const uint8_t *mask, int64_t mask_batch_stride, float *out,
                 int mode) {
    int64_t skv = p + so;
    int fail = 0;
#pragma omp parallel
    {
        double *sc = (double *)malloc(sizeof(double) * (size_t)(skv > 0 ? skv : 1));
        float *scf = (float *)malloc(sizeof(float) * (size_t)(skv > 0 ? skv : 1));
        double *acc = (double *)malloc(sizeof(double) * (size_t)d);
        float *qs = (float *)malloc(sizeof(float) * (size_t)d);
        if (!sc || !scf || !acc || !qs) fail = 1;
#pragma omp for collapse(3) schedule(static)
        for (int64_t bb = 0; bb < b; bb++)
            for (int64_t hh = 0; hh < h; hh++)
                for (int64_t i = 0; i < sq; i++) {
                    if (fail) continue;
                    const float *qr = q + ((bb * h + hh) * sq + i) * d;
                    const uint8_t *mr = mask ? mask + bb * mask_batch_stride + i * skv : NULL;
                    float *orow = out + ((bb * h + hh) * sq + i) * d;
                    if (mode == OQ_MODE_EXACT) {
                        double mx = -INFINITY;
                        for (int64_t j = 0; j < skv; j++) {
                            const float *kr = j < p ? kp + ((bb * h + hh) * p + j) * d
                                                    : ko + ((bb * h + hh) * so + (j - p)) * d;
                            double s = 0.0;
                            for (int64_t c = 0; c < d; c++) s += (double)qr[c] * kr[c];
                            s *= scale;
                            if (mr && !mr[j]) s = -INFINITY;
                            sc[j] = s;
                            if (s > mx) mx = s;
                        }
                        double sum = 0.0;
                        for (int64_t j = 0; j < skv; j++) {
                            sc[j] = exp(sc[j] - mx);
                            sum += sc[j];
                        }
                        for (int64_t c = 0; c < d; c++) acc[c] = 0.0;
                        for (int64_t j = 0; j < skv; j++) {
                            const float *vr = j < p ? vp + ((bb * h + hh) * p + j) * d
                                                    : vo + ((bb * h + hh) * so + (j - p)) * d;
                            double pj = sc[j] / sum;
                            for (int64_t c = 0; c < d; c++) acc[c] += pj * vr[c];
                        }
                        for (int64_t c = 0; c < d; c++) orow[c] = (float)acc[c];
                    } else {
                        float fs = (float)scale;
                        for (int64_t c = 0; c < d; c++) qs[c] = qr[c] * fs;
                        float mx = -INFINITY;
                        for (int64_t j = 0; j < skv; j++) {
                            const float *kr = j < p ? kp + ((bb * h + hh) * p + j) * d
                                                    : ko + ((bb * h + hh) * so + (j - p)) * d;
                            float s = 0.f;
                            for (int64_t c = 0; c < d; c++) s += qs[c] * kr[c];
                            if (mr && !mr[j]) s = -INFINITY;
                            scf[j] = s;
                            if (s > mx) mx = s;
                        }
                        float sum = 0.f;
                        for (int64_t j = 0; j < skv; j++) {
                            scf[j] = expf(scf[j] - mx);
                            sum += scf[j];
                        }
                        for (int64_t j = 0; j < skv; j++) scf[j] /= sum;
                        for (int64_t c = 0; c < d; c++) qs[c] = 0.f;
                        for (int64_t j = 0; j < skv; j++) {
                            const float *vr = j < p ? vp + ((bb * h + hh) * p + j) * d
                                                    : vo + ((bb * h + hh) * so + (j - p)) * d;
                            for (int64_t c = 0; c < d; c++) qs[c] += scf[j] * vr[c];
                        }
                        for (int64_t c = 0; c < d; c++) orow[c] = qs[c];
                    }
                }
        free(sc); free(scf); free(acc); free(qs);
    }
    return fail ? -2 : 0;
}

/* ------------------------------------------------------------------ */
/* the block                                                           */
/* ------------------------------------------------------------------ */

static inline float silu_f(float x) { return x / (1.0f + expf(-x)); }

void oq_silu_inplace(float *x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = silu_f(x[i]);
}

static int qlin(const oq_qweight *w, const float *x, int64_t m, float *y, int mode) {
    return oq_qmatmul(w->type, w->data, w->rows, w->cols, x, m, y, mode);
}

/* [B,S,H,D] -> [B,H,S,D] */
static void bshd_to_bhsd(const float *in, int64_t b, int64_t s, int64_t h, int64_t d, float *out) {
#pragma omp parallel for collapse(3) schedule(static)
    for (int64_t bb = 0; bb < b; bb++)
        for (int64_t hh = 0; hh < h; hh++)
            for (int64_t t = 0; t < s; t++)
                memcpy(out + ((bb * h + hh) * s + t) * d, in + ((bb * s + t) * h + hh) * d,
                       sizeof(float) * (size_t)d);
}

/* TransformerBlock::forward (src/quantized_transformer.rs:258-285) with
 * Attention::forward (124-152) and GatedMlp::forward (191-204). */
int oq_block_forward(const oq_block_cfg *cfg, const oq_block_weights *w,
                     const float *x, int64_t b, int64_t s,
                     const float *mod, int64_t mod_rows, const float *pe,
                     const uint8_t *mask, int64_t mask_batch_stride,
                     const uint16_t *prefix_k, const uint16_t *prefix_v, int64_t p,
                     float *x_out, float *k_out, float *v_out, int mode) {
    const int64_t hid = cfg->hidden, H = cfg->heads, D = cfg->head_dim, F = cfg->mlp;
    const int64_t M = b * s;
    if (H * D != hid || mod_rows < 1 || (mod_rows != 1 && mod_rows != s)) return -1;
    const float eps = 1e-6f;
    int rc = 0;
    float *normed = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *qb = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *kb = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *vb = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *qh = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *kh = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *vh = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *att = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *gu = (float *)malloc(sizeof(float) * (size_t)(M * 2 * F));
    float *hm = (float *)malloc(sizeof(float) * (size_t)(M * F));
    float *pk = NULL, *pv = NULL;
    if (!normed || !qb || !kb || !vb || !qh || !kh || !vh || !att || !gu || !hm) { rc = -2; goto done; }
    if (p > 0) {
        if (!prefix_k || !prefix_v) { rc = -1; goto done; }
        pk = (float *)malloc(sizeof(float) * (size_t)(b * H * p * D));
        pv = (float *)malloc(sizeof(float) * (size_t)(b * H * p * D));
        if (!pk || !pv) { rc = -2; goto done; }
        /* from_cache_entry: bf16 -> compute dtype (src/transformer.rs:43-45) */
        oq_bf16_to_f32_n(prefix_k, b * H * p * D, pk);
        oq_bf16_to_f32_n(prefix_v, b * H * p * D, pv);
    }

    /* chunk(4): scale1, gate1, scale2, gate2 (260-264) */
    const int64_t mstride = 4 * hid;
    /* normed = norm1(x) * (1 + scale1) (267-269) */
    for (int64_t bb = 0; bb < b; bb++)
        oq_layernorm_mod(x + bb * s * hid, s, hid, mod + bb * mod_rows * mstride, mstride,
                         mod_rows == 1 ? s : 1, eps, normed + bb * s * hid);
    /* q, k, v projections (133-135) */
    if ((rc = qlin(&w->to_q, normed, M, qb, mode))) goto done;
    if ((rc = qlin(&w->to_k, normed, M, kb, mode))) goto done;
    if ((rc = qlin(&w->to_v, normed, M, vb, mode))) goto done;
    /* per-head RmsNorm on [B,S,H,D], transpose to [B,H,S,D] (137-139) */
    oq_rmsnorm(qb, M * H, D, w->norm_q, eps);
    oq_rmsnorm(kb, M * H, D, w->norm_k, eps);
    bshd_to_bhsd(qb, b, s, H, D, qh);
    bshd_to_bhsd(kb, b, s, H, D, kh);
    bshd_to_bhsd(vb, b, s, H, D, vh);
    /* RoPE (141-142) */
    oq_apply_rope(qh, b * H, s, D, pe);
    oq_apply_rope(kh, b * H, s, D, pe);
    if (k_out) memcpy(k_out, kh, sizeof(float) * (size_t)(M * hid));
    if (v_out) memcpy(v_out, vh, sizeof(float) * (size_t)(M * hid));
    /* attention over [prefix ; own] (143-148) */
    if ((rc = oq_attention(qh, pk, pv, p, kh, vh, s, b, H, s, D, 1.0 / sqrt((double)D),
                           mask, mask_batch_stride, qb, mode)))
        goto done;
    /* [B,H,S,D] -> [B,S,H*D] (150) */
#pragma omp parallel for collapse(3) schedule(static)
    for (int64_t bb = 0; bb < b; bb++)
        for (int64_t hh = 0; hh < H; hh++)
            for (int64_t t = 0; t < s; t++)
                memcpy(att + ((bb * s + t) * H + hh) * D, qb + ((bb * H + hh) * s + t) * D,
                       sizeof(float) * (size_t)D);
    /* to_out (151) */
    if ((rc = qlin(&w->to_out, att, M, kb, mode))) goto done;
    /* x1 = x + tanh(gate1) * attn (271-273) */
    for (int64_t bb = 0; bb < b; bb++)
        for (int64_t t = 0; t < s; t++) {
            const float *g = mod + (bb * mod_rows + (mod_rows == 1 ? 0 : t)) * mstride + hid;
            for (int64_t c = 0; c < hid; c++) {
                int64_t i = (bb * s + t) * hid + c;
                x_out[i] = x[i] + tanhf(g[c]) * kb[i];
            }
        }
    /* normed = norm2(x1) * (1 + scale2) (276-278) */
    for (int64_t bb = 0; bb < b; bb++)
        oq_layernorm_mod(x_out + bb * s * hid, s, hid, mod + bb * mod_rows * mstride + 2 * hid,
                         mstride, mod_rows == 1 ? s : 1, eps, normed + bb * s * hid);
    /* gated MLP (191-204): [gate ; up] = gate_up(x) or (gate_layer(x), proj(x)) */
    if (w->fused_gate_up) {
        if ((rc = qlin(&w->gate_up, normed, M, gu, mode))) goto done;
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < M; r++)
            for (int64_t c = 0; c < F; c++)
                hm[r * F + c] = silu_f(gu[r * 2 * F + c]) * gu[r * 2 * F + F + c];
    } else {
        if ((rc = qlin(&w->gate_layer, normed, M, gu, mode))) goto done;
        if ((rc = qlin(&w->proj, normed, M, gu + M * F, mode))) goto done;
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < M; r++)
            for (int64_t c = 0; c < F; c++)
                hm[r * F + c] = silu_f(gu[r * F + c]) * gu[M * F + r * F + c];
    }
    if ((rc = qlin(&w->down, hm, M, kb, mode))) goto done;
    /* x2 = x1 + tanh(gate2) * mlp (280-282) */
    for (int64_t bb = 0; bb < b; bb++)
        for (int64_t t = 0; t < s; t++) {
            const float *g = mod + (bb * mod_rows + (mod_rows == 1 ? 0 : t)) * mstride + 3 * hid;
            for (int64_t c = 0; c < hid; c++) {
                int64_t i = (bb * s + t) * hid + c;
                x_out[i] = x_out[i] + tanhf(g[c]) * kb[i];
            }
        }
done:
    free(normed); free(qb); free(kb); free(vb); free(qh); free(kh); free(vh);
    free(att); free(gu); free(hm); free(pk); free(pv);
    return rc;
}

/* The same block forward for a subset of token rows (flat indices r = b*S + t
 * into [0, B*S)): K and V come from every row, since every query attends over
 * all of them, but the query side (q, attention, out-proj, both residuals and
 * the MLP) runs for the listed rows only. x_out is [nrows, hidden]; k_out /
 * v_out (optional) are the full [B,H,S,D]. Each output row is computed with
 * the operations the full forward applies to that row, so it is bit-identical
 * to that row of oq_block_forward. */
int oq_block_forward_rows(const oq_block_cfg *cfg, const oq_block_weights *w,
                          const float *x, int64_t b, int64_t s,
                          const float *mod, int64_t mod_rows, const float *pe,
                          const uint8_t *mask, int64_t mask_batch_stride,
                          const uint16_t *prefix_k, const uint16_t *prefix_v, int64_t p,
                          const int64_t *rows, int64_t nrows,
                          float *x_out, float *k_out, float *v_out, int mode) {
    const int64_t hid = cfg->hidden, H = cfg->heads, D = cfg->head_dim, F = cfg->mlp;
    const int64_t M = b * s, skv = p + s, mstride = 4 * hid;
    if (H * D != hid || mod_rows < 1 || (mod_rows != 1 && mod_rows != s) || nrows < 0) return -1;
    for (int64_t i = 0; i < nrows; i++)
        if (rows[i] < 0 || rows[i] >= M) return -1;
    const float eps = 1e-6f;
    int rc = 0;
    const int64_t R = nrows > 0 ? nrows : 1;
    float *normed = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *kb = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *vb = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *kh = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *vh = (float *)malloc(sizeof(float) * (size_t)(M * hid));
    float *xs = (float *)malloc(sizeof(float) * (size_t)(R * hid));   /* selected rows: normed, then residual */
    float *qs = (float *)malloc(sizeof(float) * (size_t)(R * hid));
    float *qg = (float *)malloc(sizeof(float) * (size_t)(R * hid));   /* q of one batch entry [H, n, D] */
    float *og = (float *)malloc(sizeof(float) * (size_t)(R * hid));
    float *att = (float *)malloc(sizeof(float) * (size_t)(R * hid));
    float *pr = (float *)malloc(sizeof(float) * (size_t)(R * D));     /* pe rows of the selected tokens */
    float *gu = (float *)malloc(sizeof(float) * (size_t)(R * 2 * F));
    float *hm = (float *)malloc(sizeof(float) * (size_t)(R * F));
    int64_t *sel = (int64_t *)malloc(sizeof(int64_t) * (size_t)R);
    uint8_t *mg = mask ? (uint8_t *)malloc((size_t)(R * (skv > 0 ? skv : 1))) : NULL;
    float *pk = NULL, *pv = NULL;
    if (!normed || !kb || !vb || !kh || !vh || !xs || !qs || !qg || !og || !att || !pr || !gu || !hm || !sel ||
        (mask && !mg)) { rc = -2; goto done; }
    if (p > 0) {
        if (!prefix_k || !prefix_v) { rc = -1; goto done; }
        pk = (float *)malloc(sizeof(float) * (size_t)(b * H * p * D));
        pv = (float *)malloc(sizeof(float) * (size_t)(b * H * p * D));
        if (!pk || !pv) { rc = -2; goto done; }
        oq_bf16_to_f32_n(prefix_k, b * H * p * D, pk);
        oq_bf16_to_f32_n(prefix_v, b * H * p * D, pv);
    }
    /* norm1 over every row (K and V need them all) */
    for (int64_t bb = 0; bb < b; bb++)
        oq_layernorm_mod(x + bb * s * hid, s, hid, mod + bb * mod_rows * mstride, mstride,
                         mod_rows == 1 ? s : 1, eps, normed + bb * s * hid);
    if ((rc = qlin(&w->to_k, normed, M, kb, mode))) goto done;
    if ((rc = qlin(&w->to_v, normed, M, vb, mode))) goto done;
    oq_rmsnorm(kb, M * H, D, w->norm_k, eps);
    bshd_to_bhsd(kb, b, s, H, D, kh);
    bshd_to_bhsd(vb, b, s, H, D, vh);
    oq_apply_rope(kh, b * H, s, D, pe);
    if (k_out) memcpy(k_out, kh, sizeof(float) * (size_t)(M * hid));
    if (v_out) memcpy(v_out, vh, sizeof(float) * (size_t)(M * hid));
    /* q for the selected rows */
    for (int64_t i = 0; i < nrows; i++) memcpy(xs + i * hid, normed + rows[i] * hid, sizeof(float) * (size_t)hid);
    if ((rc = qlin(&w->to_q, xs, nrows, qs, mode))) goto done;
    oq_rmsnorm(qs, nrows * H, D, w->norm_q, eps);
    /* attention per batch entry over [prefix ; own] of that entry */
    for (int64_t bb = 0; bb < b; bb++) {
        int64_t n = 0;
        for (int64_t i = 0; i < nrows; i++)
            if (rows[i] / s == bb) sel[n++] = i;
        if (!n) continue;
        for (int64_t j = 0; j < n; j++) {
            const int64_t t = rows[sel[j]] % s;
            memcpy(pr + j * D, pe + t * D, sizeof(float) * (size_t)D);
            for (int64_t hh = 0; hh < H; hh++)
                memcpy(qg + (hh * n + j) * D, qs + sel[j] * hid + hh * D, sizeof(float) * (size_t)D);
            if (mask)
                memcpy(mg + j * skv, mask + bb * mask_batch_stride + t * skv, (size_t)skv);
        }
        oq_apply_rope(qg, H, n, D, pr);
        if ((rc = oq_attention(qg, pk ? pk + bb * H * p * D : NULL, pv ? pv + bb * H * p * D : NULL, p,
                               kh + bb * H * s * D, vh + bb * H * s * D, s, 1, H, n, D,
                               1.0 / sqrt((double)D), mg, 0, og, mode)))
            goto done;
        for (int64_t j = 0; j < n; j++)
            for (int64_t hh = 0; hh < H; hh++)
                memcpy(att + sel[j] * hid + hh * D, og + (hh * n + j) * D, sizeof(float) * (size_t)D);
    }
    if ((rc = qlin(&w->to_out, att, nrows, qs, mode))) goto done;
    /* x1 = x + tanh(gate1) * attn, then norm2 per selected row */
    for (int64_t i = 0; i < nrows; i++) {
        const int64_t bb = rows[i] / s, t = rows[i] % s;
        const float *mr = mod + (bb * mod_rows + (mod_rows == 1 ? 0 : t)) * mstride;
        for (int64_t c = 0; c < hid; c++)
            x_out[i * hid + c] = x[rows[i] * hid + c] + tanhf(mr[hid + c]) * qs[i * hid + c];
        oq_layernorm_mod(x_out + i * hid, 1, hid, mr + 2 * hid, mstride, 1, eps, xs + i * hid);
    }
    if (w->fused_gate_up) {
        if ((rc = qlin(&w->gate_up, xs, nrows, gu, mode))) goto done;
        for (int64_t r = 0; r < nrows; r++)
            for (int64_t c = 0; c < F; c++)
                hm[r * F + c] = silu_f(gu[r * 2 * F + c]) * gu[r * 2 * F + F + c];
    } else {
        if ((rc = qlin(&w->gate_layer, xs, nrows, gu, mode))) goto done;
        if ((rc = qlin(&w->proj, xs, nrows, gu + nrows * F, mode))) goto done;
        for (int64_t r = 0; r < nrows; r++)
            for (int64_t c = 0; c < F; c++)
                hm[r * F + c] = silu_f(gu[r * F + c]) * gu[nrows * F + r * F + c];
    }
    if ((rc = qlin(&w->down, hm, nrows, qs, mode))) goto done;
    for (int64_t i = 0; i < nrows; i++) {
        const int64_t bb = rows[i] / s, t = rows[i] % s;
        const float *g = mod + (bb * mod_rows + (mod_rows == 1 ? 0 : t)) * mstride + 3 * hid;
        for (int64_t c = 0; c < hid; c++)
            x_out[i * hid + c] = x_out[i * hid + c] + tanhf(g[c]) * qs[i * hid + c];
    }
done:
    free(normed); free(kb); free(vb); free(kh); free(vh); free(xs); free(qs); free(qg); free(og);
    free(att); free(pr); free(gu); free(hm); free(sel); free(mg); free(pk); free(pv);
    return rc;
}

/* timestep_embedding (src/scheduler.rs:101-126): f_i = exp(-ln(1e4) * i/half)
 * in f32, emb = 1000 t f_i, output [cos ; sin]. */
void oq_timestep_embedding(const float *t, int64_t b, int64_t dim, float *out) {
    int64_t half = dim / 2;
    for (int64_t bb = 0; bb < b; bb++)
        for (int64_t i = 0; i < half; i++) {
            float lt = logf(10000.0f);
            float f = expf(-lt * ((float)i / (float)half));
            float e = (t[bb] * 1000.0f) * f;
            out[bb * dim + i] = cosf(e);
            out[bb * dim + half + i] = sinf(e);
        }
}
