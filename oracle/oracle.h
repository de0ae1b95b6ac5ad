/*
 * CPU oracle for the single-stream MMDiT block of Qwen-Image-2.1.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C, the arithmetic
 * of the reference engine's denoising-step hot path so that the HIP kernels can
 * be checked against it. Only the test suite, the smoke check and the CPU
 * baseline leg of the benchmark load it; the product library never links it.
 *
 * Every function cites the reference file:line (paths relative to the
 * reference repository root) or, for arithmetic that lives in the pinned
 * third-party crate candle-core 0.11.0 (absent from the reference tree), the
 * published GGML block format it restates.
 *
 * Two GEMM modes:
 *   OQ_MODE_CANDLE  candle's CPU QMatMul: activations quantized per row to the
 *                   weight's vec-dot type (Q8_0 for Q8_0 weights, Q8_K for
 *                   K-quants), integer dot products, f32 block sums.
 *   OQ_MODE_EXACT   weights dequantized to f32 exactly, activations kept in
 *                   f32, products accumulated in f64.
 */
#ifndef QIMM_ORACLE_H
#define QIMM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (GGML spec, as read by candle's gguf_file). */
enum {
    OQ_F32 = 0,
    OQ_F16 = 1,
    OQ_Q8_0 = 8,
    OQ_Q8_K = 15,
    OQ_Q4_K = 12,
    OQ_Q6_K = 14,
    OQ_BF16 = 30
};

enum { OQ_MODE_CANDLE = 0, OQ_MODE_EXACT = 1 };

/* ---- scalar conversions (half 2.7.1 semantics: round to nearest even) ---- */
float oq_f16_to_f32(uint16_t h);
uint16_t oq_f32_to_f16(float f);
float oq_bf16_to_f32(uint16_t b);
uint16_t oq_f32_to_bf16(float f);
void oq_f32_to_bf16_n(const float *x, int64_t n, uint16_t *out);
void oq_bf16_to_f32_n(const uint16_t *x, int64_t n, float *out);

/* ---- GGML block codecs ---- */
int oq_block_size(int type);          /* values per block, 0 if unknown */
int oq_block_bytes(int type);         /* bytes per block, 0 if unknown */
int64_t oq_row_bytes(int type, int64_t n);
/* x has n values (n a multiple of the block size). Returns 0 on success. */
int oq_quantize(int type, const float *x, int64_t n, void *out);
/* candle's activation rounding of m rows of k values for a wtype weight, as
 * bf16 operands bf16(d * q) (rounded once from the exact product). */
int oq_quant_act_bf16(int wtype, const float *x, int64_t m, int64_t k, uint16_t *out);
int oq_dequantize(int type, const void *in, int64_t n, float *out);

/* ---- quantized matmul: y[M,N] = x[M,K] * W[N,K]^T ---- */
int oq_qmatmul(int wtype, const void *w, int64_t N, int64_t K,
               const float *x, int64_t M, float *y, int mode);

/* ---- row ops ---- */
/* out = LayerNorm(x; eps, weight 1, bias 0) * (1 + scale[col]) per row. */
void oq_layernorm_mod(const float *x, int64_t rows, int64_t cols,
                      const float *scale, int64_t scale_row_stride,
                      int64_t rows_per_scale_row, float eps, float *out);
/* In place: x = x / sqrt(mean(x^2) + eps) * w, rows of length d. */
void oq_rmsnorm(float *x, int64_t rows, int64_t d, const float *w, float eps);

/* ---- RoPE ---- */
/* Position table of EmbedNd::forward: pe[seq][2*sum(axes)/2] = (cos, sin)
 * interleaved. shapes: nshapes x (frame, height, width). image_mask: seq. */
int oq_rope_table(const int64_t *shapes, int nshapes, const uint8_t *image_mask,
                  int64_t seq, const int64_t *axes, double theta, float *pe);
/* x [BH][S][D] rotated in place by pe [S][D] (interleaved cos, sin). */
void oq_apply_rope(float *x, int64_t bh, int64_t s, int64_t d, const float *pe);

/* ---- joint layout and mask ---- */
int oq_joint_layout(int64_t text_len, const uint8_t *text_image_mask,
                    const int64_t *cond_shapes, int ncond, int64_t th, int64_t tw,
                    int64_t *image_ids, int64_t cap, int64_t *prefix_len,
                    int64_t *target_len, int64_t *total_len);
void oq_block_causal_mask(const int64_t *image_ids, int64_t s, uint8_t *mask);

/* ---- attention ----
 * out[b,h,i,:] = softmax(scale * q[b,h,i,:] . k[b,h,j,:] over allowed j) v[b,h,j,:]
 * k/v are given as a prefix segment [B,H,P,D] (may be NULL when P == 0) and an
 * own segment [B,H,S,D]. mask (nullable) is [B or 1][Sq][P+S] bytes, nonzero
 * where attending is allowed; mask_batch_stride 0 broadcasts. */
int oq_attention(const float *q, const float *kp, const float *vp, int64_t p,
                 const float *ko, const float *vo, int64_t so,
                 int64_t b, int64_t h, int64_t sq, int64_t d, double scale,
                 const uint8_t *mask, int64_t mask_batch_stride, float *out,
                 int mode);

/* ---- the block ---- */
typedef struct {
    int type;
    const void *data;
    int64_t rows; /* out features */
    int64_t cols; /* in features */
} oq_qweight;

typedef struct {
    oq_qweight to_q, to_k, to_v, to_out;
    int fused_gate_up;          /* 1: gate_up [2*mlp, hidden]; 0: proj + gate_layer */
    oq_qweight gate_up, proj, gate_layer;
    oq_qweight down;            /* img_mlp.out [hidden, mlp] */
    const float *norm_q;        /* [head_dim] */
    const float *norm_k;        /* [head_dim] */
} oq_block_weights;

typedef struct {
    int64_t hidden, heads, head_dim, mlp;
} oq_block_cfg;

/* x [B,S,hidden] f32; mod [B, mod_rows, 4*hidden] (mod_rows 1 broadcasts);
 * pe [S, head_dim]; mask nullable [B or 1][S][P+S] with mask_batch_stride;
 * prefix_k/v bf16 [B,H,P,D] or NULL; outputs x_out [B,S,hidden] and optional
 * k_out/v_out [B,H,S,D] f32 (after norm and rope for k). */
int oq_block_forward(const oq_block_cfg *cfg, const oq_block_weights *w,
                     const float *x, int64_t b, int64_t s,
                     const float *mod, int64_t mod_rows, const float *pe,
                     const uint8_t *mask, int64_t mask_batch_stride,
                     const uint16_t *prefix_k, const uint16_t *prefix_v, int64_t p,
                     float *x_out, float *k_out, float *v_out, int mode);
/* The same forward for the token rows listed in rows[nrows] (flat b*S + t):
 * x_out [nrows, hidden], bit-identical to those rows of oq_block_forward;
 * k_out / v_out (optional) are the full [B,H,S,D]. */
int oq_block_forward_rows(const oq_block_cfg *cfg, const oq_block_weights *w,
                          const float *x, int64_t b, int64_t s,
                          const float *mod, int64_t mod_rows, const float *pe,
                          const uint8_t *mask, int64_t mask_batch_stride,
                          const uint16_t *prefix_k, const uint16_t *prefix_v, int64_t p,
                          const int64_t *rows, int64_t nrows,
                          float *x_out, float *k_out, float *v_out, int mode);

/* ---- timestep path ---- */
/* [cos(1000 t f_i), sin(1000 t f_i)], f_i = exp(-ln(1e4) i / half), dim 256. */
void oq_timestep_embedding(const float *t, int64_t b, int64_t dim, float *out);
void oq_silu_inplace(float *x, int64_t n);

/* ---- timing helper for the CPU baseline ---- */
double oq_now_seconds(void);
int oq_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
