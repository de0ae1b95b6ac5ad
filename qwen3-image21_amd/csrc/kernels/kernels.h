// Launch interface of the gfx950 kernels (host side of the .hip files).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qimm {

// Device weight formats after upload. The GGUF block bytes are the source of
// truth; these layouts only move bytes (no value changes):
//   WF_Q8_0  codes int8 [N][K] + f16 scales [N][K/32]      (34 B blocks split)
//   WF_Q4_K  GGUF 144 B blocks, 16-row groups interleaved per super-block:
//            [N/16][K/256][16] x 144 B (q4k_block in device_common.h)
//   WF_Q6_K  GGUF blocks padded to 224 B, the same 16-row interleave:
//            [N/16][K/256][16] x 224 B (q6k_block)
//   WF_BF16  bf16 [N][K]
enum : int { WF_Q8_0 = 0, WF_Q4_K = 1, WF_Q6_K = 2, WF_BF16 = 3 };

enum : int { EPI_F32 = 0, EPI_BF16 = 1, EPI_QKV = 2, EPI_RESID = 3, EPI_SWIGLU = 4 };

struct EpiParams {
    // EPI_F32 / EPI_BF16: out[m * ldo + n]
    void *out;
    int64_t ldo;
    // EPI_RESID: x_out[m*N+n] = x_in[m*N+n] + gvec[(m / g_rows_per) * g_stride + n] * acc
    const float *x_in;
    float *x_out;
    const float *gvec;
    int64_t g_stride;
    int64_t g_rows_per;
    // EPI_QKV: fused-column n + n_offset in [0, 3*hidden): q | k | v sections.
    // q, k: RmsNorm per 128-wide head, then RoPE with pe[s][128], to [B,H,S,D].
    // v: transposed to vt [B,H,D,S]; also [B,H,S,D] into v_bhsd when non-null.
    uint16_t *q;
    uint16_t *k;
    uint16_t *vt;
    uint16_t *v_bhsd;
    const float *norm_q;
    const float *norm_k;
    const float *pe;
    int64_t seq;
    int64_t heads;
    int64_t hidden;
    int64_t n_offset;
    float q_scale = 1.0f;  // multiplies q after RoPE, before the bf16 rounding
    // EPI_SWIGLU: tile columns [0,64) gate, [64,128) up -> hmid[m*ldh + n/2 + j]
    // (bf16), or hmid_f32[m*ldh + n/2 + j] (f32) when hmid_f32 is set
    uint16_t *hmid;
    int64_t ldh;
    float *hmid_f32 = nullptr;
    // EPI_SWIGLU with hmid_q8k set: hmid receives the hidden state rounded as
    // candle's Q8_K (quant_act4<256> over each 256 columns of a row, ldh and the
    // hidden width multiples of 256), and hmid_f32 is f32 scratch of the same
    // shape for it (the large-M paired kernel, else the f32 state and then the
    // rows quantizer)
    int hmid_q8k = 0;
    // EPI_SWIGLU with hmid_q8_0 set: hmid receives the hidden state rounded as
    // candle's Q8_0 activations (bf16(d q), one d per 32 columns of a row), by
    // the epilogue of the large-M kernel or the undivided 128x128 kernel;
    // every other path writes the f32 state to hmid_f32 (which must be set)
    // and rounds it in its own pass. Needs (N / 2) % 32 == 0.
    int hmid_q8_0 = 0;
    // f32 scratch of part_ws_bytes for the short-M split-K path (optional;
    // without it short M takes the 128x128 kernel)
    float *part_ws = nullptr;
    size_t part_ws_bytes = 0;
};

struct GemmWeight {
    int fmt;
    int64_t n, k;
    const uint8_t *q;       // codes / blocks
    const uint16_t *scales; // WF_Q8_0 only
};

// y = A[M,K] (bf16, row stride lda) x W[N,K]^T with the epilogue selected by epi.
// Dispatches to the 256x256 large-M kernel when qgemm_large_fits (at least 512
// rows, and more 128x128 tiles than one wave of two workgroups per CU), else to
// the 128x128 kernel.
hipError_t launch_qgemm(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda,
                        int epi, const EpiParams &ep, hipStream_t stream);
bool qgemm_large_fits(const GemmWeight &w, int64_t m);
// Compute units of the current device (0 if the runtime cannot say), read once.
int device_cu_count();

// Short-M weight-streaming path (M <= 64): split-K partial sums, added in a
// fixed order by the epilogue (in the same launch for Q4_K / Q6_K at M <= 16).
// work (qgemm_stream_workspace bytes) starts with STREAM_COUNTER_BYTES of
// arrival counters that must be zero before the first call; every call leaves
// them zero again. The partial sums follow.
constexpr size_t STREAM_COUNTER_BYTES = 64 * 1024;
bool qgemm_stream_fits(const GemmWeight &w, int64_t m);
size_t qgemm_stream_workspace(const GemmWeight &w, int64_t m);
int qgemm_stream_splits(const GemmWeight &w, int64_t m);
hipError_t launch_qgemm_stream(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                               const EpiParams &ep, float *work, hipStream_t stream);
hipError_t launch_qgemm_large(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda,
                              int epi, const EpiParams &ep, hipStream_t stream);
// The large-M kernel for quantized weights (Q4_K, Q6_K, Q8_0 with K % 256 == 0
// and N % 256 == 0): eight waves per 256x256 tile, each decoding its own 32
// weight rows into registers. launch_qgemm_large takes it where it fits (the
// q/k/v epilogue also needs hidden % 256 == 0).
bool qgemm_wide_fits(const GemmWeight &w);
// the paired SwiGLU form with the Q8_K rounding of the hidden state (EpiParams::hmid_q8k)
bool qgemm_wide_pairs_fit(const GemmWeight &w);
hipError_t launch_qgemm_wide(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                             const EpiParams &ep, hipStream_t stream);
// Sum of split-K partials part[splits][m][N] (f32) in split order, with the
// epilogue epi applied (the second kernel of the split paths).
hipError_t launch_split_epilogue(const float *part, int splits, int64_t m, int64_t N, int epi, const EpiParams &ep,
                                 hipStream_t stream);
// K split of the 128x128 kernel (64 < M < 512) when its tiles alone leave CUs
// idle; 1 = no split.
int qgemm_mid_splits(const GemmWeight &w, int64_t m);
// Scratch bytes launch_qgemm may use for (w, m) through EpiParams::part_ws
// (0 = none): the short-M path's, or the split 128x128 path's partial sums,
// each after STREAM_COUNTER_BYTES of counters. Without it the unsplit kernels run.
size_t qgemm_workspace(const GemmWeight &w, int64_t m);

// Static scratch of the allocation-free product (noalloc.hip): one file-scope
// device array per device. The split 128x128 partials stay within 32 MiB for
// every shape (at most two workgroups per CU of f32 128x128 tiles), and the
// short-M partials within 32 MiB for every projection of the reference's
// block; with the counters 48 MiB covers them. A product that needs more (one
// share of m x N x 4 bytes of partials for a very wide bf16 weight at 64
// tokens) is rejected by the allocation-free entry point.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)48 << 20;  // QIMM_NOALLOC_SCRATCH_BYTES of qimm.h
// Looks up the array's device address on `device` (which must be current)
// once, zeroes its counter area and waits; later calls return at once.
hipError_t noalloc_scratch_setup(int device);
// The device address looked up by noalloc_scratch_setup, or null before it.
void *noalloc_scratch(int device);

// Exact GGUF dequantization of raw block bytes (device) to f32 (device).
hipError_t launch_dequant(int ggml_type, const uint8_t *src, int64_t n, float *out,
                          hipStream_t stream);

// out[m][:] = bf16(LayerNorm(x[m][:]) * modp_scale[(m / rows_per) * stride + :]);
// one workgroup keeps a row in registers, so hidden <= LN_MAX_HIDDEN
// (hipErrorInvalidValue beyond).
// qblk 32 / 256: the output is candle's activation rounding of the f32 values
// instead (Q8_0 / Q8_K blocks along the row, quant_act4 of device_common.h;
// hidden % 256 == 0); 0: plain bf16.
// prep non-null: scale points at the raw modulation rows [prep_rows][4h] (1 is
// added to their scale1 part here), and the launch also writes their prepared
// form to prep: prep[r][0:h] = 1 + scale1, [h:2h] = tanh(gate1), [2h:3h] =
// 1 + scale2, [3h:4h] = tanh(gate2).
constexpr int64_t LN_MAX_HIDDEN = 8192;
hipError_t launch_ln_mod(const float *x, int64_t m, int64_t hidden, const float *scale,
                         int64_t stride, int64_t rows_per, uint16_t *out, hipStream_t stream, int qblk = 0,
                         float *prep = nullptr, int64_t prep_rows = 0);
// out[m][:] (bf16, row stride ldo) = candle's activation rounding of the f32
// rows x[m][:k] (row stride ldx) in blocks of qblk = 32 (Q8_0) or 256 (Q8_K).
hipError_t launch_quant_rows(const float *x, int64_t ldx, int64_t m, int64_t k, int qblk, uint16_t *out,
                             int64_t ldo, hipStream_t stream);
// The activation block of candle's vec-dot type for a weight format: 32 for
// Q8_0, 256 for Q4_K / Q6_K (Q8_K), 0 for float weights (a plain matmul).
inline int act_block(int fmt) { return fmt == WF_Q8_0 ? 32 : (fmt == WF_Q4_K || fmt == WF_Q6_K) ? 256 : 0; }

// Joint attention over [prefix ; own] keys. q, k_* : [B,H,S,128] bf16;
// vt_* : [B,H,128,S] bf16; out [B,Sq,H*128] bf16, or outf [B,Sq,H*128] f32
// instead when outf is set (out is then not written). out_qblk 32 / 256: out
// holds candle's activation rounding of the output instead, bf16(d q) per Q8_0
// (32 values) / Q8_K (256 values) block (quant_act4's arithmetic), the to_out
// input in the candle mode: Q8_0 in the kernels' epilogue; Q8_K by the paired
// cached-step kernel where it runs (an even head count), else through outf
// (then required, f32 scratch) and the rows quantizer.
hipError_t launch_attention(const uint16_t *q, const uint16_t *kp, const uint16_t *vtp,
                            int64_t p, const uint16_t *ko, const uint16_t *vto, int64_t so,
                            int64_t b, int64_t h, int64_t sq, float scale, uint16_t *out,
                            hipStream_t stream, float *outf = nullptr);
// Masked attention (build_block_causal_mask semantics): img [sq] image block
// ids (-1 text) for a prefix-less call where queries and keys are one
// sequence (so == sq), kvalid [b][p + so] key validity; either may be null.
// sl2 = softmax scale * log2(e), or 1 when q already carries it. lim_scratch
// (sq int32, may be null) holds each query's last visible key for the
// block-causal form; without it that form takes the register-staged kernel.
hipError_t launch_attention_masked(const uint16_t *q, const uint16_t *kp, const uint16_t *vtp, int64_t p,
                                   const uint16_t *ko, const uint16_t *vto, int64_t so, int64_t b, int64_t h,
                                   int64_t sq, float sl2, const int32_t *img, const uint8_t *kvalid,
                                   int32_t *lim_scratch, uint16_t *out, hipStream_t stream,
                                   float *outf = nullptr, const float *k_prefix_norm = nullptr,
                                   float q_norm = 0.f, float k_own_norm = 0.f, int out_qblk = 0);
// The same with q already multiplied by scale * log2(e) (the QKV epilogue's
// q_scale), so scores are in log2 units.
hipError_t launch_attention_log2(const uint16_t *q, const uint16_t *kp, const uint16_t *vtp,
                                 int64_t p, const uint16_t *ko, const uint16_t *vto, int64_t so,
                                 int64_t b, int64_t h, int64_t sq, uint16_t *out, hipStream_t stream,
                                 float *outf = nullptr, const float *k_prefix_norm = nullptr,
                                 float q_norm = 0.f, float k_own_norm = 0.f, int out_qblk = 0);
// Score bound of the fast kernels (both launches above): with q_norm >= every
// query's norm (as passed, before sl2), k_own_norm >= every own key's norm and,
// when there is a prefix, *k_prefix_norm (device) >= every prefix key's norm,
// a bound q_norm * sl2 * max(k norms) <= 64 on the scores in log2 units lets
// the kernel drop the running maximum (a fixed softmax reference). q_norm 0:
// always the running-maximum form.

// out_dev[0] = the largest Euclidean norm of the rows of k [rows][128] bf16
// (f32 sums), through part (>= QK_NORM_PARTS floats of device scratch).
constexpr int QK_NORM_PARTS = 1024;
hipError_t launch_row_norm_max(const uint16_t *k, int64_t rows, float *part, float *out_dev, hipStream_t stream);

// Per-head RmsNorm + RoPE of raw projections x [B,S,H,128] (f32) into the
// attention layouts; mode 0: q/k -> [B,H,S,128]; mode 1: v -> vt [B,H,128,S].
hipError_t launch_qk_prep(const float *x, int64_t b, int64_t s, int64_t h, const float *w,
                          const float *pe, int mode, uint16_t *out, hipStream_t stream);

// [B,H,S,128] bf16 -> [B,H,128,S] bf16 (and back when inverse != 0).
hipError_t launch_transpose_sd(const uint16_t *in, int64_t bh, int64_t s, uint16_t *out,
                               int inverse, hipStream_t stream);

// ---- the denoising step around the blocks (step.hip), all f32 ----
enum : int { ACT_NONE = 0, ACT_SILU = 1, ACT_GELU_TANH = 2 };
// y[m][n] (row stride ldy) = sum_k act(x[m][k]) * w[n][k]; x row stride ldx, w [n][k] dense.
hipError_t launch_linear_f32(const float *x, int64_t ldx, const float *w, int64_t m, int64_t n, int64_t k,
                             int act_in, float *y, int64_t ldy, hipStream_t stream);
// y = x / sqrt(mean(x^2) + eps) * w, per row of d values
hipError_t launch_rows_rmsnorm(const float *x, const float *w, int64_t rows, int64_t d, float eps, float *y,
                               hipStream_t stream);
// y = LayerNorm(x) * (1 + scale[row / rows_per][:]), per row of d values
hipError_t launch_rows_ln_scale(const float *x, const float *scale, int64_t rows, int64_t d, int64_t rows_per,
                                float eps, float *y, hipStream_t stream);
// x += dt * v
hipError_t launch_euler(float *x, const float *v, int64_t n, float dt, hipStream_t stream);
// out = neg + scale * (cond - neg)
hipError_t launch_cfg(const float *cond, const float *neg, int64_t n, float scale, float *out, hipStream_t stream);

}  // namespace qimm
