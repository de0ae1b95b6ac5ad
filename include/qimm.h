/*
 * qimm — MI355X (gfx950) kernels for the single-stream MMDiT block of
 * Qwen-Image-2.1: GGUF dequant-GEMM + joint attention over a persistent
 * prefix K/V cache.
 *
 * C ABI. Plain pointers and sizes only. Device pointers are HIP device
 * addresses on the context's device; "stream" is a hipStream_t (NULL = the
 * legacy default stream). Every call returns a qimm_status; a non-zero status
 * leaves a message retrievable with qimm_last_error(ctx).
 *
 * The reference engine (Rust, candle 0.11) has no FFI boundary of its own;
 * each entry point below names the Rust item it stands in for. Paths are
 * relative to the reference repository root.
 *
 * Threading: one context per device per host thread, as the reference gives
 * each worker thread exclusive use of its device (src/server.rs:120-148).
 */
#ifndef QIMM_H
#define QIMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QIMM_ABI_VERSION 1

typedef enum {
    QIMM_OK = 0,
    QIMM_ERR_ARG = 1,      /* null pointer, bad enum, negative size */
    QIMM_ERR_SHAPE = 2,    /* sizes inconsistent or unsupported by the kernels */
    QIMM_ERR_TYPE = 3,     /* GGML type not supported for this use */
    QIMM_ERR_OOM = 4,      /* device or host allocation failed */
    QIMM_ERR_HIP = 5,      /* a HIP runtime call failed */
    QIMM_ERR_STATE = 6,    /* object used in the wrong state (e.g. missing cache) */
    QIMM_ERR_NOT_FOUND = 7,/* named tensor or metadata key absent */
    QIMM_ERR_FORMAT = 8    /* file malformed or truncated (GGUF reader) */
} qimm_status;

/* GGML tensor type ids as stored in GGUF files (GGML spec; the values
 * candle's gguf_file reader uses). */
typedef enum {
    QIMM_TYPE_F32 = 0,
    QIMM_TYPE_F16 = 1,
    QIMM_TYPE_Q8_0 = 8,
    QIMM_TYPE_Q4_K = 12,
    QIMM_TYPE_Q6_K = 14,
    QIMM_TYPE_BF16 = 30
} qimm_ggml_type;

typedef struct qimm_ctx qimm_ctx;
typedef struct qimm_weight qimm_weight;
typedef struct qimm_block qimm_block;
typedef struct qimm_kv qimm_kv;

/* ---------------- context ---------------- */

/* One device context. Stands in for candle's Device handle as selected in
 * src/main.rs:159-162 and owned per worker thread (src/server.rs:123-155).
 * Calls through one context share its device scratch (block intermediates,
 * split-K partial sums and their arrival counters), so they must not overlap
 * on the device: issue them from one thread on one stream, or order the
 * streams with events. Separate contexts are independent. */
int qimm_ctx_create(int device, qimm_ctx **out);
int qimm_ctx_destroy(qimm_ctx *ctx);
/* Message of the last failed call on ctx (mirrors candle's bail! text,
 * e.g. src/quantized_transformer.rs:489). Never NULL. */
const char *qimm_last_error(const qimm_ctx *ctx);
const char *qimm_status_string(int status);
int qimm_abi_version(void);

/* Device memory helpers for hosts without their own device allocator
 * (candle moves tensors with Tensor::to_device, src/transformer.rs:37-45). */
int qimm_malloc(qimm_ctx *ctx, size_t bytes, void **dptr);
int qimm_free(qimm_ctx *ctx, void *dptr);
int qimm_memcpy_h2d(qimm_ctx *ctx, void *dst, const void *src, size_t bytes, void *stream);
int qimm_memcpy_d2h(qimm_ctx *ctx, void *dst, const void *src, size_t bytes, void *stream);
int qimm_stream_synchronize(qimm_ctx *ctx, void *stream);

/* ---------------- quantized weights ---------------- */

/* Upload one GGUF tensor [rows = out features, cols = in features], GGML
 * blocks running along cols, exactly as candle's quantized VarBuilder hands
 * it to QMatMul::from_arc (src/quantized_transformer.rs:31-33). bytes must be
 * rows * cols / block_size * block_bytes. The library owns the device copy
 * and may re-stride blocks for aligned loads; values are never changed. */
int qimm_weight_upload(qimm_ctx *ctx, int ggml_type, int64_t rows, int64_t cols,
                       const void *host_bytes, size_t nbytes, qimm_weight **out);
int qimm_weight_free(qimm_weight *w);
int64_t qimm_weight_device_bytes(const qimm_weight *w);

/* Exact dequantization to f32 of raw GGUF block bytes already on the device.
 * Replaces QTensor::dequantize (src/gguf_loader.rs:35-38,
 * src/quantized_transformer.rs:68,108,110). Bit-identical to the GGML
 * formulas: every scale product is exact in f32. n = number of values. */
int qimm_dequant(qimm_ctx *ctx, int ggml_type, const void *dev_bytes, int64_t n,
                 float *dev_out, void *stream);

/* y[M,N] = x[M,K] * W^T with x bf16 row-major (row stride lda elements,
 * lda % 8 == 0), y row-major [M,N] in f32 (out_type QIMM_TYPE_F32) or bf16
 * (QIMM_TYPE_BF16). Replaces QMatMul::forward as called by Linear::forward
 * (src/quantized_transformer.rs:19-29). Requires N % 128 == 0 and K a
 * multiple of 64 and of the block size. */
int qimm_qmatmul(qimm_ctx *ctx, const qimm_weight *w, const void *x_bf16, int64_t m,
                 int64_t lda, void *y, int out_type, void *stream);

/* qimm_qmatmul that allocates nothing, for callers that cannot allocate
 * device memory during a call (code under HIP graph capture, tight serving
 * loops). It has no counterpart in the reference. Same arguments, kernels and
 * results as qimm_qmatmul; the split-K partial sums and arrival counters live
 * in a static device array of QIMM_NOALLOC_SCRATCH_BYTES (48 MiB) per device,
 * set up when the device's first context is created and held until the
 * process ends, instead of the context's growable scratch. A product needs
 * qimm_qmatmul_scratch_bytes(w, m) of it; one that needs more than the array
 * returns QIMM_ERR_SHAPE (use qimm_qmatmul there). Every projection of the
 * reference's block (hidden 4096, mlp 12288: q/k/v, out, gate_up, down in
 * Q8_0, Q4_K, Q6_K or BF16) fits at any m (32 MiB at most); larger products
 * may not: up to 64 tokens the short-M kernels keep at least m * N * 4 bytes
 * of split-K partial sums (more than 48 MiB for N above ~196,000 outputs at
 * 64 tokens). All calls on one device share that array (it
 * keeps the last call's contents; the counters return to zero after every
 * call), so calls that overlap on one device, from any context or stream,
 * race: order them. */
#define QIMM_NOALLOC_SCRATCH_BYTES (48u << 20)
int qimm_qmatmul_noalloc(qimm_ctx *ctx, const qimm_weight *w, const void *x_bf16, int64_t m,
                         int64_t lda, void *y, int out_type, void *stream);
/* Bytes of device scratch the product of w with m rows takes (0 = none; -1 on
 * a bad argument): what qimm_qmatmul grows the context scratch to, and what
 * qimm_qmatmul_noalloc needs of its static array. It depends on the device's
 * compute-unit count (the split plans). No counterpart in the reference. */
int64_t qimm_qmatmul_scratch_bytes(const qimm_weight *w, int64_t m);

/* ---------------- host-side layout and RoPE ---------------- */

/* JointLayout::new (src/joint_layout.rs:52-103). text_image_mask may be NULL
 * (text-to-image). cond_shapes: ncond (h, w) pairs. image_ids receives the
 * per-token block id (-1 text) for total_len tokens; pass cap >= total_len. */
int qimm_joint_layout(int64_t text_len, const uint8_t *text_image_mask,
                      const int64_t *cond_shapes, int64_t ncond,
                      int64_t target_h, int64_t target_w,
                      int64_t *image_ids, int64_t cap,
                      int64_t *prefix_len, int64_t *target_len, int64_t *total_len);

/* EmbedNd::forward (src/rope.rs:104-211) with the tables of
 * EmbedNd::new_with_mode (src/rope.rs:37-88): pe[seq][sum(axes)] = (cos, sin)
 * interleaved per pair, frame | height | width pairs. shapes: nshapes
 * (frame, height, width) triples; image_mask: seq bytes (nonzero = image). */
int qimm_rope_table(const int64_t *shapes, int64_t nshapes, const uint8_t *image_mask,
                    int64_t seq, const int64_t axes[3], double theta, float *pe_host);

/* ---------------- prefix K/V cache ---------------- */

/* TextKvCache (src/transformer.rs:14-19): per layer (k, v) of the prefix
 * after Q/K norm and RoPE, stored bf16 (KV_CACHE_DTYPE, src/transformer.rs:24)
 * in device memory owned by the library, persistent across steps. Head dim
 * must be 128. Internally k is [B,H,P,128] and v is stored transposed
 * [B,H,128,P] for the attention kernel. */
int qimm_kv_create(qimm_ctx *ctx, int64_t layers, int64_t batch, int64_t heads,
                   int64_t prefix_len, int64_t head_dim, qimm_kv **out);
int qimm_kv_destroy(qimm_kv *kv);
/* to_cache_entry (src/transformer.rs:37-41): store one layer given in the
 * reference layout [B,H,P,D] bf16 (device pointers). */
int qimm_kv_store_layer(qimm_kv *kv, int64_t layer, const uint16_t *k_bhpd,
                        const uint16_t *v_bhpd, void *stream);
/* from_cache_entry (src/transformer.rs:43-45): read one layer back in the
 * reference layout [B,H,P,D] bf16 (device pointers). */
int qimm_kv_load_layer(const qimm_kv *kv, int64_t layer, uint16_t *k_bhpd, uint16_t *v_bhpd,
                       void *stream);
int64_t qimm_kv_prefix_len(const qimm_kv *kv);

/* The host-resident cache of set_kv_cache_offload / --kv-cache-cpu
 * (src/transformer.rs:26-41, src/main.rs:169-172): the same object, but the
 * layers live in pinned host memory and a layer is copied to the device only
 * while it is used. Two device slots of one layer each stage the copies.
 * Every call that takes a qimm_kv works on both kinds; on a host cache, a call
 * that needs a layer not staged copies it first on its own stream. */
int qimm_kv_create_host(qimm_ctx *ctx, int64_t layers, int64_t batch, int64_t heads,
                        int64_t prefix_len, int64_t head_dim, qimm_kv **out);
int qimm_kv_is_host(const qimm_kv *kv);
/* Starts copying one layer of a host cache into a device slot on `stream`
 * (a copy stream, so that layer l+1 moves while layer l computes); the next
 * call using that layer, on any stream, waits for the copy on the device. A
 * slot is reused only after the kernels reading it have finished (events), so
 * at most the layer in use and one prefetched layer are resident. No-op on a
 * device cache. (The reference copies synchronously inside from_cache_entry,
 * src/transformer.rs:43-45; the prefetch is this library's overlap of it.) */
int qimm_kv_prefetch(qimm_kv *kv, int64_t layer, void *stream);

/* ---------------- attention ---------------- */

/* Per-head RmsNorm (eps 1e-6, weight norm_w[128] device f32) then RoPE with
 * pe [S,128] (device f32) on raw projections x [B,S,H,128] f32 (device),
 * written as bf16 [B,H,S,128] — the q/k half of Attention::forward
 * (src/quantized_transformer.rs:137-142). */
int qimm_qk_norm_rope(qimm_ctx *ctx, const float *x, int64_t batch, int64_t seq,
                      int64_t heads, const float *norm_w, const float *pe, uint16_t *out,
                      void *stream);
/* Raw values x [B,S,H,128] f32 -> bf16 [B,H,128,S] (the kernel's V layout). */
int qimm_v_transpose(qimm_ctx *ctx, const float *x, int64_t batch, int64_t seq,
                     int64_t heads, uint16_t *vt_out, void *stream);

/* The activation rounding of QMatMul::forward (src/quantized_transformer.rs:19-29:
 * candle's CPU QMatMul quantizes its f32 input rows to the weight's vec-dot
 * type, candle-core 0.11 BlockQ8_0 / BlockQ8K::from_float): rows x[m][0:k] f32
 * (row stride ldx) to out[m][0:k] bf16 (row stride ldo) = bf16(d * q), the
 * quantized value rounded once to nearest even, in blocks of 32 values (Q8_0
 * weights: d = f16(amax/127), q = round(x * (1/(amax/127)))) or 256 (Q4_K /
 * Q6_K weights, Q8_K: iscale = -128/x_max with x_max the first value of largest
 * magnitude, q = min(127, round(iscale * x)), d = 1/iscale); round() is half
 * away from zero. Feeding out to qimm_qmatmul reproduces QMatMul::forward's
 * rounding. weight_type: Q8_0, Q4_K or Q6_K (QIMM_ERR_TYPE otherwise); k a
 * multiple of the block, ldx and ldo >= k and multiples of 4, x and out 16-byte
 * aligned (device pointers). */
int qimm_quantize_act(qimm_ctx *ctx, int weight_type, const float *x, int64_t m, int64_t k,
                      int64_t ldx, uint16_t *out, int64_t ldo, void *stream);

/* Unmasked joint attention of queries q [B,H,Sq,128] over keys
 * [prefix layer of kv ; own] with own keys k_own [B,H,So,128] and own values
 * transposed vt_own [B,H,128,So] (bf16, device). kv may be NULL (no prefix).
 * out [B,Sq,H*128] bf16. Replaces chunked_attention / flash_attention
 * (src/transformer.rs:246-296) on the cached step, where the mask is None
 * (src/quantized_transformer.rs:526-532) and the keys are
 * cat([from_cache_entry(prefix), own]) (143-146). scale = 1/sqrt(128) there.
 * q, k_own, vt_own and out must be 16-byte aligned. */
int qimm_attention(qimm_ctx *ctx, const uint16_t *q, int64_t batch, int64_t heads,
                   int64_t sq, const qimm_kv *kv, int64_t layer, const uint16_t *k_own,
                   const uint16_t *vt_own, int64_t so, float scale, uint16_t *out,
                   void *stream);

/* ---------------- the block ---------------- */

typedef struct {
    int64_t hidden;    /* heads * head_dim (Config::hidden_size, src/transformer.rs:81-84) */
    int64_t heads;
    int64_t head_dim;  /* must be 128 */
    int64_t mlp;       /* Config::mlp_hidden_size = 3 * hidden (src/transformer.rs:86-88) */
} qimm_block_config;

/* One GGUF tensor in host memory, as the quantized VarBuilder returns it. */
typedef struct {
    int ggml_type;
    int64_t rows;      /* out features (GGUF ne[1]) */
    int64_t cols;      /* in features (GGUF ne[0]) */
    const void *data;  /* NULL = absent */
    size_t nbytes;
} qimm_tensor;

/* The tensors of transformer_blocks.{i} (src/quantized_transformer.rs:99-111,
 * 173-188): attn.to_q/to_k/to_v/to_out.0, attn.norm_q/norm_k [128],
 * img_mlp.gate_up (fused [2*mlp, hidden]) or img_mlp.proj + img_mlp.gate_layer,
 * img_mlp.out. */
typedef struct {
    qimm_tensor to_q, to_k, to_v, to_out;
    qimm_tensor norm_q, norm_k;
    qimm_tensor gate_up;
    qimm_tensor proj, gate_layer;
    qimm_tensor mlp_out;
} qimm_block_tensors;

/* TransformerBlock::new (src/quantized_transformer.rs:249-256): uploads the
 * block's weights (q/k/v fused along N when their types match, gate/up rows
 * interleaved per 64 for the SwiGLU epilogue; block bytes unchanged). */
int qimm_block_create(qimm_ctx *ctx, const qimm_block_config *cfg,
                      const qimm_block_tensors *tensors, qimm_block **out);
int qimm_block_destroy(qimm_block *blk);

/* TransformerBlock::forward (src/quantized_transformer.rs:258-285) on the
 * cached step: attention_mask None, prefix = layer `layer` of kv (kv NULL =
 * no prefix). All pointers are device pointers:
 *   x        [B,S,hidden] f32; x_out may alias x
 *   mod      [B,1,4*hidden] f32 = (scale1, gate1, scale2, gate2) rows
 *   pe       [S,head_dim] f32 (cos, sin interleaved), rows of this call's tokens
 *   k_out/v_out  optional bf16 [B,H,S,head_dim]: this call's own k (after
 *            norm and RoPE) and v, the tuple's 2nd/3rd members stored as
 *            to_cache_entry would (src/quantized_transformer.rs:388). */
int qimm_block_forward(qimm_block *blk, const float *x, float *x_out, int64_t batch,
                       int64_t seq, const float *mod, const float *pe, const qimm_kv *kv,
                       int64_t layer, uint16_t *k_out, uint16_t *v_out, void *stream);

/* Arithmetic at the inputs of the block's quantized matmuls (q/k/v, to_out,
 * gate_up, down: Linear::forward, src/quantized_transformer.rs:19-29, called at
 * 133-135, 151, 196-202).
 *  QIMM_ACT_CANDLE, the default: each f32 input row is rounded as candle's CPU
 *    QMatMul::forward rounds it before its integer dot products (candle-core
 *    0.11 quantized/k_quants.rs, the weight's vec-dot type): to Q8_K per 256
 *    values (scale -128 / the first value of largest magnitude) for Q4_K and
 *    Q6_K weights, to Q8_0 per 32 values (scale amax/127 kept as f16) for Q8_0
 *    weights; float-stored weights take the values unrounded, as candle's plain
 *    matmul does. The MFMA operand is the quantized value d*q rounded once to
 *    bf16 (qimm_quantize_act), so the block follows the reference CPU path's
 *    rounding.
 *  QIMM_ACT_BF16: the f32 values rounded to bf16, no int8 step: closer to exact
 *    arithmetic than the reference, and slightly faster (no f32 staging of the
 *    attention output and the SwiGLU hidden state). */
#define QIMM_ACT_CANDLE 0
#define QIMM_ACT_BF16 1
int qimm_block_set_act_mode(qimm_block *blk, int mode);
int qimm_block_act_mode(const qimm_block *blk);

/* Sizes the context's device scratch for forwards of this block with up to
 * batch x seq tokens and mod_rows modulation rows (1 or seq). A forward that
 * needs more than the scratch holds grows it, which synchronizes the device
 * and reallocates; after a reserve, forwards within these sizes (on this
 * block, or on any block of the context with the same shapes) neither
 * allocate nor synchronize. The reference allocates per call through candle
 * and has no counterpart; this is for serving loops that must not stall. */
int qimm_block_reserve(qimm_block *blk, int64_t batch, int64_t seq, int64_t mod_rows);
/* A forward captured into a HIP graph keeps the scratch addresses it was
 * captured with: while such a graph may still be replayed, no call on the
 * context may grow the scratch (a larger forward, a qimm_qmatmul of a larger
 * product, qimm_attention_masked over more queries), since growing frees the
 * old buffers. Reserve the largest sizes first. */

/* An attention mask, the product of build_block_causal_mask
 * (src/attention_mask.rs:18-66) kept as its two inputs (device pointers):
 *   image_ids  int32 [S]: JointLayout::image_ids of the call's tokens, -1 for
 *              text; query i sees key j if i >= j or both lie in the same
 *              image block. NULL: no block-causal term (every key visible).
 *              Only for calls without a prefix cache, where queries and keys
 *              are the same S tokens.
 *   key_valid  uint8 [B][P+S] over the keys [prefix ; own], 0 = padding
 *              (key_valid, src/quantized_transformer.rs:349-356). NULL: all
 *              keys valid. */
typedef struct {
    const int32_t *image_ids;
    const uint8_t *key_valid;
} qimm_attn_mask;

/* TransformerBlock::forward (src/quantized_transformer.rs:258-285) with
 * Some(attention_mask) and modulation rows [B, mod_rows, 4*hidden]
 * (mod_rows 1 broadcasts, mod_rows == S gives each token its own row).
 * The prefix pass that fills the cache (prefix_kv,
 * src/quantized_transformer.rs:359-392): kv NULL, mask = block-causal over the
 * prefix tokens, the t=0 modulation row, k_out/v_out the layer's cache entry.
 * The uncached full-sequence step (:508-543): kv NULL, mod_rows == S (t=0
 * rows for the prefix, the step's row for the targets). The cached step with
 * padded text: kv given, mask->key_valid only. */
int qimm_block_forward_masked(qimm_block *blk, const float *x, float *x_out, int64_t batch,
                              int64_t seq, const float *mod, int64_t mod_rows, const float *pe,
                              const qimm_attn_mask *mask, const qimm_kv *kv, int64_t layer,
                              uint16_t *k_out, uint16_t *v_out, void *stream);

/* qimm_attention with a mask: chunked_attention (src/transformer.rs:259-296)
 * called with Some(mask) (the masked branch adds -inf where the mask is 0).
 * With mask->image_ids, kv must be NULL and so == sq, and the call keeps each
 * query's last visible key (sq int32) in the context scratch, growing it
 * first when it is smaller (a device-wide synchronize and an allocation);
 * after qimm_block_reserve on this context, or any earlier call of that size,
 * it neither allocates nor synchronizes. Like every call through one context,
 * it must not overlap another on the device. */
int qimm_attention_masked(qimm_ctx *ctx, const uint16_t *q, int64_t batch, int64_t heads,
                          int64_t sq, const qimm_kv *kv, int64_t layer, const uint16_t *k_own,
                          const uint16_t *vt_own, int64_t so, float scale,
                          const qimm_attn_mask *mask, uint16_t *out, void *stream);

/* Stage timing of qimm_block_forward, the device-side counterpart of the
 * reference's per-phase wall-clock prints (src/service.rs:190-203). While
 * enabled, each forward records HIP events on its stream around its stages;
 * qimm_block_stage_times waits for the last forward and writes the durations
 * in ms of its QIMM_BLOCK_STAGES stages:
 *   0 modulation prep + norm1   1 q/k/v projection + norm + RoPE
 *   2 attention                 3 rounding of the attention output (candle mode)
 *   4 output projection + gated residual
 *   5 norm2                     6 gate_up projection + SwiGLU
 *   7 rounding of the SwiGLU hidden state (candle mode)
 *   8 down projection + gated residual
 * Stages 3 and 7 are empty under QIMM_ACT_BF16. */
#define QIMM_BLOCK_STAGES 9
int qimm_block_profile(qimm_block *blk, int enable);
int qimm_block_stage_times(qimm_block *blk, float *ms_out, int n);

/* ---------------- the denoising step around the blocks ---------------- */

/* The whole quantized transformer: the global layers around the blocks plus
 * the caller's blocks (QwenImageTransformerQuantized, src/quantized_transformer.rs:311-331,
 * 399-427). The global linears run in f32 over weights dequantized once at
 * creation (exact), as the reference runs its unquantized ones in F32. */
typedef struct qimm_model qimm_model;

typedef struct {
    int64_t in_channels; /* latent channels (Config::in_channels = 64, src/transformer.rs:67) */
    int64_t joint_dim;   /* txt_in input width (Config::joint_attention_dim); 0 = no txt_in */
    int64_t hidden;      /* must equal the blocks' hidden */
    int64_t layers;      /* number of blocks */
} qimm_model_config;

/* Global tensors, each [out, in] as in GGUF (rows = out, cols = in):
 * img_in [hidden, in_channels]; time_text_embed.timestep_embedder.linear_1
 * [hidden, 256] and linear_2 [hidden, hidden]; modulation.1 [4 hidden, hidden];
 * norm_out.linear [hidden, hidden]; proj_out [in_channels, hidden];
 * txt_in.text_norm [joint_dim] as stored (scale - 1, src/quantized_transformer.rs:65-68),
 * txt_in.in_layer [hidden, joint_dim], txt_in.out_layer [hidden, hidden]
 * (the txt_in three may be absent: data NULL). Types F32, F16, BF16, Q8_0,
 * Q4_K, Q6_K. */
typedef struct {
    qimm_tensor img_in, t_linear_1, t_linear_2, modulation, norm_out, proj_out;
    qimm_tensor txt_norm, txt_in, txt_out;
} qimm_model_tensors;

/* QwenImageTransformerQuantized::new_with_dtype (src/quantized_transformer.rs:399-427).
 * blocks: cfg->layers blocks made by qimm_block_create, not owned; they must
 * outlive the model. */
int qimm_model_create(qimm_ctx *ctx, const qimm_model_config *cfg, const qimm_model_tensors *t,
                      qimm_block *const *blocks, qimm_model **out);
int qimm_model_destroy(qimm_model *m);

/* timestep_embedding(t, 256) (src/scheduler.rs:101-126): cos | sin of
 * 1000 t exp(-ln(1e4) i / 128), i < 128, for batch timesteps t (host),
 * written as f32 [batch][256] to out (device). */
int qimm_timestep_embedding(qimm_ctx *ctx, const float *t, int64_t batch, float *out, void *stream);

/* The cached step of forward_conditioned (src/quantized_transformer.rs:471-551
 * with a filled prefix cache): t_emb = linear_2(silu(linear_1(t_sin))),
 * modulation = modulation.1(silu(t_emb)), h = img_in(latents), the blocks over
 * [prefix ; h] (qimm_block_forward, or the key-validity form when key_valid is
 * given), pred = proj_out(LayerNorm(h) * (1 + norm_out.linear(silu(t_emb)))).
 * latents, pred: [batch, seq, in_channels] f32 (device); t_sin [batch, 256]
 * f32 from qimm_timestep_embedding; pe [seq, 128] f32 (the target rows of the
 * joint table); kv: the prefix cache (or NULL without prefix); key_valid
 * uint8 [batch][P + seq] or NULL. */
int qimm_model_forward(qimm_model *m, const float *latents, int64_t batch, int64_t seq, const float *t_sin,
                       const float *pe, const qimm_kv *kv, const uint8_t *key_valid, float *pred, void *stream);

/* prefix_kv (src/quantized_transformer.rs:359-392): runs the prefix through
 * every block under the t = 0 modulation (zero_modulation, :334-343) and the
 * block-causal mask, storing each layer's k, v into kv.
 * txt [batch, text_len, joint_dim] f32 (before txt_in); cond [batch,
 * cond_len, in_channels] f32 condition latents (before img_in) or NULL;
 * pieces: npieces (kind, start, len) triples in layout order, kind 0 = text
 * rows, 1 = condition rows (JointLayout::assemble, src/joint_layout.rs:112-126;
 * qimm_joint_layout_pieces); image_ids int32 [P] and key_valid uint8
 * [batch][P] (or NULL) on the device; pe [P, 128] f32. P = kv's prefix_len. */
int qimm_model_prefix_fill(qimm_model *m, const float *txt, int64_t text_len, const float *cond, int64_t cond_len,
                           int64_t batch, const int64_t *pieces, int64_t npieces, const int32_t *image_ids,
                           const uint8_t *key_valid, const float *pe, qimm_kv *kv, void *stream);

/* The prefix pieces of JointLayout::new (src/joint_layout.rs:52-103): writes
 * (kind, start, len) triples, kind 0 = Text { start, len } over prompt rows,
 * 1 = Condition { index } as (1, cond_offsets[index], h*w); the target piece
 * is not listed. cap = capacity in triples. */
int qimm_joint_layout_pieces(int64_t text_len, const uint8_t *text_image_mask, const int64_t *cond_shapes,
                             int64_t ncond, int64_t *pieces, int64_t cap, int64_t *npieces);

/* FlowMatchEuler::new (src/scheduler.rs:24-37): the shifted sigma schedule,
 * f32 arithmetic in the reference's order; sigmas gets steps values. */
int qimm_flow_match_sigmas(int64_t steps, int64_t image_seq_len, float *sigmas);
/* FlowMatchEuler::step (src/scheduler.rs:54-66): latents += dt * pred over n
 * f32 values, dt = sigmas[i+1] - sigmas[i] (or -sigmas[i] at the last step). */
int qimm_euler_step(qimm_ctx *ctx, float *latents, const float *pred, int64_t n, float dt, void *stream);
/* Classifier-free guidance (src/pipeline.rs:180-186): out = neg + scale * (cond - neg). */
int qimm_cfg_combine(qimm_ctx *ctx, const float *cond, const float *neg, int64_t n, float scale, float *out,
                     void *stream);

/* ---------------- GGUF files (host only, no device needed) ---------------- */

/* A memory-mapped, parsed GGUF file (format versions 2 and 3). Stands in for
 * candle's gguf_file::Content::read + Content::tensor as used by the quantized
 * VarBuilder in load_transformer (src/service.rs:246-258) and by
 * load_gguf_as_safetensors (src/gguf_loader.rs:15-40). Tensor data pointers
 * stay valid until qimm_gguf_close. */
typedef struct qimm_gguf qimm_gguf;

typedef struct {
    const char *name;  /* NUL-terminated, owned by the file handle */
    int ggml_type;     /* GGML type id (any; sizes known for the non-IQ types) */
    int32_t n_dims;    /* 1..4 */
    int64_t ne[4];     /* ne[0] innermost: in features of a weight, 1 past n_dims */
    const void *data;  /* host pointer into the mapping; NULL if the type's size is unknown */
    size_t nbytes;     /* 0 if the type's size is unknown */
    uint64_t offset;   /* byte offset of the data from the start of the file */
} qimm_gguf_tensor_info;

/* Opens and validates the whole file: magic "GGUF", version 2 or 3, every
 * metadata value, every tensor info, general.alignment (default 32), and that
 * every tensor of known type lies inside the file at an aligned offset.
 * QIMM_ERR_ARG: cannot open/map; QIMM_ERR_FORMAT: malformed (err gets the
 * reason when err_len > 0). */
int qimm_gguf_open(const char *path, qimm_gguf **out, char *err, size_t err_len);
int qimm_gguf_close(qimm_gguf *g);
/* Format version, tensor count, metadata count, alignment, data-section offset. */
int qimm_gguf_header(const qimm_gguf *g, uint32_t *version, int64_t *n_tensors, int64_t *n_kv,
                     uint32_t *alignment, uint64_t *data_offset);

int qimm_gguf_tensor_at(const qimm_gguf *g, int64_t i, qimm_gguf_tensor_info *info);
/* By exact name, else under the ComfyUI prefix "model.diffusion_model." that
 * load_transformer strips (src/service.rs:250-256). QIMM_ERR_NOT_FOUND if absent. */
int qimm_gguf_find(const qimm_gguf *g, const char *name, qimm_gguf_tensor_info *info);

/* GGUF metadata value types (GGUF spec). */
typedef enum {
    QIMM_GGUF_U8 = 0, QIMM_GGUF_I8 = 1, QIMM_GGUF_U16 = 2, QIMM_GGUF_I16 = 3,
    QIMM_GGUF_U32 = 4, QIMM_GGUF_I32 = 5, QIMM_GGUF_F32 = 6, QIMM_GGUF_BOOL = 7,
    QIMM_GGUF_STRING = 8, QIMM_GGUF_ARRAY = 9, QIMM_GGUF_U64 = 10, QIMM_GGUF_I64 = 11,
    QIMM_GGUF_F64 = 12
} qimm_gguf_value_type;

/* Metadata entry i: its key (NUL-terminated, owned by the handle), value type
 * and, for arrays, the element type and count (else elem_type = -1, count 1). */
int qimm_gguf_meta_at(const qimm_gguf *g, int64_t i, const char **key, int *type, int *elem_type,
                      uint64_t *count);
/* Scalar metadata by key: integers and bools widen to int64 (u64 above
 * INT64_MAX is QIMM_ERR_TYPE), floats to double; arrays/strings are QIMM_ERR_TYPE. */
int qimm_gguf_meta_int(const qimm_gguf *g, const char *key, int64_t *out);
int qimm_gguf_meta_float(const qimm_gguf *g, const char *key, double *out);
/* String metadata: pointer into the mapping plus length (not NUL-terminated). */
int qimm_gguf_meta_string(const qimm_gguf *g, const char *key, const char **str, uint64_t *len);

/* 1 if the name is one the model loads (map_gguf_name / is_mappable,
 * src/gguf_mapping.rs:13-60, plus the fused img_mlp.gate_up.weight of
 * src/quantized_transformer.rs:181), after stripping the ComfyUI prefix; else 0. */
int qimm_gguf_is_known_name(const char *name);

/* The tensors of transformer_blocks.{layer} as qimm_block_create takes them
 * (host pointers into the mapping): attn.to_q/k/v/out.0, attn.norm_q/norm_k,
 * img_mlp.gate_up when present else img_mlp.proj + img_mlp.gate_layer
 * (src/quantized_transformer.rs:173-188), img_mlp.out. Each weight's rows =
 * ne[1], cols = ne[0]. QIMM_ERR_NOT_FOUND names the first missing tensor. */
int qimm_gguf_block_tensors(const qimm_gguf *g, int64_t layer, qimm_block_tensors *out, char *err,
                            size_t err_len);
/* The global tensors for qimm_model_create (QwenImageTransformerQuantized::new_with_dtype,
 * src/quantized_transformer.rs:399-427): img_in, time_text_embed.timestep_embedder.linear_1/2,
 * modulation.1, norm_out.linear, proj_out, and txt_in.text_norm / in_layer /
 * out_layer when txt_in.in_layer.weight exists (:406-411). */
int qimm_gguf_model_tensors(const qimm_gguf *g, qimm_model_tensors *out, char *err, size_t err_len);

#ifdef __cplusplus
}
#endif
#endif /* QIMM_H */
