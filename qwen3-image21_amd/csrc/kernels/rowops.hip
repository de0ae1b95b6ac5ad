// Memory-bound helpers of the block step on gfx950: exact GGUF dequant,
// adaLN modulation prep, LayerNorm*(1+scale) to bf16, per-head RmsNorm+RoPE
// prep for standalone attention inputs, and the bf16 [S,D] <-> [D,S]
// transpose used by the prefix cache.
#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

// ---- exact dequantization (QTensor::dequantize, src/gguf_loader.rs:35-38) ----
// One thread per 32 output values. All scale products are exact in f32, so
// the only rounding is Q4_K's final subtraction, as on the CPU.

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

__device__ void q4k_sc_m(const uint8_t *s, int j, float &sc, float &mn) {
    uint32_t a, b;
    if (j < 4) {
        a = s[j] & 63u;
        b = s[j + 4] & 63u;
    } else {
        a = (s[j + 4] & 0xFu) | ((uint32_t)(s[j - 4] >> 6) << 4);
        b = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
    sc = (float)a;
    mn = (float)b;
}

__global__ void dequant_kernel(int type, const uint8_t *__restrict__ src, int64_t ngroups,
                               float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= ngroups) return;
    float *o = out + i * 32;
    if (type == 8) {  // Q8_0: 34 B = f16 d + 32 x i8
        const uint8_t *b = src + i * 34;
        const float d = f16_bits_to_f32(ld_u16(b));
        for (int l = 0; l < 32; l++) o[l] = (float)(int8_t)b[2 + l] * d;
    } else if (type == 12) {  // Q4_K: 144 B
        const uint8_t *b = src + (i >> 3) * 144;
        const int j = (int)(i & 7), c = j >> 1;
        const float d = f16_bits_to_f32(ld_u16(b)), dmin = f16_bits_to_f32(ld_u16(b + 2));
        float sc, mn;
        q4k_sc_m(b + 4, j, sc, mn);
        const float ds = d * sc, dm = dmin * mn;
        const uint8_t *qs = b + 16 + 32 * c;
        for (int l = 0; l < 32; l++) {
            const uint32_t q = (j & 1) ? (qs[l] >> 4) : (qs[l] & 0xFu);
            o[l] = ds * (float)q - dm;
        }
    } else if (type == 14) {  // Q6_K: 210 B = ql[128] qh[64] sc[16] d
        const uint8_t *b = src + (i >> 3) * 210;
        const int w = (int)(i & 7), hh = w >> 2, r = w & 3;
        const float d = f16_bits_to_f32(ld_u16(b + 208));
        for (int l = 0; l < 32; l++) {
            const uint8_t qlb = b[64 * hh + l + 32 * (r & 1)];
            const uint32_t lo = r < 2 ? (qlb & 0xFu) : (uint32_t)(qlb >> 4);
            const uint32_t hi = (b[128 + 32 * hh + l] >> (2 * r)) & 3u;
            const int q = (int)(lo | (hi << 4)) - 32;
            const float ds = d * (float)(int8_t)b[192 + 8 * hh + (32 * r + l) / 16];
            o[l] = ds * (float)q;
        }
    } else if (type == 0) {
        const float *s = (const float *)src + i * 32;
        for (int l = 0; l < 32; l++) o[l] = s[l];
    } else if (type == 1) {
        const uint16_t *s = (const uint16_t *)src + i * 32;
        for (int l = 0; l < 32; l++) o[l] = f16_bits_to_f32(s[l]);
    } else {  // 30: BF16
        const uint16_t *s = (const uint16_t *)src + i * 32;
        for (int l = 0; l < 32; l++) o[l] = bf16_bits_to_f32(s[l]);
    }
}

// ---- adaLN modulation rows (src/quantized_transformer.rs:259-282) ----
// prepared element i of rows [r][4h]: 1 + scale1 | tanh(gate1) | 1 + scale2 | tanh(gate2)
__device__ __forceinline__ float mod_prep_value(const float *__restrict__ mod, int64_t i, int64_t hidden) {
    const int64_t part = (i % (4 * hidden)) / hidden;
    const float v = mod[i];
    return (part & 1) ? tanhf(v) : v + 1.0f;
}

// ---- LayerNorm (weight 1, bias 0, eps 1e-6) * (1 + scale) -> bf16 ----
// src/quantized_transformer.rs:231-237, 267-269, 276-278. One 256-thread
// workgroup per row; the row stays in registers for the two-pass variance.
// With QBLK 32 or 256 the output is the bf16 operand of candle's activation
// quantization instead (quant_act4): thread t holds chunk t + 256 i, so for
// iteration i wave w holds the 256 consecutive values of block 4 i + w (hidden
// is a multiple of 256: whole waves are in or out of the row).
constexpr int LN_MAXV = (int)(LN_MAX_HIDDEN / 4 / 256);  // float4 chunks per thread

// NI > 0: hidden == 1024 NI, every thread holds NI chunks (no guards, so the
// NI roundings of a thread are independent straight-line code the scheduler
// interleaves); NI == 0: any hidden, guarded chunks.
// With `prep` set, scale points at the raw modulation rows (the scale part, 1
// added here) and the workgroups also write the prepared rows of all of them
// to prep (grid-strided), which the block's later
// stages read.
template <int QBLK, int NI>
__global__ __launch_bounds__(256) void ln_mod_kernel(const float *__restrict__ x, int64_t hidden,
                                                     const float *__restrict__ scale, int64_t stride,
                                                     int64_t rows_per, uint16_t *__restrict__ out,
                                                     const float *__restrict__ mod, float *__restrict__ prep,
                                                     int64_t prep_n) {
    __shared__ float red[8];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    if (prep)
        for (int64_t i = row * 256 + tid; i < prep_n; i += (int64_t)gridDim.x * 256)
            prep[i] = mod_prep_value(mod, i, hidden);
    const float *xr = x + row * hidden;
    const int nv = NI > 0 ? 256 * NI : (int)(hidden / 4);
    // the modulation row is loaded with x, so its latency overlaps the row's
    const float *sc = scale + (row / rows_per) * stride;
    f32x4 v[NI > 0 ? NI : LN_MAXV], sv[NI > 0 ? NI : LN_MAXV];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < (NI > 0 ? NI : LN_MAXV); i++) {
        const int c = tid + 256 * i;
        if (c < nv) {
            v[i] = *(const f32x4 *)(xr + 4 * c);
            sv[i] = *(const f32x4 *)(sc + 4 * c);
            s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
        }
    }
    if (prep) {
        // 1 + scale, the same rounding as the prepared rows
#pragma unroll
        for (int i = 0; i < (NI > 0 ? NI : LN_MAXV); i++)
#pragma unroll
            for (int e = 0; e < 4; e++) sv[i][e] = sv[i][e] + 1.0f;
    }
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)hidden;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < (NI > 0 ? NI : LN_MAXV); i++) {
        const int c = tid + 256 * i;
        if (c < nv) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float t = v[i][e] - mean;
                ss += t * t;
            }
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[4 + (tid >> 6)] = ss;
    __syncthreads();
    const float var = (red[4] + red[5] + red[6] + red[7]) / (float)hidden;
    const float rstd = 1.0f / sqrtf(var + 1e-6f);
    uint16_t *orow = out + row * hidden;
    if constexpr (NI > 0 && QBLK != 0) {
        // the NI chunks rounded together (their reductions interleave)
        f32x4 y[NI];
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) y[i][e] = (v[i][e] - mean) * rstd * sv[i][e];
        u32x2 o[NI];
        quant_act4_n<QBLK, NI>(y, o);
#pragma unroll
        for (int i = 0; i < NI; i++) *(u32x2 *)(orow + 4 * (tid + 256 * i)) = o[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < (NI > 0 ? NI : LN_MAXV); i++) {
        const int c = tid + 256 * i;
        if (c < nv) {
            const f32x4 s4 = sv[i];
            const f32x4 y{(v[i][0] - mean) * rstd * s4[0], (v[i][1] - mean) * rstd * s4[1],
                          (v[i][2] - mean) * rstd * s4[2], (v[i][3] - mean) * rstd * s4[3]};
            if constexpr (QBLK == 0)
                *(u32x2 *)(orow + 4 * c) = u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
            else
                *(u32x2 *)(orow + 4 * c) = quant_act4<QBLK>(y);
        }
    }
}

// The same for hidden == 1024 NI, RPW consecutive rows per workgroup: the
// next row's x loads are issued before the current row's reductions, so they
// are in flight while it is normalised, rounded and stored (one resident round
// of workgroups streams the rows, instead of rounds that all load, then all
// compute). The rows are straight-line code (rows past m clamped to the last
// row, which is then written again with the same values), so every wait for a
// load is exact. The modulation row is loaded again only where the row's
// changes. The same arithmetic as ln_mod_kernel.
template <int QBLK, int NI, int RPW>
__global__ __launch_bounds__(256) void ln_mod_run_kernel(const float *__restrict__ x, int64_t m,
                                                         const float *__restrict__ scale, int64_t stride,
                                                         int64_t rows_per, uint16_t *__restrict__ out,
                                                         const float *__restrict__ mod, float *__restrict__ prep,
                                                         int64_t prep_n) {
    constexpr int64_t hidden = 1024 * NI;
    __shared__ float red[8];
    const int tid = threadIdx.x;
    if (prep)
        for (int64_t i = (int64_t)blockIdx.x * 256 + tid; i < prep_n; i += (int64_t)gridDim.x * 256)
            prep[i] = mod_prep_value(mod, i, hidden);
    const int64_t r0 = (int64_t)blockIdx.x * RPW;
    f32x4 v[NI], sv[NI];
    auto load_scale = [&](int64_t sr) __attribute__((always_inline)) {
        const float *sc = scale + sr * stride;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            sv[i] = *(const f32x4 *)(sc + 4 * (tid + 256 * i));
            // 1 + scale, the same rounding as the prepared rows
            if (prep)
#pragma unroll
                for (int e = 0; e < 4; e++) sv[i][e] = sv[i][e] + 1.0f;
        }
    };
    int64_t srow = min(r0, m - 1) / rows_per;
#pragma unroll
    for (int i = 0; i < NI; i++) v[i] = *(const f32x4 *)(x + min(r0, m - 1) * hidden + 4 * (tid + 256 * i));
    load_scale(srow);
#pragma unroll
    for (int k = 0; k < RPW; k++) {
        const int64_t row = min(r0 + k, m - 1), next = min(r0 + k + 1, m - 1);
        f32x4 vn[NI];
        if (k + 1 < RPW)
#pragma unroll
            for (int i = 0; i < NI; i++) vn[i] = *(const f32x4 *)(x + next * hidden + 4 * (tid + 256 * i));
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NI; i++) s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
        s = wave_sum(s);
        if ((tid & 63) == 0) red[tid >> 6] = s;
        __syncthreads();
        const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)hidden;
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float t = v[i][e] - mean;
                ss += t * t;
            }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[4 + (tid >> 6)] = ss;
        __syncthreads();
        const float var = (red[4] + red[5] + red[6] + red[7]) / (float)hidden;
        const float rstd = 1.0f / sqrtf(var + 1e-6f);
        f32x4 y[NI];
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) y[i][e] = (v[i][e] - mean) * rstd * sv[i][e];
        uint16_t *orow = out + row * hidden;
        if constexpr (QBLK == 0) {
#pragma unroll
            for (int i = 0; i < NI; i++)
                *(u32x2 *)(orow + 4 * (tid + 256 * i)) = u32x2{pack_bf16x2(y[i][0], y[i][1]), pack_bf16x2(y[i][2], y[i][3])};
        } else {
            u32x2 o[NI];
            quant_act4_n<QBLK, NI>(y, o);
#pragma unroll
            for (int i = 0; i < NI; i++) *(u32x2 *)(orow + 4 * (tid + 256 * i)) = o[i];
        }
        if (k + 1 < RPW) {
#pragma unroll
            for (int i = 0; i < NI; i++) v[i] = vn[i];
            const int64_t sr = next / rows_per;
            if (sr != srow) {
                srow = sr;
                load_scale(sr);
            }
        }
    }
}

// ---- candle's activation quantization of f32 rows (QMatMul::forward's
// quantize step, src/quantized_transformer.rs:19-29 -> candle-core 0.11
// BlockQ8_0 / BlockQ8K::from_float) to the bf16 operands bf16(d * q) ----
// One wave per QR_CH x 256 values of a row (four per lane and chunk, all
// chunks' loads in flight before the first rounding): each chunk a Q8_K
// block or eight Q8_0 blocks. Rows of k values (k % 256 == 0 for Q8_K,
// k % 32 == 0 for Q8_0); chunks past the row end are zeros and not stored
// (whole waves for Q8_K, whole 8-lane groups for Q8_0).
constexpr int QR_CH = 4;

template <int QBLK>
__global__ __launch_bounds__(256) void quant_rows_kernel(const float *__restrict__ x, int64_t ldx, int64_t m,
                                                         int64_t k, uint16_t *__restrict__ out, int64_t ldo) {
    const int64_t wpr = (k + 256 * QR_CH - 1) / (256 * QR_CH);
    const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= m * wpr) return;  // whole waves
    const int64_t row = gw / wpr, c0 = (gw % wpr) * (256 * QR_CH) + 4 * (threadIdx.x & 63);
    f32x4 v[QR_CH];
#pragma unroll
    for (int j = 0; j < QR_CH; j++) {
        const int64_t c = c0 + 256 * j;
        v[j] = c < k ? *(const f32x4 *)(x + row * ldx + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    u32x2 r[QR_CH];
    quant_act4_n<QBLK, QR_CH>(v, r);
#pragma unroll
    for (int j = 0; j < QR_CH; j++) {
        const int64_t c = c0 + 256 * j;
        if (c < k) *(u32x2 *)(out + row * ldo + c) = r[j];
    }
}

// ---- the largest key norm of a cache layer (the attention's score bound) ----
// Two passes, no atomics: workgroup g takes rows g, g + G, ... (16 lanes per
// row of 128 bf16, 16 rows per workgroup step) and writes its maximum; one
// workgroup then reduces the G partial maxima.
__global__ __launch_bounds__(256) void row_norm_part_kernel(const uint16_t *__restrict__ k, int64_t rows,
                                                            float *__restrict__ part) {
    __shared__ float red[16];
    const int tid = threadIdx.x, sub = tid & 15;
    float best = 0.f;
    for (int64_t r = (int64_t)blockIdx.x * 16 + (tid >> 4); r < rows; r += (int64_t)gridDim.x * 16) {
        const u32x4 v = *(const u32x4 *)(k + r * 128 + sub * 8);
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float a = bf16_bits_to_f32(v[i] & 0xffffu), b = bf16_bits_to_f32(v[i] >> 16);
            ss += a * a + b * b;
        }
        best = fmaxf(best, sqrtf(group_sum(ss, 16)));
    }
    if (sub == 0) red[tid >> 4] = best;  // the 16 lanes of a row group hold the same value
    __syncthreads();
    if (tid == 0) {
        float m = red[0];
        for (int i = 1; i < 16; i++) m = fmaxf(m, red[i]);
        part[blockIdx.x] = m;
    }
}

__global__ __launch_bounds__(256) void max_reduce_kernel(const float *__restrict__ part, int n,
                                                         float *__restrict__ out) {
    __shared__ float red[4];
    float m = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, part[i]);
    m = max_wave(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) out[0] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ---- per-head RmsNorm + RoPE prep (src/quantized_transformer.rs:137-142) ----
// x [B,S,H,128] f32. mode 0: out [B,H,S,128] bf16 after norm (w) and RoPE
// (pe [S,128]); mode 1 (values): out = vt [B,H,128,S] bf16, no norm.
__global__ __launch_bounds__(256) void qk_prep_kernel(const float *__restrict__ x, int64_t B, int64_t S,
                                                      int64_t H, const float *__restrict__ w,
                                                      const float *__restrict__ pe,
                                                      uint16_t *__restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t row = gid >> 4;  // (b, s, h) row of 128
    const int cg = (int)(gid & 15) * 8;
    const bool ok = row < B * S * H;
    const int64_t rr = ok ? row : 0;
    const float *xr = x + rr * 128 + cg;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = xr[i];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) ss += v[i] * v[i];
    ss = group_sum(ss, 16);
    if (!ok) return;
    const float rs = 1.0f / sqrtf(ss * (1.0f / 128.0f) + 1e-6f);
    const int64_t h = rr % H, s = (rr / H) % S, b = rr / (H * S);
    const float *pr = pe + s * 128 + cg;
    uint32_t pk[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float x0 = v[2 * i] * rs * w[cg + 2 * i], x1 = v[2 * i + 1] * rs * w[cg + 2 * i + 1];
        const float c = pr[2 * i], sn = pr[2 * i + 1];
        pk[i] = pack_bf16x2(x0 * c - x1 * sn, x0 * sn + x1 * c);
    }
    *(u32x4 *)(out + ((b * H + h) * S + s) * 128 + cg) = u32x4{pk[0], pk[1], pk[2], pk[3]};
}

__global__ void v_prep_kernel(const float *__restrict__ x, int64_t B, int64_t S, int64_t H,
                              uint16_t *__restrict__ vt) {
    // element (b, h, d, s) with s fastest: coalesced writes, strided reads
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * H * 128 * S) return;
    const int64_t s = i % S, d = (i / S) % 128, h = (i / (S * 128)) % H, b = i / (S * 128 * H);
    vt[i] = (uint16_t)(pack_bf16x2(x[((b * S + s) * H + h) * 128 + d], 0.f) & 0xffffu);
}

// ---- [BH][S][128] <-> [BH][128][S] bf16 via 64x64 LDS tiles ----
__global__ __launch_bounds__(256) void transpose_sd_kernel(const uint16_t *__restrict__ in, int64_t S,
                                                           uint16_t *__restrict__ out, int inverse) {
    __shared__ uint16_t tile[64][65];
    const int64_t bh = blockIdx.z;
    const int64_t s0 = (int64_t)blockIdx.x * 64, d0 = (int64_t)blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    // source rows: forward reads [S][128] (row = s), inverse reads [128][S] (row = d)
    for (int r = ty; r < 64; r += 4) {
        if (!inverse) {
            const int64_t s = s0 + r, d = d0 + tx;
            tile[r][tx] = s < S ? in[(bh * S + s) * 128 + d] : (uint16_t)0;
        } else {
            const int64_t d = d0 + r, s = s0 + tx;
            tile[tx][r] = s < S ? in[(bh * 128 + d) * S + s] : (uint16_t)0;
        }
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        if (!inverse) {
            const int64_t d = d0 + r, s = s0 + tx;
            if (s < S) out[(bh * 128 + d) * S + s] = tile[tx][r];
        } else {
            const int64_t s = s0 + r, d = d0 + tx;
            if (s < S) out[(bh * S + s) * 128 + d] = tile[r][tx];
        }
    }
}

}  // namespace

hipError_t launch_dequant(int ggml_type, const uint8_t *src, int64_t n, float *out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t groups = n / 32;
    dequant_kernel<<<dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, stream>>>(ggml_type, src, groups, out);
    return hipGetLastError();
}

hipError_t launch_ln_mod(const float *x, int64_t m, int64_t hidden, const float *scale, int64_t stride,
                         int64_t rows_per, uint16_t *out, hipStream_t stream, int qblk, float *prep,
                         int64_t prep_rows) {
    if (m <= 0) return hipSuccess;
    if (hidden > LN_MAX_HIDDEN || hidden % 4) return hipErrorInvalidValue;
    if (qblk && hidden % 256) return hipErrorInvalidValue;
    if (qblk != 0 && qblk != 32 && qblk != 256) return hipErrorInvalidValue;
    const dim3 block(256);
    // hidden = 1024 n with 16 to 20 rows per CU: runs of 4 rows per workgroup,
    // 4 or 5 workgroups per CU, all resident at once (at most 88 VGPRs
    // allocated: 5 waves per SIMD). More rows would leave a short second round.
    const int64_t cus = device_cu_count();
    const bool runs = cus > 0 && m >= 16 * cus && m <= 20 * cus;
    auto go = [&](auto qb, auto ni) {
        constexpr int QB = decltype(qb)::value, NI = decltype(ni)::value;
        const int64_t prep_n = prep ? prep_rows * 4 * hidden : 0;
        if constexpr (NI > 0)
            if (runs) {
                ln_mod_run_kernel<QB, NI, 4><<<dim3((unsigned)((m + 3) / 4)), block, 0, stream>>>(
                    x, m, scale, stride, rows_per, out, scale, prep, prep_n);
                return;
            }
        ln_mod_kernel<QB, NI><<<dim3((unsigned)m), block, 0, stream>>>(x, hidden, scale, stride, rows_per, out,
                                                                      scale, prep, prep_n);
    };
    using Q0 = std::integral_constant<int, 0>;
    using Q32 = std::integral_constant<int, 32>;
    using Q256 = std::integral_constant<int, 256>;
    auto by_q = [&](auto ni) {
        if (qblk == 0) go(Q0{}, ni);
        else if (qblk == 32) go(Q32{}, ni);
        else go(Q256{}, ni);
    };
    switch (hidden % 1024 ? 0 : hidden / 1024) {
    case 3: by_q(std::integral_constant<int, 3>{}); break;
    case 4: by_q(std::integral_constant<int, 4>{}); break;
    default: by_q(std::integral_constant<int, 0>{}); break;
    }
    return hipGetLastError();
}

hipError_t launch_quant_rows(const float *x, int64_t ldx, int64_t m, int64_t k, int qblk, uint16_t *out, int64_t ldo,
                             hipStream_t stream) {
    if (m <= 0 || k <= 0) return hipSuccess;
    if ((qblk != 32 && qblk != 256) || k % qblk || k % 4 || ldx % 4 || ldo % 4 || ldx < k || ldo < k)
        return hipErrorInvalidValue;
    const int64_t waves = m * ((k + 256 * QR_CH - 1) / (256 * QR_CH));
    const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
    if (qblk == 32)
        quant_rows_kernel<32><<<grid, block, 0, stream>>>(x, ldx, m, k, out, ldo);
    else
        quant_rows_kernel<256><<<grid, block, 0, stream>>>(x, ldx, m, k, out, ldo);
    return hipGetLastError();
}

hipError_t launch_row_norm_max(const uint16_t *k, int64_t rows, float *part, float *out_dev, hipStream_t stream) {
    const int64_t g = std::min<int64_t>(QK_NORM_PARTS, std::max<int64_t>(1, (rows + 15) / 16));
    row_norm_part_kernel<<<dim3((unsigned)g), dim3(256), 0, stream>>>(k, rows, part);
    max_reduce_kernel<<<dim3(1), dim3(256), 0, stream>>>(part, (int)g, out_dev);
    return hipGetLastError();
}

hipError_t launch_qk_prep(const float *x, int64_t b, int64_t s, int64_t h, const float *w, const float *pe,
                          int mode, uint16_t *out, hipStream_t stream) {
    const int64_t rows = b * s * h;
    if (rows <= 0) return hipSuccess;
    if (mode == 0) {
        const int64_t threads = rows * 16;
        qk_prep_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream>>>(x, b, s, h, w, pe, out);
    } else {
        const int64_t n = rows * 128;
        v_prep_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(x, b, s, h, out);
    }
    return hipGetLastError();
}

hipError_t launch_transpose_sd(const uint16_t *in, int64_t bh, int64_t s, uint16_t *out, int inverse,
                               hipStream_t stream) {
    if (bh <= 0 || s <= 0) return hipSuccess;
    dim3 grid((unsigned)((s + 63) / 64), 2u, (unsigned)bh);
    transpose_sd_kernel<<<grid, dim3(256), 0, stream>>>(in, s, out, inverse);
    return hipGetLastError();
}

}  // namespace qimm
