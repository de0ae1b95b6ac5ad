// Kernels of the denoising step around the blocks (the transformer's outer
// forward and the sampler), all in f32:
//   linear_f32: the bias-free global linears (img_in, the timestep embedder,
//     modulation.1, norm_out.linear, proj_out, txt_in) over f32 weights,
//     src/quantized_transformer.rs:14-33, 43-54, 56-81, 213-228, 288-310;
//   rows_rmsnorm: txt_in's ZeroCenterRMSNorm (weight + 1 applied at upload);
//   rows_ln_scale: norm_out = LayerNorm(x) * (1 + scale) (:300-309);
//   euler: FlowMatchEuler::step (src/scheduler.rs:54-66);
//   cfg: neg + scale * (cond - neg) (src/pipeline.rs:180-186).
// These run a few times per step (about 0.3% of its FLOPs next to 32 blocks),
// so they favour exactness: weights are dequantized to f32 once at upload and
// accumulation is f32, as the reference's F32 matmuls.
#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

constexpr int LT = 64;  // output tile (rows x columns) per workgroup
constexpr int LK = 32;  // k chunk staged through LDS
constexpr int LP = LT + 4;

__device__ __forceinline__ float act(float v, int a) {
    if (a == ACT_SILU) return v / (1.0f + expf(-v));
    if (a == ACT_GELU_TANH) {
        const float c = 0.7978845608028654f;  // sqrt(2 / pi)
        return 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
    }
    return v;
}

// y[m, n] = sum_k act(x[m, k]) * w[n, k]. 256 threads, each a 4 x 4 block of
// the 64 x 64 tile; x and w chunks are stored k-major in LDS so the inner loop
// reads 4 consecutive rows / columns per thread.
__global__ __launch_bounds__(256) void linear_f32_kernel(const float *__restrict__ x, int64_t ldx,
                                                         const float *__restrict__ w, int64_t M, int64_t N,
                                                         int64_t K, int a, float *__restrict__ y, int64_t ldy) {
    __shared__ float xs[LK][LP];
    __shared__ float ws[LK][LP];
    const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
    const int64_t m0 = (int64_t)blockIdx.y * LT, n0 = (int64_t)blockIdx.x * LT;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < K; k0 += LK) {
        // 64 rows x 32 k of each operand: 8 values per thread, k fastest
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int idx = t + 256 * e, r = idx >> 5, kk = idx & 31;
            const int64_t k = k0 + kk;
            const int64_t m = m0 + r, n = n0 + r;
            xs[kk][r] = (m < M && k < K) ? act(x[m * ldx + k], a) : 0.f;
            ws[kk][r] = (n < N && k < K) ? w[n * K + k] : 0.f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < LK; kk++) {
            const float4 av = *(const float4 *)&xs[kk][4 * ty];
            const float4 bv = *(const float4 *)&ws[kk][4 * tx];
            const float ar[4] = {av.x, av.y, av.z, av.w}, br[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(ar[i], br[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t m = m0 + 4 * ty + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t n = n0 + 4 * tx + j;
            if (n < N) y[m * ldy + n] = acc[i][j];
        }
    }
}

// one 256-thread workgroup per row: block sum of v over the row
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// y = x / sqrt(mean(x^2) + eps) * w   (candle_nn::RmsNorm)
__global__ __launch_bounds__(256) void rows_rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                           int64_t D, float eps, float *__restrict__ y) {
    __shared__ float red[4];
    const float *xr = x + (int64_t)blockIdx.x * D;
    float *yr = y + (int64_t)blockIdx.x * D;
    float ss = 0.f;
    for (int64_t i = threadIdx.x; i < D; i += 256) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    for (int64_t i = threadIdx.x; i < D; i += 256) yr[i] = xr[i] * r * w[i];
}

// y = (x - mean) / sqrt(var + eps) * (1 + scale[row / rows_per])   (two-pass variance)
__global__ __launch_bounds__(256) void rows_ln_scale_kernel(const float *__restrict__ x,
                                                            const float *__restrict__ scale, int64_t D,
                                                            int64_t rows_per, float eps, float *__restrict__ y) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float *xr = x + row * D;
    const float *sr = scale + (row / rows_per) * D;
    float *yr = y + row * D;
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < D; i += 256) s += xr[i];
    const float mean = block_sum(s, red) / (float)D;
    float v = 0.f;
    for (int64_t i = threadIdx.x; i < D; i += 256) {
        const float d = xr[i] - mean;
        v += d * d;
    }
    const float rstd = 1.0f / sqrtf(block_sum(v, red) / (float)D + eps);
    for (int64_t i = threadIdx.x; i < D; i += 256) yr[i] = (xr[i] - mean) * rstd * (1.0f + sr[i]);
}

__global__ void euler_kernel(float *__restrict__ x, const float *__restrict__ v, int64_t n, float dt) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + v[i] * dt;
}

__global__ void cfg_kernel(const float *__restrict__ cond, const float *__restrict__ neg, int64_t n, float s,
                           float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = neg[i] + (cond[i] - neg[i]) * s;
}

unsigned grid1(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_linear_f32(const float *x, int64_t ldx, const float *w, int64_t m, int64_t n, int64_t k, int act_in,
                             float *y, int64_t ldy, hipStream_t stream) {
    if (m <= 0 || n <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n + LT - 1) / LT), (unsigned)((m + LT - 1) / LT));
    linear_f32_kernel<<<grid, dim3(256), 0, stream>>>(x, ldx, w, m, n, k, act_in, y, ldy);
    return hipGetLastError();
}

hipError_t launch_rows_rmsnorm(const float *x, const float *w, int64_t rows, int64_t d, float eps, float *y,
                               hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    rows_rmsnorm_kernel<<<dim3((unsigned)rows), dim3(256), 0, stream>>>(x, w, d, eps, y);
    return hipGetLastError();
}

hipError_t launch_rows_ln_scale(const float *x, const float *scale, int64_t rows, int64_t d, int64_t rows_per,
                                float eps, float *y, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    rows_ln_scale_kernel<<<dim3((unsigned)rows), dim3(256), 0, stream>>>(x, scale, d, rows_per, eps, y);
    return hipGetLastError();
}

hipError_t launch_euler(float *x, const float *v, int64_t n, float dt, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    euler_kernel<<<dim3(grid1(n)), dim3(256), 0, stream>>>(x, v, n, dt);
    return hipGetLastError();
}

hipError_t launch_cfg(const float *cond, const float *neg, int64_t n, float scale, float *out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    cfg_kernel<<<dim3(grid1(n)), dim3(256), 0, stream>>>(cond, neg, n, scale, out);
    return hipGetLastError();
}

}  // namespace qimm
