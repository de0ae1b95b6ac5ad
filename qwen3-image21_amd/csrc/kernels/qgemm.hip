// Dequant-GEMM for gfx950: C[M,N] = A[M,K] (bf16) x W[N,K]^T (GGUF blocks).
//
// Replaces candle's QMatMul::forward as called through Linear::forward
// (src/quantized_transformer.rs:19-33; call sites 133-135, 151, 194-199, 202).
//
// Tile 128x128x64, 256 threads = 4 waves in a 2x2 grid, each wave 64x64 as
// 2x2 v_mfma_f32_32x32x16_bf16 tiles. A is staged to LDS as bf16; W is read
// as raw quantized bytes with 128-bit loads, dequantized in registers
// (exact f32 value d*sc*q - dmin*m, then round-to-nearest-even to bf16) and
// staged to LDS next to A. Two LDS stages: the global loads for step k+1 are
// in flight while the MFMAs of step k run. The epilogue goes through LDS as
// an f32 tile so each variant (plain store, fused QKV RmsNorm+RoPE, gated
// residual, SwiGLU) writes whole rows with 128-bit stores.
#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LP = 72;                 // bf16 pitch of an A/B stage row (64 + 8 pad)
constexpr int CP = 132;                // f32 pitch of the epilogue tile row
constexpr int STAGE = 2 * 128 * LP;    // bf16 elements per stage (A rows, then B rows)
constexpr int LDS_ELEMS = 2 * STAGE;   // 73728 B

struct WRaw {
    u32x4 v[4];
    uint32_t s;
};

__device__ __forceinline__ uint32_t byte_of(const u32x4 &x, int i) {
    return (x[i >> 2] >> (8 * (i & 3))) & 0xffu;
}

// Q4_K 6-bit scale and min of sub-block j from the 12 packed bytes, which
// sit at bytes 4..15 of the block header word h (GGML layout).
__device__ __forceinline__ void q4k_sc_m(const u32x4 &h, int j, float &sc, float &mn) {
    uint32_t s, m;
    if (j < 4) {
        s = byte_of(h, 4 + j) & 63u;
        m = byte_of(h, 8 + j) & 63u;
    } else {
        s = (byte_of(h, 8 + j) & 0xFu) | ((byte_of(h, j) >> 6) << 4);
        m = (byte_of(h, 8 + j) >> 4) | ((byte_of(h, 4 + j) >> 6) << 4);
    }
    sc = (float)s;
    mn = (float)m;
}

// 4 unsigned bytes of x -> 4 floats v*ds + off, packed to 2 bf16x2 words.
__device__ __forceinline__ u32x2 cvt4(uint32_t x, float ds, float off) {
    float f0 = (float)(x & 0xffu), f1 = (float)((x >> 8) & 0xffu);
    float f2 = (float)((x >> 16) & 0xffu), f3 = (float)(x >> 24);
    return u32x2{pack_bf16x2(__builtin_fmaf(f0, ds, off), __builtin_fmaf(f1, ds, off)),
                 pack_bf16x2(__builtin_fmaf(f2, ds, off), __builtin_fmaf(f3, ds, off))};
}

// 16 codes held as bytes of a u32x4 -> 16 bf16 (two u32x4).
__device__ __forceinline__ void cvt16(const u32x4 &x, float ds, float off, u32x4 &o0, u32x4 &o1) {
    const u32x2 a = cvt4(x[0], ds, off), b = cvt4(x[1], ds, off);
    const u32x2 c = cvt4(x[2], ds, off), d = cvt4(x[3], ds, off);
    o0 = u32x4{a[0], a[1], b[0], b[1]};
    o1 = u32x4{c[0], c[1], d[0], d[1]};
}

template <int FMT>
__device__ __forceinline__ void load_w(const GemmWeight &w, int64_t n, int64_t k0, int h, WRaw &r) {
    const int64_t K = w.k;
    if constexpr (FMT == WF_Q8_0) {
        const uint8_t *p = w.q + n * K + k0 + 32 * h;
        r.v[0] = *(const u32x4 *)p;
        r.v[1] = *(const u32x4 *)(p + 16);
        r.s = w.scales[n * (K / 32) + k0 / 32 + h];
    } else if constexpr (FMT == WF_Q4_K) {
        const uint8_t *blk = q4k_block(w.q, n, k0 / 256, K / 256);
        const int c = (int)((k0 & 255) >> 6);
        r.v[0] = *(const u32x4 *)blk;
        r.v[1] = *(const u32x4 *)(blk + 16 + 32 * c + 16 * h);
    } else if constexpr (FMT == WF_Q6_K) {
        const uint8_t *blk = q6k_block(w.q, n, k0 / 256, K / 256);
        const int hh = (int)((k0 & 255) >> 7);
        r.v[0] = *(const u32x4 *)(blk + 64 * hh + 16 * h);
        r.v[1] = *(const u32x4 *)(blk + 64 * hh + 32 + 16 * h);
        r.v[2] = *(const u32x4 *)(blk + 128 + 32 * hh + 16 * h);
        r.v[3] = *(const u32x4 *)(blk + 192);
        r.s = *(const uint16_t *)(blk + 208);
    } else {
        const uint8_t *p = w.q + (n * K + k0 + 32 * h) * 2;
        r.v[0] = *(const u32x4 *)p;
        r.v[1] = *(const u32x4 *)(p + 16);
        r.v[2] = *(const u32x4 *)(p + 32);
        r.v[3] = *(const u32x4 *)(p + 48);
    }
}

// Dequantize one thread's 32 values of row n_local and store them as bf16 in
// the B stage: Q8_0/BF16 cover k in [32h, 32h+32); Q4_K/Q6_K cover
// [16h, 16h+16) and [32+16h, 32+16h+16).
template <int FMT>
__device__ __forceinline__ void store_w(uint16_t *bs, int nl, int h, int64_t k0, const WRaw &r) {
    uint16_t *row = bs + nl * LP;
    if constexpr (FMT == WF_Q8_0) {
        const float d = f16_bits_to_f32(r.s);
        const float off = -128.f * d;  // codes biased to unsigned: (q+128)*d - 128*d, exact
        u32x4 a = r.v[0] ^ 0x80808080u, b = r.v[1] ^ 0x80808080u;
        u32x4 o0, o1, o2, o3;
        cvt16(a, d, off, o0, o1);
        cvt16(b, d, off, o2, o3);
        *(u32x4 *)(row + 32 * h) = o0;
        *(u32x4 *)(row + 32 * h + 8) = o1;
        *(u32x4 *)(row + 32 * h + 16) = o2;
        *(u32x4 *)(row + 32 * h + 24) = o3;
    } else if constexpr (FMT == WF_Q4_K) {
        const int c = (int)((k0 & 255) >> 6);
        const float d = f16_bits_to_f32(r.v[0][0] & 0xffffu);
        const float dmin = f16_bits_to_f32(r.v[0][0] >> 16);
        float sc0, m0, sc1, m1;
        q4k_sc_m(r.v[0], 2 * c, sc0, m0);
        q4k_sc_m(r.v[0], 2 * c + 1, sc1, m1);
        const float ds0 = d * sc0, dm0 = dmin * m0, ds1 = d * sc1, dm1 = dmin * m1;
        u32x4 lo = r.v[1] & 0x0F0F0F0Fu, hi = (r.v[1] >> 4) & 0x0F0F0F0Fu;
        u32x4 o0, o1, o2, o3;
        cvt16(lo, ds0, -dm0, o0, o1);
        cvt16(hi, ds1, -dm1, o2, o3);
        *(u32x4 *)(row + 16 * h) = o0;
        *(u32x4 *)(row + 16 * h + 8) = o1;
        *(u32x4 *)(row + 32 + 16 * h) = o2;
        *(u32x4 *)(row + 32 + 16 * h + 8) = o3;
    } else if constexpr (FMT == WF_Q6_K) {
        const int hh = (int)((k0 & 255) >> 7), o = (int)((k0 & 127) >> 6);
        const float d = f16_bits_to_f32(r.s);
        const int ra = 2 * o, rb = 2 * o + 1;
        const float sa = (float)(int8_t)byte_of(r.v[3], 8 * hh + 4 * o + h);
        const float sb = (float)(int8_t)byte_of(r.v[3], 8 * hh + 4 * o + 2 + h);
        const float dsa = d * sa, dsb = d * sb;
        u32x4 la = o ? ((r.v[0] >> 4) & 0x0F0F0F0Fu) : (r.v[0] & 0x0F0F0F0Fu);
        u32x4 lb = o ? ((r.v[1] >> 4) & 0x0F0F0F0Fu) : (r.v[1] & 0x0F0F0F0Fu);
        u32x4 qa = la | (((r.v[2] >> (2 * ra)) & 0x03030303u) << 4);
        u32x4 qb = lb | (((r.v[2] >> (2 * rb)) & 0x03030303u) << 4);
        u32x4 o0, o1, o2, o3;
        cvt16(qa, dsa, -32.f * dsa, o0, o1);  // (q+32)*ds - 32*ds, exact
        cvt16(qb, dsb, -32.f * dsb, o2, o3);
        *(u32x4 *)(row + 16 * h) = o0;
        *(u32x4 *)(row + 16 * h + 8) = o1;
        *(u32x4 *)(row + 32 + 16 * h) = o2;
        *(u32x4 *)(row + 32 + 16 * h + 8) = o3;
    } else {
        *(u32x4 *)(row + 32 * h) = r.v[0];
        *(u32x4 *)(row + 32 * h + 8) = r.v[1];
        *(u32x4 *)(row + 32 * h + 16) = r.v[2];
        *(u32x4 *)(row + 32 * h + 24) = r.v[3];
    }
}

// silu with the hardware reciprocal (about 1 ulp) instead of an IEEE divide
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

template <int FMT, int EPI>
__global__ __launch_bounds__(256, 2) void qgemm_kernel(const uint16_t *__restrict__ A, int64_t M,
                                                       int64_t lda, GemmWeight w, EpiParams ep) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int64_t K = w.k;
    // split K (gridDim.z > 1): this workgroup covers k steps [kt0, kt0 + KT)
    // and writes its f32 partial sums to slice blockIdx.z of ep.out
    const int KT = (int)(K / BK / gridDim.z);
    const int kt0 = (int)blockIdx.z * KT;

    // loader roles
    const int a_row = tid >> 3, a_kc = (tid & 7) * 8;
    const int w_nl = tid >> 1, w_h = tid & 1;

    u32x4 ra[4];
    WRaw rw;

    // rows past M are clamped to row M-1: they only feed unwritten output rows
    auto load_a = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t gm = min(m0 + a_row + 32 * i, M - 1);
            ra[i] = *(const u32x4 *)(A + gm * lda + k0 + a_kc);
        }
    };
    auto store_a = [&](uint16_t *as) {
#pragma unroll
        for (int i = 0; i < 4; i++) *(u32x4 *)(as + (a_row + 32 * i) * LP + a_kc) = ra[i];
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    load_a((int64_t)kt0 * BK);
    load_w<FMT>(w, n0 + w_nl, (int64_t)kt0 * BK, w_h, rw);
    store_a(lds);
    store_w<FMT>(lds + 128 * LP, w_nl, w_h, (int64_t)kt0 * BK, rw);
    __syncthreads();

    for (int kt = kt0; kt < kt0 + KT; kt++) {
        const int cur = (kt - kt0) & 1;
        const bool more = kt + 1 < kt0 + KT;
        if (more) {
            load_a((int64_t)(kt + 1) * BK);
            load_w<FMT>(w, n0 + w_nl, (int64_t)(kt + 1) * BK, w_h, rw);
        }
        const uint16_t *as = lds + cur * STAGE;
        const uint16_t *bs = as + 128 * LP;
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            bf16x8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                af[i] = *(const bf16x8 *)(as + (wm * 64 + i * 32 + (lane & 31)) * LP + kk * 16 + (lane >> 5) * 8);
#pragma unroll
            for (int j = 0; j < 2; j++)
                bf[j] = *(const bf16x8 *)(bs + (wn * 64 + j * 32 + (lane & 31)) * LP + kk * 16 + (lane >> 5) * 8);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            uint16_t *an = lds + (cur ^ 1) * STAGE;
            store_a(an);
            store_w<FMT>(an + 128 * LP, w_nl, w_h, (int64_t)(kt + 1) * BK, rw);
        }
        __syncthreads();
    }

    // accumulators -> f32 tile in LDS
    float *cs = (float *)lds;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int col = wn * 64 + j * 32 + (lane & 31);
                cs[row * CP + col] = acc[i][j][r];
            }
    __syncthreads();

    const int64_t N = w.n;
    if constexpr (EPI == EPI_F32 || EPI == EPI_BF16 || EPI == EPI_RESID) {
        const int cg = (tid & 15) * 8;
#pragma unroll 1
        for (int pass = 0; pass < 8; pass++) {
            const int row = pass * 16 + (tid >> 4);
            const int64_t m = m0 + row;
            if (m >= M) continue;
            f32x4 v0 = *(const f32x4 *)(cs + row * CP + cg);
            f32x4 v1 = *(const f32x4 *)(cs + row * CP + cg + 4);
            if constexpr (EPI == EPI_F32) {
                float *o = (float *)ep.out + (int64_t)blockIdx.z * M * ep.ldo + m * ep.ldo + n0 + cg;
                *(f32x4 *)o = v0;
                *(f32x4 *)(o + 4) = v1;
            } else if constexpr (EPI == EPI_BF16) {
                u32x4 pk{pack_bf16x2(v0[0], v0[1]), pack_bf16x2(v0[2], v0[3]),
                         pack_bf16x2(v1[0], v1[1]), pack_bf16x2(v1[2], v1[3])};
                *(u32x4 *)((uint16_t *)ep.out + m * ep.ldo + n0 + cg) = pk;
            } else {
                const int64_t idx = m * N + n0 + cg;
                const float *g = ep.gvec + (m / ep.g_rows_per) * ep.g_stride + n0 + cg;
                f32x4 x0 = *(const f32x4 *)(ep.x_in + idx), x1 = *(const f32x4 *)(ep.x_in + idx + 4);
                f32x4 g0 = *(const f32x4 *)g, g1 = *(const f32x4 *)(g + 4);
                *(f32x4 *)(ep.x_out + idx) = x0 + g0 * v0;
                *(f32x4 *)(ep.x_out + idx + 4) = x1 + g1 * v1;
            }
        }
    } else if constexpr (EPI == EPI_SWIGLU) {
        const int j0 = (tid & 7) * 8;
#pragma unroll 1
        for (int pass = 0; pass < 4; pass++) {
            const int row = pass * 32 + (tid >> 3);
            const int64_t m = m0 + row;
            if (m >= M) continue;
            const float *cr = cs + row * CP;
            uint32_t pk[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float h0 = silu(cr[j0 + 2 * i]) * cr[64 + j0 + 2 * i];
                float h1 = silu(cr[j0 + 2 * i + 1]) * cr[64 + j0 + 2 * i + 1];
                pk[i] = pack_bf16x2(h0, h1);
            }
            *(u32x4 *)(ep.hmid + m * ep.ldh + n0 / 2 + j0) = u32x4{pk[0], pk[1], pk[2], pk[3]};
        }
    } else {  // EPI_QKV
        const int64_t nb = n0 + ep.n_offset;
        const int sec = (int)(nb / ep.hidden);
        const int64_t head = (nb % ep.hidden) / 128;
        const int64_t S = ep.seq, H = ep.heads;
        if (sec < 2) {
            const float *nw = sec == 0 ? ep.norm_q : ep.norm_k;
            uint16_t *dst = sec == 0 ? ep.q : ep.k;
            const float osc = sec == 0 ? ep.q_scale : 1.0f;
            const int cg = (tid & 15) * 8;
            float wv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) wv[i] = nw[cg + i];
#pragma unroll 1
            for (int pass = 0; pass < 8; pass++) {
                const int row = pass * 16 + (tid >> 4);
                const int64_t m = m0 + row;
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = cs[row * CP + cg + i];
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) ss += v[i] * v[i];
                ss = group_sum(ss, 16);
                const float rs = 1.0f / sqrtf(ss * (1.0f / 128.0f) + 1e-6f);
                if (m >= M) continue;
                const int64_t b = m / S, s = m % S;
                const float *pr = ep.pe + s * 128 + cg;
                uint32_t pk[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float x0 = v[2 * i] * rs * wv[2 * i];
                    const float x1 = v[2 * i + 1] * rs * wv[2 * i + 1];
                    const float c = pr[2 * i], sn = pr[2 * i + 1];
                    pk[i] = pack_bf16x2((x0 * c - x1 * sn) * osc, (x0 * sn + x1 * c) * osc);
                }
                *(u32x4 *)(dst + ((b * H + head) * S + s) * 128 + cg) = u32x4{pk[0], pk[1], pk[2], pk[3]};
            }
        } else {
            const int d = tid & 127;
            const int rbase = (tid >> 7) * 64;
#pragma unroll 1
            for (int g = 0; g < 8; g++) {
                const int r0 = rbase + 8 * g;
                const int64_t m = m0 + r0;
                if (m >= M) break;
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = cs[(r0 + i) * CP + d];
                const int64_t b = m / S, s = m % S;
                if ((S & 7) == 0 && (s & 7) == 0 && m + 7 < M) {
                    u32x4 pk{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                             pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
                    *(u32x4 *)(ep.vt + ((b * H + head) * 128 + d) * S + s) = pk;
                } else {
                    for (int i = 0; i < 8; i++) {
                        const int64_t mi = m + i;
                        if (mi >= M) break;
                        const int64_t bi = mi / S, si = mi % S;
                        ep.vt[((bi * H + head) * 128 + d) * S + si] =
                            (uint16_t)(pack_bf16x2(v[i], 0.f) & 0xffffu);
                    }
                }
            }
            if (ep.v_bhsd) {
                const int cg = (tid & 15) * 8;
#pragma unroll 1
                for (int pass = 0; pass < 8; pass++) {
                    const int row = pass * 16 + (tid >> 4);
                    const int64_t m = m0 + row;
                    if (m >= M) continue;
                    const int64_t b = m / S, s = m % S;
                    const float *cr = cs + row * CP + cg;
                    u32x4 pk{pack_bf16x2(cr[0], cr[1]), pack_bf16x2(cr[2], cr[3]),
                             pack_bf16x2(cr[4], cr[5]), pack_bf16x2(cr[6], cr[7])};
                    *(u32x4 *)(ep.v_bhsd + ((b * H + head) * S + s) * 128 + cg) = pk;
                }
            }
        }
    }
}

template <int FMT>
hipError_t launch_fmt(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                      const EpiParams &ep, hipStream_t stream, int splits = 1) {
    dim3 grid((unsigned)(w.n / BN), (unsigned)((m + BM - 1) / BM), (unsigned)splits);
    dim3 block(256);
    switch (epi) {
    case EPI_F32: qgemm_kernel<FMT, EPI_F32><<<grid, block, 0, stream>>>(a, m, lda, w, ep); break;
    case EPI_BF16: qgemm_kernel<FMT, EPI_BF16><<<grid, block, 0, stream>>>(a, m, lda, w, ep); break;
    case EPI_QKV: qgemm_kernel<FMT, EPI_QKV><<<grid, block, 0, stream>>>(a, m, lda, w, ep); break;
    case EPI_RESID: qgemm_kernel<FMT, EPI_RESID><<<grid, block, 0, stream>>>(a, m, lda, w, ep); break;
    case EPI_SWIGLU: qgemm_kernel<FMT, EPI_SWIGLU><<<grid, block, 0, stream>>>(a, m, lda, w, ep); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

int device_cus() {
    static int cus = -1;
    if (cus < 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
            cus = v;
        else
            cus = 0;
    }
    return cus;
}

hipError_t launch_any(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi, const EpiParams &ep,
                      hipStream_t stream, int splits) {
    switch (w.fmt) {
    case WF_Q8_0: return launch_fmt<WF_Q8_0>(w, a, m, lda, epi, ep, stream, splits);
    case WF_Q4_K: return launch_fmt<WF_Q4_K>(w, a, m, lda, epi, ep, stream, splits);
    case WF_Q6_K: return launch_fmt<WF_Q6_K>(w, a, m, lda, epi, ep, stream, splits);
    case WF_BF16: return launch_fmt<WF_BF16>(w, a, m, lda, epi, ep, stream, splits);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

// K split of the 128x128 kernel when its tiles alone would leave CUs idle:
// doubled (up to 8) while the doubled grid still fits the two resident
// workgroups per CU (a second one hides the first one's load waits) and each
// share stays a whole number of 512-value groups. The partial sums cost
// 8 s m N bytes of traffic (written once, read once); at these token counts
// an idle CU costs more.
int qgemm_mid_splits(const GemmWeight &w, int64_t m) {
    if (m <= 0 || qgemm_large_fits(w, m) || qgemm_stream_fits(w, m)) return 1;
    const int64_t tiles = (w.n / BN) * ((m + BM - 1) / BM), cus = device_cus();
    int s = 1;
    while (s < 8 && tiles * 2 * s <= 2 * cus && w.k % (512 * 2 * s) == 0) s *= 2;
    return s;
}

namespace {

// Rows of a large-M product handed to the shorter-M paths so that the 256x256
// kernel runs whole waves: when the 256x256 tiles leave a last, partial wave
// of at most a quarter of the CUs made of whole 256-row tile rows (4352 tokens
// x N = 4096: 272 tiles for 256 CUs), those rows go to the split-K 128x128
// kernel (or the short-M path) instead. Plain outputs only (their rows are
// independent of the token index); 0 = none.
int64_t large_tail_rows(const GemmWeight &w, int64_t m) {
    if (!qgemm_large_fits(w, m)) return 0;
    const int64_t mt = (m + 255) / 256, nt = w.n / 256, tiles = mt * nt, cus = device_cus();
    const int64_t r = cus > 0 ? tiles % cus : 0;
    if (tiles <= cus || r == 0 || r > cus / 4 || r % nt) return 0;
    const int64_t tail = m - (mt - r / nt) * 256;
    return (tail < 512 && m - tail >= 512) ? tail : 0;
}

size_t mid_workspace(const GemmWeight &w, int64_t m) {
    const int s = qgemm_mid_splits(w, m);
    return s > 1 ? STREAM_COUNTER_BYTES + (size_t)s * (size_t)m * (size_t)w.n * 4 : 0;
}

size_t small_workspace(const GemmWeight &w, int64_t m) {
    return qgemm_stream_fits(w, m) ? qgemm_stream_workspace(w, m) : mid_workspace(w, m);
}

// M < 512: the short-M path when it fits and its scratch is there, else the
// 128x128 kernel, split over K when its tiles leave CUs idle and scratch is
// there.
hipError_t launch_small(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi, const EpiParams &ep,
                        hipStream_t stream) {
    if (qgemm_stream_fits(w, m) && ep.part_ws && ep.part_ws_bytes >= qgemm_stream_workspace(w, m))
        return launch_qgemm_stream(w, a, m, lda, epi, ep, ep.part_ws, stream);
    const int splits = qgemm_mid_splits(w, m);
    if (splits > 1 && ep.part_ws && ep.part_ws_bytes >= qgemm_workspace(w, m)) {
        // partial sums [splits][m][n] after the counter area, then the fixed-order
        // reduction that applies the epilogue
        float *part = (float *)((char *)ep.part_ws + STREAM_COUNTER_BYTES);
        EpiParams pe{};
        pe.out = part;
        pe.ldo = w.n;
        const hipError_t e = launch_any(w, a, m, lda, EPI_F32, pe, stream, splits);
        if (e != hipSuccess) return e;
        return launch_split_epilogue(part, splits, m, w.n, epi, ep, stream);
    }
    return launch_any(w, a, m, lda, epi, ep, stream, 1);
}

}  // namespace

size_t qgemm_workspace(const GemmWeight &w, int64_t m) {
    if (qgemm_large_fits(w, m)) {
        const int64_t tail = large_tail_rows(w, m);
        return tail ? small_workspace(w, tail) : 0;
    }
    return small_workspace(w, m);
}

hipError_t launch_qgemm(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                        const EpiParams &ep, hipStream_t stream) {
    if (m <= 0) return hipSuccess;
    if (qgemm_large_fits(w, m)) {
        const int64_t tail = (epi == EPI_F32 || epi == EPI_BF16) ? large_tail_rows(w, m) : 0;
        if (tail && ep.part_ws && ep.part_ws_bytes >= small_workspace(w, tail)) {
            const int64_t head = m - tail;
            const hipError_t e = launch_qgemm_large(w, a, head, lda, epi, ep, stream);
            if (e != hipSuccess) return e;
            EpiParams et = ep;
            et.out = (char *)ep.out + (size_t)head * (size_t)ep.ldo * (epi == EPI_F32 ? 4 : 2);
            return launch_small(w, a + head * lda, tail, lda, epi, et, stream);
        }
        return launch_qgemm_large(w, a, m, lda, epi, ep, stream);
    }
    return launch_small(w, a, m, lda, epi, ep, stream);
}

}  // namespace qimm
