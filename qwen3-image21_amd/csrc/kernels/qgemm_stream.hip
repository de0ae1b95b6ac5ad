// Weight-streaming dequant-GEMM for gfx950 at small token counts (M <= 64):
// C = A (bf16, M x K) x W^T (GGUF blocks, N x K). At these sizes the time is
// the weight bytes over HBM bandwidth, so the kernel is shaped for streaming:
//
//  - 64 weight rows x one K chunk per workgroup (4 waves x 16 rows), the K
//    range split over workgroups so that the grid holds several workgroups per
//    CU; partial sums go to an f32 workspace [split][M][N] and a second kernel
//    adds them in a fixed order (deterministic) and applies the epilogue.
//  - each lane dequantizes its own B fragment of v_mfma_f32_16x16x32_bf16
//    (W row = lane % 16, 8 consecutive k) straight from the raw GGUF bytes in
//    registers (exact f32 d*sc*q - dmin*m, RNE to bf16), so weights never pass
//    through LDS; the raw bytes of a stage are loaded two stages ahead.
//  - the activations (shared by every wave) are staged in LDS, 128 k per
//    stage, double-buffered, rows XOR-swizzled; the next stage's rows are
//    loaded into registers while the current one is consumed.
//
// Replaces candle's QMatMul::forward (src/quantized_transformer.rs:19-33) for
// short token counts: the per-row vec-dot regime of the reference CPU path.
#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

constexpr int SK = 128;          // k per LDS stage (two 64-k weight steps)
constexpr int MAXM = 64;         // token rows per workgroup
constexpr int XROWB = SK * 2;    // bytes per activation row in LDS (256)
constexpr int XSTAGE = MAXM * XROWB;  // 16 KB

typedef __attribute__((address_space(3))) void *lds_ptr_t;

__device__ __forceinline__ uint32_t byte_of(const u32x4 &x, int i) {
    return (x[i >> 2] >> (8 * (i & 3))) & 0xffu;
}

// 8 unsigned byte codes (two words) -> 8 bf16 of code*ds + off (exact f32
// value, rounded to nearest even).
__device__ __forceinline__ bf16x8 cvt8(uint32_t x0, uint32_t x1, float ds, float off) {
    auto f = [&](uint32_t x, int i) { return __builtin_fmaf((float)((x >> (8 * i)) & 0xffu), ds, off); };
    return __builtin_bit_cast(bf16x8, u32x4{pack_bf16x2(f(x0, 0), f(x0, 1)), pack_bf16x2(f(x0, 2), f(x0, 3)),
                                            pack_bf16x2(f(x1, 0), f(x1, 1)), pack_bf16x2(f(x1, 2), f(x1, 3))});
}

// Q4_K 6-bit scale / min of sub-block j (GGML packing, header bytes 4..15).
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

// Raw bytes one lane needs for one 64-k step of its W row: values
// k0 + 32 s + 8 kg + i for slices s = 0, 1 and i = 0..7.
struct WStep {
    u32x4 a;     // Q4_K header | Q6_K scales | Q8_0 codes of both slices (2 x 8 B) | BF16 slice 0
    u32x4 b;     // Q6_K ql (2 x 8 B) | BF16 slice 1
    u32x2 c;     // Q4_K qs | Q6_K qh
    uint32_t s;  // Q8_0 scales (2 x f16) | Q6_K d
};

template <int FMT>
__device__ __forceinline__ void load_step(const GemmWeight &w, int64_t n, int64_t k0, int kg, WStep &r) {
    const int64_t K = w.k;
    if constexpr (FMT == WF_Q4_K) {
        const uint8_t *blk = q4k_block(w.q, n, k0 / 256, K / 256);
        const int c = (int)((k0 & 255) >> 6);
        r.a = *(const u32x4 *)blk;
        r.c = *(const u32x2 *)(blk + 16 + 32 * c + 8 * kg);
    } else if constexpr (FMT == WF_Q6_K) {
        const uint8_t *blk = q6k_block(w.q, n, k0 / 256, K / 256);
        const int hh = (int)((k0 & 255) >> 7);
        const u32x2 l0 = *(const u32x2 *)(blk + 64 * hh + 8 * kg);
        const u32x2 l1 = *(const u32x2 *)(blk + 64 * hh + 32 + 8 * kg);
        r.b = u32x4{l0[0], l0[1], l1[0], l1[1]};
        r.c = *(const u32x2 *)(blk + 128 + 32 * hh + 8 * kg);
        r.a = *(const u32x4 *)(blk + 192);
        r.s = *(const uint16_t *)(blk + 208);
    } else if constexpr (FMT == WF_Q8_0) {
        const uint8_t *p = w.q + n * K + k0 + 8 * kg;
        const u32x2 c0 = *(const u32x2 *)p;
        const u32x2 c1 = *(const u32x2 *)(p + 32);
        r.a = u32x4{c0[0], c0[1], c1[0], c1[1]};
        r.s = *(const uint32_t *)(w.scales + n * (K / 32) + k0 / 32);
    } else {
        const uint16_t *p = (const uint16_t *)w.q + n * K + k0 + 8 * kg;
        r.a = *(const u32x4 *)p;
        r.b = *(const u32x4 *)(p + 32);
    }
}

// bf16 B fragment of slice s (compile time) of a step.
template <int FMT>
__device__ __forceinline__ bf16x8 frag(const WStep &r, int s, int64_t k0, int kg) {
    if constexpr (FMT == WF_Q4_K) {
        const int c = (int)((k0 & 255) >> 6);
        const float d = f16_bits_to_f32(r.a[0] & 0xffffu), dmin = f16_bits_to_f32(r.a[0] >> 16);
        float sc, mn;
        q4k_sc_m(r.a, 2 * c + s, sc, mn);
        const uint32_t sh = 4u * (uint32_t)s;  // sub-block 2c: low nibbles, 2c+1: high
        return cvt8((r.c[0] >> sh) & 0x0F0F0F0Fu, (r.c[1] >> sh) & 0x0F0F0F0Fu, d * sc, -(dmin * mn));
    } else if constexpr (FMT == WF_Q6_K) {
        // values 32 r6 + l, r6 = 2 o + s: ql low (o = 0) / high (o = 1)
        // nibble, qh bits >> 2 r6, scale 8 hh + 2 r6 + l / 16
        const int hh = (int)((k0 & 255) >> 7), o = (int)((k0 & 127) >> 6);
        const int r6 = 2 * o + s;
        const uint32_t qsh = 4u * (uint32_t)o, hsh = 2u * (uint32_t)r6;
        const uint32_t q0 = r.b[2 * s] >> qsh, q1 = r.b[2 * s + 1] >> qsh;
        const uint32_t c0 = (q0 & 0x0F0F0F0Fu) | (((r.c[0] >> hsh) & 0x03030303u) << 4);
        const uint32_t c1 = (q1 & 0x0F0F0F0Fu) | (((r.c[1] >> hsh) & 0x03030303u) << 4);
        const float ds = f16_bits_to_f32(r.s) * (float)(int8_t)byte_of(r.a, 8 * hh + 2 * r6 + (kg >> 1));
        return cvt8(c0, c1, ds, -32.f * ds);  // (q+32)*ds - 32*ds, exact
    } else if constexpr (FMT == WF_Q8_0) {
        const float d = f16_bits_to_f32(s ? (r.s >> 16) : (r.s & 0xffffu));
        return cvt8(r.a[2 * s] ^ 0x80808080u, r.a[2 * s + 1] ^ 0x80808080u, d, -128.f * d);  // biased codes
    } else {
        return __builtin_bit_cast(bf16x8, s ? r.b : r.a);
    }
}

// LDS activation tile of a stage: row m (256 B = 16 chunks of 8 k) holds chunk
// c at slot c ^ (m & 15): the 16 rows of an A-fragment read cover all 64 banks.
__device__ __forceinline__ int x_off(int m, int c) { return m * XROWB + ((c ^ (m & 15)) << 4); }

template <int FMT>
__global__ __launch_bounds__(256) void qgemm_stream_kernel(const uint16_t *__restrict__ A, int64_t M, int64_t lda,
                                                           GemmWeight w, float *__restrict__ part, int nt,
                                                           int kc_stages) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * XSTAGE];
    const int lane = threadIdx.x & 63, l16 = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int ks = blockIdx.x / nt, ntile = blockIdx.x % nt;
    const int64_t n = (int64_t)ntile * 64 + wave * 16 + l16;  // this lane's W row
    const int64_t kbase = (int64_t)ks * kc_stages * SK;
    const int mt = (int)((M + 15) >> 4);  // 16-token tiles
    const int64_t N = w.n;

    // activations of a stage: thread (wave, lane) loads 16 B of rows
    // 4(4 wave + i) + lane / 16 (i < 4) at chunk slot lane % 16 and stores them
    // to the swizzled LDS tile; rows past M repeat row M-1
    const uint16_t *xsrc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = 4 * (4 * wave + i) + (lane >> 4);
        const int c = (lane & 15) ^ (m & 15);
        xsrc[i] = A + (int64_t)min((int64_t)m, M - 1) * lda + 8 * c;
    }
    u32x4 xr[4];
    auto load_x = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (4 * (4 * wave + i) < 16 * mt) xr[i] = *(const u32x4 *)(xsrc[i] + k0);  // wave-uniform skip
    };
    auto store_x = [&](int stage) {
        uint8_t *base = lds + stage * XSTAGE;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (4 * (4 * wave + i) < 16 * mt) *(u32x4 *)(base + (4 * wave + i) * 1024 + 16 * lane) = xr[i];
    };
    // LDS hand-off without a memory fence: the fence of __syncthreads would
    // also wait for the weight loads in flight for later stages
    auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    f32x4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // raw weights of three stages (six 64-k steps) rotate through registers
    WStep ws[3][2];
    auto load_stage = [&](WStep *dst, int j) {
        const int jj = min(j, kc_stages - 1);
#pragma unroll
        for (int h = 0; h < 2; h++) load_step<FMT>(w, n, kbase + (int64_t)jj * SK + 64 * h, kg, dst[h]);
    };
    auto compute = [&](int stage, const WStep *src, int j) {
        const uint8_t *xs = lds + stage * XSTAGE;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t k0 = kbase + (int64_t)j * SK + 64 * h;
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const bf16x8 b = frag<FMT>(src[h], s, k0, kg);
                const int c = 8 * h + 4 * s + kg;  // 8-k chunk of the stage row
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    if (t < mt) {
                        const bf16x8 a = *(const bf16x8 *)(xs + x_off(16 * t + l16, c));
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[t], 0, 0, 0);
                    }
                }
            }
        }
    };

    load_x(kbase);
    load_stage(ws[0], 0);
    store_x(0);
    load_x(kbase + (int64_t)min(1, kc_stages - 1) * SK);
    load_stage(ws[1], 1);
    lds_barrier();
    // On entry to stage j: x of stage j is in LDS stage j&1, xr holds x of
    // stage j+1 and ws[j%3], ws[(j+1)%3] the raw weights of stages j, j+1.
    // Loads are issued oldest-needed first (x of j+2, then W of j+2), so the
    // wait for xr never waits for weights that are only needed later.
    int j = 0;
    auto step = [&](int cur, int wsi, int wsn) {
        store_x(cur ^ 1);  // stage cur^1 was last read in stage j-1, before the barrier
        load_x(kbase + (int64_t)min(j + 2, kc_stages - 1) * SK);
        load_stage(ws[wsn], j + 2);
        compute(cur, ws[wsi], j);
        lds_barrier();
        j++;
    };
    while (j + 6 <= kc_stages) {
        step(0, 0, 2);
        step(1, 1, 0);
        step(0, 2, 1);
        step(1, 0, 2);
        step(0, 1, 0);
        step(1, 2, 1);
    }
    // fewer than six stages left: the same rotation, one stage at a time, with
    // branches that keep every register-set index a compile-time constant
    while (j < kc_stages) {
        const int cur = j & 1, wsi = j % 3;
        if (wsi == 0) {
            if (cur == 0) step(0, 0, 2); else step(1, 0, 2);
        } else if (wsi == 1) {
            if (cur == 0) step(0, 1, 0); else step(1, 1, 0);
        } else {
            if (cur == 0) step(0, 2, 1); else step(1, 2, 1);
        }
    }

    // partial sums: acc[t][i] = token 16 t + 4 kg + i, W row n
    float *dst = part + (int64_t)ks * M * N;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        if (t < mt) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t m = 16 * t + 4 * kg + i;
                if (m < M) dst[m * N + n] = acc[t][i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_K at M <= 16: MFMA on the raw 4-bit codes, scales applied afterwards.
//
// For sub-block j (32 values) of row n: w = ds_j q - dm_j with ds_j = d sc_j,
// dm_j = dmin m_j. The B operand is the exact bf16 of 128 + q (bits 0x4300 |
// q), so one v_mfma_f32_16x16x32_bf16 gives S'_j = sum x (128 + q) for 16
// tokens x 16 rows, and
//     sum_k x w = sum_j ds_j S'_j - sum_j (128 ds_j + dm_j) X_j,
// X_j = sum of x over the sub-block. The first sum is 4 FMAs per lane per
// sub-block; the second is an f32 MFMA (16x16x4) per four sub-blocks, its
// A operand X from a bf16 MFMA with row-selector ones, so no per-value
// dequantization runs at all. The result is the exact product of the bf16
// activations and the exact Q4_K weights up to f32 summation order.
//
// One workgroup per CU (8 waves, 131 KB LDS holding x[16][4096] bf16): x is
// copied to LDS once by direct loads, then each wave streams its share of the
// (16-row group, super-block) tiles -- 2304 contiguous bytes in the device
// layout -- through a register ring four tiles deep. Waves split the
// workgroup's tiles evenly; the partial tile sums of a wave are reduced in LDS
// in wave order (deterministic) and written to part[c][m][n] for the
// split-K epilogue.
namespace m16 {

constexpr int NW = 8;       // waves per workgroup
constexpr int KC = 4096;    // k per workgroup (x[16][KC] in LDS)
constexpr int SBC = KC / 256;
constexpr int ROWB = KC * 2 + 16;  // padded row: the 16 rows of a fragment read hit distinct banks
constexpr int DEPTH = 4;    // tiles in flight per wave

struct Raw {
    u32x4 h;
    u32x2 q[4];
};

// B fragments of 8 consecutive codes (two words): bf16 128 + q of the low and
// of the high nibbles, by byte permutes against a 0x43 source register.
__device__ __forceinline__ void codes8(uint32_t w0, uint32_t w1, u32x4 &lo, u32x4 &hi) {
    const uint32_t C43 = 0x43434343u;
    const uint32_t l0 = w0 & 0x0F0F0F0Fu, l1 = w1 & 0x0F0F0F0Fu;
    const uint32_t h0 = (w0 >> 4) & 0x0F0F0F0Fu, h1 = (w1 >> 4) & 0x0F0F0F0Fu;
    lo = u32x4{__builtin_amdgcn_perm(C43, l0, 0x04010400u), __builtin_amdgcn_perm(C43, l0, 0x04030402u),
               __builtin_amdgcn_perm(C43, l1, 0x04010400u), __builtin_amdgcn_perm(C43, l1, 0x04030402u)};
    hi = u32x4{__builtin_amdgcn_perm(C43, h0, 0x04010400u), __builtin_amdgcn_perm(C43, h0, 0x04030402u),
               __builtin_amdgcn_perm(C43, h1, 0x04010400u), __builtin_amdgcn_perm(C43, h1, 0x04030402u)};
}

__device__ __forceinline__ float cvt_f16_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float cvt_f16_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// PER tiles per wave (compile time, so every wait on the ring is exact).
// Grid: NG n-groups x C k-chunks; group g holds T 16-row tiles.
template <int PER>
__global__ __launch_bounds__(512) void q4k_m16_kernel(const uint16_t *__restrict__ A, int M, int64_t lda,
                                                      GemmWeight w, int C, int T, float *__restrict__ part) {
    __shared__ __attribute__((aligned(16))) uint8_t xs[16 * ROWB];
    __shared__ __attribute__((aligned(16))) float red[NW][2][256];
    __shared__ int tags[NW][2];
    constexpr int D = DEPTH < PER ? DEPTH : PER;
    constexpr int R = D + 1;  // ring slots: tile u + D is requested before tile u is computed
    const int lane = threadIdx.x & 63, l16 = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t N = w.n, SB = w.k / 256;
    const int NG = (int)((N / 16) / T);
    const int ng = blockIdx.x % NG, c = blockIdx.x / NG;
    const int64_t k0 = (int64_t)c * KC;
    const int t0 = wave * PER;

    // x chunk -> LDS by direct loads (instruction i of wave w fills 64
    // consecutive 16 B chunks of one row); rows past M repeat row M - 1
    {
        constexpr int NI = 16 * KC / 8 / 64 / NW;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int q0 = (i * NW + wave) * 64;
            const int m = q0 / (KC / 8), s0 = q0 % (KC / 8);
            const uint16_t *src = A + (int64_t)min(m, M - 1) * lda + k0 + 8 * (s0 + lane);
            __builtin_amdgcn_global_load_lds((const void *)src, (lds_ptr_t)(xs + m * ROWB + 16 * s0), 16, 0, 0);
        }
    }
    // the wave's tiles in (n-tile, super-block) order
    Raw ring[R];
    const int nt0 = t0 / SBC, sb0 = t0 % SBC;
    auto load_tile = [&](Raw &r, int u) {
        const int ntl = nt0 + (sb0 + u) / SBC, sbl = (sb0 + u) % SBC;
        const int64_t n = (int64_t)(ng * T + ntl) * 16 + l16;
        const uint8_t *b = q4k_block(w.q, n, (int64_t)c * SBC + sbl, SB);
        r.h = *(const u32x4 *)b;
#pragma unroll
        for (int cc = 0; cc < 4; cc++) r.q[cc] = *(const u32x2 *)(b + 16 + 32 * cc + 8 * kg);
    };
#pragma unroll
    for (int u = 0; u < D; u++) load_tile(ring[u], u);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(5 * D) : "memory");

    // A operands of the sub-block sums: rows 4 s .. 4 s + 3 of ones[s] are 1
    bf16x8 ones[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const uint32_t v = (l16 >> 2) == s ? 0x3F803F80u : 0u;
        ones[s] = __builtin_bit_cast(bf16x8, u32x4{v, v, v, v});
    }
    f32x4 accA = {0.f, 0.f, 0.f, 0.f}, accM = {0.f, 0.f, 0.f, 0.f};
    int seg = 0;
    const uint8_t *xlane = xs + l16 * ROWB + 16 * kg;
    auto tile = [&](const Raw &r, int u) {
        const int ntl = nt0 + (sb0 + u) / SBC, sbl = (sb0 + u) % SBC;
        const uint32_t hx = r.h[0], hy = r.h[1], hz = r.h[2], hw = r.h[3];
        const float d = cvt_f16_lo(hx), dmin = cvt_f16_hi(hx);
        // 6-bit scales / mins of sub-blocks 0..3 (lo) and 4..7 (hi), one per byte
        const uint32_t sc_lo = hy & 0x3F3F3F3Fu, m_lo = hz & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (hw & 0x0F0F0F0Fu) | ((hy >> 2) & 0x30303030u);
        const uint32_t m_hi = ((hw >> 4) & 0x0F0F0F0Fu) | ((hz >> 2) & 0x30303030u);
        // f32-MFMA B operand: 128 ds_j + dm_j of sub-blocks kg and 4 + kg
        const uint32_t sh = 8u * (uint32_t)kg;
        const float cc0 = fmaf(128.f, d * (float)((sc_lo >> sh) & 0xffu), dmin * (float)((m_lo >> sh) & 0xffu));
        const float cc1 = fmaf(128.f, d * (float)((sc_hi >> sh) & 0xffu), dmin * (float)((m_hi >> sh) & 0xffu));
        const uint8_t *xt = xlane + sbl * 512;
        bf16x8 af[8];
#pragma unroll
        for (int j = 0; j < 8; j++) af[j] = *(const bf16x8 *)(xt + 64 * j);
        // X[m][j0 + kg] in the A layout of the f32 MFMA (all four registers)
        f32x4 xq0 = {0.f, 0.f, 0.f, 0.f}, xq1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            xq0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones[j], af[j], xq0, 0, 0, 0);
            xq1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones[j], af[4 + j], xq1, 0, 0, 0);
        }
        accM = __builtin_amdgcn_mfma_f32_16x16x4f32(xq0[0], cc0, accM, 0, 0, 0);
        accM = __builtin_amdgcn_mfma_f32_16x16x4f32(xq1[0], cc1, accM, 0, 0, 0);
        // the eight code products (independent accumulators), then the scales
        u32x4 bq[8];
#pragma unroll
        for (int cc = 0; cc < 4; cc++) codes8(r.q[cc][0], r.q[cc][1], bq[2 * cc], bq[2 * cc + 1]);
        f32x4 tv[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            tv[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[j], __builtin_bit_cast(bf16x8, bq[j]),
                                                            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float ds = d * (float)(((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3))) & 0xffu);
#pragma unroll
            for (int e = 0; e < 4; e++) accA[e] = fmaf(ds, tv[j][e], accA[e]);
        }
        if (sbl == SBC - 1 || u == PER - 1) {  // end of this n-tile's part in the wave
#pragma unroll
            for (int e = 0; e < 4; e++) red[wave][seg][(4 * kg + e) * 16 + l16] = accA[e] - accM[e];
            if (lane == 0) tags[wave][seg] = ntl;
            seg++;
            accA = f32x4{0.f, 0.f, 0.f, 0.f};
            accM = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
#pragma unroll
    for (int u = 0; u < PER; u++) {
        if (u + D < PER) load_tile(ring[(u + D) % R], u + D);
        tile(ring[u % R], u);
    }
    if (lane == 0 && seg < 2) tags[wave][1] = -1;
    __syncthreads();
    // per-tile sums over the waves that covered it, in wave order
    for (int p = threadIdx.x; p < T * 256; p += 64 * NW) {
        const int tt = p >> 8, e = p & 255, m = e >> 4, nl = e & 15;
        float s = 0.f;
        for (int wv = 0; wv < NW; wv++)
            for (int sg = 0; sg < 2; sg++)
                if (tags[wv][sg] == tt) s += red[wv][sg][e];
        if (m < M) part[((int64_t)c * M + m) * N + (int64_t)(ng * T + tt) * 16 + nl] = s;
    }
}

// Grid of the M <= 16 kernel, or false when the shape does not tile exactly:
// K a multiple of 4096 (C chunks), NG n-groups of T 16-row tiles with
// NG * C equal to the CU count, each wave covering at most two n-tiles.
bool plan(const GemmWeight &w, int64_t m, int cus, int &C, int &T, int &NG) {
    if (w.fmt != WF_Q4_K || m < 1 || m > 16 || w.k % KC || w.n % 16 || cus <= 0) return false;
    C = (int)(w.k / KC);
    const int64_t tiles16 = w.n / 16;
    if ((tiles16 * C) % cus) return false;
    T = (int)(tiles16 * C / cus);
    if (T < 1 || T > 8 || tiles16 % T) return false;
    NG = (int)(tiles16 / T);
    return (int64_t)NG * C == cus;
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

hipError_t launch(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, float *part, int C, int T, int NG,
                  hipStream_t stream) {
    const dim3 grid((unsigned)(NG * C)), block(64 * NW);
    switch (2 * T) {
    case 2: q4k_m16_kernel<2><<<grid, block, 0, stream>>>(a, (int)m, lda, w, C, T, part); break;
    case 4: q4k_m16_kernel<4><<<grid, block, 0, stream>>>(a, (int)m, lda, w, C, T, part); break;
    case 6: q4k_m16_kernel<6><<<grid, block, 0, stream>>>(a, (int)m, lda, w, C, T, part); break;
    case 8: q4k_m16_kernel<8><<<grid, block, 0, stream>>>(a, (int)m, lda, w, C, T, part); break;
    case 10: q4k_m16_kernel<10><<<grid, block, 0, stream>>>(a, (int)m, lda, w, C, T, part); break;
    case 12: q4k_m16_kernel<12><<<grid, block, 0, stream>>>(a, (int)m, lda, w, C, T, part); break;
    case 14: q4k_m16_kernel<14><<<grid, block, 0, stream>>>(a, (int)m, lda, w, C, T, part); break;
    case 16: q4k_m16_kernel<16><<<grid, block, 0, stream>>>(a, (int)m, lda, w, C, T, part); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace m16

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Sum of the split-K partials of C[m][n], in split order.
__device__ __forceinline__ float csum(const float *part, int splits, int64_t MN, int64_t idx) {
    float v = 0.f;
    for (int s = 0; s < splits; s++) v += part[s * MN + idx];
    return v;
}

// Elementwise epilogues: one thread per output element (SwiGLU: per output
// column of the hidden, gate and up read from the interleaved layout).
template <int EPI>
__global__ __launch_bounds__(256) void stream_epi_kernel(const float *__restrict__ part, int splits, int64_t M,
                                                         int64_t N, EpiParams ep) {
    const int64_t MN = M * N;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if constexpr (EPI == EPI_SWIGLU) {
        // hidden column h = 64 g + j (j < 64): gate at device column 128 g + j, up at 128 g + 64 + j
        const int64_t F = N / 2;
        if (idx >= M * F) return;
        const int64_t m = idx / F, h = idx % F;
        const int64_t cg = (h >> 6) * 128 + (h & 63);
        const float gt = csum(part, splits, MN, m * N + cg), up = csum(part, splits, MN, m * N + cg + 64);
        ep.hmid[m * ep.ldh + h] = (uint16_t)(pack_bf16x2(silu(gt) * up, 0.f) & 0xffffu);
    } else {
        if (idx >= MN) return;
        const int64_t m = idx / N, n = idx % N;
        const float v = csum(part, splits, MN, idx);
        if constexpr (EPI == EPI_F32) {
            ((float *)ep.out)[m * ep.ldo + n] = v;
        } else if constexpr (EPI == EPI_BF16) {
            ((uint16_t *)ep.out)[m * ep.ldo + n] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
        } else {  // EPI_RESID
            const float *grow = ep.gvec + (int64_t)((int)m / (int)ep.g_rows_per) * ep.g_stride;
            ep.x_out[m * N + n] = ep.x_in[m * N + n] + grow[n] * v;
        }
    }
}

// QKV epilogue: one wave per (token, head); lane j holds the RoPE pair
// (2j, 2j+1) of the head's 128 columns.
__global__ __launch_bounds__(256) void stream_qkv_kernel(const float *__restrict__ part, int splits, int64_t M,
                                                         int64_t N, EpiParams ep) {
    const int64_t MN = M * N;
    const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (token, head slot)
    const int lane = threadIdx.x & 63;
    const int64_t heads_here = N / 128;
    if (g >= M * heads_here) return;
    const int64_t m = g / heads_here, hs = g % heads_here;
    const int64_t nb = hs * 128 + ep.n_offset;  // fused column of the head start
    const int sec = (int)(nb / ep.hidden);
    const int64_t head = (nb % ep.hidden) / 128;
    const int64_t S = ep.seq, H = ep.heads;
    const int64_t b = m / S, s = m % S;
    const int64_t c0 = hs * 128 + 2 * lane;
    float x0 = csum(part, splits, MN, m * N + c0), x1 = csum(part, splits, MN, m * N + c0 + 1);
    if (sec < 2) {
        const float *nw = sec == 0 ? ep.norm_q : ep.norm_k;
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float rs = 1.0f / sqrtf(ss * (1.0f / 128.0f) + 1e-6f);
        x0 = x0 * rs * nw[2 * lane];
        x1 = x1 * rs * nw[2 * lane + 1];
        const float *pr = ep.pe + s * 128 + 2 * lane;
        const float cs = pr[0], sn = pr[1];
        const float osc = sec == 0 ? ep.q_scale : 1.0f;
        const float y0 = (x0 * cs - x1 * sn) * osc, y1 = (x0 * sn + x1 * cs) * osc;
        uint16_t *dst = sec == 0 ? ep.q : ep.k;
        *(uint32_t *)(dst + ((b * H + head) * S + s) * 128 + 2 * lane) = pack_bf16x2(y0, y1);
    } else {
        const uint32_t pk = pack_bf16x2(x0, x1);
        ep.vt[((b * H + head) * 128 + 2 * lane) * S + s] = (uint16_t)(pk & 0xffffu);
        ep.vt[((b * H + head) * 128 + 2 * lane + 1) * S + s] = (uint16_t)(pk >> 16);
        if (ep.v_bhsd) *(uint32_t *)(ep.v_bhsd + ((b * H + head) * S + s) * 128 + 2 * lane) = pk;
    }
}

template <int FMT>
hipError_t launch_fmt(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, float *part, int splits,
                      hipStream_t stream) {
    const int nt = (int)(w.n / 64);
    const int kc_stages = (int)(w.k / SK / splits);
    qgemm_stream_kernel<FMT><<<dim3((unsigned)(nt * splits)), dim3(256), 0, stream>>>(a, m, lda, w, part, nt,
                                                                                     kc_stages);
    return hipGetLastError();
}

}  // namespace

// The K split: doubled while the grid has fewer than 1024 workgroups, the
// chunks stay whole 256-value groups and the partial sums (written and read
// once each) stay under half the weight bytes.
int qgemm_stream_splits(const GemmWeight &w, int64_t m) {
    int C, T, NG;
    if (m16::plan(w, m, m16::device_cus(), C, T, NG)) return C;
    const int64_t nt = w.n / 64, kst = w.k / 256;
    const double wbytes = (double)w.n * (double)w.k * (w.fmt == WF_Q4_K ? 0.5625 : w.fmt == WF_Q6_K ? 0.875
                                                       : w.fmt == WF_Q8_0 ? 1.0625 : 2.0);
    int s = 1;
    while (nt * s < 1024 && kst % (2 * s) == 0 && (double)(2 * s) * (double)m * (double)w.n * 8.0 <= 0.5 * wbytes)
        s *= 2;
    return s;
}

bool qgemm_stream_fits(const GemmWeight &w, int64_t m) {
    return m >= 1 && m <= MAXM && w.n % 64 == 0 && w.k % 256 == 0;
}

size_t qgemm_stream_workspace(const GemmWeight &w, int64_t m) {
    return (size_t)qgemm_stream_splits(w, m) * (size_t)m * (size_t)w.n * 4;
}

hipError_t launch_qgemm_stream(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                               const EpiParams &ep, float *part, hipStream_t stream) {
    int splits = qgemm_stream_splits(w, m);
    hipError_t e;
    int C, T, NG;
    switch (w.fmt) {
    case WF_Q8_0: e = launch_fmt<WF_Q8_0>(w, a, m, lda, part, splits, stream); break;
    case WF_Q4_K:
        if (m16::plan(w, m, m16::device_cus(), C, T, NG)) {
            splits = C;
            e = m16::launch(w, a, m, lda, part, C, T, NG, stream);
        } else {
            e = launch_fmt<WF_Q4_K>(w, a, m, lda, part, splits, stream);
        }
        break;
    case WF_Q6_K: e = launch_fmt<WF_Q6_K>(w, a, m, lda, part, splits, stream); break;
    case WF_BF16: e = launch_fmt<WF_BF16>(w, a, m, lda, part, splits, stream); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    const int64_t N = w.n;
    const int64_t elems = epi == EPI_SWIGLU ? m * N / 2 : m * N;
    const dim3 grid((unsigned)((elems + 255) / 256)), block(256);
    switch (epi) {
    case EPI_F32: stream_epi_kernel<EPI_F32><<<grid, block, 0, stream>>>(part, splits, m, N, ep); break;
    case EPI_BF16: stream_epi_kernel<EPI_BF16><<<grid, block, 0, stream>>>(part, splits, m, N, ep); break;
    case EPI_RESID: stream_epi_kernel<EPI_RESID><<<grid, block, 0, stream>>>(part, splits, m, N, ep); break;
    case EPI_SWIGLU: stream_epi_kernel<EPI_SWIGLU><<<grid, block, 0, stream>>>(part, splits, m, N, ep); break;
    case EPI_QKV: {
        const int64_t waves = m * (N / 128);
        stream_qkv_kernel<<<dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream>>>(part, splits, m, N, ep);
        break;
    }
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qimm
