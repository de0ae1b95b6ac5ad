// Dequant-GEMM for gfx950: C[M,N] = A[M,K] (bf16) x W[N,K]^T (GGUF blocks),
// the tile for 64 < M < 512 token rows (and the split-K shares of short
// products).
//
// Replaces candle's QMatMul::forward as called through Linear::forward
// (src/quantized_transformer.rs:19-33; call sites 133-135, 151, 194-199, 202).
//
// Tile 128x128x64, 256 threads = 4 waves in a 2x2 grid, each wave 64x64 as
// 2x2 v_mfma_f32_32x32x16_bf16 tiles, two workgroups per CU. Operand tiles
// live in LDS as dense 128 B rows with XOR-swizzled 16 B chunks (swz in
// device_common.h: conflict-free staging writes and fragment reads), two
// stages per operand. Both operands are loaded into register rings three k
// steps ahead (activation rows as bf16, weight half-rows as raw GGUF bytes);
// while the MFMAs of step k run, step k+1 goes from the ring to the other LDS
// stage, the weights dequantized on the way (v_fma_mix: exact f32
// d*sc*q - dmin*m, then round-to-nearest-even to bf16). One barrier per step.
// Every load goes to registers (no direct-to-LDS loads), so the compiler
// waits for each ring slot by an exact count and the loads of the next three
// steps stay in flight. The epilogue goes through LDS as an f32 tile so each
// variant (plain store, fused QKV RmsNorm+RoPE, gated residual, SwiGLU)
// writes whole rows with 128-bit stores.
#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int TILEB = 128 * 128;        // bytes of one 128-row operand tile
constexpr int STAGE = 2 * TILEB;        // A tile then W tile
constexpr int RING = 2;                 // k steps in flight in registers
constexpr int CP = 132;                 // f32 pitch of the epilogue tile row
constexpr int MAX_MID_SPLITS = 16;      // K shares; the split-K reduction kernel sums at most 16
constexpr int LDS_BYTES = BM * CP * 4;  // 67.6 KB (the two 64 KB operand stages fit): two workgroups per CU
static_assert(2 * STAGE <= LDS_BYTES, "operand stages fit the epilogue tile");
static_assert(RING == 2, "the step loop is unrolled by the ring size");

// Raw bytes of one half row (32 values) of a k step.
struct WRaw {
    u32x4 v[4];
    uint32_t s;
};

// A word whose value the optimizer must not look through.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ uint32_t byte_of(const u32x4 &x, int i) {
    return (x[i >> 2] >> (8 * (i & 3))) & 0xffu;
}

// Half h of row n for the k step at k0: Q8_0 / BF16 values [32h, 32h+32) of
// the step; Q4_K / Q6_K values [16h, 16h+16) and [32+16h, 32+16h+16).
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
#pragma unroll
        for (int i = 0; i < 4; i++) r.v[i] = *(const u32x4 *)(p + 16 * i);
    }
}

// Global loads load_w issues per thread (the pipeline's wait counts).
template <int FMT>
constexpr int w_loads() { return FMT == WF_Q8_0 ? 3 : FMT == WF_Q4_K ? 2 : FMT == WF_Q6_K ? 5 : 4; }

// Step dequant constants of a half row.
struct WScale {
    float a0, b0, a1, b1;
};

template <int FMT>
__device__ __forceinline__ WScale w_scales(const WRaw &r, int64_t k0, int h) {
    WScale s{};
    if constexpr (FMT == WF_Q8_0) {
        const float d = f16_to_f32(r.s & 0xffffu);
        s.a0 = d * 0x1p24f;  // codes biased to unsigned: (q+128)*d - 128*d, exact
        s.b0 = -128.f * d;
    } else if constexpr (FMT == WF_Q4_K) {
        const int c = (int)((k0 & 255) >> 6);
        const float d = f16_to_f32(r.v[0][0] & 0xffffu), dmin = f16_to_f32(r.v[0][0] >> 16);
        // the 12 packed scale/min bytes sit at header bytes 4..15 (GGML layout);
        // sub-blocks 2c (low nibbles) and 2c+1 (high nibbles). Both packings
        // are decoded and one is kept by a mask: c is uniform but known only at
        // run time, and a select on it compiles to a branch that would split the
        // step into separately scheduled blocks.
        const uint32_t hi = opaque(0u - (uint32_t)(c >> 1));  // all ones for sub-blocks 4-7
        float sc[2], mn[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int jl = (2 * c + e) & 3;
            const uint32_t b4 = byte_of(r.v[0], 4 + jl), b8 = byte_of(r.v[0], 8 + jl), b12 = byte_of(r.v[0], 12 + jl);
            const uint32_t s_lo = b4 & 63u, m_lo = b8 & 63u;
            const uint32_t s_hi = (b12 & 0xFu) | ((b4 >> 6) << 4), m_hi = (b12 >> 4) | ((b8 >> 6) << 4);
            sc[e] = (float)((s_lo & ~hi) | (s_hi & hi));
            mn[e] = (float)((m_lo & ~hi) | (m_hi & hi));
        }
        s.a0 = d * sc[0] * 0x1p24f;  // low nibbles at f16 bits 0-3
        s.b0 = -(dmin * mn[0]);
        s.a1 = d * sc[1] * 0x1p20f;  // high nibbles at f16 bits 4-7
        s.b1 = -(dmin * mn[1]);
    } else if constexpr (FMT == WF_Q6_K) {
        const int hh = (int)((k0 & 255) >> 7), o = (int)((k0 & 127) >> 6);
        const float d = f16_to_f32(r.s);
        const float da = d * (float)(int8_t)byte_of(r.v[3], 8 * hh + 4 * o + h);
        const float db = d * (float)(int8_t)byte_of(r.v[3], 8 * hh + 4 * o + 2 + h);
        s.a0 = da * 0x1p24f;  // (q)*ds - 32*ds with both products exact, one rounding
        s.b0 = -32.f * da;
        s.a1 = db * 0x1p24f;
        s.b1 = -32.f * db;
    }
    return s;
}

// Chunk j (8 values) of the half row as bf16 and the LDS chunk it fills:
// Q8_0 / BF16 chunk 4h + j; Q4_K / Q6_K chunks 2h, 2h+1, 4+2h, 5+2h.
template <int FMT>
__device__ __forceinline__ u32x4 w_chunk(const WRaw &r, const WScale &s, int j, int64_t k0) {
    if constexpr (FMT == WF_Q8_0) {
        const uint32_t u0 = r.v[j >> 1][2 * (j & 1)] ^ 0x80808080u, u1 = r.v[j >> 1][2 * (j & 1) + 1] ^ 0x80808080u;
        const uint32_t p0 = u0 & 0x00FF00FFu, p1 = __builtin_amdgcn_perm(0u, u0, 0x0C030C01u);
        const uint32_t p2 = u1 & 0x00FF00FFu, p3 = __builtin_amdgcn_perm(0u, u1, 0x0C030C01u);
        const float a = s.a0, b = s.b0;
        return u32x4{pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)), pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                     pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)), pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))};
    } else if constexpr (FMT == WF_Q4_K) {
        // j < 2: low nibbles of qs bytes [8j, 8j+8); j >= 2: high nibbles of
        // bytes [8(j-2), ...). The halves of (y & m) hold bytes 0 and 2, those
        // of ((y >> 8) & m) bytes 1 and 3.
        const int jb = j & 1;
        const uint32_t y0 = r.v[1][2 * jb], y1 = r.v[1][2 * jb + 1];
        const uint32_t m = j < 2 ? 0x000F000Fu : 0x00F000F0u;
        const float a = j < 2 ? s.a0 : s.a1, b = j < 2 ? s.b0 : s.b1;
        const uint32_t p0 = y0 & m, p1 = (y0 >> 8) & m, p2 = y1 & m, p3 = (y1 >> 8) & m;
        return u32x4{pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)), pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                     pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)), pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))};
    } else if constexpr (FMT == WF_Q6_K) {
        // j < 2: value rows ra = 2o (ql piece v[0]), j >= 2: rb = 2o + 1 (v[1]);
        // low nibbles when o == 0, high when o == 1; qh bits 2r .. 2r+1 of v[2]
        const int o = (int)((k0 & 127) >> 6);
        const int jb = j & 1, rr = 2 * o + (j >> 1);
        const u32x4 &L = j < 2 ? r.v[0] : r.v[1];
        const uint32_t q0 = L[2 * jb] >> (4 * o), q1 = L[2 * jb + 1] >> (4 * o);
        const uint32_t c0 = (q0 & 0x0F0F0F0Fu) | (((r.v[2][2 * jb] >> (2 * rr)) & 0x03030303u) << 4);
        const uint32_t c1 = (q1 & 0x0F0F0F0Fu) | (((r.v[2][2 * jb + 1] >> (2 * rr)) & 0x03030303u) << 4);
        const float a = j < 2 ? s.a0 : s.a1, b = j < 2 ? s.b0 : s.b1;
        const uint32_t p0 = c0 & 0x00FF00FFu, p1 = __builtin_amdgcn_perm(0u, c0, 0x0C030C01u);
        const uint32_t p2 = c1 & 0x00FF00FFu, p3 = __builtin_amdgcn_perm(0u, c1, 0x0C030C01u);
        return u32x4{pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)), pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                     pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)), pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))};
    } else {
        return r.v[j];
    }
}

template <int FMT>
__device__ __forceinline__ int w_slot(int j, int h) {
    if constexpr (FMT == WF_Q4_K || FMT == WF_Q6_K) return (j < 2 ? 2 * h : 4 + 2 * h) + (j & 1);
    else return 4 * h + j;
}

// silu with the hardware reciprocal (about 1 ulp) instead of an IEEE divide
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

template <int FMT, int EPI>
__global__ __launch_bounds__(256, 2) void qgemm_kernel(const uint16_t *__restrict__ A, int64_t M,
                                                       int64_t lda, GemmWeight w, EpiParams ep) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, l32 = lane & 31, g = lane >> 5;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int64_t K = w.k;
    // split K (gridDim.z > 1): this workgroup covers k steps [kt0, kt0 + KT)
    // and writes its f32 partial sums to slice blockIdx.z of ep.out
    const int KT = (int)(K / BK / gridDim.z);
    const int kt0 = (int)blockIdx.z * KT;
    // step q of this share, clamped to the last (redundant loads, no branches)
    auto kofs = [&](int q) __attribute__((always_inline)) { return (int64_t)(kt0 + min(q, KT - 1)) * BK; };

    // A: chunk a_kc of rows a_row + 32 i (rows past M clamped to row M-1: they
    // only feed output rows the epilogue never writes)
    const int a_row = tid >> 3, a_kc = tid & 7;
    const uint16_t *asrc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) asrc[i] = A + min(m0 + a_row + 32 * i, M - 1) * lda + 8 * a_kc;
    // W: half w_h of row n0 + w_nl
    const int w_nl = tid >> 1, w_h = tid & 1;
    const int64_t wrow = n0 + w_nl;

    u32x4 ra[RING][4];
    WRaw rw[RING];
    auto load = [&](int slot, int q) __attribute__((always_inline)) {
        const int64_t k0 = kofs(q);
#pragma unroll
        for (int i = 0; i < 4; i++) ra[slot][i] = *(const u32x4 *)(asrc[i] + k0);
        load_w<FMT>(w, wrow, k0, w_h, rw[slot]);
    };
    // ring slot -> LDS stage (the weights dequantized on the way)
    auto stage_in = [&](int slot, int q, int stage) __attribute__((always_inline)) {
        uint8_t *as = lds + stage * STAGE, *bs = as + TILEB;
#pragma unroll
        for (int i = 0; i < 4; i++) *(u32x4 *)(as + swz(a_row + 32 * i, a_kc)) = ra[slot][i];
        const int64_t k0 = kofs(q);
        const WScale sc = w_scales<FMT>(rw[slot], k0, w_h);
#pragma unroll
        for (int j = 0; j < 4; j++) *(u32x4 *)(bs + swz(w_nl, w_slot<FMT>(j, w_h))) = w_chunk<FMT>(rw[slot], sc, j, k0);
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // operand fragments of one 16-wide k slice, double-buffered across slices
    bf16x8 fa[2][2], fb[2][2];
    auto rd = [&](int buf, int stage, int kk) __attribute__((always_inline)) {
        const uint8_t *as = lds + stage * STAGE, *bs = as + TILEB;
#pragma unroll
        for (int i = 0; i < 2; i++) fa[buf][i] = *(const bf16x8 *)(as + swz(wm * 64 + i * 32 + l32, 2 * kk + g));
#pragma unroll
        for (int j = 0; j < 2; j++) fb[buf][j] = *(const bf16x8 *)(bs + swz(wn * 64 + j * 32 + l32, 2 * kk + g));
    };
    auto mm = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[buf][i], fb[buf][j], acc[i][j], 0, 0, 0);
    };

    // prologue: steps 0 .. RING-1 in flight, step 0 staged, its slice 0 read
#pragma unroll
    for (int q = 0; q < RING; q++) load(q, q);
    stage_in(0, 0, 0);
    __syncthreads();
    rd(0, 0, 0);

    // Step q: ring slot c = q % RING (compile time after unrolling) held step
    // q, already staged; it now receives step q + RING. On entry fa/fb[0] hold
    // slice 0 of step q. The next slice is read while the current one
    // computes, and step q+1 goes from slot (q+1) % RING into the other stage
    // (its loads were issued two steps ago). ONE barrier per step, before the
    // last slice, whose operands are then in registers: it publishes the
    // other stage and frees this one, whose slice 0 of step q+1 is read while
    // the last two slices compute.
    auto step = [&](int q, auto c_) __attribute__((always_inline)) {
        constexpr int c = decltype(c_)::value, c1 = (c + 1) % RING;
        const int st = q & 1;
        load(c, q + RING);
        __builtin_amdgcn_sched_barrier(0);  // the loads issue here, ahead of the staging that waits on older ones
        rd(1, st, 1);
        mm(0);
        stage_in(c1, q + 1, st ^ 1);
        rd(0, st, 2);
        mm(1);
        rd(1, st, 3);
        __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);
        __syncthreads();
        mm(0);
        rd(0, st ^ 1, 0);
        mm(1);
    };
    int q = 0;
    for (; q + 2 <= KT; q += 2) {
        step(q, std::integral_constant<int, 0>{});
        step(q + 1, std::integral_constant<int, 1>{});
    }
    if (q < KT) step(q, std::integral_constant<int, 0>{});
    __syncthreads();  // every wave is done reading the operand stages

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
            float h[8];
#pragma unroll
            for (int i = 0; i < 8; i++) h[i] = silu(cr[j0 + i]) * cr[64 + j0 + i];
            const int64_t o = m * ep.ldh + n0 / 2 + j0;
            if (ep.hmid_q8_0) {
                // the Q8_0 block of these 8 columns is the 32 of lanes 4q .. 4q + 3
                // (one row: all four in or out of range together)
                float a = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) a = fmaxf(a, fabsf(h[i]));
                a = fmaxf(a, __shfl_xor(a, 1));
                a = fmaxf(a, __shfl_xor(a, 2));
                float sc, dq;
                q8_0_scales(a, sc, dq);
                const u32x2 lo = q8_0_values4(f32x4{h[0], h[1], h[2], h[3]}, sc, dq);
                const u32x2 hi = q8_0_values4(f32x4{h[4], h[5], h[6], h[7]}, sc, dq);
                *(u32x4 *)(ep.hmid + o) = u32x4{lo[0], lo[1], hi[0], hi[1]};
            } else if (ep.hmid_f32) {
                *(f32x4 *)(ep.hmid_f32 + o) = f32x4{h[0], h[1], h[2], h[3]};
                *(f32x4 *)(ep.hmid_f32 + o + 4) = f32x4{h[4], h[5], h[6], h[7]};
            } else {
                *(u32x4 *)(ep.hmid + o) = u32x4{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]),
                                               pack_bf16x2(h[4], h[5]), pack_bf16x2(h[6], h[7])};
            }
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

int device_cus() { return device_cu_count(); }

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

int device_cu_count() {
    // initialised once, by the first caller (a function-local static: thread-safe)
    static const int cus = [] {
        int dev = 0, v = 0;
        return (hipGetDevice(&dev) == hipSuccess &&
                hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
                   ? v
                   : 0;
    }();
    return cus;
}

// K split of the 128x128 kernel, chosen by a cost estimate in microseconds:
// each workgroup's k steps at 0.64 us per 64-k step when it has its CU to
// itself, 0.58 us per step and workgroup when two or more share a CU (two are
// resident at once; the second hides little of the first's issue-bound loop);
// then, for a split product, the reduction launch (8.4 us) and the partial sums
// written and read once (8 s m N bytes at ~6.5 TB/s), and for an unsplit one
// the fused epilogue (9.6 us). Shares are whole 256-value super-blocks of at
// least 512 k, and a split grid stays within two workgroups per CU, which also
// bounds the partial sums by 2 x CUs f32 128x128 tiles. Fitted to the Q8_0,
// Q4_K and Q6_K projections of hidden 3072 and 4096 at 256 and 384 tokens, it
// picks the measured best share count or one within 3% of it on each, e.g.
// Q8_0 3072x9216 at 256 tokens: 4 shares, 36.7 us (2 shares: 59.7), and
// 9216x3072: 3 shares, 37.5 us (unsplit: 40.3).
int qgemm_mid_splits(const GemmWeight &w, int64_t m) {
    if (m <= 0 || qgemm_large_fits(w, m) || qgemm_stream_fits(w, m)) return 1;
    const int64_t tiles = (w.n / BN) * ((m + BM - 1) / BM), cus = device_cus(), steps = w.k / BK;
    if (cus <= 0) return 1;
    auto cost = [&](int s) {
        const int64_t per_cu = (tiles * s + cus - 1) / cus;
        const double st = (double)(steps / s);
        const double loop = per_cu <= 1 ? 0.64 * st : 0.58 * (double)per_cu * st;
        return loop + (s == 1 ? 9.6 : 8.4 + 8.0 * s * (double)m * (double)w.n / 6.5e6);
    };
    int best = 1;
    double best_cost = cost(1);
    for (int s = 2; s <= MAX_MID_SPLITS; s++) {
        if (w.k % (256 * s) || w.k / s < 512 || tiles * s > 2 * cus) continue;
        const double c = cost(s);
        if (c < best_cost) {
            best_cost = c;
            best = s;
        }
    }
    return best;
}

namespace {

// Rows of a large-M product handed to the shorter-M paths so that the 256x256
// kernel runs whole waves: when the 256x256 tiles leave a last, partial wave
// of at most a quarter of the CUs made of whole 256-row tile rows (4352 tokens
// x N = 4096: 272 tiles for 256 CUs), those rows go to the split-K 128x128
// kernel (or the short-M path) instead (tail_rows below names the epilogues
// whose rows can be shifted); 0 = none. `pairs`: the paired SwiGLU form, whose
// workgroups take two tiles each (its rounds are counted in pairs).
int64_t large_tail_rows(const GemmWeight &w, int64_t m, bool pairs = false) {
    if (!qgemm_large_fits(w, m)) return 0;
    const int64_t mt = (m + 255) / 256, nt = w.n / 256 / (pairs ? 2 : 1), tiles = mt * nt, cus = device_cus();
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
enum class SmallPath { STREAM, SPLIT, WHOLE };
SmallPath small_path(const GemmWeight &w, int64_t m, const EpiParams &ep) {
    if (qgemm_stream_fits(w, m) && ep.part_ws && ep.part_ws_bytes >= qgemm_stream_workspace(w, m))
        return SmallPath::STREAM;
    if (qgemm_mid_splits(w, m) > 1 && ep.part_ws && ep.part_ws_bytes >= qgemm_workspace(w, m)) return SmallPath::SPLIT;
    return SmallPath::WHOLE;
}

hipError_t launch_small(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi, const EpiParams &ep,
                        hipStream_t stream) {
    const SmallPath path = small_path(w, m, ep);
    if (path == SmallPath::STREAM) return launch_qgemm_stream(w, a, m, lda, epi, ep, ep.part_ws, stream);
    if (path == SmallPath::SPLIT) {
        const int splits = qgemm_mid_splits(w, m);
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
        size_t need = 0;
        for (bool pairs : {false, true})
            if (const int64_t tail = large_tail_rows(w, m, pairs)) need = std::max(need, small_workspace(w, tail));
        return need;
    }
    return small_workspace(w, m);
}

namespace {

// The large-M tail (large_tail_rows) of a product whose epilogue's rows can be
// shifted: plain outputs, SwiGLU, the gated residual when the tail's rows
// share one gate row, and q/k/v when they lie in one sequence and take the
// undivided 128x128 kernel (its epilogue then sees positions 0 .. of outputs
// shifted to the tail's first position; the split q/k/v reduction takes whole
// sequences only); 0 = none.
int64_t tail_rows(const GemmWeight &w, int64_t m, int epi, const EpiParams &ep) {
    const int64_t tail = large_tail_rows(w, m, epi == EPI_SWIGLU && ep.hmid_q8k && qgemm_wide_pairs_fit(w));
    if (!tail || !ep.part_ws || ep.part_ws_bytes < small_workspace(w, tail)) return 0;
    if (epi == EPI_F32 || epi == EPI_BF16 || epi == EPI_SWIGLU) return tail;
    if (epi == EPI_RESID && ep.g_rows_per > 0 && (m - tail) / ep.g_rows_per == (m - 1) / ep.g_rows_per)
        return tail;
    if (epi == EPI_QKV && ep.seq > 0 && (m - tail) / ep.seq == (m - 1) / ep.seq &&
        small_path(w, tail, ep) == SmallPath::WHOLE)
        return tail;
    return 0;
}

// The epilogue of rows head .. of a product as that of a product of its own
EpiParams rows_from(const EpiParams &ep, int epi, const GemmWeight &w, int64_t head) {
    EpiParams e = ep;
    if (epi == EPI_F32 || epi == EPI_BF16) {
        e.out = (char *)ep.out + (size_t)head * (size_t)ep.ldo * (epi == EPI_F32 ? 4 : 2);
    } else if (epi == EPI_RESID) {
        e.x_in = ep.x_in + head * w.n;
        e.x_out = ep.x_out + head * w.n;
        e.gvec = ep.gvec + (head / ep.g_rows_per) * ep.g_stride;
    } else if (epi == EPI_SWIGLU) {
        e.hmid = ep.hmid + head * ep.ldh;
        if (ep.hmid_f32) e.hmid_f32 = ep.hmid_f32 + head * ep.ldh;
    } else if (epi == EPI_QKV) {
        // sequence b0 from position s0: with positions 0 .. (m < seq - s0) the
        // epilogue's rows ((b H + h) S + s) land at ((b0 H + h) S + s0 + m)
        const int64_t S = ep.seq, H = ep.heads, b0 = head / S, s0 = head % S;
        if (ep.q) e.q = ep.q + (b0 * H * S + s0) * 128;
        if (ep.k) e.k = ep.k + (b0 * H * S + s0) * 128;
        if (ep.vt) e.vt = ep.vt + b0 * H * 128 * S + s0;
        if (ep.v_bhsd) e.v_bhsd = ep.v_bhsd + (b0 * H * S + s0) * 128;
        if (ep.pe) e.pe = ep.pe + s0 * 128;
    }
    return e;
}

}  // namespace

hipError_t launch_qgemm(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                        const EpiParams &ep, hipStream_t stream) {
    if (m <= 0) return hipSuccess;
    // a last, nearly empty round of 256x256 tiles: those rows as a shorter-M
    // product of their own (whole rounds above, the 128x128 or short-M path
    // for the tail), each part with its own form of the epilogue
    if (const int64_t tail = tail_rows(w, m, epi, ep)) {
        const int64_t head = m - tail;
        const hipError_t e = launch_qgemm(w, a, head, lda, epi, ep, stream);
        if (e != hipSuccess) return e;
        return launch_qgemm(w, a + head * lda, tail, lda, epi, rows_from(ep, epi, w, head), stream);
    }
    if (epi == EPI_SWIGLU && ep.hmid_q8k) {
        // the Q8_K rounding of the hidden state: inside the paired large-M
        // kernel where it runs, else the f32 state and then the rows quantizer
        if (!ep.hmid || !ep.hmid_f32 || ep.ldh % 256 || (w.n / 2) % 256) return hipErrorInvalidValue;
        if (qgemm_large_fits(w, m) && qgemm_wide_pairs_fit(w)) return launch_qgemm_large(w, a, m, lda, epi, ep, stream);
        EpiParams e = ep;
        e.hmid_q8k = 0;
        const hipError_t err = launch_qgemm(w, a, m, lda, EPI_SWIGLU, e, stream);
        if (err != hipSuccess) return err;
        return launch_quant_rows(ep.hmid_f32, ep.ldh, m, w.n / 2, 256, ep.hmid, ep.ldh, stream);
    }
    if (epi == EPI_SWIGLU && ep.hmid_q8_0) {
        // the Q8_0 rounding of the hidden state: in the epilogue of the large-M
        // kernel or the undivided 128x128 kernel where one of them runs, else
        // the f32 state and then the rows quantizer
        if (!ep.hmid || !ep.hmid_f32 || (w.n / 2) % 32) return hipErrorInvalidValue;
        if (qgemm_large_fits(w, m) ? qgemm_wide_fits(w) : small_path(w, m, ep) == SmallPath::WHOLE)
            return qgemm_large_fits(w, m) ? launch_qgemm_large(w, a, m, lda, epi, ep, stream)
                                          : launch_small(w, a, m, lda, epi, ep, stream);
        EpiParams e = ep;
        e.hmid_q8_0 = 0;
        const hipError_t err = launch_qgemm(w, a, m, lda, EPI_SWIGLU, e, stream);
        if (err != hipSuccess) return err;
        return launch_quant_rows(ep.hmid_f32, ep.ldh, m, w.n / 2, 32, ep.hmid, ep.ldh, stream);
    }
    if (qgemm_large_fits(w, m)) return launch_qgemm_large(w, a, m, lda, epi, ep, stream);
    return launch_small(w, a, m, lda, epi, ep, stream);
}

}  // namespace qimm
