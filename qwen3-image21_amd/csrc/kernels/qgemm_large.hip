// Large-M dequant-GEMM for gfx950 (M >= 512 token rows): C = A (bf16) x W^T
// (GGUF blocks), same epilogues as the 128x128 kernel. Quantized weights with
// K % 256 == 0 take the eight-wave kernel of qgemm_wide.hip instead; this one
// serves bf16-stored weights and the remaining quantized shapes.
//
// Replaces candle's QMatMul::forward (src/quantized_transformer.rs:19-33) on
// the block's token-parallel projections (call sites 133-135, 151, 196, 202).
//
// Tile 256x256x64, 256 threads = 4 waves in a 2x2 grid, each wave 128x128 as
// 4x4 v_mfma_f32_32x32x16_bf16 tiles (accumulators live in AGPRs), one
// workgroup per CU. Per 16-wide k slice a wave reads 8 KB of operands from LDS
// for 16 MFMAs, half the LDS traffic per flop of a 64x64 wave tile. LDS rows
// are dense 128 B with the 16 B chunk index XOR-swizzled by (row & 7), so both
// the staging writes and the MFMA operand reads are bank-conflict free.
// The A tile goes global->LDS directly (no registers); the raw weights are
// loaded two steps ahead and those of step k+1 are dequantized into the other
// LDS stage between the MFMAs of step k. One barrier per 64-wide k step; the
// operand fragments of the next 16-wide slice are read while the current
// slice's MFMAs run. The q/k/v epilogue stages its outputs through LDS; the
// others work on the accumulators in place.
// Tiles are ordered XCD-aware: each XCD gets a contiguous range of tiles,
// grouped 4 M-tiles at a time so concurrently resident tiles share A rows and
// W columns in that XCD's L2.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int ROWB = 128;                      // bytes per LDS row: 64 bf16
constexpr int STAGE = 2 * 256 * ROWB;          // A rows then B rows: 64 KB
constexpr int QP = 132;                        // f32 pitch of the q/k epilogue rows (128 + 4: conflict free)
constexpr int LDS_BYTES = 4 * 64 * QP * 4;     // 132 KB: the two operand stages (128 KB) or four waves' q/k rows
static_assert(LDS_BYTES >= 2 * STAGE, "operand stages fit");
constexpr int GROUP_M = 4;

// A word whose value the optimizer must not look through (keeps nibble masks as
// whole-word ops so the byte converts below stay v_cvt_f32_ubyte{0..3}).
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ uint32_t byte_of(const u32x4 &x, int i) {
    return (x[i >> 2] >> (8 * (i & 3))) & 0xffu;
}

// Q4_K 6-bit scale/min of sub-block j from the 12 packed bytes at bytes 4..15
// of the block header word (GGML layout).
// Branch-free: j comes from the k step at run time, and a branch here would
// split the step's scheduling region.
__device__ __forceinline__ void q4k_sc_m(const u32x4 &h, int j, float &sc, float &mn) {
    // the 12 packed bytes sit at header bytes 4..15: scales[i] = byte 4 + i
    const int jl = j & 3;
    const uint32_t b4 = byte_of(h, 4 + jl), b8 = byte_of(h, 8 + jl), b12 = byte_of(h, 12 + jl);
    const uint32_t s_lo = b4 & 63u, m_lo = b8 & 63u;                         // sub-blocks 0-3
    const uint32_t s_hi = (b12 & 0xFu) | ((b4 >> 6) << 4);                   // sub-blocks 4-7
    const uint32_t m_hi = (b12 >> 4) | ((b8 >> 6) << 4);
    sc = (float)(j < 4 ? s_lo : s_hi);
    mn = (float)(j < 4 ? m_lo : m_hi);
}

// 8 unsigned byte codes (two words) -> 8 bf16 of code*ds + off (exact f32 value,
// rounded to nearest even).
__device__ __forceinline__ u32x4 cvt8(uint32_t x0, uint32_t x1, float ds, float off) {
    auto f = [&](uint32_t x, int i) { return __builtin_fmaf((float)((x >> (8 * i)) & 0xffu), ds, off); };
    return u32x4{pack_bf16x2(f(x0, 0), f(x0, 1)), pack_bf16x2(f(x0, 2), f(x0, 3)),
                 pack_bf16x2(f(x1, 0), f(x1, 1)), pack_bf16x2(f(x1, 2), f(x1, 3))};
}

__device__ __forceinline__ uint32_t word(const u32x4 *v, int byte_off) {
    return v[byte_off >> 4][(byte_off >> 2) & 3];
}

// Raw bytes of one weight row for one 64-wide k step.
struct WRaw {
    u32x4 v[8];
    uint32_t s;
};

template <int FMT>
__device__ __forceinline__ void load_w(const GemmWeight &w, int64_t n, int64_t k0, WRaw &r) {
    const int64_t K = w.k;
    if constexpr (FMT == WF_Q8_0) {
        const uint8_t *p = w.q + n * K + k0;
#pragma unroll
        for (int i = 0; i < 4; i++) r.v[i] = *(const u32x4 *)(p + 16 * i);
        r.s = *(const uint32_t *)(w.scales + n * (K / 32) + k0 / 32);
    } else if constexpr (FMT == WF_Q4_K) {
        const uint8_t *blk = q4k_block(w.q, n, k0 / 256, K / 256);
        const int c = (int)((k0 & 255) >> 6);
        r.v[0] = *(const u32x4 *)blk;
        r.v[1] = *(const u32x4 *)(blk + 16 + 32 * c);
        r.v[2] = *(const u32x4 *)(blk + 32 + 32 * c);
    } else if constexpr (FMT == WF_Q6_K) {
        const uint8_t *blk = q6k_block(w.q, n, k0 / 256, K / 256);
        const int hh = (int)((k0 & 255) >> 7);
#pragma unroll
        for (int i = 0; i < 4; i++) r.v[i] = *(const u32x4 *)(blk + 64 * hh + 16 * i);
        r.v[4] = *(const u32x4 *)(blk + 128 + 32 * hh);
        r.v[5] = *(const u32x4 *)(blk + 144 + 32 * hh);
        r.v[6] = *(const u32x4 *)(blk + 192);
        r.s = *(const uint16_t *)(blk + 208);
    } else {
        const uint8_t *p = w.q + (n * K + k0) * 2;
#pragma unroll
        for (int i = 0; i < 8; i++) r.v[i] = *(const u32x4 *)(p + 16 * i);
    }
}

// Per-step dequant constants of one row.
struct WScale {
    float a0, b0, a1, b1, a2, b2, a3, b3;
};

template <int FMT>
__device__ __forceinline__ WScale w_scales(const WRaw &r, int64_t k0) {
    WScale s{};
    if constexpr (FMT == WF_Q8_0) {
        const float d0 = f16_bits_to_f32(r.s & 0xffffu), d1 = f16_bits_to_f32(r.s >> 16);
        s.a0 = d0;  // codes biased to unsigned: (q+128)*d - 128*d, exact
        s.b0 = -128.f * d0;
        s.a1 = d1;
        s.b1 = -128.f * d1;
    } else if constexpr (FMT == WF_Q4_K) {
        const int c = (int)((k0 & 255) >> 6);
        const float d = f16_bits_to_f32(r.v[0][0] & 0xffffu), dmin = f16_bits_to_f32(r.v[0][0] >> 16);
        float sc0, m0, sc1, m1;
        q4k_sc_m(r.v[0], 2 * c, sc0, m0);
        q4k_sc_m(r.v[0], 2 * c + 1, sc1, m1);
        // low nibbles (sub-block 2c) sit at f16 bits 0-3, high nibbles
        // (sub-block 2c+1) at bits 4-7: the scales carry 2^24 and 2^20
        s.a0 = d * sc0 * 0x1p24f;
        s.b0 = -(dmin * m0);
        s.a1 = d * sc1 * 0x1p20f;
        s.b1 = -(dmin * m1);
    } else if constexpr (FMT == WF_Q6_K) {
        // values 32 r + l of half hh, r in {2o, 2o+1}; scale index 8hh + 2r + l/16
        const int hh = (int)((k0 & 255) >> 7), o = (int)((k0 & 127) >> 6);
        const float d = f16_bits_to_f32(r.s);
        const int base = 8 * hh + 4 * o;
        const float d0 = d * (float)(int8_t)byte_of(r.v[6], base + 0);
        const float d1 = d * (float)(int8_t)byte_of(r.v[6], base + 1);
        const float d2 = d * (float)(int8_t)byte_of(r.v[6], base + 2);
        const float d3 = d * (float)(int8_t)byte_of(r.v[6], base + 3);
        // codes sit at f16 bits 0-5 (the subnormal q * 2^-24), so the scales carry
        // 2^24; q*ds - 32*ds with both products exact and one rounding
        s.a0 = d0 * 0x1p24f;
        s.a1 = d1 * 0x1p24f;
        s.a2 = d2 * 0x1p24f;
        s.a3 = d3 * 0x1p24f;
        s.b0 = -32.f * d0;
        s.b1 = -32.f * d1;
        s.b2 = -32.f * d2;
        s.b3 = -32.f * d3;
    }
    return s;
}

// bf16 values k in [8j, 8j+8) of the step.
template <int FMT>
__device__ __forceinline__ u32x4 w_chunk(const WRaw &r, const WScale &s, int j, int64_t k0) {
    if constexpr (FMT == WF_Q8_0) {
        const uint32_t x0 = opaque(word(r.v, 8 * j) ^ 0x80808080u), x1 = opaque(word(r.v, 8 * j + 4) ^ 0x80808080u);
        return j < 4 ? cvt8(x0, x1, s.a0, s.b0) : cvt8(x0, x1, s.a1, s.b1);
    } else if constexpr (FMT == WF_Q4_K) {
        // k < 32: low nibbles of qs bytes [8j, 8j+8); k >= 32: high nibbles of
        // bytes [8(j-4), ...). The halves of (y & m) hold bytes 0 and 2, those
        // of ((y >> 8) & m) bytes 1 and 3.
        const int jb = j & 3;
        const uint32_t y0 = word(r.v + 1, 8 * jb), y1 = word(r.v + 1, 8 * jb + 4);
        const uint32_t m = j < 4 ? 0x000F000Fu : 0x00F000F0u;
        const float a = j < 4 ? s.a0 : s.a1, b = j < 4 ? s.b0 : s.b1;
        const uint32_t p0 = y0 & m, p1 = (y0 >> 8) & m, p2 = y1 & m, p3 = (y1 >> 8) & m;
        return u32x4{pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)), pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                     pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)), pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))};
    } else if constexpr (FMT == WF_Q6_K) {
        // k = 32 rl + l with rl = j/4, l in [8(j%4), +8): low 4 bits from ql byte
        // 32 rl + l (low nibble when o == 0, else high), high 2 bits from qh byte l
        // >> 2r with r = 2o + rl; scale index 2 rl + l/16.
        const int o = (int)((k0 & 127) >> 6);
        const int rl = j >> 2, l0 = 8 * (j & 3);
        const int rr = 2 * o + rl;
        uint32_t q0 = word(r.v, 32 * rl + l0), q1 = word(r.v, 32 * rl + l0 + 4);
        if (o) {
            q0 >>= 4;
            q1 >>= 4;
        }
        const uint32_t h0 = word(r.v + 4, l0), h1 = word(r.v + 4, l0 + 4);
        const uint32_t c0 = opaque((q0 & 0x0F0F0F0Fu) | (((h0 >> (2 * rr)) & 0x03030303u) << 4));
        const uint32_t c1 = opaque((q1 & 0x0F0F0F0Fu) | (((h1 >> (2 * rr)) & 0x03030303u) << 4));
        const int si = 2 * rl + (l0 >> 4);
        const float a = si == 0 ? s.a0 : (si == 1 ? s.a1 : (si == 2 ? s.a2 : s.a3));
        const float b = si == 0 ? s.b0 : (si == 1 ? s.b1 : (si == 2 ? s.b2 : s.b3));
        // the 6-bit codes fill whole bytes (<= 63): the halves of (c & 0x00FF00FF)
        // hold bytes 0 and 2, those of perm(c) bytes 1 and 3
        const uint32_t p0 = c0 & 0x00FF00FFu, p1 = __builtin_amdgcn_perm(0u, c0, 0x0C030C01u);
        const uint32_t p2 = c1 & 0x00FF00FFu, p3 = __builtin_amdgcn_perm(0u, c1, 0x0C030C01u);
        return u32x4{pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)), pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                     pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)), pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))};
    } else {
        return r.v[j];
    }
}

// silu with the hardware reciprocal (about 1 ulp): an IEEE divide here is ~8
// instructions per value, a third of the SwiGLU epilogue's code.
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

template <int FMT, int EPI>
__global__ __launch_bounds__(256, 1) void qgemm_large_kernel(const uint16_t *__restrict__ A, int64_t M,
                                                             int64_t lda, GemmWeight w, EpiParams ep,
                                                             int mt, int nt) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
    // the wave index as a scalar: the LDS destinations of the direct loads are
    // then scalar values set into M0 without a lane read per load
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, l32 = lane & 31, g = lane >> 5;

    // XCD-aware, M-grouped tile order
    const int total = mt * nt;
    int L = blockIdx.x;
    if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
    const int per_group = GROUP_M * nt;
    const int grp = L / per_group;
    const int first_m = grp * GROUP_M;
    const int gm = min(mt - first_m, GROUP_M);
    const int mtile = first_m + (L % per_group) % gm;
    const int ntile = (L % per_group) / gm;
    const int64_t m0 = (int64_t)mtile * BM, n0 = (int64_t)ntile * BN;
    const int64_t K = w.k;
    const int KT = (int)(K / BK);

    // A staging by direct global->LDS loads (16 B per lane, lane l lands at
    // base + 16 l): instruction i of wave w fills LDS rows 8(8w+i) .. +8, lane l
    // row 8(8w+i) + l/8 at slot l%8, which must hold logical chunk
    // (l%8) ^ swz_key(row). Rows past M are clamped to row M-1: they only feed
    // output rows the epilogue never writes.
    const uint16_t *asrc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int row = 8 * (8 * wave + i) + (lane >> 3);
        const int c = (lane & 7) ^ swz_key(row);
        asrc[i] = A + min(m0 + row, M - 1) * lda + 8 * c;
    }
    auto dma_a = [&](int stage, int64_t k0) {
        uint8_t *base = lds + stage * STAGE;
#pragma unroll
        for (int i = 0; i < 8; i++)
            __builtin_amdgcn_global_load_lds((const void *)(asrc[i] + k0), (lds_ptr_t)(base + (8 * wave + i) * 8 * ROWB),
                                             16, 0, 0);
    };
    // bf16 weights (a dequantized copy, [N][K]) take the A path: direct
    // global->LDS loads into the B rows of the stage, same swizzle
    const uint16_t *bsrc[8];
    if constexpr (FMT == WF_BF16) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int row = 8 * (8 * wave + i) + (lane >> 3);
            const int c = (lane & 7) ^ swz_key(row);
            bsrc[i] = (const uint16_t *)w.q + (n0 + row) * K + 8 * c;
        }
    }
    auto dma_b = [&](int stage, int64_t k0) {
        uint8_t *base = lds + stage * STAGE + 256 * ROWB;
#pragma unroll
        for (int i = 0; i < 8; i++)
            __builtin_amdgcn_global_load_lds((const void *)(bsrc[i] + k0), (lds_ptr_t)(base + (8 * wave + i) * 8 * ROWB),
                                             16, 0, 0);
    };
    // W staging (quantized): row n0 + tid, all 8 chunks, through registers
    // (dequantized); raw weights double-buffered two steps ahead
    const int64_t wrow = n0 + tid;
    WRaw rw[2];

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // operand fragments of one 16-wide k slice, double-buffered across slices
    // (buffer and slice indices are compile-time after unrolling)
    bf16x8 fa[2][4], fb[2][4];
    auto rd = [&](int buf, int stage, int kk) __attribute__((always_inline)) {
        const uint8_t *as = lds + stage * STAGE;
        const uint8_t *bs = as + 256 * ROWB;
#pragma unroll
        for (int i = 0; i < 4; i++) fa[buf][i] = *(const bf16x8 *)(as + swz(wm * 128 + i * 32 + l32, 2 * kk + g));
#pragma unroll
        for (int j = 0; j < 4; j++) fb[buf][j] = *(const bf16x8 *)(bs + swz(wn * 128 + j * 32 + l32, 2 * kk + g));
        // bf16 weights: the reads stay ahead of the MFMAs that follow (those
        // use the other buffer); left alone, the scheduler sinks each read to
        // just before its first use and waits out the LDS latency there (q/k/v
        // shape 441-458 -> 416-424 us). The dequantizing forms keep the
        // scheduler's order: their decode VALU already fills that latency, and
        // Q6_K measured 507 -> 585 us with the reads pinned.
        if constexpr (FMT == WF_BF16) __builtin_amdgcn_sched_barrier(0);
    };
    auto mm = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int i = q >> 2, j = q & 3;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[buf][i], fb[buf][j], acc[i][j], 0, 0, 0);
        }
    };

    if constexpr (FMT == WF_BF16) {
        // both operands of steps 0 and 1 in flight, then the same one-barrier
        // step as below without the dequantization
        dma_a(0, 0);
        dma_b(0, 0);
        dma_a(1, (int64_t)min(1, KT - 1) * BK);
        dma_b(1, (int64_t)min(1, KT - 1) * BK);
        __builtin_amdgcn_s_waitcnt(WAIT_VM0_LGKM0);  // vmcnt(0) lgkmcnt(0)
        __syncthreads();
        rd(0, 0, 0);
        auto step_b = [&](int kt, auto sc_) __attribute__((always_inline)) {
            constexpr int s = decltype(sc_)::value, t = s ^ 1;
            rd(1, s, 1);
            mm(0);
            rd(0, s, 2);
            mm(1);
            rd(1, s, 3);
            mm(0);
            __builtin_amdgcn_s_waitcnt(WAIT_VM0_LGKM0);  // stage t's loads (issued a step ago) landed
            __syncthreads();
            dma_a(s, (int64_t)min(kt + 2, KT - 1) * BK);
            dma_b(s, (int64_t)min(kt + 2, KT - 1) * BK);
            rd(0, t, 0);
            mm(1);
        };
        int kt = 0;
        for (; kt + 1 < KT; kt += 2) {
            step_b(kt, std::integral_constant<int, 0>{});
            step_b(kt + 1, std::integral_constant<int, 1>{});
        }
        if (kt < KT) step_b(kt, std::integral_constant<int, 0>{});
    } else {
    // prologue: step 0 staged in stage 0; raw weights of steps 1 and 2 and the
    // A tile of step 1 loaded (step indices clamped to the last step: redundant
    // loads, no branches)
    load_w<FMT>(w, wrow, 0, rw[0]);
    dma_a(0, 0);
    __builtin_amdgcn_s_waitcnt(WAIT_VM0);  // vmcnt(0)
    {
        const WScale sc = w_scales<FMT>(rw[0], 0);
        uint8_t *bn = lds + 256 * ROWB;
#pragma unroll
        for (int j = 0; j < 8; j++) *(u32x4 *)(bn + swz(tid, j)) = w_chunk<FMT>(rw[0], sc, j, 0);
    }
    load_w<FMT>(w, wrow, (int64_t)min(1, KT - 1) * BK, rw[1]);
    dma_a(1, (int64_t)min(1, KT - 1) * BK);
    load_w<FMT>(w, wrow, (int64_t)min(2, KT - 1) * BK, rw[0]);
    __builtin_amdgcn_s_waitcnt(WAIT_VM0_LGKM0);  // vmcnt(0) lgkmcnt(0)
    __syncthreads();
    rd(0, 0, 0);

    // Step kt, stage s = kt & 1, t = s ^ 1. On entry fa/fb[0] hold slice 0 of
    // step kt, rw[t] holds the raw weights of step kt+1, rw[s] those of step
    // kt+2 and stage t holds the A tile of step kt+1. Slices 0-2 dequantize step
    // kt+1 into stage t while their MFMAs run; then ONE barrier per step: stage t
    // is complete, and every wave is done reading stage s (its last slice sits
    // in registers). After it, stage s receives the A tile of step kt+2 and
    // rw[t] the raw weights of step kt+3 while slice 3 computes and slice 0 of
    // step kt+1 is read. The vmcnt(0) before the barrier covers loads issued a
    // whole step earlier.
    auto step = [&](int kt, auto sc_) __attribute__((always_inline)) {
        constexpr int s = decltype(sc_)::value, t = s ^ 1;
        const int64_t knext = (int64_t)min(kt + 1, KT - 1) * BK;
        uint8_t *bn = lds + t * STAGE + 256 * ROWB;
        const WScale sc = w_scales<FMT>(rw[t], knext);
        rd(1, s, 1);
        mm(0);
#pragma unroll
        for (int c = 0; c < 3; c++) *(u32x4 *)(bn + swz(tid, c)) = w_chunk<FMT>(rw[t], sc, c, knext);
        rd(0, s, 2);
        mm(1);
#pragma unroll
        for (int c = 3; c < 6; c++) *(u32x4 *)(bn + swz(tid, c)) = w_chunk<FMT>(rw[t], sc, c, knext);
        rd(1, s, 3);
        mm(0);
#pragma unroll
        for (int c = 6; c < 8; c++) *(u32x4 *)(bn + swz(tid, c)) = w_chunk<FMT>(rw[t], sc, c, knext);
        __builtin_amdgcn_s_waitcnt(WAIT_VM0_LGKM0);  // vmcnt(0) lgkmcnt(0)
        __syncthreads();
        dma_a(s, (int64_t)min(kt + 2, KT - 1) * BK);
        load_w<FMT>(w, wrow, (int64_t)min(kt + 3, KT - 1) * BK, rw[t]);
        rd(0, t, 0);
        mm(1);
    };
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
        step(kt, std::integral_constant<int, 0>{});
        step(kt + 1, std::integral_constant<int, 1>{});
    }
    if (kt < KT) step(kt, std::integral_constant<int, 0>{});
    }
    __builtin_amdgcn_s_waitcnt(WAIT_VM0);  // vmcnt(0): no load into LDS still in flight

    // ---- epilogue, straight from the accumulators ----
    // acc[i][j][r] holds row wm*128 + 32i + 8(r/4) + 4g + (r%4) and column
    // wn*128 + 32j + l32 of the tile: each lane owns one column of 16 rows per
    // (i, j), 32 lanes cover 32 consecutive columns.
    const int64_t N = w.n;
    const int64_t nw = n0 + wn * 128;  // first global column of this wave
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t mi = m0 + wm * 128 + i * 32 + 4 * g;
        if constexpr (EPI == EPI_F32 || EPI == EPI_BF16) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = mi + 8 * (r >> 2) + (r & 3);
                if (m >= M) continue;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int64_t n = nw + j * 32 + l32;
                    const float v = acc[i][j][r];
                    if constexpr (EPI == EPI_F32) {
                        ((float *)ep.out)[m * ep.ldo + n] = v;
                    } else {
                        ((uint16_t *)ep.out)[m * ep.ldo + n] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
                    }
                }
            }
        } else if constexpr (EPI == EPI_RESID) {
            // Every load of the 16 rows x 4 columns first (rows past M clamped
            // to M-1), then the stores: one memory round trip per 32 rows
            // instead of one per row. x_out may alias x_in: each element is read
            // and written by the same lane, loads before stores.
            float xv[16][4], gv[16][4];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = min(mi + 8 * (r >> 2) + (r & 3), M - 1);
                const float *grow = ep.gvec + (int64_t)((int)m / (int)ep.g_rows_per) * ep.g_stride;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int64_t n = nw + j * 32 + l32;
                    xv[r][j] = ep.x_in[m * N + n];
                    gv[r][j] = grow[n];
                }
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = mi + 8 * (r >> 2) + (r & 3);
                if (m >= M) continue;
#pragma unroll
                for (int j = 0; j < 4; j++) ep.x_out[m * N + nw + j * 32 + l32] = xv[r][j] + gv[r][j] * acc[i][j][r];
            }
        } else if constexpr (EPI == EPI_SWIGLU) {
            // columns 32j + l32 (j < 2) are gate, 64 + 32j + l32 the matching up
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = mi + 8 * (r >> 2) + (r & 3);
                if (m >= M) continue;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float h = silu(acc[i][j][r]) * acc[i][j + 2][r];
                    const int64_t o = m * ep.ldh + nw / 2 + j * 32 + l32;
                    if (ep.hmid_f32)
                        ep.hmid_f32[o] = h;
                    else
                        ep.hmid[o] = (uint16_t)(pack_bf16x2(h, 0.f) & 0xffffu);
                }
            }
        }
    }
    if constexpr (EPI == EPI_QKV) {
        // This wave's 128 columns are one head of q, k or v; its 128 rows are
        // staged as bf16 in a private 32 KB LDS tile (q/k row-major [t][d], v
        // transposed [d][t]) and then stored as whole 16 B chunks.
        __syncthreads();  // every wave is done reading the last operand stage
        uint16_t *tile = (uint16_t *)lds + wave * 128 * 128;
        const int64_t nb = nw + ep.n_offset;
        const int sec = (int)(nb / ep.hidden);
        const int64_t head = (nb % ep.hidden) / 128;
        const int S = (int)ep.seq;
        const int64_t H = ep.heads;
        const int64_t mw = m0 + wm * 128;  // first row of this wave
        if (sec < 2) {
            // q/k: RMSNorm over the head's 128 columns, RoPE on (2i, 2i+1), q
            // also scaled, bf16 rows to [B,H,S,128]; one 64-row half at a
            // time with one token row per lane. The half's accumulators go to
            // this wave's 33 KB of LDS as f32 rows with a pitch of 132 floats
            // (16 B reads of 16 rows then cover all 64 banks once), and each
            // lane reads its row back 16 B at a time, so the row reduction and
            // the RoPE partner stay inside the lane. The code stays compact:
            // the same work done in the accumulator layout unrolls to ~10K
            // instructions that stream through the instruction cache once per
            // tile.
            float *ft = (float *)lds + wave * 64 * QP;
            // the norm weights are the same for every lane and unchanged by the
            // kernel: read through the constant address space (scalar loads)
            typedef __attribute__((address_space(4))) const f32x4 cf32x4;
            const __attribute__((address_space(4))) float *nwt =
                (const __attribute__((address_space(4))) float *)(sec == 0 ? ep.norm_q : ep.norm_k);
            const float osc = sec == 0 ? ep.q_scale : 1.0f;
            uint16_t *dst = sec == 0 ? ep.q : ep.k;
            const uint32_t Su = (uint32_t)S, Mlast = (uint32_t)(M - 1);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                // the second half's accumulators stay in place until the first is done
                __builtin_amdgcn_sched_barrier(0);
                // rows of the half to LDS, row-major with a pitch of QP floats:
                // register 4q + k of tile (ii, j) is row 32 ii + 8 q + 4 g + k,
                // column 32 j + l32
#pragma unroll
                for (int ii = 0; ii < 2; ii++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
#pragma unroll
                        for (int r = 0; r < 16; r++)
                            ft[(ii * 32 + 8 * (r >> 2) + 4 * g + (r & 3)) * QP + j * 32 + l32] = acc[2 * h + ii][j][r];
                const int64_t m = mw + h * 64 + lane;
                const uint32_t mc = min((uint32_t)m, Mlast);
                const uint32_t s = mc % Su;
                const float *pr = ep.pe + (int64_t)s * 128;  // (cos, sin) of pair i at 2i, 2i + 1
                // the row's RoPE table in four batches of 32 columns, each
                // batch's loads issued a batch ahead (the first before the sum
                // of squares)
                f32x4 pt[2][8];
#pragma unroll
                for (int e = 0; e < 8; e++) pt[0][e] = *(const f32x4 *)(pr + 4 * e);
                __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);  // lgkmcnt(0): the wave's LDS writes landed
                __builtin_amdgcn_wave_barrier();
                // each lane reads its own row back, 16 B at a time, twice: for
                // the sum of squares, then for the rotation
                const float *frow = ft + lane * QP;
                float ss4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < 128; c += 4) {
                    const f32x4 x = *(const f32x4 *)(frow + c);
                    ss4[0] += x.x * x.x;
                    ss4[1] += x.y * x.y;
                    ss4[2] += x.z * x.z;
                    ss4[3] += x.w * x.w;
                }
                const float rs = 1.0f / sqrtf(((ss4[0] + ss4[1]) + (ss4[2] + ss4[3])) * (1.0f / 128.0f) + 1e-6f);
#pragma unroll
                for (int bt = 0; bt < 4; bt++) {
                    if (bt < 3) {
#pragma unroll
                        for (int e = 0; e < 8; e++) pt[(bt + 1) & 1][e] = *(const f32x4 *)(pr + 32 * (bt + 1) + 4 * e);
                    }
#pragma unroll
                    for (int cc = 0; cc < 4; cc++) {
                        const int c0 = 32 * bt + 8 * cc;
                        const f32x4 x0v = *(const f32x4 *)(frow + c0), x1v = *(const f32x4 *)(frow + c0 + 4);
                        const f32x4 cs0 = pt[bt & 1][2 * cc], cs1 = pt[bt & 1][2 * cc + 1];
                        const f32x4 w0 = *(const cf32x4 *)(nwt + c0), w1 = *(const cf32x4 *)(nwt + c0 + 4);
                        const float xv[8] = {x0v.x, x0v.y, x0v.z, x0v.w, x1v.x, x1v.y, x1v.z, x1v.w};
                        const float cs[8] = {cs0.x, cs0.y, cs0.z, cs0.w, cs1.x, cs1.y, cs1.z, cs1.w};
                        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                        u32x4 o;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float x0 = xv[2 * e] * rs * wv[2 * e];
                            const float x1 = xv[2 * e + 1] * rs * wv[2 * e + 1];
                            const float co = cs[2 * e], sn = cs[2 * e + 1];
                            o[e] = pack_bf16x2((x0 * co - x1 * sn) * osc, (x0 * sn + x1 * co) * osc);
                        }
                        // back into the lane's own row (bytes already read)
                        *(u32x4 *)((uint16_t *)frow + c0) = o;
                    }
                }
                __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);
                __builtin_amdgcn_wave_barrier();
                // the half's bf16 rows out with 16 lanes per 256 B row, so every
                // store covers whole lines (row-per-lane stores leave partial
                // lines that reach memory more than once)
#pragma unroll 4
                for (int it = 0; it < 16; it++) {
                    const int rr = it * 4 + (lane >> 4), ch = lane & 15;
                    const int64_t mr = mw + h * 64 + rr;
                    if (mr < M) {
                        const uint32_t sr = (uint32_t)mr % Su, br = (uint32_t)mr / Su;
                        *(u32x4 *)(dst + (((int64_t)br * H + head) * S + sr) * 128 + ch * 8) =
                            *(const u32x4 *)((const uint16_t *)(ft + rr * QP) + ch * 8);
                    }
                }
                __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);
                __builtin_amdgcn_wave_barrier();  // the half is read before the next one is written
            }
        } else {
            // V^T: tile[d][t], 8-token groups XOR-swizzled by d. Registers
            // 4q .. 4q+3 hold 4 consecutive tokens (4-aligned; the swizzle
            // only flips bits 3-6): one 8 B write each. One 32-row block of
            // accumulators at a time (a scheduling fence each), so they are
            // not all copied out of the accumulator registers at once.
#pragma unroll
            for (int i = 0; i < 4; i++) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int d = j * 32 + l32;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int t = i * 32 + 8 * q + 4 * g;
                        *(u32x2 *)(tile + d * 128 + (t ^ ((d & 15) << 3))) =
                            u32x2{pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                                  pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
                    }
                }
            }
            __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);
            __builtin_amdgcn_wave_barrier();
            // one d row (128 tokens = 256 B) per 16 lanes, 16 B (8 tokens) per lane
#pragma unroll 4
            for (int pass = 0; pass < 32; pass++) {
                const int d = pass * 4 + (lane >> 4), ch = lane & 15;
                const int64_t m = mw + ch * 8;
                if (m >= M) continue;
                const u32x4 v = *(const u32x4 *)(tile + d * 128 + ((ch * 8) ^ ((d & 15) << 3)));
                const int64_t b = m / S, s = m % S;
                if ((S & 7) == 0 && m + 7 < M) {
                    *(u32x4 *)(ep.vt + ((b * H + head) * 128 + d) * S + s) = v;
                } else {
                    for (int e = 0; e < 8; e++) {
                        const int64_t me = m + e;
                        if (me >= M) break;
                        ep.vt[((me / S * H + head) * 128 + d) * S + me % S] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
                    }
                }
            }
            if (ep.v_bhsd) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int64_t m = mw + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                        if (m >= M) continue;
                        const int64_t b = m / S, s = m % S;
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            ep.v_bhsd[((b * H + head) * S + s) * 128 + j * 32 + l32] =
                                (uint16_t)(pack_bf16x2(acc[i][j][r], 0.f) & 0xffffu);
                    }
                }
            }
        }
    }
}

template <int FMT>
hipError_t launch_fmt(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                      const EpiParams &ep, hipStream_t stream) {
    const int mt = (int)((m + BM - 1) / BM), nt = (int)(w.n / BN);
    dim3 grid((unsigned)(mt * nt)), block(256);
    switch (epi) {
    case EPI_F32: qgemm_large_kernel<FMT, EPI_F32><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    case EPI_BF16: qgemm_large_kernel<FMT, EPI_BF16><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    case EPI_QKV: qgemm_large_kernel<FMT, EPI_QKV><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    case EPI_RESID: qgemm_large_kernel<FMT, EPI_RESID><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    case EPI_SWIGLU: qgemm_large_kernel<FMT, EPI_SWIGLU><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

// The 128x128 kernel (split over K where its tiles are still too few) is
// faster whenever its whole grid runs as one wave of its two resident
// workgroups per CU; beyond that its second, partial wave costs more than the
// 256x256 kernel's idle CUs. Measured: Q4_K 4096 x 4096 at 1024 tokens 109 ->
// 66 us and Q6_K 4096 x 12288 352 -> 215 us (256 tiles of 128x128), at 2048
// tokens 2-4% faster (512 tiles); the block step at 1024 image tokens 0.90 ->
// 0.71 ms. At 2304 tokens (576 tiles), 3072, and gate_up at 512 the 256x256
// kernel is faster.
bool qgemm_large_fits(const GemmWeight &w, int64_t m) {
    if (m < 512 || w.n % BN || w.k % BK) return false;
    const int64_t mid_tiles = ((m + 127) / 128) * (w.n / 128);
    return mid_tiles > 2 * (int64_t)device_cu_count();
}

hipError_t launch_qgemm_large(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                              const EpiParams &ep, hipStream_t stream) {
    if (qgemm_wide_fits(w) && (epi != EPI_QKV || ep.hidden % BN == 0))
        return launch_qgemm_wide(w, a, m, lda, epi, ep, stream);
    switch (w.fmt) {
    case WF_Q8_0: return launch_fmt<WF_Q8_0>(w, a, m, lda, epi, ep, stream);
    case WF_Q4_K: return launch_fmt<WF_Q4_K>(w, a, m, lda, epi, ep, stream);
    case WF_Q6_K: return launch_fmt<WF_Q6_K>(w, a, m, lda, epi, ep, stream);
    case WF_BF16: return launch_fmt<WF_BF16>(w, a, m, lda, epi, ep, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace qimm
