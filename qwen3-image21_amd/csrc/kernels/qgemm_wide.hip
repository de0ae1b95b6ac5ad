// Large-M dequant-GEMM for gfx950 with quantized weights (Q4_K, Q6_K, Q8_0;
// M >= 512 token rows, K % 256 == 0): C = A (bf16) x W^T, the epilogues of
// the other GEMM kernels.
//
// Replaces candle's QMatMul::forward (src/quantized_transformer.rs:19-33) on
// the block's token-parallel projections (call sites 133-135, 151, 196, 202).
//
// Tile 256 tokens x 256 weight rows x 64 k, 512 threads = 8 waves, two per
// SIMD. Each wave owns 32 weight rows and all 256 tokens: per 16-wide k slice
// it decodes ONE weight fragment (32 rows x 16 k, 8 values per lane) straight
// from the raw GGUF bytes in its registers and runs 8 v_mfma_f32_32x32x16_bf16
// against the 8 token fragments of the slice, read from LDS. So decoded
// weights never pass through LDS, every decoded value feeds 8 MFMAs, and the
// only LDS traffic is the activation tile (copied HBM->LDS by direct loads,
// double-buffered, rows XOR-swizzled) and its fragment reads.
//
// The weights are the MFMA's A operand and the tokens its B operand, so a
// lane's accumulator registers hold 16 weight rows of one token: row
// 8 (r / 4) + 4 g + r % 4 of the wave's 32 in register r of lane (g, token).
// Four consecutive rows per lane make 16 B stores, RoPE pairs sit in one lane,
// and the SwiGLU gate and up rows of a hidden column are two registers of the
// same lane (the wave's rows are 16 gate rows then the matching 16 up rows).
//
// The k order inside a 64-k step is free as long as both operands use it: each
// format's lanes take the byte run of their row that one 16 B load brings in,
// and the token fragments are read from the LDS chunks holding the same k.
// Steps are unrolled by four (one Q4_K / Q6_K super-block), so block-scale
// decoding has compile-time sub-block indices.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

constexpr int BM = 256, BN = 256, NW = 8, BK = 64;
constexpr int ROWB = 128;         // bytes per LDS row of an activation stage: 64 bf16
constexpr int STAGE = BM * ROWB;  // 32 KB
constexpr int GROUP_M = 4;
// Epilogue code of the paired SwiGLU form (EpiParams::hmid_q8k): a workgroup
// takes the n tiles 2u and 2u + 1 of one token tile in turn, whose 128 + 128
// hidden columns are one Q8_K block of every token row.
constexpr int EPI_SWIGLU_Q8K = 16;

__device__ __forceinline__ uint32_t byte_of(const u32x4 &x, int i) {
    return (x[i >> 2] >> (8 * (i & 3))) & 0xffu;
}

// silu with the hardware reciprocal (about 1 ulp)
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// 8 codes held as f16 subnormals in the halves of four words -> 8 bf16 of
// code * a + b (exact f32, rounded to nearest even): p0 / p1 hold codes
// (0, 2) / (1, 3), p2 / p3 codes (4, 6) / (5, 7).
__device__ __forceinline__ bf16x8 mix8(uint32_t p0, uint32_t p1, uint32_t p2, uint32_t p3, float a, float b) {
    return __builtin_bit_cast(bf16x8, u32x4{pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)),
                                            pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                                            pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)),
                                            pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))});
}

// ---- per-format weight streams: one lane, one weight row, half g of a step ----
//
// issue<c>(kt) runs after the barrier that ends step kt (kt % 4 == c) and
// loads what step kt + 2 needs (clamped to the last step: redundant loads, no
// branches); scales<c>() and frag<c>(kk) decode step kt's slice kk;
// chunk(kk, g) is the LDS chunk (8 k) of the activation row holding the same k.
template <int FMT>
struct WStream;

// Q4_K (144 B blocks, 16-row groups interleaved per super-block): lane half g
// takes bytes [32 c + 16 g, +16) of the 128 code bytes at sub-block pair c:
// low nibbles are k = 16 g + 0..15, high nibbles k = 32 + 16 g + 0..15.
template <>
struct WStream<WF_Q4_K> {
    const uint8_t *row, *code;
    u32x4 q[2], hcur, hnext;
    float a0, b0, a1, b1;
    __device__ __forceinline__ void init(const GemmWeight &w, int64_t n, int g, int KT) {
        row = q4k_block(w.q, n, 0, w.k / 256);
        code = row + 16 + 16 * g;
        hnext = hdr(0);
        q[0] = ldq(0);
        q[1] = ldq(min(1, KT - 1));
    }
    __device__ __forceinline__ u32x4 ldq(int kt) const {
        return *(const u32x4 *)(code + (int64_t)(kt >> 2) * (16 * 144) + 32 * (kt & 3));
    }
    __device__ __forceinline__ u32x4 hdr(int kt) const { return *(const u32x4 *)(row + (int64_t)(kt >> 2) * (16 * 144)); }
    template <int C>
    __device__ __forceinline__ void issue(int kt, int KT) {
        const int kn = min(kt + 2, KT - 1);
        q[C & 1] = ldq(kn);
        if constexpr (C == 2) hnext = hdr(kn);
    }
    // sub-blocks 2c and 2c + 1: 6-bit scale and min from header bytes 4..15
    template <int C>
    __device__ __forceinline__ void scales() {
        if constexpr (C == 0) hcur = hnext;
        const float d = f16_to_f32(hcur[0] & 0xffffu), dmin = f16_to_f32(hcur[0] >> 16);
        float sc[2], mn[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            constexpr int j0 = 2 * C;
            const int j = j0 + h, jl = j & 3;
            const uint32_t b4 = byte_of(hcur, 4 + jl), b8 = byte_of(hcur, 8 + jl), b12 = byte_of(hcur, 12 + jl);
            sc[h] = (float)(j < 4 ? (b4 & 63u) : ((b12 & 0xFu) | ((b4 >> 6) << 4)));
            mn[h] = (float)(j < 4 ? (b8 & 63u) : ((b12 >> 4) | ((b8 >> 6) << 4)));
        }
        // low nibbles sit at f16 bits 0-3 (scale carries 2^24), high at 4-7 (2^20)
        a0 = d * sc[0] * 0x1p24f;
        b0 = -(dmin * mn[0]);
        a1 = d * sc[1] * 0x1p20f;
        b1 = -(dmin * mn[1]);
    }
    template <int C>
    __device__ __forceinline__ bf16x8 frag(int kk) const {
        const u32x4 &r = q[C & 1];
        const uint32_t y0 = r[2 * (kk & 1)], y1 = r[2 * (kk & 1) + 1];
        const uint32_t m = kk < 2 ? 0x000F000Fu : 0x00F000F0u;
        const float a = kk < 2 ? a0 : a1, b = kk < 2 ? b0 : b1;
        return mix8(y0 & m, (y0 >> 8) & m, y1 & m, (y1 >> 8) & m, a, b);
    }
    __device__ __forceinline__ static int chunk(int kk, int g) { return 4 * (kk >> 1) + 2 * g + (kk & 1); }
};

// Q8_0 (codes [N][K], f16 scales [N][K/32]): lane half g takes the 32-code
// block 2 kt + g of the step: k = 32 g + 8 kk + 0..7 in slice kk. Codes biased
// to unsigned (q + 128) sit in f16 halves as subnormals; one v_fma_mix gives
// (q + 128) d - 128 d = q d exactly.
template <>
struct WStream<WF_Q8_0> {
    const uint8_t *code;
    const uint16_t *sc;
    u32x4 q[2][2];
    uint32_t s[2];
    float a, b;
    __device__ __forceinline__ void init(const GemmWeight &w, int64_t n, int g, int KT) {
        code = w.q + n * w.k + 32 * g;
        sc = w.scales + n * (w.k / 32) + g;
        load(0, 0);
        load(1, min(1, KT - 1));
    }
    __device__ __forceinline__ void load(int slot, int kt) {
        q[slot][0] = *(const u32x4 *)(code + 64 * (int64_t)kt);
        q[slot][1] = *(const u32x4 *)(code + 64 * (int64_t)kt + 16);
        s[slot] = sc[2 * kt];
    }
    template <int C>
    __device__ __forceinline__ void issue(int kt, int KT) {
        load(C & 1, min(kt + 2, KT - 1));
    }
    template <int C>
    __device__ __forceinline__ void scales() {
        const float d = f16_to_f32(s[C & 1]);
        a = d * 0x1p24f;
        b = -128.f * d;
    }
    template <int C>
    __device__ __forceinline__ bf16x8 frag(int kk) const {
        const u32x4 &r = q[C & 1][kk >> 1];
        const uint32_t x0 = r[2 * (kk & 1)] ^ 0x80808080u, x1 = r[2 * (kk & 1) + 1] ^ 0x80808080u;
        return mix8(x0 & 0x00FF00FFu, __builtin_amdgcn_perm(0u, x0, 0x0C030C01u), x1 & 0x00FF00FFu,
                    __builtin_amdgcn_perm(0u, x1, 0x0C030C01u), a, b);
    }
    __device__ __forceinline__ static int chunk(int kk, int g) { return 4 * g + kk; }
};

// Q6_K (224 B blocks: ql[128], qh[64], int8 scales[16], f16 d; 16-row groups
// interleaved per super-block). Step c of a super-block is half hh = c / 2,
// part o = c % 2; lane half g takes quarter 2 o + g of the half, its 32 values
// l = 0..31 at k = 32 g + l: the low (o = 0) or high (o = 1) nibbles of ql
// bytes [64 hh + 32 g + l] and bits 2 (2 o + g) of qh bytes [32 hh + l], scale
// 8 hh + 2 (2 o + g) + l / 16. A half's 64 bytes per lane are loaded once for
// its two steps.
template <>
struct WStream<WF_Q6_K> {
    const uint8_t *row;
    int g;
    u32x4 ql[2][2], qh[2][2], hcur, hnext;
    uint32_t dcur, dnext;
    float a[2], b[2];
    __device__ __forceinline__ void init(const GemmWeight &w, int64_t n, int g_, int KT) {
        g = g_;
        row = q6k_block(w.q, n, 0, w.k / 256);
        hnext = *(const u32x4 *)(row + 192);
        dnext = *(const uint16_t *)(row + 208);
        load_half(0, 0);
        if (KT > 2) load_half(1, 2);
    }
    __device__ __forceinline__ void load_half(int slot, int kt) {
        const uint8_t *blk = row + (int64_t)(kt >> 2) * (16 * 224);
        const int hh = (kt & 3) >> 1;
        ql[slot][0] = *(const u32x4 *)(blk + 64 * hh + 32 * g);
        ql[slot][1] = *(const u32x4 *)(blk + 64 * hh + 32 * g + 16);
        qh[slot][0] = *(const u32x4 *)(blk + 128 + 32 * hh);
        qh[slot][1] = *(const u32x4 *)(blk + 144 + 32 * hh);
    }
    template <int C>
    __device__ __forceinline__ void issue(int kt, int KT) {
        // after step c = 0 (c = 2) the other half's slot is free: it receives
        // the half of step kt + 2
        if constexpr ((C & 1) == 0) {
            const int kn = kt + 2;
            if (kn < KT) {
                load_half(((C + 2) >> 1) & 1, kn);
                if constexpr (C == 2) {
                    const uint8_t *blk = row + (int64_t)(kn >> 2) * (16 * 224);
                    hnext = *(const u32x4 *)(blk + 192);
                    dnext = *(const uint16_t *)(blk + 208);
                }
            }
        }
    }
    template <int C>
    __device__ __forceinline__ void scales() {
        if constexpr (C == 0) {
            hcur = hnext;
            dcur = dnext;
        }
        constexpr int hh = C >> 1, o = C & 1;
        const float d = f16_to_f32(dcur);
        // scale bytes 8 hh + 4 o + 2 g (+1): word 2 hh + o, bytes 2 g, 2 g + 1
        const uint32_t wv = hcur[2 * hh + o];
        const int sh = 16 * g;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            // the builtin returns the sign-extended field as an unsigned int:
            // convert it as a signed one
            const float ds = d * (float)(int)__builtin_amdgcn_sbfe((int)wv, sh + 8 * h, 8);
            a[h] = ds * 0x1p24f;  // codes at f16 bits 0-5: the subnormal q 2^-24
            b[h] = -32.f * ds;
        }
    }
    template <int C>
    __device__ __forceinline__ bf16x8 frag(int kk) const {
        constexpr int hh = C >> 1, o = C & 1, slot = hh & 1;
        const u32x4 &l = ql[slot][kk >> 1];
        const u32x4 &h = qh[slot][kk >> 1];
        uint32_t q0 = l[2 * (kk & 1)], q1 = l[2 * (kk & 1) + 1];
        if constexpr (o) {
            q0 >>= 4;
            q1 >>= 4;
        }
        const int sh = 2 * (2 * o + g);
        const uint32_t c0 = (q0 & 0x0F0F0F0Fu) | (((h[2 * (kk & 1)] >> sh) & 0x03030303u) << 4);
        const uint32_t c1 = (q1 & 0x0F0F0F0Fu) | (((h[2 * (kk & 1) + 1] >> sh) & 0x03030303u) << 4);
        const float av = a[kk >> 1], bv = b[kk >> 1];
        return mix8(c0 & 0x00FF00FFu, __builtin_amdgcn_perm(0u, c0, 0x0C030C01u), c1 & 0x00FF00FFu,
                    __builtin_amdgcn_perm(0u, c1, 0x0C030C01u), av, bv);
    }
    __device__ __forceinline__ static int chunk(int kk, int g) { return 4 * g + kk; }
};

template <int FMT, int EPI>
__global__ __launch_bounds__(64 * NW, 1) void qgemm_wide_kernel(const uint16_t *__restrict__ A, int64_t M, int64_t lda,
                                                               GemmWeight w, EpiParams ep, int mt, int nt) {
    constexpr bool PAIR = EPI == EPI_SWIGLU_Q8K;
    // the two activation stages; in the paired form then the first tile's
    // per-token largest magnitude, and the block column of its first
    // occurrence times 2 plus its sign bit (one LDS object, so the compiler
    // tells the direct loads into one stage from the reads of the other)
    // (the q/k/v epilogue stages both heads' rows, 2 x 64 KB, and its
    // reduction table, 8 KB, past the activation stages' 64 KB)
    __shared__ __attribute__((aligned(16))) uint8_t
        lds[2 * STAGE + (PAIR ? 2 * BM * 4 : 0) + (EPI == EPI_QKV ? 2 * STAGE + NW * BM * 4 : 0)];
    float *pair_amax = (float *)(lds + 2 * STAGE);
    int *pair_first = (int *)(lds + 2 * STAGE + BM * 4);
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // XCD-aware, M-grouped order of the (token tile, n unit) pairs; an n unit
    // is one tile, or two in the paired form
    const int nu = PAIR ? nt / 2 : nt;
    const int total = mt * nu;
    int L = blockIdx.x;
    if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
    const int per_group = GROUP_M * nu;
    const int grp = L / per_group;
    const int first_m = grp * GROUP_M;
    const int gm = min(mt - first_m, GROUP_M);
    const int mtile = first_m + (L % per_group) % gm;
    const int nunit = (L % per_group) / gm;
    const int64_t m0 = (int64_t)mtile * BM;
    const int KT = (int)(w.k / BK);

    // one tile (t: its index in the workgroup's n unit)
    auto tile = [&](auto t_) __attribute__((always_inline)) {
        constexpr int t = decltype(t_)::value;
        const int64_t n0 = (int64_t)(PAIR ? 2 * nunit + t : nunit) * BN;
        // every lane-dependent value of a tile derives from this copy of the
        // thread index, which the compiler cannot see through: in the paired
        // form nothing of the second tile's addressing is computed early and
        // kept live across the first tile's loop. The mask after it keeps the
        // lane's range known (the fragment reads of one stage provably miss
        // the other stage's direct loads, so they wait for no load).
        int lane = tid;
        if constexpr (PAIR) asm volatile("" : "+v"(lane));
        lane &= 63;
        const int l32 = lane & 31, g = lane >> 5;

        // activation stage by direct global->LDS loads (16 B per lane, lane l at
        // base + 16 l): instruction i of wave v fills rows 8 (4 v + i) .. +8, lane l
        // row 8 (4 v + i) + l / 8 at slot l % 8, which holds chunk (l % 8) ^ key(row).
        // Rows past M repeat row M - 1; their outputs are never written.
        const uint16_t *asrc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 8 * (4 * wave + i) + (lane >> 3);
            const int c = (lane & 7) ^ swz_key(row);
            asrc[i] = A + min(m0 + row, M - 1) * lda + 8 * c;
        }
        auto dma = [&](int stage, int64_t k0) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                __builtin_amdgcn_global_load_lds((const void *)(asrc[i] + k0),
                                                 (lds_ptr_t)(lds + stage * STAGE + (4 * wave + i) * 8 * ROWB), 16, 0, 0);
        };

        // LDS offsets of the token fragments: row l32 (+ 32 i), chunk(kk, g)
        const int key = swz_key(l32);
        int aoff[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) aoff[kk] = l32 * ROWB + ((WStream<FMT>::chunk(kk, g) ^ key) << 4);

        // this lane's weight row (the A-operand row l32 of the wave's fragment)
        int64_t wrow;
        if constexpr (EPI == EPI_SWIGLU || PAIR) {
            // rows interleaved per 64 (gate | up): the wave takes 16 gate rows and
            // the 16 up rows of the same hidden columns
            const int G = wave >> 2, sub = wave & 3;
            wrow = n0 + 128 * G + (l32 < 16 ? 16 * sub + l32 : 64 + 16 * sub + l32 - 16);
        } else {
            wrow = n0 + 32 * wave + l32;
        }
        WStream<FMT> ws;
        ws.init(w, wrow, g, KT);

        f32x16 acc[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][r] = 0.f;

        dma(0, 0);
        dma(1, (int64_t)min(1, KT - 1) * BK);
        __builtin_amdgcn_s_waitcnt(WAIT_VM0_LGKM0);  // vmcnt(0) lgkmcnt(0)
        __syncthreads();

        // Step kt (kt % 4 == C), stage s = C & 1: slice kk decodes its weight
        // fragment and runs 8 MFMAs against the slice's token fragments, which
        // were read ahead. After slice 3: the wait for the next step's activation
        // stage (issued a step ago) and ONE barrier, after which stage s receives
        // the activations of step kt + 2, the weight stream loads for step kt + 2,
        // and the first token fragments of step kt + 1 are read. Every read is
        // pinned ahead of the MFMAs it overlaps by a scheduling barrier.
        if constexpr (FMT != WF_Q6_K) {
            // the 8 fragments of slice kk + 1 are read while slice kk's MFMAs run
            bf16x8 fa[2][8];
            auto rd = [&](int buf, int stage, int kk) __attribute__((always_inline)) {
                const uint8_t *st = lds + stage * STAGE + aoff[kk];
#pragma unroll
                for (int i = 0; i < 8; i++) fa[buf][i] = *(const bf16x8 *)(st + i * 32 * ROWB);
                __builtin_amdgcn_sched_barrier(0);
            };
            rd(0, 0, 0);
            ws.template scales<0>();
            bf16x8 wf0 = ws.template frag<0>(0);  // slice 0 of the coming step
            auto step = [&](int kt, auto c_) __attribute__((always_inline)) {
                constexpr int C = decltype(c_)::value, s = C & 1, CN = (C + 1) & 3;
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const bf16x8 wf = kk == 0 ? wf0 : ws.template frag<C>(kk);
                    const int buf = kk & 1;
                    if (kk < 3) {
                        rd(buf ^ 1, s, kk + 1);
                    } else {
                        // slice 3's operands are in registers: the barrier comes
                        // before its MFMAs, so the next step's first reads and its
                        // slice-0 decode overlap them
                        __builtin_amdgcn_s_waitcnt(WAIT_VM0_LGKM0);
                        __syncthreads();
                        dma(s, (int64_t)min(kt + 2, KT - 1) * BK);
                        ws.template issue<C>(kt, KT);
                        rd(0, s ^ 1, 0);
                        ws.template scales<CN>();
                        wf0 = ws.template frag<CN>(0);
                    }
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, fa[buf][i], acc[i], 0, 0, 0);
                }
            };
            for (int kt = 0; kt < KT; kt += 4) {
                step(kt, std::integral_constant<int, 0>{});
                step(kt + 1, std::integral_constant<int, 1>{});
                step(kt + 2, std::integral_constant<int, 2>{});
                step(kt + 3, std::integral_constant<int, 3>{});
            }
        } else {
            // Q6_K holds twice the raw bytes of Q4_K in registers, so its token
            // fragments are read half a slice ahead (four at a time)
            bf16x8 fh[2][4];
            auto rdh = [&](int buf, int stage, int kk, int h) __attribute__((always_inline)) {
                const uint8_t *st = lds + stage * STAGE + aoff[kk] + h * 4 * 32 * ROWB;
#pragma unroll
                for (int i = 0; i < 4; i++) fh[buf][i] = *(const bf16x8 *)(st + i * 32 * ROWB);
                __builtin_amdgcn_sched_barrier(0);
            };
            rdh(0, 0, 0, 0);
            auto step = [&](int kt, auto c_) __attribute__((always_inline)) {
                constexpr int C = decltype(c_)::value, s = C & 1;
                ws.template scales<C>();
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const bf16x8 wf = ws.template frag<C>(kk);
                    rdh(1, s, kk, 1);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, fh[0][i], acc[i], 0, 0, 0);
                    if (kk < 3) {
                        rdh(0, s, kk + 1, 0);
                    } else {
                        // the last four fragments are in registers: the barrier
                        // comes before their MFMAs
                        __builtin_amdgcn_s_waitcnt(WAIT_VM0_LGKM0);
                        __syncthreads();
                        dma(s, (int64_t)min(kt + 2, KT - 1) * BK);
                        ws.template issue<C>(kt, KT);
                        rdh(0, s ^ 1, 0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[4 + i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, fh[1][i], acc[4 + i], 0, 0, 0);
                }
            };
            for (int kt = 0; kt < KT; kt += 4) {
                step(kt, std::integral_constant<int, 0>{});
                step(kt + 1, std::integral_constant<int, 1>{});
                step(kt + 2, std::integral_constant<int, 2>{});
                step(kt + 3, std::integral_constant<int, 3>{});
            }
        }
        __builtin_amdgcn_s_waitcnt(WAIT_VM0_LGKM0);  // no load into LDS still in flight

        // ---- epilogue: lane (g, l32) of token tile i holds token m0 + 32 i + l32,
        // register r the wave's weight row p(r) = 8 (r / 4) + 4 g + r % 4 ----
        if constexpr (EPI == EPI_F32 || EPI == EPI_BF16 || EPI == EPI_RESID) {
            const int64_t nw = n0 + 32 * wave + 4 * g;  // + 8 j: the lane's run j of four rows
            const int64_t N = w.n;
            // the gated residual of a tile whose rows share one gate row: the
            // x_in loads of four token rows in flight before their stores
            // (x_out may alias x_in: each element is read and written by the
            // same lane, its load before its store)
            bool resid_done = false;
            if constexpr (EPI == EPI_RESID) {
                const int64_t gp = ep.g_rows_per, last = (m0 + BM < M ? m0 + BM : M) - 1;
                if (m0 / gp == last / gp) {
                    const float *grow = ep.gvec + (m0 / gp) * ep.g_stride;
                    f32x4 gv[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) gv[j] = *(const f32x4 *)(grow + nw + 8 * j);
#pragma unroll
                    for (int i0 = 0; i0 < 8; i0 += 4) {
                        f32x4 xv[4][4];
#pragma unroll
                        for (int ii = 0; ii < 4; ii++) {
                            const int64_t m = m0 + 32 * (i0 + ii) + l32;
                            if (m < M)
#pragma unroll
                                for (int j = 0; j < 4; j++) xv[ii][j] = *(const f32x4 *)(ep.x_in + m * N + nw + 8 * j);
                        }
#pragma unroll
                        for (int ii = 0; ii < 4; ii++) {
                            const int64_t m = m0 + 32 * (i0 + ii) + l32;
                            if (m >= M) continue;
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                f32x4 o;
#pragma unroll
                                for (int e = 0; e < 4; e++) o[e] = xv[ii][j][e] + gv[j][e] * acc[i0 + ii][4 * j + e];
                                *(f32x4 *)(ep.x_out + m * N + nw + 8 * j) = o;
                            }
                        }
                    }
                    resid_done = true;
                }
            }
            if (!resid_done)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int64_t m = m0 + 32 * i + l32;
                if (m >= M) continue;
                if constexpr (EPI == EPI_F32) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        *(f32x4 *)((float *)ep.out + m * ep.ldo + nw + 8 * j) =
                            f32x4{acc[i][4 * j], acc[i][4 * j + 1], acc[i][4 * j + 2], acc[i][4 * j + 3]};
                } else if constexpr (EPI == EPI_BF16) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        *(u32x2 *)((uint16_t *)ep.out + m * ep.ldo + nw + 8 * j) =
                            u32x2{pack_bf16x2(acc[i][4 * j], acc[i][4 * j + 1]),
                                  pack_bf16x2(acc[i][4 * j + 2], acc[i][4 * j + 3])};
                } else {
                    // x_out may alias x_in: each element is read and written by
                    // the same lane, every load of the row before its stores
                    const float *grow = ep.gvec + (int64_t)((int)m / (int)ep.g_rows_per) * ep.g_stride;
                    f32x4 xv[4], gv[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        xv[j] = *(const f32x4 *)(ep.x_in + m * N + nw + 8 * j);
                        gv[j] = *(const f32x4 *)(grow + nw + 8 * j);
                    }
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        f32x4 o;
#pragma unroll
                        for (int e = 0; e < 4; e++) o[e] = xv[j][e] + gv[j][e] * acc[i][4 * j + e];
                        *(f32x4 *)(ep.x_out + m * N + nw + 8 * j) = o;
                    }
                }
            }
        } else if constexpr (EPI == EPI_SWIGLU) {
            // registers r < 8 are gate rows 16 sub + p(r), r + 8 the up rows of the
            // same hidden columns
            const int G = wave >> 2, sub = wave & 3;
            const int64_t hc = (n0 + 128 * G) / 2 + 16 * sub + 4 * g;  // + 8 j
            auto hval = [&](int i, int r) __attribute__((always_inline)) { return silu(acc[i][r]) * acc[i][8 + r]; };
            if (ep.hmid_q8_0) {
                // candle's Q8_0 rounding: a 32-column block is the 16 columns of
                // waves sub and sub ^ 1, so each token's largest magnitude comes
                // from the lane's 8, its partner half (lane ^ 32) and the sibling
                // wave's through LDS; the values are formed again for the stores
                float *red = (float *)lds;  // [8 waves][256 tokens]
                __syncthreads();            // every wave is done with the operand stages
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float a = 0.f;
#pragma unroll
                    for (int r = 0; r < 8; r++) a = fmaxf(a, fabsf(hval(i, r)));
                    float lo = a, hi = a;
                    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
                    if (g == 0) red[wave * BM + 32 * i + l32] = fmaxf(lo, hi);
                }
                __syncthreads();
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int tk = 32 * i + l32;
                    const int64_t m = m0 + tk;
                    if (m >= M) continue;
                    float sc, dq;
                    q8_0_scales(fmaxf(red[wave * BM + tk], red[(wave ^ 1) * BM + tk]), sc, dq);
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        f32x4 hv;
#pragma unroll
                        for (int e = 0; e < 4; e++) hv[e] = hval(i, 4 * j + e);
                        *(u32x2 *)(ep.hmid + m * ep.ldh + hc + 8 * j) = q8_0_values4(hv, sc, dq);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int64_t m = m0 + 32 * i + l32;
                    if (m >= M) continue;
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        float h[4];
#pragma unroll
                        for (int e = 0; e < 4; e++) h[e] = hval(i, 4 * j + e);
                        const int64_t o = m * ep.ldh + hc + 8 * j;
                        if (ep.hmid_f32)
                            *(f32x4 *)(ep.hmid_f32 + o) = f32x4{h[0], h[1], h[2], h[3]};
                        else
                            *(u32x2 *)(ep.hmid + o) = u32x2{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
                    }
                }
            }
        } else if constexpr (PAIR) {
            // candle's Q8_K rounding of the hidden state (the down projection's
            // input), in the arithmetic of quant_act4<256>: the first tile's f32
            // values go to hmid_f32 (scratch) and its per-token largest magnitude
            // and first column to LDS; after the second tile the block's x_max is
            // the first of largest magnitude over both, and both halves are
            // written to hmid as bf16(d q). Register r < 8 of token tile i is gate
            // row 16 sub + p(r), r + 8 its up row: hidden column hc + 8 (r / 4) + r % 4.
            const int G = wave >> 2, sub = wave & 3;
            const int64_t hc = n0 / 2 + 64 * G + 16 * sub + 4 * g;
            const int cb = (int)(hc & 255);  // its column in the Q8_K block
            // second tile: this lane's own f32 stores of the first tile, 128
            // columns back, loaded first so they arrive during the work below
            f32x4 ha[8][2];
            if constexpr (t == 1) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int64_t m = min(m0 + 32 * i + l32, M - 1);
                    const float *frow = ep.hmid_f32 + m * ep.ldh + hc - 128;
#pragma unroll
                    for (int j = 0; j < 2; j++) ha[i][j] = *(const f32x4 *)(frow + 8 * j);
                }
            }
            float h[8][8];
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int r = 0; r < 8; r++) h[i][r] = silu(acc[i][r]) * acc[i][8 + r];
            if constexpr (t == 0) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int64_t m = m0 + 32 * i + l32;
                    if (m >= M) continue;
                    float *frow = ep.hmid_f32 + m * ep.ldh + hc;
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        *(f32x4 *)(frow + 8 * j) = f32x4{h[i][4 * j], h[i][4 * j + 1], h[i][4 * j + 2], h[i][4 * j + 3]};
                }
            }
            float *red = (float *)lds;                    // [8 waves][256 tokens]
            int *redi = (int *)(lds + NW * BM * 4);       // [8 waves][256 tokens]
            float *tmax = (float *)(lds + 2 * NW * BM * 4);  // [256] per token
            float *tsc = tmax + BM, *tdq = tmax + 2 * BM;    // [256] s and d per token
            __syncthreads();  // every wave is done with the operand stages
            // largest magnitude per token: the lane's 8, its partner half (lane ^ 32), the 8 waves
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float a = 0.f;
#pragma unroll
                for (int r = 0; r < 8; r++) a = fmaxf(a, fabsf(h[i][r]));
                float lo = a, hi = a;
                asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
                if (g == 0) red[wave * BM + 32 * i + l32] = fmaxf(lo, hi);
            }
            __syncthreads();
            if (tid < BM) {
                float a = red[tid];
#pragma unroll
                for (int v = 1; v < NW; v++) a = fmaxf(a, red[v * BM + tid]);
                tmax[tid] = a;
            }
            __syncthreads();
            // its first occurrence: the smallest (column << 1 | sign) holding it
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float a = tmax[32 * i + l32];
                int f = 0x7fffffff;
#pragma unroll
                for (int r = 7; r >= 0; r--) {
                    const int code = ((cb + 8 * (r >> 2) + (r & 3)) << 1) | (h[i][r] < 0.f ? 1 : 0);
                    f = fabsf(h[i][r]) == a ? code : f;
                }
                int lo = f, hi = f;
                asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
                if (g == 0) redi[wave * BM + 32 * i + l32] = min(lo, hi);
            }
            __syncthreads();
            if (tid < BM) {
                int f = redi[tid];
#pragma unroll
                for (int v = 1; v < NW; v++) f = min(f, redi[v * BM + tid]);
                float a = tmax[tid];
                if constexpr (t == 0) {
                    pair_amax[tid] = a;
                    pair_first[tid] = f;
                } else {
                    // the first tile's columns come first: it wins ties
                    if (!(a > pair_amax[tid])) {
                        a = pair_amax[tid];
                        f = pair_first[tid];
                    }
                    float sc, dq;
                    q8k_scales(a, (f & 1) ? -a : a, sc, dq);
                    tsc[tid] = sc;
                    tdq[tid] = dq;
                }
            }
            __syncthreads();  // (first tile) the next tile's stages overwrite these tables
            if constexpr (t == 1) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int64_t m = m0 + 32 * i + l32;
                    if (m >= M) continue;
                    const float sc = tsc[32 * i + l32], dq = tdq[32 * i + l32];
                    uint16_t *hrow = ep.hmid + m * ep.ldh + hc;
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const float *v = &h[i][4 * j];
                        const f32x4 u = ha[i][j];
                        *(u32x2 *)(hrow + 8 * j) = q8k_values4(f32x4{v[0], v[1], v[2], v[3]}, sc, dq);
                        *(u32x2 *)(hrow - 128 + 8 * j) = q8k_values4(u, sc, dq);
                    }
                }
            }
        } else if constexpr (EPI == EPI_QKV) {
            // waves 4 G .. 4 G + 3 hold one head (128 fused columns), wave sub its
            // dims 32 sub + p(r)
            const int G = wave >> 2, sub = wave & 3;
            const int64_t nb = n0 + 128 * G + ep.n_offset;
            const int sec = (int)(nb / ep.hidden);
            const int64_t head = (nb % ep.hidden) / 128;
            const uint32_t Su = (uint32_t)ep.seq;
            const int64_t H = ep.heads, S = ep.seq;
            // (batch, position) of token m0 + t: with sequences of at least 256
            // tokens the tile's 256 consecutive tokens span at most two, so one
            // division for the tile's first token and a compare per row; shorter
            // sequences divide per row. (Rows past M get a position below S.)
            const uint32_t b0 = (uint32_t)m0 / Su, s0 = (uint32_t)m0 % Su;
            auto tok = [&](int t, uint32_t &b, uint32_t &s) __attribute__((always_inline)) {
                if (Su >= 256) {
                    const uint32_t x = s0 + (uint32_t)t;
                    const bool w = x >= Su;
                    s = w ? x - Su : x;
                    b = b0 + (w ? 1u : 0u);
                } else {
                    const uint32_t m = (uint32_t)min(m0 + t, M - 1);
                    s = m % Su;
                    b = m / Su;
                }
            };
            if (sec < 2) {
                // RmsNorm over the head: each lane's 16 squares, the partner half
                // (lane ^ 32), then the head's four waves through LDS. The RoPE
                // (cos, sin) of the lane's 16 dims for its token of tile i are
                // loaded one tile ahead (the first before the reduction), with
                // the row clamped so that every load is unconditional.
                const int dbase = 32 * sub + 4 * g;  // + 8 j
                f32x4 cs[2][4];
                auto load_pe = [&](int i) __attribute__((always_inline)) {
                    uint32_t b, s;
                    tok(32 * i + l32, b, s);
                    const float *pr = ep.pe + (int64_t)s * 128;  // (cos, sin) of pair i at 2i, 2i + 1
#pragma unroll
                    for (int j = 0; j < 4; j++) cs[i & 1][j] = *(const f32x4 *)(pr + dbase + 8 * j);
                };
                load_pe(0);
                typedef __attribute__((address_space(4))) const f32x4 cf32x4;
                const __attribute__((address_space(4))) float *nwt =
                    (const __attribute__((address_space(4))) float *)(sec == 0 ? ep.norm_q : ep.norm_k);
                f32x4 wv[4];
#pragma unroll
                for (int j = 0; j < 4; j++) wv[j] = *(const cf32x4 *)(nwt + dbase + 8 * j);
                float *red = (float *)(lds + 4 * STAGE);  // [8 waves][256 tokens], past the row staging
                __syncthreads();                           // every wave is done with the operand stages
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float ss = 0.f;
#pragma unroll
                    for (int r = 0; r < 16; r++) ss += acc[i][r] * acc[i][r];
                    float lo = ss, hi = ss;
                    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
                    if (g == 0) red[wave * 256 + 32 * i + l32] = lo + hi;
                }
                __syncthreads();
                const float osc = sec == 0 ? ep.q_scale : 1.0f;
                uint16_t *dst = sec == 0 ? ep.q : ep.k;
                // the rows go through LDS: head G's 256 tokens x 128 dims of bf16
                // in its own 64 KB (256 B rows, 16 B chunk c of row t at slot
                // c ^ (t % 16)), then both heads are stored as whole 256 B rows
                uint16_t *stg = (uint16_t *)lds + G * (256 * 128);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (i + 1 < 8) load_pe(i + 1);
                    const int t = 32 * i + l32;
                    const float *rr = red + 4 * G * 256 + t;
                    const float rs = 1.0f / sqrtf(((rr[0] + rr[256]) + (rr[512] + rr[768])) * (1.0f / 128.0f) + 1e-6f);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        uint32_t o[2];
#pragma unroll
                        for (int e = 0; e < 2; e++) {
                            const float x0 = acc[i][4 * j + 2 * e] * rs * wv[j][2 * e];
                            const float x1 = acc[i][4 * j + 2 * e + 1] * rs * wv[j][2 * e + 1];
                            const float co = cs[i & 1][j][2 * e], sn = cs[i & 1][j][2 * e + 1];
                            o[e] = pack_bf16x2((x0 * co - x1 * sn) * osc, (x0 * sn + x1 * co) * osc);
                        }
                        // dims dbase + 8 j: chunk 4 sub + j, half g of it
                        const int c = (4 * sub + j) ^ (t & 15);
                        *(u32x2 *)(stg + t * 128 + 8 * c + 4 * g) = u32x2{o[0], o[1]};
                    }
                }
                __syncthreads();
                const int64_t head0 = head - G;  // the tile's first head
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    const int ch = tid + 512 * k, hg = ch >> 12, t = (ch >> 4) & 255, c = ch & 15;
                    if (m0 + t >= M) continue;
                    uint32_t b, s;
                    tok(t, b, s);
                    *(u32x4 *)(dst + (((int64_t)b * H + head0 + hg) * S + s) * 128 + 8 * c) =
                        *(const u32x4 *)((uint16_t *)lds + hg * (256 * 128) + t * 128 + 8 * (c ^ (t & 15)));
                }
            } else {
                // v: transposed to vt [B,H,128,S] (consecutive lanes hold
                // consecutive tokens of a d row), and [B,H,S,128] when v_bhsd is set
                const int dbase = 32 * sub + 4 * g;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (m0 + 32 * i + l32 >= M) continue;
                    uint32_t b, s;
                    tok(32 * i + l32, b, s);
                    uint16_t *vrow = ep.vt + ((int64_t)b * H + head) * 128 * S + s;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int d = dbase + 8 * (r >> 2) + (r & 3);
                        vrow[(int64_t)d * S] = (uint16_t)(pack_bf16x2(acc[i][r], 0.f) & 0xffffu);
                    }
                    if (ep.v_bhsd) {
                        uint16_t *brow = ep.v_bhsd + (((int64_t)b * H + head) * S + s) * 128;
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            *(u32x2 *)(brow + dbase + 8 * j) = u32x2{pack_bf16x2(acc[i][4 * j], acc[i][4 * j + 1]),
                                                                     pack_bf16x2(acc[i][4 * j + 2], acc[i][4 * j + 3])};
                    }
                }
            }
        }
    };
    tile(std::integral_constant<int, 0>{});
    if constexpr (PAIR) tile(std::integral_constant<int, 1>{});
}

template <int FMT>
hipError_t launch_fmt(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi, const EpiParams &ep,
                      hipStream_t stream) {
    const int mt = (int)((m + BM - 1) / BM), nt = (int)(w.n / BN);
    const dim3 block(64 * NW);
    if (epi == EPI_SWIGLU && ep.hmid_q8k) {
        if (nt % 2 || !ep.hmid || !ep.hmid_f32) return hipErrorInvalidValue;
        qgemm_wide_kernel<FMT, EPI_SWIGLU_Q8K>
            <<<dim3((unsigned)(mt * nt / 2)), block, 0, stream>>>(a, m, lda, w, ep, mt, nt);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)(mt * nt));
    switch (epi) {
    case EPI_F32: qgemm_wide_kernel<FMT, EPI_F32><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    case EPI_BF16: qgemm_wide_kernel<FMT, EPI_BF16><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    case EPI_QKV: qgemm_wide_kernel<FMT, EPI_QKV><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    case EPI_RESID: qgemm_wide_kernel<FMT, EPI_RESID><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    case EPI_SWIGLU: qgemm_wide_kernel<FMT, EPI_SWIGLU><<<grid, block, 0, stream>>>(a, m, lda, w, ep, mt, nt); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool qgemm_wide_fits(const GemmWeight &w) {
    return (w.fmt == WF_Q4_K || w.fmt == WF_Q6_K || w.fmt == WF_Q8_0) && w.n % BN == 0 && w.k % 256 == 0 && w.k > 0;
}

bool qgemm_wide_pairs_fit(const GemmWeight &w) { return qgemm_wide_fits(w) && w.n % (2 * BN) == 0; }

hipError_t launch_qgemm_wide(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                             const EpiParams &ep, hipStream_t stream) {
    switch (w.fmt) {
    case WF_Q8_0: return launch_fmt<WF_Q8_0>(w, a, m, lda, epi, ep, stream);
    case WF_Q4_K: return launch_fmt<WF_Q4_K>(w, a, m, lda, epi, ep, stream);
    case WF_Q6_K: return launch_fmt<WF_Q6_K>(w, a, m, lda, epi, ep, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace qimm
