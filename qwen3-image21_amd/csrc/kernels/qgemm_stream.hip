// Weight-streaming dequant-GEMM for gfx950 at small token counts (M <= 64):
// C = A (bf16, M x K) x W^T (GGUF blocks, N x K). At these sizes the time is
// the weight bytes over HBM bandwidth, so the kernels are shaped for streaming.
//
// Q4_K, Q6_K and Q8_0 with K % 1024 == 0 take the one-launch kernel in
// namespace ws (its description is there). Everything else takes the split-K
// kernel:
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
#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

constexpr int SK = 128;          // k per LDS stage (two 64-k weight steps)
constexpr int MAXM = 64;         // token rows per workgroup
constexpr int XROWB = SK * 2;    // bytes per activation row in LDS (256)
constexpr int XSTAGE = MAXM * XROWB;  // 16 KB

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
        const float d = f16_to_f32(r.a[0] & 0xffffu), dmin = f16_to_f32(r.a[0] >> 16);
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
        const float ds = f16_to_f32(r.s) * (float)(int8_t)byte_of(r.a, 8 * hh + 2 * r6 + (kg >> 1));
        return cvt8(c0, c1, ds, -32.f * ds);  // (q+32)*ds - 32*ds, exact
    } else if constexpr (FMT == WF_Q8_0) {
        const float d = f16_to_f32(s ? (r.s >> 16) : (r.s & 0xffffu));
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
// Q4_K code products (used by the M <= 16 kernel below).
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
namespace m16 {

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

int device_cus() { return device_cu_count(); }

}  // namespace m16

// silu with the hardware reciprocal (about 1 ulp) instead of an IEEE divide
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
// one SwiGLU hidden value: bf16 into hmid, or f32 into hmid_f32 when set
__device__ __forceinline__ void store_hidden(const EpiParams &ep, int64_t o, float h) {
    if (ep.hmid_f32)
        ep.hmid_f32[o] = h;
    else
        ep.hmid[o] = (uint16_t)(pack_bf16x2(h, 0.f) & 0xffffu);
}

// ---------------------------------------------------------------------------
// M <= 64, Q4_K / Q6_K / Q8_0, K % 1024 == 0: one launch per product.
//
// Work item = (16-row weight group g, 1024-wide k chunk c) = four (group,
// super-block) tiles, contiguous in the device layout, against MT = 1, 2 or 4
// tiles of 16 tokens. Workgroup b keeps chunk c = b % C of the activations in
// LDS (x[16 MT][1024] bf16, loaded once by direct loads) and its waves (four,
// or eight for MT = 4) grid-stride over the groups: at step t wave v takes
// group (t * WPC + b / C) * NW + v. Workgroups with neighbouring ids read
// neighbouring groups, so the bytes in flight at any time are one compact
// window of the weight matrix (the pattern of a plain streaming read). Raw
// tiles go straight to registers, four in flight per wave, one item ahead.
//
// Q4_K uses the exact code products described above up to 16 tokens (the
// sub-block sums X_j of the chunk are computed once per wave and token tile)
// and beyond that decodes each value once for all token tiles. Q6_K dequantizes
// each lane's 8 values of a step with v_fma_mix (the 6-bit codes as f16
// subnormals, scales carrying 2^24; RNE to bf16) once for all token tiles; a
// lane's 8 values of a step are 8 consecutive k of one 16-value sub-block and
// the matching activations are one 16 B LDS read, so the lane reads its ql /
// qh bytes as 16 B pieces.
//
// The partial sums of an item, [16 MT tokens][16 rows] f32, go to
// part[c][g] with system-scope stores; the wave that completes the last item
// of an epilogue unit (a counter per unit) reads the C partials of the unit
// back the same way, adds them in chunk order -- deterministic -- applies the
// epilogue and resets the counter for the next launch. Units: a group (F32,
// BF16, residual), the gate and up groups of 16 hidden columns (SwiGLU), a
// 128-column head (q/k/v).
namespace ws {

constexpr int KCH = 1024;           // k per chunk
constexpr int SBC = KCH / 256;      // tiles per item
constexpr int XROW = KCH * 2 + 16;  // padded LDS row: a fragment's 16 rows hit distinct bank groups
constexpr int MAX_STEPS = 4;        // items per wave (compile-time unrolled)

// Token tiles of 16 per item (MT), and per MT the waves per workgroup and the
// workgroups resident per CU (LDS: 16 MT rows of XROW bytes per workgroup).
constexpr int nwaves(int mt) { return mt == 4 ? 8 : 4; }
constexpr int wg_per_cu(int mt) { return mt == 1 ? 3 : mt == 2 ? 2 : 1; }

struct Plan {
    int C, G, WPC, steps, units, per_unit, MT;
};

size_t part_bytes(const GemmWeight &w, int64_t m);

bool plan(const GemmWeight &w, int64_t m, int epi, int cus, Plan &p) {
    if ((w.fmt != WF_Q4_K && w.fmt != WF_Q6_K && w.fmt != WF_Q8_0) || m < 1 || m > 64 || w.k % KCH || w.n % 16 ||
        cus <= 0)
        return false;
    if ((epi == EPI_SWIGLU || epi == EPI_QKV) && w.n % 128) return false;
    p.MT = m <= 16 ? 1 : m <= 32 ? 2 : 4;
    const int nw = nwaves(p.MT);
    p.C = (int)(w.k / KCH);
    p.G = (int)(w.n / 16);
    const int need = (p.G + nw - 1) / nw;  // workgroups per chunk that have work at step 0
    p.WPC = std::max(1, std::min(wg_per_cu(p.MT) * cus / p.C, need));
    p.steps = (p.G + nw * p.WPC - 1) / (nw * p.WPC);
    p.per_unit = epi == EPI_QKV ? 8 : epi == EPI_SWIGLU ? 2 : 1;
    p.units = p.G / p.per_unit;
    // partial sums addressed by 32-bit byte offsets
    return p.steps <= MAX_STEPS && (size_t)p.units * 4 <= STREAM_COUNTER_BYTES && part_bytes(w, m) < ((size_t)1 << 31);
}

// partial sums: [C][G][item] f32, an item holding token m of row r at
// pidx(m, r): the four consecutive tokens 4i .. 4i+3 of a row are contiguous,
// the MFMA result of one lane, one 16 B access
__host__ __device__ constexpr int pidx(int m, int r) { return ((m >> 2) * 16 + r) * 4 + (m & 3); }
size_t part_bytes(const GemmWeight &w, int64_t m) {
    const int mt = m <= 16 ? 1 : m <= 32 ? 2 : 4;
    return (size_t)(w.k / KCH) * (size_t)w.n * 64 * mt;
}

struct TileQ4 {
    u32x4 h;
    u32x2 q[4];
};
struct TileQ6 {
    u32x4 l0, l1, h0, h1, sc;
    uint32_t d;
};

struct TileQ8 {
    u32x4 c[4], s;
};

template <int FMT>
using Tile = typename std::conditional<FMT == WF_Q4_K, TileQ4,
                                       typename std::conditional<FMT == WF_Q6_K, TileQ6, TileQ8>::type>::type;

// The A fragment of step s of a 256-k tile for lane group kg (8 consecutive
// k, 16 B): its byte offset in a tile row. Q4_K steps are the 32-k
// sub-blocks; a Q6_K or Q8_0 step pair covers a 64-k block, in which group
// kg holds 16 consecutive k and the step's parity picks 8 of them.
template <int FMT>
__device__ __forceinline__ int xoff(int s, int kg) {
    return FMT == WF_Q4_K ? 64 * s + 16 * kg : 128 * (s >> 1) + 32 * kg + 16 * (s & 1);
}

// A fragments from an activation row in LDS (token tile tt 16 rows further).
template <int FMT>
struct XLds {
    const uint8_t *row;
    int kg;
    __device__ __forceinline__ bf16x8 operator()(int s, int tt) const {
        if constexpr (FMT == WF_Q4_K) return *(const bf16x8 *)(row + tt * 16 * XROW + 64 * s + 16 * kg);
        else if constexpr (FMT == WF_Q6_K)
            return *(const bf16x8 *)(row + tt * 16 * XROW + 256 * (s >> 2) + 128 * ((s >> 1) & 1) + 32 * kg + 16 * (s & 1));
        else return *(const bf16x8 *)(row + tt * 16 * XROW + 128 * (s >> 1) + 32 * kg + 16 * (s & 1));
    }
};

// Q8_0 (device layout: codes [N][K], f16 scales [N][K/32]): lane kg holds the
// 16-code pieces at k = 64 q + 16 kg (q < 4) of its row and the row's 8
// scales of the super-block-sized tile.
__device__ __forceinline__ void load_tile(const GemmWeight &w, int64_t g, int64_t sb, int64_t SB, int l16, int kg,
                                          TileQ8 &r) {
    const int64_t n = 16 * g + l16, K = SB * 256;
    const uint8_t *p = w.q + n * K + sb * 256 + 16 * kg;
#pragma unroll
    for (int q = 0; q < 4; q++) r.c[q] = *(const u32x4 *)(p + 64 * q);
    r.s = *(const u32x4 *)(w.scales + n * (K / 32) + sb * 8);
}

__device__ __forceinline__ void load_tile(const GemmWeight &w, int64_t g, int64_t sb, int64_t SB, int l16, int kg,
                                          TileQ4 &r) {
    const uint8_t *b = w.q + ((g * SB + sb) * 16 + l16) * 144;  // q4k_block(16 g + l16, sb)
    r.h = *(const u32x4 *)b;
#pragma unroll
    for (int cc = 0; cc < 4; cc++) r.q[cc] = *(const u32x2 *)(b + 16 + 32 * cc + 8 * kg);
}

// Lane kg = 2 r1 + h': ql bytes [32 r1 + 16 h', +16) of each half, qh bytes
// [16 h', +16) of each half, the 16 scales and d (a 4-byte load: d and the
// first two pad bytes of the 224-byte device block).
__device__ __forceinline__ void load_tile(const GemmWeight &w, int64_t g, int64_t sb, int64_t SB, int l16, int kg,
                                          TileQ6 &r) {
    const uint8_t *b = w.q + ((g * SB + sb) * 16 + l16) * 224;  // q6k_block(16 g + l16, sb)
    const int qo = 32 * (kg >> 1) + 16 * (kg & 1), ho = 128 + 16 * (kg & 1);
    r.l0 = *(const u32x4 *)(b + qo);
    r.l1 = *(const u32x4 *)(b + 64 + qo);
    r.h0 = *(const u32x4 *)(b + ho);
    r.h1 = *(const u32x4 *)(b + ho + 32);
    r.sc = *(const u32x4 *)(b + 192);
    r.d = *(const uint32_t *)(b + 208);  // d and two pad bytes
}

// The raw registers pass through an empty asm first, so no decoding of a tile
// is hoisted to where its loads were issued (that would wait for them there).
__device__ __forceinline__ void pin(TileQ6 &r) {
    asm volatile("" : "+v"(r.l0), "+v"(r.l1), "+v"(r.h0), "+v"(r.h1), "+v"(r.sc), "+v"(r.d));
}
__device__ __forceinline__ void pin(TileQ4 &r) {
    asm volatile("" : "+v"(r.h), "+v"(r.q[0]), "+v"(r.q[1]), "+v"(r.q[2]), "+v"(r.q[3]));
}
__device__ __forceinline__ void pin(TileQ8 &r) {
    asm volatile("" : "+v"(r.c[0]), "+v"(r.c[1]), "+v"(r.c[2]), "+v"(r.c[3]), "+v"(r.s));
}

// One Q8_0 tile into acc[0..MT). Step s = 2 q + h: the lane's 8 codes
// k = 64 q + 16 kg + 8 h + i, all in 32-value block 2 q + kg / 2; codes biased
// to unsigned (q + 128) sit in f16 halves as subnormals, one v_fma_mix each
// gives (q + 128) d - 128 d = q d exactly, then RNE to bf16.
template <int MT, class XF>
__device__ __forceinline__ void tile_q8(TileQ8 r, XF xf, int kg, f32x4 *acc) {
    pin(r);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        // block 2 q + kg / 2: its scale is half kg / 2 of scale word q
        const uint32_t sw = (kg >> 1) ? (r.s[q] >> 16) : (r.s[q] & 0xffffu);
        const float d = m16::cvt_f16_lo(sw);
        const float a = d * 0x1p24f, b = -128.f * d;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t u0 = r.c[q][2 * h] ^ 0x80808080u, u1 = r.c[q][2 * h + 1] ^ 0x80808080u;
            const uint32_t p0 = u0 & 0x00FF00FFu, p1 = __builtin_amdgcn_perm(0u, u0, 0x0C030C01u);
            const uint32_t p2 = u1 & 0x00FF00FFu, p3 = __builtin_amdgcn_perm(0u, u1, 0x0C030C01u);
            const u32x4 bw = {pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)), pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                              pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)), pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))};
#pragma unroll
            for (int tt = 0; tt < MT; tt++) {
                const bf16x8 av = xf(2 * q + h, tt);
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, bw), acc[tt], 0, 0, 0);
            }
        }
    }
}

// One Q6_K tile (16 rows x 256 k) into acc[0..MT) (token tiles 16 tt + l16
// at xrow + 16 tt XROW). Step s: half hh = s / 4, nibble n = (s / 2) % 2,
// 8-byte half h8 = s % 2 of the lane's 16 B pieces; the values are
// k = 128 hh + 32 (r1 + 2 n) + 16 h' + 8 h8 + i of the super-block, scale
// index 8 hh + 4 n + kg. Each step's B fragment serves every token tile.
template <int MT, class XF>
__device__ __forceinline__ void tile_q6(TileQ6 r, XF xf, int kg, f32x4 *acc) {
    pin(r);
    const float d = m16::cvt_f16_lo(r.d);
    const uint32_t hsh = 2u * (uint32_t)(kg >> 1);  // qh bit pair of quadrant r1 (+4 for n = 1)
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int hh = s >> 2, n = (s >> 1) & 1, h8 = s & 1;
        const u32x4 &L = hh ? r.l1 : r.l0;
        const u32x4 &H = hh ? r.h1 : r.h0;
        const float ds = d * (float)(int8_t)((r.sc[2 * hh + n] >> (8 * kg)) & 0xffu);
        const float a = ds * 0x1p24f, b = -32.f * ds;
        uint32_t c[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t lo = (L[2 * h8 + i] >> (4 * n)) & 0x0F0F0F0Fu;
            const uint32_t hi = ((H[2 * h8 + i] >> (hsh + 4u * n)) & 0x03030303u) << 4;
            c[i] = lo | hi;
        }
        const uint32_t p0 = c[0] & 0x00FF00FFu, p1 = __builtin_amdgcn_perm(0u, c[0], 0x0C030C01u);
        const uint32_t p2 = c[1] & 0x00FF00FFu, p3 = __builtin_amdgcn_perm(0u, c[1], 0x0C030C01u);
        const u32x4 bw = {pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)), pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                          pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)), pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))};
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            const bf16x8 av = xf(s, tt);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, bw), acc[tt], 0, 0, 0);
        }
    }
}

// One Q4_K tile by code products (see the m16 notes above) into accA / accM
// of each token tile; xq0[tt] / xq1[tt] hold the sub-block sums X_kg,
// X_{4+kg} of token 16 tt + l16 for this super-block.
template <int MT, class XF>
__device__ __forceinline__ void tile_q4(TileQ4 r, XF xf, int kg, const float *xq0, const float *xq1,
                                        f32x4 *accA, f32x4 *accM) {
    pin(r);
    const uint32_t hx = r.h[0], hy = r.h[1], hz = r.h[2], hw = r.h[3];
    const float d = m16::cvt_f16_lo(hx), dmin = m16::cvt_f16_hi(hx);
    const uint32_t sc_lo = hy & 0x3F3F3F3Fu, m_lo = hz & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (hw & 0x0F0F0F0Fu) | ((hy >> 2) & 0x30303030u);
    const uint32_t m_hi = ((hw >> 4) & 0x0F0F0F0Fu) | ((hz >> 2) & 0x30303030u);
    const uint32_t sh = 8u * (uint32_t)kg;
    const float cc0 = fmaf(128.f, d * (float)((sc_lo >> sh) & 0xffu), dmin * (float)((m_lo >> sh) & 0xffu));
    const float cc1 = fmaf(128.f, d * (float)((sc_hi >> sh) & 0xffu), dmin * (float)((m_hi >> sh) & 0xffu));
#pragma unroll
    for (int tt = 0; tt < MT; tt++) {
        accM[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xq0[tt], cc0, accM[tt], 0, 0, 0);
        accM[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xq1[tt], cc1, accM[tt], 0, 0, 0);
    }
    // two halves of four sub-blocks: four independent products in flight,
    // scaled into accA as the next products run
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        u32x4 bq[4];
#pragma unroll
        for (int cc = 0; cc < 2; cc++)
            m16::codes8(r.q[2 * hf + cc][0], r.q[2 * hf + cc][1], bq[2 * cc], bq[2 * cc + 1]);
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            f32x4 tv[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const bf16x8 av = xf(4 * hf + jj, tt);
                tv[jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, bq[jj]),
                                                                 f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int j = 4 * hf + jj;
                const float ds = d * (float)(((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3))) & 0xffu);
#pragma unroll
                for (int e = 0; e < 4; e++) accA[tt][e] = fmaf(ds, tv[jj][e], accA[tt][e]);
            }
        }
    }
}

// One Q4_K tile by dequantization into acc[0..MT): the 8 B fragments of a
// lane (sub-block j = 2 cc + nib, its 8 values k = 32 j + 8 kg + i) are
// decoded once with v_fma_mix and serve every token tile. A nibble masked into
// an f16 half is the subnormal q 2^-24 (low, bits 0-3) or q 2^-20 (high, bits
// 4-7), so with the scale carrying 2^24 or 2^20 one fma gives d sc q - dmin m
// with a single rounding, then RNE to bf16 (the value every other Q4_K path
// here feeds the MFMA). Cheaper than the code products once the fragment
// serves two or more token tiles.
template <int MT, class XF>
__device__ __forceinline__ void tile_q4d(TileQ4 r, XF xf, int kg, f32x4 *acc) {
    pin(r);
    const uint32_t hx = r.h[0], hy = r.h[1], hz = r.h[2], hw = r.h[3];
    const float d = m16::cvt_f16_lo(hx), dmin = m16::cvt_f16_hi(hx);
    const uint32_t sc_lo = hy & 0x3F3F3F3Fu, m_lo = hz & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (hw & 0x0F0F0F0Fu) | ((hy >> 2) & 0x30303030u);
    const uint32_t m_hi = ((hw >> 4) & 0x0F0F0F0Fu) | ((hz >> 2) & 0x30303030u);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int cc = j >> 1, nib = j & 1;
        const uint32_t scw = j < 4 ? sc_lo : sc_hi, mw = j < 4 ? m_lo : m_hi;
        const float a = d * (float)((scw >> (8 * (j & 3))) & 0xffu) * (nib ? 0x1p20f : 0x1p24f);
        const float b = -(dmin * (float)((mw >> (8 * (j & 3))) & 0xffu));
        const uint32_t msk = nib ? 0x00F000F0u : 0x000F000Fu;
        const uint32_t y0 = r.q[cc][0], y1 = r.q[cc][1];
        const uint32_t p0 = y0 & msk, p1 = (y0 >> 8) & msk, p2 = y1 & msk, p3 = (y1 >> 8) & msk;
        const u32x4 bw = {pack_bf16x2(mix_lo(p0, a, b), mix_lo(p1, a, b)), pack_bf16x2(mix_hi(p0, a, b), mix_hi(p1, a, b)),
                          pack_bf16x2(mix_lo(p2, a, b), mix_lo(p3, a, b)), pack_bf16x2(mix_hi(p2, a, b), mix_hi(p3, a, b))};
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            const bf16x8 av = xf(j, tt);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, bw), acc[tt], 0, 0, 0);
        }
    }
}

// Q4_K tiles by code products up to this many token tiles, by dequantization
// beyond (the code products' per-tile-and-token-tile scaling outgrows one
// decode per value).
#ifndef QIMM_Q4_CP_MAX_MT
#define QIMM_Q4_CP_MAX_MT 1
#endif
constexpr bool q4_code_products(int mt) { return mt <= QIMM_Q4_CP_MAX_MT; }

// Partial sums cross workgroups on different XCDs: stored and loaded with
// system scope (sc0 sc1: written through to, and read from, memory).
// The partial sums as a buffer resource: four consecutive floats per 16 B
// access with the same system-scope bits (sc0 sc1), which a 16 B atomic or
// volatile access does not give (volatile loads each wait for the one before).
// Accesses past `bytes` read zero and drop their stores.
struct PartBuf {
    __amdgpu_buffer_rsrc_t r;
    static constexpr int SYS = 1 | 16;  // cache policy sc0 | sc1
    __device__ __forceinline__ PartBuf(const float *base, uint32_t bytes)
        : r(__builtin_amdgcn_make_buffer_rsrc((void *)base, 0, (int)bytes, 0x00020000)) {}
    __device__ __forceinline__ void put4(uint32_t idx, f32x4 v) const {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, idx * 4u, 0, SYS);
    }
    __device__ __forceinline__ f32x4 get4(uint32_t idx) const {
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, idx * 4u, 0, SYS));
    }
};
// one float with the same bits (the q/k/v gather reads column pairs)
__device__ __forceinline__ float get_coherent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Sums over the C chunks of NS slices at once: slice s is the four partial
// elements (row r, tokens 16 tts[s] + 4 kg + e) of a lane in group gs[s],
// summed in chunk order. Every slice's loads of a batch of CB chunks go out
// together (VB values in flight per lane), so the whole unit costs
// ceil(C / CB) memory round trips instead of one or more per slice.
// IS = floats per item.
template <int NS, int VB>
__device__ __forceinline__ void psum_slices(const PartBuf &pb, int C, int G, int IS, const int64_t (&gs)[NS],
                                            const int (&tts)[NS], int kg, int r, f32x4 (&out)[NS]) {
    constexpr int CB = VB / (4 * NS) > 0 ? VB / (4 * NS) : 1;
    uint32_t base[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        base[s] = (uint32_t)(gs[s] * IS + pidx(16 * tts[s] + 4 * kg, r));
        out[s] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int c0 = 0; c0 < C; c0 += CB) {
        float v[NS][CB][4];
#pragma unroll
        for (int cc = 0; cc < CB; cc++) {
            if (c0 + cc >= C) break;  // wave-uniform: no loads past the last chunk
            const uint32_t off = (uint32_t)(c0 + cc) * (uint32_t)G * (uint32_t)IS;
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const f32x4 t = pb.get4(base[s] + off);
#pragma unroll
                for (int e = 0; e < 4; e++) v[s][cc][e] = t[e];
            }
        }
#pragma unroll
        for (int cc = 0; cc < CB; cc++)
            if (c0 + cc < C) {
#pragma unroll
                for (int s = 0; s < NS; s++)
#pragma unroll
                    for (int e = 0; e < 4; e++) out[s][e] += v[s][cc][e];
            }
    }
}

template <int EPI, int MT>
__device__ void unit_epilogue(const float *part, const Plan &p, int64_t unit, int M, int64_t N, const EpiParams &ep,
                              int lane) {
    constexpr int TOK = 16 * MT, IS = 16 * TOK;
    const int l16 = lane & 15, kg = lane >> 4;
    const PartBuf pb(part, (uint32_t)p.C * (uint32_t)p.G * (uint32_t)IS * 4u);
    if constexpr (EPI == EPI_QKV) {
        // head unit: lane j holds columns (2j, 2j+1) of the head; TB tokens x
        // CB chunks per batch of loads (chunk sums in chunk order; 64 values
        // per lane where registers are scarce, 128 otherwise)
        const int64_t g = unit * 8 + (lane >> 3);
        const int r = 2 * (lane & 7);
        const int64_t nb = unit * 128 + ep.n_offset;
        const int sec = (int)(nb / ep.hidden);
        const int64_t head = (nb % ep.hidden) / 128;
        const int64_t S = ep.seq, H = ep.heads;
        constexpr int TB = MT == 1 ? 8 : 16, CB = 4;
        for (int m0 = 0; m0 < M; m0 += TB) {
            float sx[TB][2];
#pragma unroll
            for (int i = 0; i < TB; i++) sx[i][0] = sx[i][1] = 0.f;
            for (int c0 = 0; c0 < p.C; c0 += CB) {
                float v[CB][TB][2];
#pragma unroll
                for (int cc = 0; cc < CB; cc++) {
                    const float *pc = part + ((int64_t)min(c0 + cc, p.C - 1) * p.G + g) * IS;
#pragma unroll
                    for (int i = 0; i < TB; i++) {
                        const int m = min(m0 + i, TOK - 1);
                        v[cc][i][0] = get_coherent(pc + pidx(m, r));
                        v[cc][i][1] = get_coherent(pc + pidx(m, r + 1));
                    }
                }
#pragma unroll
                for (int cc = 0; cc < CB; cc++)
                    if (c0 + cc < p.C) {
#pragma unroll
                        for (int i = 0; i < TB; i++) {
                            sx[i][0] += v[cc][i][0];
                            sx[i][1] += v[cc][i][1];
                        }
                    }
            }
#pragma unroll
            for (int i = 0; i < TB; i++) {
                const int m = m0 + i;
                if (m >= M) break;
                float x0 = sx[i][0], x1 = sx[i][1];
                const int64_t b = m / S, s = m % S;
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
        }
    } else if constexpr (EPI == EPI_SWIGLU) {
        // hidden columns 64 blk + 16 q + l16: gate group 8 blk + q, up group 8 blk + 4 + q
        // (every token tile's partials were stored, so all MT tiles load)
        const int64_t blk = unit >> 2, q = unit & 3;
        const int64_t gg = 8 * blk + q, gu = gg + 4;
        int64_t gs[2 * MT];
        int tts[2 * MT];
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            gs[2 * tt] = gg;
            gs[2 * tt + 1] = gu;
            tts[2 * tt] = tts[2 * tt + 1] = tt;
        }
        f32x4 sum[2 * MT];
        psum_slices<2 * MT, MT == 1 ? 64 : 128>(pb, p.C, p.G, IS, gs, tts, kg, l16, sum);
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = 16 * tt + 4 * kg + e;
                if (m < M) store_hidden(ep, m * ep.ldh + 64 * blk + 16 * q + l16, silu(sum[2 * tt][e]) * sum[2 * tt + 1][e]);
            }
        }
    } else {
        const int64_t n = unit * 16 + l16;
        int64_t gs[MT];
        int tts[MT];
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            gs[tt] = unit;
            tts[tt] = tt;
        }
        f32x4 sum[MT];
        psum_slices<MT, MT == 1 ? 64 : 128>(pb, p.C, p.G, IS, gs, tts, kg, l16, sum);
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = 16 * tt + 4 * kg + e;
                if (m < M) {
                    const float v = sum[tt][e];
                    if constexpr (EPI == EPI_F32) {
                        ((float *)ep.out)[m * ep.ldo + n] = v;
                    } else if constexpr (EPI == EPI_BF16) {
                        ((uint16_t *)ep.out)[m * ep.ldo + n] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
                    } else {  // EPI_RESID
                        const float *grow = ep.gvec + (int64_t)(m / (int)ep.g_rows_per) * ep.g_stride;
                        ep.x_out[m * N + n] = ep.x_in[m * N + n] + grow[n] * v;
                    }
                }
            }
        }
    }
}

template <int FMT, int EPI, int STEPS, int MT>
__global__ __launch_bounds__(64 * nwaves(MT), wg_per_cu(MT) * nwaves(MT) / 4) void ws_kernel(const uint16_t *__restrict__ A, int M, int64_t lda,
                                                             GemmWeight w, float *__restrict__ part,
                                                             uint32_t *__restrict__ counters, Plan p, EpiParams ep) {
    constexpr int NW = nwaves(MT), TOK = 16 * MT, IS = 16 * TOK;
    __shared__ __attribute__((aligned(16))) uint8_t xs[TOK * XROW];
    const PartBuf pb(part, (uint32_t)p.C * (uint32_t)p.G * (uint32_t)IS * 4u);
    const int lane = threadIdx.x & 63, l16 = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = blockIdx.x % p.C, slot = blockIdx.x / p.C;
    const int64_t SB = w.k / 256, N = w.n;
    const int64_t gstep = (int64_t)p.WPC * NW;
    int64_t g = (int64_t)slot * NW + wave;

    // x chunk -> LDS by direct loads: instruction i of wave v fills 64
    // consecutive 16 B pieces of one row; rows past M repeat row M - 1
#pragma unroll
    for (int i = 0; i < TOK * (KCH / 8) / 64 / NW; i++) {
        const int q0 = (i * NW + wave) * 64;
        const int m = q0 / (KCH / 8), s0 = q0 % (KCH / 8);
        const uint16_t *src = A + (int64_t)min(m, M - 1) * lda + (int64_t)c * KCH + 8 * (s0 + lane);
        __builtin_amdgcn_global_load_lds((const void *)src, (lds_ptr_t)(xs + m * XROW + 16 * s0), 16, 0, 0);
    }
    if (g >= p.G) {  // no item for this wave: its x pieces still have to land
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        return;
    }
    Tile<FMT> ring[SBC];
#pragma unroll
    for (int t = 0; t < SBC; t++) {
        load_tile(w, g, (int64_t)c * SBC + t, SB, l16, kg, ring[t]);
        __builtin_amdgcn_sched_barrier(0);  // tiles issue in order: each wait covers one tile
    }
    // the x pieces were issued before the tiles: wait for them alone, then for
    // every wave's pieces
    constexpr int TL = FMT == WF_Q6_K ? 6 : 5;  // loads per tile
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(SBC * TL) : "memory");

    const uint8_t *xrow = xs + l16 * XROW;
    constexpr bool CP = FMT == WF_Q4_K && q4_code_products(MT);
    float xq0[SBC][MT], xq1[SBC][MT];
    if constexpr (CP) {
        // X_kg and X_{4+kg} of token 16 tt + l16 for the chunk's four
        // super-blocks, in the A layout of the f32 MFMA (bf16 MFMA against
        // row-selector ones)
        bf16x8 ones[4];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t v = (l16 >> 2) == s ? 0x3F803F80u : 0u;
            ones[s] = __builtin_bit_cast(bf16x8, u32x4{v, v, v, v});
        }
#pragma unroll
        for (int t = 0; t < SBC; t++)
#pragma unroll
            for (int tt = 0; tt < MT; tt++) {
                const uint8_t *xr = xrow + tt * 16 * XROW + 512 * t;
                f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const bf16x8 f0 = *(const bf16x8 *)(xr + 64 * j + 16 * kg);
                    const bf16x8 f1 = *(const bf16x8 *)(xr + 64 * (4 + j) + 16 * kg);
                    a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones[j], f0, a0, 0, 0, 0);
                    a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones[j], f1, a1, 0, 0, 0);
                }
                xq0[t][tt] = a0[0];
                xq1[t][tt] = a1[0];
            }
    }

    // items: the last one is peeled so the prefetch of the next item is
    // unconditional in the loop (the load counts stay exact for the waits)
    const int64_t g0 = g;
    auto item = [&](auto prefetch) {
        const int64_t gn = min(g + gstep, (int64_t)p.G - 1);
        f32x4 acc[MT], accM[MT];
#pragma unroll
        for (int tt = 0; tt < MT; tt++) acc[tt] = accM[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < SBC; t++) {
            const XLds<FMT> xt{xrow + 512 * t, kg};
            if constexpr (CP) tile_q4<MT>(ring[t], xt, kg, xq0[t], xq1[t], acc, accM);
            else if constexpr (FMT == WF_Q4_K) tile_q4d<MT>(ring[t], xt, kg, acc);
            else if constexpr (FMT == WF_Q6_K) tile_q6<MT>(ring[t], xt, kg, acc);
            else tile_q8<MT>(ring[t], xt, kg, acc);
            // finish this tile's arithmetic here: left alone, the compiler sinks
            // it past the loads and keeps every tile's products live
#pragma unroll
            for (int tt = 0; tt < MT; tt++)
#pragma unroll
                for (int e = 0; e < 4; e++) asm volatile("" : "+v"(acc[tt][e]));
            if constexpr (decltype(prefetch)::value) load_tile(w, gn, (int64_t)c * SBC + t, SB, l16, kg, ring[t]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // partial sums of the item: acc[tt][e] = token 16 tt + 4 kg + e, row 16 g + l16
        const uint32_t dst = ((uint32_t)c * (uint32_t)p.G + (uint32_t)g) * (uint32_t)IS;
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            if constexpr (CP) acc[tt] -= accM[tt];
            pb.put4(dst + pidx(16 * tt + 4 * kg, l16), acc[tt]);
        }
    };
    // straight-line over the (compile-time) step count: a loop here makes the
    // compiler wait for every outstanding load at its head. Every step but the
    // last prefetches (a wave with fewer items re-reads its last group's tiles
    // once instead of branching, which would also cost register copies).
    static_assert(STEPS >= 1 && STEPS <= MAX_STEPS, "steps");
    item(std::integral_constant<bool, (STEPS > 1)>{});
    if constexpr (STEPS > 1) {
        g += gstep;
        if (g < p.G) {
            item(std::integral_constant<bool, (STEPS > 2)>{});
            if constexpr (STEPS > 2) {
                g += gstep;
                if (g < p.G) {
                    item(std::integral_constant<bool, (STEPS > 3)>{});
                    if constexpr (STEPS > 3) {
                        g += gstep;
                        if (g < p.G) item(std::false_type{});
                    }
                }
            }
        }
    }

    // arrivals, once per wave after all of its items. The partial sums were
    // written through to memory (system-coherent stores, no dirty L2 lines), so
    // waiting for their completion publishes them to every XCD before the
    // counter moves; the completing wave reads them back the same way. (A
    // device-scope fence instead writes back and invalidates the whole L2.)
    // All of the wave's counter increments go out as one instruction (lane i
    // counts item i: one round trip), then the wave finishes every unit it
    // completed.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    auto unit_of = [&](int64_t gi) { return EPI == EPI_QKV ? gi / 8 : EPI == EPI_SWIGLU ? 4 * (gi / 8) + (gi & 3) : gi; };
    uint32_t old = 0;
    {
        const int64_t gl = g0 + (int64_t)lane * gstep;
        if (lane < STEPS && gl < p.G) old = atomicAdd(&counters[unit_of(gl)], 1u);
    }
#pragma unroll
    for (int i = 0; i < STEPS; i++) {
        const int64_t gi = g0 + i * gstep;
        if (gi >= p.G) break;
        if (__shfl(old, i) == (uint32_t)(p.C * p.per_unit - 1)) {
            const int64_t unit = unit_of(gi);
            unit_epilogue<EPI, MT>(part, p, unit, M, N, ep, lane);
            if (lane == 0) __hip_atomic_store(&counters[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int FMT, int STEPS, int MT>
hipError_t launch_steps(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep,
                        float *part, uint32_t *counters, const Plan &p, hipStream_t stream) {
    const dim3 grid((unsigned)(p.WPC * p.C)), block(64 * nwaves(MT));
    switch (epi) {
    case EPI_F32: ws_kernel<FMT, EPI_F32, STEPS, MT><<<grid, block, 0, stream>>>(a, m, lda, w, part, counters, p, ep); break;
    case EPI_BF16: ws_kernel<FMT, EPI_BF16, STEPS, MT><<<grid, block, 0, stream>>>(a, m, lda, w, part, counters, p, ep); break;
    case EPI_RESID: ws_kernel<FMT, EPI_RESID, STEPS, MT><<<grid, block, 0, stream>>>(a, m, lda, w, part, counters, p, ep); break;
    case EPI_SWIGLU: ws_kernel<FMT, EPI_SWIGLU, STEPS, MT><<<grid, block, 0, stream>>>(a, m, lda, w, part, counters, p, ep); break;
    case EPI_QKV: ws_kernel<FMT, EPI_QKV, STEPS, MT><<<grid, block, 0, stream>>>(a, m, lda, w, part, counters, p, ep); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int FMT, int MT>
hipError_t launch_mt(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep,
                     float *part, uint32_t *counters, const Plan &p, hipStream_t stream) {
    switch (p.steps) {
    case 1: return launch_steps<FMT, 1, MT>(w, a, m, lda, epi, ep, part, counters, p, stream);
    case 2: return launch_steps<FMT, 2, MT>(w, a, m, lda, epi, ep, part, counters, p, stream);
    case 3: return launch_steps<FMT, 3, MT>(w, a, m, lda, epi, ep, part, counters, p, stream);
    case 4: return launch_steps<FMT, 4, MT>(w, a, m, lda, epi, ep, part, counters, p, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int FMT>
hipError_t launch(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep,
                  float *part, uint32_t *counters, const Plan &p, hipStream_t stream) {
    switch (p.MT) {
    case 1: return launch_mt<FMT, 1>(w, a, m, lda, epi, ep, part, counters, p, stream);
    case 2: return launch_mt<FMT, 2>(w, a, m, lda, epi, ep, part, counters, p, stream);
    case 4: return launch_mt<FMT, 4>(w, a, m, lda, epi, ep, part, counters, p, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ws

// ---------------------------------------------------------------------------
// M <= 16, Q4_K / Q6_K / Q8_0, K <= 4096 with K % 1024 == 0, plain, residual or
// SwiGLU outputs with at least one workgroup step per CU: the split-K sum of a
// unit inside one workgroup.
//
// All of x (16 rows x K) sits in LDS (132 KB at K = 4096), so one workgroup of
// eight waves per CU holds every k chunk. Wave v always takes chunk v % C of
// group slot v / C; a step covers NW / (C * per_unit) whole epilogue units
// (a SwiGLU unit's gate and up groups, or single groups), and the workgroup
// walks its steps (grid-strided over the units) with the next step's tiles in
// registers, as in the cross-workgroup kernel. The partial sums of a step go
// to LDS (double-buffered by step), one barrier, and the chunk-0 wave of each
// unit adds them in chunk order (deterministic) and applies the epilogue.
// Against the cross-workgroup kernel this drops the partial-sum stores and
// loads through memory, the arrival counters and the three memory round trips
// at the tail.
namespace wl {

constexpr int NW = 8;    // waves per workgroup (one workgroup per CU)
constexpr int MAXC = 4;  // k chunks of x held in LDS

struct Plan {
    int C, G, UPS, per_unit, total, steps;
};

bool plan(const GemmWeight &w, int64_t m, int epi, int cus, Plan &p) {
    if ((w.fmt != WF_Q4_K && w.fmt != WF_Q6_K && w.fmt != WF_Q8_0) || m < 1 || m > 16 || w.k % ws::KCH ||
        w.n % 16 || cus <= 0 || epi == EPI_QKV)
        return false;
    if (epi == EPI_SWIGLU && w.n % 128) return false;
    p.C = (int)(w.k / ws::KCH);
    p.per_unit = epi == EPI_SWIGLU ? 2 : 1;
    const int items = p.C * p.per_unit;  // items per unit
    if (p.C > MAXC || NW % items) return false;
    p.UPS = NW / items;
    p.G = (int)(w.n / 16);
    const int units = p.G / p.per_unit;
    if (units % p.UPS) return false;
    p.total = units / p.UPS;
    // fewer workgroup steps than CUs leave CUs idle: the cross-workgroup
    // kernel spreads such products wider
    if (p.total < cus) return false;
    p.steps = (p.total + cus - 1) / cus;
    return p.steps <= ws::MAX_STEPS;
}

template <int FMT, int EPI, int STEPS>
__global__ __launch_bounds__(64 * NW, 1) void wl_kernel(const uint16_t *__restrict__ A, int M, int64_t lda, GemmWeight w,
                                                        Plan p, EpiParams ep) {
    using namespace ws;
    __shared__ __attribute__((aligned(16))) uint8_t xs[MAXC * 16 * XROW];
    __shared__ __attribute__((aligned(16))) float red[2][NW][256];
    const int lane = threadIdx.x & 63, l16 = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = wave % p.C, gi = wave / p.C;  // this wave's chunk and group slot
    const int64_t SB = w.k / 256, N = w.n;
    const int64_t grid = gridDim.x;
    // group of this wave at workgroup step st
    auto group_of = [&](int64_t st) __attribute__((always_inline)) {
        const int64_t unit = st * p.UPS + gi / p.per_unit;
        if constexpr (EPI == EPI_SWIGLU) return 8 * (unit >> 2) + (unit & 3) + 4 * (gi & 1);  // gate, then up
        else return unit;
    };

    // all of x -> LDS by direct loads: instruction i of wave v fills 64
    // consecutive 16 B pieces of one row of one chunk; rows past M repeat row M - 1
    const int pieces = p.C * 16 * (KCH / 8);
    for (int q0 = wave * 64; q0 < pieces; q0 += NW * 64) {
        const int cc = q0 / (16 * (KCH / 8)), rem = q0 % (16 * (KCH / 8));
        const int m = rem / (KCH / 8), s0 = rem % (KCH / 8);
        const uint16_t *src = A + (int64_t)min(m, M - 1) * lda + (int64_t)cc * KCH + 8 * (s0 + lane);
        __builtin_amdgcn_global_load_lds((const void *)src, (lds_ptr_t)(xs + (cc * 16 + m) * XROW + 16 * s0), 16, 0, 0);
    }
    int64_t st = blockIdx.x;
    int64_t g = group_of(st);
    Tile<FMT> ring[SBC];
#pragma unroll
    for (int t = 0; t < SBC; t++) {
        load_tile(w, g, (int64_t)c * SBC + t, SB, l16, kg, ring[t]);
        __builtin_amdgcn_sched_barrier(0);  // tiles issue in order: each wait covers one tile
    }
    // the x pieces were issued before the tiles: wait for them alone, then for
    // every wave's pieces
    constexpr int TL = FMT == WF_Q6_K ? 6 : 5;  // loads per tile
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(SBC * TL) : "memory");

    const uint8_t *xrow = xs + (c * 16 + l16) * XROW;
    constexpr bool CP = FMT == WF_Q4_K && q4_code_products(1);
    float xq0[SBC], xq1[SBC];
    if constexpr (CP) {
        // X_kg and X_{4+kg} of token l16 for the chunk's four super-blocks
        bf16x8 ones[4];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t v = (l16 >> 2) == s ? 0x3F803F80u : 0u;
            ones[s] = __builtin_bit_cast(bf16x8, u32x4{v, v, v, v});
        }
#pragma unroll
        for (int t = 0; t < SBC; t++) {
            const uint8_t *xr = xrow + 512 * t;
            f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bf16x8 f0 = *(const bf16x8 *)(xr + 64 * j + 16 * kg);
                const bf16x8 f1 = *(const bf16x8 *)(xr + 64 * (4 + j) + 16 * kg);
                a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones[j], f0, a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones[j], f1, a1, 0, 0, 0);
            }
            xq0[t] = a0[0];
            xq1[t] = a1[0];
        }
    }

    // one workgroup step: this wave's item, its partial sums to LDS, the
    // barrier, then the unit's chunk-0 wave reduces and stores
    auto step = [&](int s, auto prefetch) __attribute__((always_inline)) {
        const int64_t gn = group_of(min(st + grid, (int64_t)p.total - 1));
        f32x4 acc[1], accM[1];
        acc[0] = accM[0] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < SBC; t++) {
            const XLds<FMT> xt{xrow + 512 * t, kg};
            if constexpr (CP) tile_q4<1>(ring[t], xt, kg, &xq0[t], &xq1[t], acc, accM);
            else if constexpr (FMT == WF_Q4_K) tile_q4d<1>(ring[t], xt, kg, acc);
            else if constexpr (FMT == WF_Q6_K) tile_q6<1>(ring[t], xt, kg, acc);
            else tile_q8<1>(ring[t], xt, kg, acc);
#pragma unroll
            for (int e = 0; e < 4; e++) asm volatile("" : "+v"(acc[0][e]));
            if constexpr (decltype(prefetch)::value) load_tile(w, gn, (int64_t)c * SBC + t, SB, l16, kg, ring[t]);
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (CP) acc[0] -= accM[0];
        float *mine = red[s & 1][wave];
#pragma unroll
        for (int e = 0; e < 4; e++) mine[(4 * kg + e) * 16 + l16] = acc[0][e];
        __syncthreads();
        // chunk sums in chunk order; lane holds tokens 4 kg + e of column l16
        auto csum = [&](int slot) __attribute__((always_inline)) {
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            for (int cc = 0; cc < p.C; cc++) {
                const float *r = red[s & 1][slot * p.C + cc];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] += r[(4 * kg + e) * 16 + l16];
            }
            return v;
        };
        if (c == 0 && (EPI != EPI_SWIGLU || (gi & 1) == 0)) {
            const f32x4 v = csum(gi);
            if constexpr (EPI == EPI_SWIGLU) {
                const f32x4 up = csum(gi + 1);
                const int64_t unit = st * p.UPS + gi / 2, blk = unit >> 2, q = unit & 3;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int m = 4 * kg + e;
                    if (m < M) store_hidden(ep, m * ep.ldh + 64 * blk + 16 * q + l16, silu(v[e]) * up[e]);
                }
            } else {
                const int64_t n = g * 16 + l16;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int m = 4 * kg + e;
                    if (m < M) {
                        if constexpr (EPI == EPI_F32) {
                            ((float *)ep.out)[m * ep.ldo + n] = v[e];
                        } else if constexpr (EPI == EPI_BF16) {
                            ((uint16_t *)ep.out)[m * ep.ldo + n] = (uint16_t)(pack_bf16x2(v[e], 0.f) & 0xffffu);
                        } else {  // EPI_RESID
                            const float *grow = ep.gvec + (int64_t)(m / (int)ep.g_rows_per) * ep.g_stride;
                            ep.x_out[m * N + n] = ep.x_in[m * N + n] + grow[n] * v[e];
                        }
                    }
                }
            }
        }
        st += grid;
        g = gn;
    };
    // straight-line over the compile-time step count (see the cross-workgroup
    // kernel); the guard is uniform over the workgroup, so every wave meets
    // the same barriers
    static_assert(STEPS >= 1 && STEPS <= MAX_STEPS, "steps");
    step(0, std::integral_constant<bool, (STEPS > 1)>{});
    if constexpr (STEPS > 1) {
        if (st < p.total) {
            step(1, std::integral_constant<bool, (STEPS > 2)>{});
            if constexpr (STEPS > 2) {
                if (st < p.total) {
                    step(2, std::integral_constant<bool, (STEPS > 3)>{});
                    if constexpr (STEPS > 3) {
                        if (st < p.total) step(3, std::false_type{});
                    }
                }
            }
        }
    }
}

template <int FMT, int STEPS>
hipError_t launch_steps(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep,
                        const Plan &p, int grid, hipStream_t stream) {
    const dim3 g((unsigned)grid), block(64 * NW);
    switch (epi) {
    case EPI_F32: wl_kernel<FMT, EPI_F32, STEPS><<<g, block, 0, stream>>>(a, m, lda, w, p, ep); break;
    case EPI_BF16: wl_kernel<FMT, EPI_BF16, STEPS><<<g, block, 0, stream>>>(a, m, lda, w, p, ep); break;
    case EPI_RESID: wl_kernel<FMT, EPI_RESID, STEPS><<<g, block, 0, stream>>>(a, m, lda, w, p, ep); break;
    case EPI_SWIGLU: wl_kernel<FMT, EPI_SWIGLU, STEPS><<<g, block, 0, stream>>>(a, m, lda, w, p, ep); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t launch(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep,
                  const Plan &p, int cus, hipStream_t stream) {
    switch (p.steps) {
    case 1: return launch_steps<FMT, 1>(w, a, m, lda, epi, ep, p, cus, stream);
    case 2: return launch_steps<FMT, 2>(w, a, m, lda, epi, ep, p, cus, stream);
    case 3: return launch_steps<FMT, 3>(w, a, m, lda, epi, ep, p, cus, stream);
    case 4: return launch_steps<FMT, 4>(w, a, m, lda, epi, ep, p, cus, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace wl

// ---------------------------------------------------------------------------
// M <= 16, Q4_K / Q6_K / Q8_0, plain or residual outputs with about one 16-row
// group per CU (the 4096-row down and out projections: 256 groups) and K a
// multiple of 2048: one workgroup per group over the whole K, so no partial
// sums leave the workgroup.
//
// The eight waves split K into slices of TPW consecutive 256-k tiles (which
// wave takes which slice rotates with the workgroup, so that CUs running in
// step read different x lines). Every A fragment then serves one wave only, so
// x is not staged in LDS:
// a wave loads its fragments from global memory (16 x K bf16, L2-resident after
// the first workgroups touch it) straight into registers, XD tiles ahead, while
// its weight tiles (up to RD) are all requested at the start. The eight
// partial sums meet in LDS; wave 0 adds them in K order (deterministic) and
// applies the epilogue. Against the cross-workgroup kernel this drops the
// partial-sum stores and loads through memory and the arrival counters, and
// every CU keeps all of its weight bytes in flight from the first instruction.
namespace wx {

constexpr int NW = 8;    // waves per workgroup (one workgroup per CU)
constexpr int RD = 6;    // weight tiles in flight per wave
constexpr int XD = 2;    // x tiles loaded ahead
constexpr int MAXT = 8;  // tiles per wave

bool plan(const GemmWeight &w, int64_t m, int epi, int cus, int &tpw) {
    if ((w.fmt != WF_Q4_K && w.fmt != WF_Q6_K && w.fmt != WF_Q8_0) || m < 1 || m > 16 || w.n % 16 || cus <= 0 ||
        (epi != EPI_F32 && epi != EPI_BF16 && epi != EPI_RESID) || w.k % (256 * NW))
        return false;
    const int64_t G = w.n / 16;
    tpw = (int)(w.k / (256 * NW));
    // Every workgroup reads all of x (M x K bf16). Beyond K = 4096, once that
    // passes about twice the group's weight bytes it costs more than the
    // cross-workgroup kernel's partial sums (measured: Q6_K at K = 12288 wins
    // up to 13 tokens, Q8_0 at K = 16384 up to 16).
    const int wb = w.fmt == WF_Q4_K ? 144 : w.fmt == WF_Q6_K ? 224 : 272;  // device bytes per 256 weights
    if (w.k > 4096 && m * 2 * 256 >= 2 * 16 * wb) return false;
    // more groups than CUs share x better in the LDS-staged kernels; far fewer
    // leave CUs idle
    return tpw >= 1 && tpw <= MAXT && 2 * G >= cus && G <= cus;
}

// A fragments of one tile held in registers (step s -> fragment s)
struct XReg {
    const bf16x8 *f;
    __device__ __forceinline__ bf16x8 operator()(int s, int) const { return f[s]; }
};

template <int FMT, int EPI, int TPW>
__global__ __launch_bounds__(64 * NW, 1) void wx_kernel(const uint16_t *__restrict__ A, int M, int64_t lda, GemmWeight w,
                                                        EpiParams ep) {
    using namespace ws;
    constexpr int R = TPW < RD ? TPW : RD, X = TPW < XD ? TPW : XD;
    __shared__ __attribute__((aligned(16))) float red[NW][256];
    const int lane = threadIdx.x & 63, l16 = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t g = blockIdx.x, SB = w.k / 256, N = w.n;
    // K slice of this wave, rotated by workgroup: the same wave of every CU
    // would otherwise read the same x lines at the same time
    const int slice = (wave + (int)(g % NW)) % NW;
    const int64_t sb0 = (int64_t)slice * TPW;
    // this lane's token row (rows past M repeat row M - 1) at the wave's first tile
    const uint8_t *xr = (const uint8_t *)(A + (int64_t)min(l16, M - 1) * lda) + sb0 * 512;
    Tile<FMT> ring[R];
    bf16x8 xf[X][8];
    auto load_x = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < 8; s++) xf[t % X][s] = *(const bf16x8 *)(xr + t * 512 + xoff<FMT>(s, kg));
    };
    // issue order x0 w0 x1 w1 w2 ...: the first tile waits for its own bytes only
#pragma unroll
    for (int t = 0; t < R; t++) {
        if (t < X) load_x(t);
        load_tile(w, g, sb0 + t, SB, l16, kg, ring[t]);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Q4_K by code products (exact weights, as in the other kernels up to 16
    // tokens): X_kg and X_{4+kg} of token l16 from the tile's fragments by
    // bf16 MFMA against row-selector ones
    constexpr bool CP = FMT == WF_Q4_K && q4_code_products(1);
    bf16x8 ones[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const uint32_t v = (l16 >> 2) == s ? 0x3F803F80u : 0u;
        ones[s] = __builtin_bit_cast(bf16x8, u32x4{v, v, v, v});
    }
    f32x4 acc[1], accM[1];
    acc[0] = accM[0] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const XReg xt{xf[t % X]};
        if constexpr (CP) {
            f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones[j], xf[t % X][j], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones[j], xf[t % X][4 + j], a1, 0, 0, 0);
            }
            const float xq0 = a0[0], xq1 = a1[0];
            tile_q4<1>(ring[t % R], xt, kg, &xq0, &xq1, acc, accM);
        } else if constexpr (FMT == WF_Q4_K) tile_q4d<1>(ring[t % R], xt, kg, acc);
        else if constexpr (FMT == WF_Q6_K) tile_q6<1>(ring[t % R], xt, kg, acc);
        else tile_q8<1>(ring[t % R], xt, kg, acc);
#pragma unroll
        for (int e = 0; e < 4; e++) asm volatile("" : "+v"(acc[0][e]));
        if (t + R < TPW) load_tile(w, g, sb0 + t + R, SB, l16, kg, ring[t % R]);
        if (t + X < TPW) load_x(t + X);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (CP) acc[0] -= accM[0];
    // acc[0][e] = token 4 kg + e, row 16 g + l16
#pragma unroll
    for (int e = 0; e < 4; e++) red[slice][(4 * kg + e) * 16 + l16] = acc[0][e];
    __syncthreads();
    if (wave != 0) return;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NW; c++)
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] += red[c][(4 * kg + e) * 16 + l16];
    const int64_t n = g * 16 + l16;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int m = 4 * kg + e;
        if (m < M) {
            if constexpr (EPI == EPI_F32) {
                ((float *)ep.out)[m * ep.ldo + n] = v[e];
            } else if constexpr (EPI == EPI_BF16) {
                ((uint16_t *)ep.out)[m * ep.ldo + n] = (uint16_t)(pack_bf16x2(v[e], 0.f) & 0xffffu);
            } else {  // EPI_RESID
                const float *grow = ep.gvec + (int64_t)(m / (int)ep.g_rows_per) * ep.g_stride;
                ep.x_out[m * N + n] = ep.x_in[m * N + n] + grow[n] * v[e];
            }
        }
    }
}

template <int FMT, int TPW>
hipError_t launch_tpw(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep,
                      hipStream_t stream) {
    const dim3 grid((unsigned)(w.n / 16)), block(64 * NW);
    switch (epi) {
    case EPI_F32: wx_kernel<FMT, EPI_F32, TPW><<<grid, block, 0, stream>>>(a, m, lda, w, ep); break;
    case EPI_BF16: wx_kernel<FMT, EPI_BF16, TPW><<<grid, block, 0, stream>>>(a, m, lda, w, ep); break;
    case EPI_RESID: wx_kernel<FMT, EPI_RESID, TPW><<<grid, block, 0, stream>>>(a, m, lda, w, ep); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t launch(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep, int tpw,
                  hipStream_t stream) {
    switch (tpw) {
    case 1: return launch_tpw<FMT, 1>(w, a, m, lda, epi, ep, stream);
    case 2: return launch_tpw<FMT, 2>(w, a, m, lda, epi, ep, stream);
    case 3: return launch_tpw<FMT, 3>(w, a, m, lda, epi, ep, stream);
    case 4: return launch_tpw<FMT, 4>(w, a, m, lda, epi, ep, stream);
    case 5: return launch_tpw<FMT, 5>(w, a, m, lda, epi, ep, stream);
    case 6: return launch_tpw<FMT, 6>(w, a, m, lda, epi, ep, stream);
    case 7: return launch_tpw<FMT, 7>(w, a, m, lda, epi, ep, stream);
    case 8: return launch_tpw<FMT, 8>(w, a, m, lda, epi, ep, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace wx

// ---------------------------------------------------------------------------
// 17-64 tokens, K = 4096, plain or SwiGLU outputs with 4 or 6 weight
// groups (16 rows each) per CU: each workgroup keeps its groups over the whole
// K, so no partial sums leave it.
//
// Two waves per group, one for the even and one for the odd 256-k tiles. x
// goes through LDS in 512-wide sub-chunks (one tile per wave), double-buffered
// and staged through registers one sub-chunk ahead (register loads only, so the
// compiler's load waits stay exact); each wave keeps R weight tiles in flight.
// After the last sub-chunk the two waves of a group add their sums in LDS (even
// wave first) and the epilogue runs per unit. Against the cross-workgroup
// kernel this drops the split-K partial sums (C x 64 x N x 4 bytes written and
// read back), the arrival counters and the memory round trips at the tail, for
// eight x sub-chunk reads from L2 per workgroup instead of one chunk.
namespace wk {

constexpr int SKC = 512;           // k per x sub-chunk (two 256-k tiles)
constexpr int XP = SKC * 2 + 16;   // padded LDS row: a fragment's 16 rows hit distinct bank groups
constexpr int KS = 4096 / SKC;     // sub-chunks (K = 4096)

struct Plan {
    int GPW, UPW, per_unit;
};

bool plan(const GemmWeight &w, int64_t m, int epi, int cus, Plan &p) {
    if ((w.fmt != WF_Q4_K && w.fmt != WF_Q6_K && w.fmt != WF_Q8_0) || m < 17 || m > 64 || cus <= 0 ||
        (epi != EPI_F32 && epi != EPI_BF16 && epi != EPI_SWIGLU) || w.k != 4096 || w.n % 128)
        return false;
    const int64_t G = w.n / 16;
    if (G % cus) return false;
    p.GPW = (int)(G / cus);
    p.per_unit = epi == EPI_SWIGLU ? 2 : 1;
    p.UPW = p.GPW / p.per_unit;
    return p.GPW == 4 || p.GPW == 6;
}

// A fragments from an x sub-chunk row in LDS (token tile tt 16 rows further)
template <int FMT>
struct XSub {
    const uint8_t *row;
    int kg;
    __device__ __forceinline__ bf16x8 operator()(int s, int tt) const {
        return *(const bf16x8 *)(row + tt * 16 * XP + ws::xoff<FMT>(s, kg));
    }
};

template <int FMT, int EPI, int MT, int GPW>
__global__ __launch_bounds__(128 * GPW, 1) void wk_kernel(const uint16_t *__restrict__ A, int M, int64_t lda,
                                                          GemmWeight w, Plan p, EpiParams ep) {
    constexpr int NWV = 2 * GPW, NT = 64 * NWV, TOK = 16 * MT;
    constexpr int PIECES = TOK * (SKC / 8);  // 16 B pieces of a sub-chunk
    constexpr int NP = (PIECES + NT - 1) / NT;
    // weight tiles in flight per wave (Q8_0 tiles take 20 registers: two at
    // 64 tokens with three waves per SIMD)
    constexpr int R = FMT == WF_Q4_K ? 4 : (FMT == WF_Q8_0 && MT == 4 && GPW == 6) ? 2 : 3;
    static_assert(2 * TOK * XP >= NWV * TOK * 16 * 4, "the reduction reuses the x buffers");
    using ws::Tile;
    using ws::load_tile;
    __shared__ __attribute__((aligned(16))) uint8_t xs[2 * TOK * XP];
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gs = wave >> 1, par = wave & 1;  // group slot, tile parity
    const int64_t unit = (int64_t)blockIdx.x * p.UPW + gs / p.per_unit;
    int64_t g;
    if constexpr (EPI == EPI_SWIGLU) g = 8 * (unit >> 2) + (unit & 3) + 4 * (gs & 1);  // gate, then up
    else g = unit;
    const int64_t SB = w.k / 256;

    // x sub-chunk j <-> registers <-> LDS buffer; rows past M repeat row M - 1
    u32x4 xr[NP];
    auto x_load = [&](int j) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int pc = tid + i * NT;
            if (PIECES % NT == 0 || pc < PIECES) {
                const int m = pc / (SKC / 8), s = pc % (SKC / 8);
                xr[i] = *(const u32x4 *)(A + (int64_t)min(m, M - 1) * lda + (int64_t)j * SKC + 8 * s);
            }
        }
    };
    auto x_store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int pc = tid + i * NT;
            if (PIECES % NT == 0 || pc < PIECES) {
                const int m = pc / (SKC / 8), s = pc % (SKC / 8);
                *(u32x4 *)(xs + buf * TOK * XP + m * XP + 16 * s) = xr[i];
            }
        }
    };

    // the tile of sub-chunk j for this wave is super-block 2 j + par
    Tile<FMT> ring[R];
    x_load(0);
    x_store(0);
    x_load(1);
#pragma unroll
    for (int r = 0; r < R; r++) {
        load_tile(w, g, 2 * r + par, SB, l16, kg, ring[r]);
        __builtin_amdgcn_sched_barrier(0);  // tiles issue in order: each wait covers one tile
    }
    __syncthreads();

    f32x4 acc[MT];
#pragma unroll
    for (int tt = 0; tt < MT; tt++) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // straight-line over the sub-chunks (ring slots are compile-time indices)
#pragma unroll
    for (int j = 0; j < KS; j++) {
        if (j + 1 < KS) x_store((j + 1) & 1);  // buffer of sub-chunk j - 1: freed by the last barrier
        if (j + 2 < KS) x_load(j + 2);
        const XSub<FMT> xt{xs + (j & 1) * TOK * XP + l16 * XP + 512 * par, kg};
        Tile<FMT> &t = ring[j % R];
        if constexpr (FMT == WF_Q4_K) ws::tile_q4d<MT>(t, xt, kg, acc);
        else if constexpr (FMT == WF_Q6_K) ws::tile_q6<MT>(t, xt, kg, acc);
        else ws::tile_q8<MT>(t, xt, kg, acc);
        // finish this tile's arithmetic here, not past the loads
#pragma unroll
        for (int tt = 0; tt < MT; tt++)
#pragma unroll
            for (int e = 0; e < 4; e++) asm volatile("" : "+v"(acc[tt][e]));
        if (j + R < KS) load_tile(w, g, 2 * (j + R) + par, SB, l16, kg, t);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // sub-chunk j + 1 written, sub-chunk j's buffer free
    }

    // the waves' sums meet in LDS (the x buffers, free after the last barrier):
    // red[wave][token][row], lane holding tokens 16 tt + 4 kg + e of row l16
    float *red = (float *)xs;
#pragma unroll
    for (int tt = 0; tt < MT; tt++)
#pragma unroll
        for (int e = 0; e < 4; e++) red[(wave * TOK + 16 * tt + 4 * kg + e) * 16 + l16] = acc[tt][e];
    __syncthreads();
    auto gsum = [&](int slot, int tt) __attribute__((always_inline)) {  // even wave, then odd
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = 16 * tt + 4 * kg + e;
            v[e] = red[((2 * slot) * TOK + m) * 16 + l16] + red[((2 * slot + 1) * TOK + m) * 16 + l16];
        }
        return v;
    };
    if (par == 0 && (EPI != EPI_SWIGLU || (gs & 1) == 0)) {
#pragma unroll
        for (int tt = 0; tt < MT; tt++) {
            const f32x4 v = gsum(gs, tt);
            if constexpr (EPI == EPI_SWIGLU) {
                const f32x4 up = gsum(gs + 1, tt);
                const int64_t blk = unit >> 2, q = unit & 3;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int m = 16 * tt + 4 * kg + e;
                    if (m < M) store_hidden(ep, m * ep.ldh + 64 * blk + 16 * q + l16, silu(v[e]) * up[e]);
                }
            } else {
                const int64_t n = g * 16 + l16;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int m = 16 * tt + 4 * kg + e;
                    if (m < M) {
                        if constexpr (EPI == EPI_F32) ((float *)ep.out)[m * ep.ldo + n] = v[e];
                        else ((uint16_t *)ep.out)[m * ep.ldo + n] = (uint16_t)(pack_bf16x2(v[e], 0.f) & 0xffffu);
                    }
                }
            }
        }
    }
}

template <int FMT, int MT, int GPW>
hipError_t launch_g(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep,
                    const Plan &p, hipStream_t stream) {
    const dim3 grid((unsigned)(w.n / 16 / GPW)), block(128 * GPW);
    switch (epi) {
    case EPI_F32: wk_kernel<FMT, EPI_F32, MT, GPW><<<grid, block, 0, stream>>>(a, m, lda, w, p, ep); break;
    case EPI_BF16: wk_kernel<FMT, EPI_BF16, MT, GPW><<<grid, block, 0, stream>>>(a, m, lda, w, p, ep); break;
    case EPI_SWIGLU: wk_kernel<FMT, EPI_SWIGLU, MT, GPW><<<grid, block, 0, stream>>>(a, m, lda, w, p, ep); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t launch(const GemmWeight &w, const uint16_t *a, int m, int64_t lda, int epi, const EpiParams &ep,
                  const Plan &p, hipStream_t stream) {
    if (m <= 32) return p.GPW == 4 ? launch_g<FMT, 2, 4>(w, a, m, lda, epi, ep, p, stream)
                                   : launch_g<FMT, 2, 6>(w, a, m, lda, epi, ep, p, stream);
    return p.GPW == 4 ? launch_g<FMT, 4, 4>(w, a, m, lda, epi, ep, p, stream)
                      : launch_g<FMT, 4, 6>(w, a, m, lda, epi, ep, p, stream);
}

}  // namespace wk

// Sum of the split-K partials of 4 consecutive outputs at idx (16 B aligned),
// in split order; every share's 16 B load is issued before the adds.
constexpr int MAX_SPLITS = 16;  // qgemm_stream_splits and qgemm_mid_splits stay within it
__device__ __forceinline__ f32x4 csum4(const float *part, int splits, int64_t MN, int64_t idx) {
    f32x4 p[MAX_SPLITS];
#pragma unroll
    for (int s = 0; s < MAX_SPLITS; s++)
        if (s < splits) p[s] = *(const f32x4 *)(part + s * MN + idx);
    f32x4 v = p[0];
#pragma unroll
    for (int s = 1; s < MAX_SPLITS; s++)
        if (s < splits) v += p[s];
    return v;
}

// Elementwise epilogues: one thread per 4 consecutive outputs (SwiGLU: per 4
// output columns of the hidden, gate and up read from the interleaved layout).
template <int EPI>
__global__ __launch_bounds__(256) void stream_epi_kernel(const float *__restrict__ part, int splits, int64_t M,
                                                         int64_t N, EpiParams ep) {
    const int64_t MN = M * N;
    const uint32_t q = blockIdx.x * 256u + threadIdx.x;  // quad index (M * N < 2^31, N % 4 == 0)
    if constexpr (EPI == EPI_SWIGLU) {
        // hidden column h = 64 g + j (j < 64): gate at device column 128 g + j, up at 128 g + 64 + j
        const uint32_t F = (uint32_t)(N / 2);
        if ((int64_t)q * 4 >= M * F) return;
        const uint32_t m = q * 4 / F, h = q * 4 % F;
        const int64_t cg = (int64_t)(h >> 6) * 128 + (h & 63);
        const f32x4 gt = csum4(part, splits, MN, (int64_t)m * N + cg), up = csum4(part, splits, MN, (int64_t)m * N + cg + 64);
        const f32x4 hv{silu(gt[0]) * up[0], silu(gt[1]) * up[1], silu(gt[2]) * up[2], silu(gt[3]) * up[3]};
        if (ep.hmid_f32)
            *(f32x4 *)(ep.hmid_f32 + (int64_t)m * ep.ldh + h) = hv;
        else
            *(u32x2 *)(ep.hmid + (int64_t)m * ep.ldh + h) = u32x2{pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3])};
    } else {
        const int64_t idx = (int64_t)q * 4;
        if (idx >= MN) return;
        const uint32_t m = (uint32_t)(idx / N), n = (uint32_t)(idx % N);
        const f32x4 v = csum4(part, splits, MN, idx);
        if constexpr (EPI == EPI_F32) {
            *(f32x4 *)((float *)ep.out + (int64_t)m * ep.ldo + n) = v;
        } else if constexpr (EPI == EPI_BF16) {
            *(u32x2 *)((uint16_t *)ep.out + (int64_t)m * ep.ldo + n) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        } else {  // EPI_RESID
            const float *grow = ep.gvec + (int64_t)((int)m / (int)ep.g_rows_per) * ep.g_stride;
            const f32x4 x = *(const f32x4 *)(ep.x_in + idx), gv = *(const f32x4 *)(grow + n);
            *(f32x4 *)(ep.x_out + idx) = x + gv * v;
        }
    }
}

// QKV epilogue in one launch. Workgroups [0, nqk): one wave per (token, HG
// consecutive q or k heads), lane j holding the RoPE pair (2j, 2j+1) of each
// head's 128 columns (every load of the wave issued before the sums, the HG
// row reductions independent).
// The rest: one workgroup per (batch, 32 tokens, v head), which sums the
// shares of 32 tokens x 128 columns (16 B per thread and share, rows read
// whole), writes the [B,H,S,D] copy directly and goes through an LDS tile
// [d][token] for vt [B,H,D,S], whose rows then take 32 consecutive tokens per
// store run instead of one 2-byte store per value.
constexpr int VT_T = 32;  // tokens per v workgroup
constexpr int VT_P = 33;  // bf16 pitch of the transpose tile rows: the 32 rows 4 c of one write go to distinct banks
template <int HG>
__global__ __launch_bounds__(256) void stream_qkv_kernel(const float *__restrict__ part, int splits, int64_t M,
                                                         int64_t N, EpiParams ep, int64_t nqk, int64_t c_first,
                                                         int64_t heads_v) {
    __shared__ uint16_t tile[128 * VT_P];
    const int64_t MN = M * N;
    const int64_t S = ep.seq, H = ep.heads;
    if ((int64_t)blockIdx.x >= nqk) {
        const int64_t sblocks = (S + VT_T - 1) / VT_T;
        int64_t L = (int64_t)blockIdx.x - nqk;
        const int64_t hv = L % heads_v;
        L /= heads_v;
        const int64_t s0 = (L % sblocks) * VT_T, b = L / sblocks;
        const int64_t col = c_first + hv * 128;                          // the head's first column in this product
        const int64_t head = (col + ep.n_offset - 2 * ep.hidden) / 128;  // its index among the v heads
        const int tid = threadIdx.x, c = tid & 31;
#pragma unroll
        for (int r = 0; r < VT_T / 8; r++) {
            const int i = (tid >> 5) + 8 * r;  // token s0 + i, columns 4 c .. 4 c + 3
            const int64_t s = min(s0 + i, S - 1);
            const int64_t m = b * S + s;
            const f32x4 v = csum4(part, splits, MN, m * N + col + 4 * c);
            const u32x2 pk{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            if (ep.v_bhsd && s0 + i < S) *(u32x2 *)(ep.v_bhsd + ((b * H + head) * S + s) * 128 + 4 * c) = pk;
            tile[(4 * c) * VT_P + i] = (uint16_t)(pk[0] & 0xffffu);
            tile[(4 * c + 1) * VT_P + i] = (uint16_t)(pk[0] >> 16);
            tile[(4 * c + 2) * VT_P + i] = (uint16_t)(pk[1] & 0xffffu);
            tile[(4 * c + 3) * VT_P + i] = (uint16_t)(pk[1] >> 16);
        }
        __syncthreads();
        // row d = tid / 2, tokens 16 (tid % 2) .. + 16 of the block
        const int d = tid >> 1, t0 = (VT_T / 2) * (tid & 1);
        const int nt = (int)min((int64_t)(VT_T / 2), S - s0 - t0);
        if (nt <= 0) return;
        uint16_t *dst = ep.vt + ((b * H + head) * 128 + d) * S + s0 + t0;
        const uint16_t *src = tile + d * VT_P + t0;
        if (nt == VT_T / 2 && (S & 7) == 0) {
            // 16 B aligned: S and s0 + t0 are multiples of 8
#pragma unroll
            for (int j = 0; j < VT_T / 16; j++) {
                u32x4 w;
#pragma unroll
                for (int e = 0; e < 4; e++) w[e] = (uint32_t)src[8 * j + 2 * e] | ((uint32_t)src[8 * j + 2 * e + 1] << 16);
                *(u32x4 *)(dst + 8 * j) = w;
            }
        } else {
            for (int j = 0; j < nt; j++) dst[j] = src[j];
        }
        return;
    }
    const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (token, head group)
    const int lane = threadIdx.x & 63;
    const int64_t groups = N / (128 * HG);
    if (g >= M * groups) return;
    const int64_t m = g / groups, hs = (g % groups) * HG;
    const int64_t nb = hs * 128 + ep.n_offset;  // fused column of the group's first head
    const int sec = (int)(nb / ep.hidden);      // a group stays in one section (heads per section % HG == 0)
    if (sec >= 2) return;                       // v heads: the workgroups after nqk
    const int64_t head = (nb % ep.hidden) / 128;
    const int64_t b = m / S, s = m % S;
    const float *nw = sec == 0 ? ep.norm_q : ep.norm_k;
    const float2 w2 = *(const float2 *)(nw + 2 * lane);
    const float2 cs2 = *(const float2 *)(ep.pe + s * 128 + 2 * lane);  // (cos, sin) of pair lane
    float2 x[HG];
#pragma unroll
    for (int h = 0; h < HG; h++) {
        const int64_t c0 = m * N + (hs + h) * 128 + 2 * lane;
        x[h] = make_float2(0.f, 0.f);
        for (int sp = 0; sp < splits; sp++) {
            const float2 v = *(const float2 *)(part + sp * MN + c0);
            x[h].x += v.x;
            x[h].y += v.y;
        }
    }
    const float osc = sec == 0 ? ep.q_scale : 1.0f;
    uint16_t *dst = sec == 0 ? ep.q : ep.k;
#pragma unroll
    for (int h = 0; h < HG; h++) {
        const float ss = wave_sum(x[h].x * x[h].x + x[h].y * x[h].y);
        const float rs = 1.0f / sqrtf(ss * (1.0f / 128.0f) + 1e-6f);
        const float x0 = x[h].x * rs * w2.x, x1 = x[h].y * rs * w2.y;
        const float y0 = (x0 * cs2.x - x1 * cs2.y) * osc, y1 = (x0 * cs2.y + x1 * cs2.x) * osc;
        *(uint32_t *)(dst + ((b * H + head + h) * S + s) * 128 + 2 * lane) = pack_bf16x2(y0, y1);
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
    size_t need = (size_t)qgemm_stream_splits(w, m) * (size_t)m * (size_t)w.n * 4;
    ws::Plan p;
    if (ws::plan(w, m, EPI_F32, m16::device_cus(), p)) need = std::max(need, ws::part_bytes(w, m));
    return STREAM_COUNTER_BYTES + need;
}

hipError_t launch_qgemm_stream(const GemmWeight &w, const uint16_t *a, int64_t m, int64_t lda, int epi,
                               const EpiParams &ep, float *work, hipStream_t stream) {
    uint32_t *counters = (uint32_t *)work;
    float *part = (float *)((char *)work + STREAM_COUNTER_BYTES);
    const int cus = m16::device_cus();
    wl::Plan lp;
    if (wl::plan(w, m, epi, cus, lp)) {
        switch (w.fmt) {
        case WF_Q4_K: return wl::launch<WF_Q4_K>(w, a, (int)m, lda, epi, ep, lp, cus, stream);
        case WF_Q6_K: return wl::launch<WF_Q6_K>(w, a, (int)m, lda, epi, ep, lp, cus, stream);
        default: return wl::launch<WF_Q8_0>(w, a, (int)m, lda, epi, ep, lp, cus, stream);
        }
    }
    int tpw;
    if (wx::plan(w, m, epi, cus, tpw)) {
        switch (w.fmt) {
        case WF_Q4_K: return wx::launch<WF_Q4_K>(w, a, (int)m, lda, epi, ep, tpw, stream);
        case WF_Q6_K: return wx::launch<WF_Q6_K>(w, a, (int)m, lda, epi, ep, tpw, stream);
        default: return wx::launch<WF_Q8_0>(w, a, (int)m, lda, epi, ep, tpw, stream);
        }
    }
    wk::Plan kp;
    if (wk::plan(w, m, epi, cus, kp)) {
        switch (w.fmt) {
        case WF_Q4_K: return wk::launch<WF_Q4_K>(w, a, (int)m, lda, epi, ep, kp, stream);
        case WF_Q6_K: return wk::launch<WF_Q6_K>(w, a, (int)m, lda, epi, ep, kp, stream);
        default: return wk::launch<WF_Q8_0>(w, a, (int)m, lda, epi, ep, kp, stream);
        }
    }
    ws::Plan wp;
    if (ws::plan(w, m, epi, m16::device_cus(), wp)) {
        switch (w.fmt) {
        case WF_Q4_K: return ws::launch<WF_Q4_K>(w, a, (int)m, lda, epi, ep, part, counters, wp, stream);
        case WF_Q6_K: return ws::launch<WF_Q6_K>(w, a, (int)m, lda, epi, ep, part, counters, wp, stream);
        default: return ws::launch<WF_Q8_0>(w, a, (int)m, lda, epi, ep, part, counters, wp, stream);
        }
    }
    const int splits = qgemm_stream_splits(w, m);
    hipError_t e;
    switch (w.fmt) {
    case WF_Q8_0: e = launch_fmt<WF_Q8_0>(w, a, m, lda, part, splits, stream); break;
    case WF_Q4_K: e = launch_fmt<WF_Q4_K>(w, a, m, lda, part, splits, stream); break;
    case WF_Q6_K: e = launch_fmt<WF_Q6_K>(w, a, m, lda, part, splits, stream); break;
    case WF_BF16: e = launch_fmt<WF_BF16>(w, a, m, lda, part, splits, stream); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    return launch_split_epilogue(part, splits, m, w.n, epi, ep, stream);
}

hipError_t launch_split_epilogue(const float *part, int splits, int64_t m, int64_t N, int epi, const EpiParams &ep,
                                 hipStream_t stream) {
    if (splits < 1 || splits > MAX_SPLITS || N % 4 || m * N >= (int64_t)1 << 31) return hipErrorInvalidValue;
    const int64_t quads = (epi == EPI_SWIGLU ? m * N / 2 : m * N) / 4;
    const dim3 grid((unsigned)((quads + 255) / 256)), block(256);
    switch (epi) {
    case EPI_F32: stream_epi_kernel<EPI_F32><<<grid, block, 0, stream>>>(part, splits, m, N, ep); break;
    case EPI_BF16: stream_epi_kernel<EPI_BF16><<<grid, block, 0, stream>>>(part, splits, m, N, ep); break;
    case EPI_RESID: stream_epi_kernel<EPI_RESID><<<grid, block, 0, stream>>>(part, splits, m, N, ep); break;
    case EPI_SWIGLU: stream_epi_kernel<EPI_SWIGLU><<<grid, block, 0, stream>>>(part, splits, m, N, ep); break;
    case EPI_QKV: {
        // q / k heads one wave each, then the v heads (fused columns [2 hidden,
        // 3 hidden)) by (batch, 32 tokens, head)
        if (ep.seq <= 0 || m % ep.seq) return hipErrorInvalidValue;
        // heads per q / k wave: groups never straddle a section boundary
        const int64_t hps = ep.hidden / 128, off = ep.n_offset / 128, nh = N / 128;
        const int hg = (hps % 4 == 0 && off % 4 == 0 && nh % 4 == 0) ? 4 : (hps % 2 == 0 && off % 2 == 0 && nh % 2 == 0) ? 2 : 1;
        const int64_t nqk = (m * (nh / hg) + 3) / 4;
        const int64_t v0 = std::max<int64_t>(0, 2 * ep.hidden - ep.n_offset);
        const int64_t v1 = std::min<int64_t>(N, 3 * ep.hidden - ep.n_offset);
        const int64_t heads_v = v1 > v0 ? (v1 - v0) / 128 : 0;
        const int64_t nv = heads_v * (m / ep.seq) * ((ep.seq + VT_T - 1) / VT_T);
        const dim3 grid((unsigned)(nqk + nv));
        const int64_t hv = std::max<int64_t>(heads_v, 1);
        if (hg == 4) stream_qkv_kernel<4><<<grid, dim3(256), 0, stream>>>(part, splits, m, N, ep, nqk, v0, hv);
        else if (hg == 2) stream_qkv_kernel<2><<<grid, dim3(256), 0, stream>>>(part, splits, m, N, ep, nqk, v0, hv);
        else stream_qkv_kernel<1><<<grid, dim3(256), 0, stream>>>(part, splits, m, N, ep, nqk, v0, hv);
        break;
    }
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qimm
