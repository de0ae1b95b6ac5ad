// Joint attention for gfx950: image-token queries over [cached prefix K/V ;
// own K/V], non-causal, head_dim 128, bf16 MFMA with f32 online softmax.
//
// Replaces the unmasked cached-step call of chunked_attention /
// flash_attention (src/transformer.rs:246-296) made from Attention::forward
// (src/quantized_transformer.rs:143-148). The two key segments are read in
// place (no concatenation copy, src/quantized_transformer.rs:143-146).
//
// Common formulation: each wave computes S^T = K_blk Q^T for 32 queries with
// v_mfma_f32_32x32x16_bf16, so every lane owns one query column and the row
// max / row sum need only the lane and its partner lane^32. The probabilities
// stay in registers and are the B operand of O^T += V^T P^T.
//
// Two kernels:
//  - attn_fast_kernel (both segment lengths multiples of 8): 8 waves x 32
//    queries per workgroup; 64-key K and V^T tiles copied HBM -> LDS with
//    global_load_lds (no staging registers) into XOR-swizzled, conflict-free
//    layouts, double-buffered; the K rows of a 32-key half are read in a
//    bit-swapped order so that each lane's P^T registers hold 8 consecutive
//    keys and every V^T fragment is one 16 B LDS read; the running maximum is
//    folded into the S accumulator start (C = -m) and only moves when it grew
//    by more than 2^8, so the common path is p = exp2(s) (q pre-scaled by
//    scale*log2 e) and the rescale of O is a rare wave-uniform branch; row
//    sums use v_dot2_f32_bf16 over the packed bf16 probabilities, the same
//    values the PV product uses.
//    With MASKED it also applies the key mask of build_block_causal_mask
//    (image ids) and key validity, per 64-key window and wave: a window whose
//    keys all lie before the wave's first query, or all share the queries'
//    image block, runs unmasked; one with no visible key is skipped; the
//    others test each score. A workgroup stops at the last key any of its
//    queries may see (key_limit_kernel).
//  - attn_any_kernel (any lengths): 4 waves x 32 queries, K/V^T staged through
//    registers with per-element bounds, the reference shape for ragged tails.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

struct Seg {
    const uint16_t *k;   // [BH][len][128]
    const uint16_t *vt;  // [BH][128][len]
    int64_t len;
};

// Key mask of build_block_causal_mask (src/attention_mask.rs:18-66): query i
// sees key j when key_valid[b][j] and (i >= j or i and j lie in the same
// image block, img >= 0). img indexes the one sequence that queries and keys
// share (no prefix); key_valid indexes the concatenated [prefix ; own] keys.
struct KeyMask {
    const int32_t *img;     // [Sq] image block id, -1 for text; null: no block-causal term
    const uint8_t *kvalid;  // [B][kv_len]; null: every key valid
    int64_t kv_len;
};

// A bound on every score (log2 units): q_norm >= max ||q|| (as the kernel
// sees q, scale folded in), k_own >= max ||k|| of the own keys, *k_prefix >= max
// ||k|| of the prefix keys (null: no prefix). When q_norm * max(k_own,
// *k_prefix) <= STATIC_MAX every |score| <= STATIC_MAX (Cauchy-Schwarz), and
// the kernel takes p = exp2(score) against the fixed reference 0: no running
// maximum, no rescaling. exp2 of at most 2^STATIC_MAX summed over any key count
// stays far below f32 overflow, and floating-point sums keep their relative
// precision at any scale, so the result is the softmax's. q_norm = 0 disables.
struct ScoreBound {
    const float *k_prefix;
    float q_norm, k_own;
};
constexpr float STATIC_MAX = 64.0f;

// v_permlane32_swap exchanges the upper 32 lanes of its first operand with
// the lower 32 lanes of its second; with both operands holding x, each lane
// ends up with x and x of lane ^ 32 in the pair. Inline asm because the
// compiler folds a max or sum over the builtin's two results when both
// inputs are the same value.
__device__ __forceinline__ void swap32(float &a, float &b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float xmax32(float x) {
    float a = x, b = x;
    swap32(a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float xsum32(float x) {
    float a = x, b = x;
    swap32(a, b);
    return a + b;
}
// acc + lo + hi of a packed bf16 pair
__device__ __forceinline__ float dot2_ones(uint32_t pair, float acc) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), one, acc, false);
}

// Under the block-causal mask query q sees key k when q >= k or both lie in
// the same image block, so the last key it may see is
// lim[q] - 1 = max(q, last index of its image id). One workgroup: the last
// index of every id in LDS (ids outside [0, S) see every key), then lim.
constexpr int LIMIT_MAX_S = 16384;

__global__ __launch_bounds__(1024) void key_limit_kernel(const int32_t *__restrict__ img, int S,
                                                         int32_t *__restrict__ lim) {
    __shared__ int32_t last[LIMIT_MAX_S];
    for (int i = threadIdx.x; i < S; i += 1024) last[i] = -1;
    __syncthreads();
    for (int k = threadIdx.x; k < S; k += 1024) {
        const int id = img[k];
        if (id >= 0 && id < S) atomicMax(&last[id], k);
    }
    __syncthreads();
    for (int q = threadIdx.x; q < S; q += 1024) {
        const int id = img[q];
        lim[q] = (id >= S ? S - 1 : id >= 0 ? max(q, last[id]) : q) + 1;
    }
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    return v;
}

// f32 output of a wave's 32 queries x 128 d (O^T accumulators: lane l32 owns
// query q0 + l32, o[dt][4 rq + e] is d = 32 dt + 8 rq + 4 g + e), in two
// 64-wide passes through the wave's f32 staging rows (pitch PITCH floats) so
// that every store covers 256 B of a row. All waves of the workgroup call it.
template <int PITCH>
__device__ __forceinline__ void store_out_f32(float *osf, const f32x16 (&o)[4], float inv, int lane,
                                              float *__restrict__ outf, int64_t bb, int64_t Sq, int64_t row_len,
                                              int64_t col0, int64_t q0) {
    const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        __syncthreads();
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
#pragma unroll
            for (int rq = 0; rq < 4; rq++) {
                const int t = 2 * hf + dt, d = dt * 32 + 8 * rq + 4 * g;
                *(f32x4 *)(osf + l32 * PITCH + d) = f32x4{o[t][4 * rq] * inv, o[t][4 * rq + 1] * inv,
                                                          o[t][4 * rq + 2] * inv, o[t][4 * rq + 3] * inv};
            }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int r = i * 4 + (lane >> 4), c = (lane & 15) * 4;
            const int64_t qi = q0 + r;
            if (qi < Sq) *(f32x4 *)(outf + (bb * Sq + qi) * row_len + col0 + 64 * hf + c) = *(const f32x4 *)(osf + r * PITCH + c);
        }
    }
}

// bf16 output of a wave's 32 queries x 128 d (the same accumulator layout)
// into its staging rows (pitch PITCH bf16). With q8 every 32-d slice dt of a
// query, 16 values in this lane and 16 in its partner half (lane ^ 32), is
// first rounded as candle's Q8_0 activation block (quant_act4<32>'s
// arithmetic): the to_out projection's input when its weight is Q8_0.
template <int PITCH>
__device__ __forceinline__ void stage_out_bf16(uint16_t *os, const f32x16 (&o)[4], float inv, int lane, bool q8) {
    const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = o[dt][r] * inv;
        if (q8) {
            float a = 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) a = fmaxf(a, fabsf(v[r]));
            float sc, dq;
            q8_0_scales(xmax32(a), sc, dq);
#pragma unroll
            for (int rq = 0; rq < 4; rq++)
                *(u32x2 *)(os + l32 * PITCH + dt * 32 + 8 * rq + 4 * g) =
                    q8_0_values4(f32x4{v[4 * rq], v[4 * rq + 1], v[4 * rq + 2], v[4 * rq + 3]}, sc, dq);
        } else {
#pragma unroll
            for (int rq = 0; rq < 4; rq++)
                *(u32x2 *)(os + l32 * PITCH + dt * 32 + 8 * rq + 4 * g) =
                    u32x2{pack_bf16x2(v[4 * rq], v[4 * rq + 1]), pack_bf16x2(v[4 * rq + 2], v[4 * rq + 3])};
        }
    }
}

// Candle's Q8_K rounding of the output across a head pair (256 values of a
// query = two heads): this head's part of a query's largest magnitude and the
// first column holding it, as (column << 1 | sign), column col0 + d (col0 =
// 128 for the pair's second head); lane and partner half (lane ^ 32) agree.
__device__ __forceinline__ void q8k_query_max(const f32x16 (&o)[4], float inv, int g, int col0, float &amax,
                                              int &first) {
    float a = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) a = fmaxf(a, fabsf(o[dt][r] * inv));
    a = xmax32(a);
    int f = 0x7fffffff;
#pragma unroll
    for (int dt = 3; dt >= 0; dt--)
#pragma unroll
        for (int r = 15; r >= 0; r--) {
            const float v = o[dt][r] * inv;
            const int code = ((col0 + 32 * dt + 8 * (r >> 2) + 4 * (g) + (r & 3)) << 1) | (v < 0.f ? 1 : 0);
            f = fabsf(v) == a ? code : f;
        }
    float lo = __int_as_float(f), hi = lo;
    swap32(lo, hi);
    amax = a;
    first = min(__float_as_int(lo), __float_as_int(hi));
}

// The f32 output of a wave's 32 queries x 128 d that store_out_f32 wrote, read
// back into the accumulator layout (v[dt][r] = d 32 dt + 8 (r / 4) + 4 g + r % 4)
// through the same staging rows: whole 256 B row pieces from memory, then each
// lane its own values. Rows past Sq are not read (their values are not used).
template <int PITCH>
__device__ __forceinline__ void load_back_f32(float *osf, float (&v)[4][16], int lane, const float *__restrict__ outf,
                                              int64_t bb, int64_t Sq, int64_t row_len, int64_t col0, int64_t q0) {
    const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int r = i * 4 + (lane >> 4), c = (lane & 15) * 4;
            const int64_t qi = q0 + r;
            if (qi < Sq) *(f32x4 *)(osf + r * PITCH + c) = *(const f32x4 *)(outf + (bb * Sq + qi) * row_len + col0 + 64 * hf + c);
        }
        __syncthreads();
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
#pragma unroll
            for (int rq = 0; rq < 4; rq++) {
                const f32x4 x = *(const f32x4 *)(osf + l32 * PITCH + dt * 32 + 8 * rq + 4 * g);
#pragma unroll
                for (int e = 0; e < 4; e++) v[2 * hf + dt][4 * rq + e] = x[e];
            }
    }
}

namespace fast {

// A workgroup of NW waves (8, or 4 where 8-wave workgroups leave CUs idle)
// takes 32 NW queries of one head; each wave owns 32 of them.
constexpr int KB = 64;           // keys per block
constexpr int HD = 128;
constexpr int TILE = KB * HD * 2;     // 16 KB: K (64 rows x 256 B) or V^T (128 rows x 128 B)
constexpr int STAGE = 2 * TILE;       // K tile then V^T tile
constexpr int OP = 136;               // bf16 pitch of the output staging rows
constexpr int OPF = 68;               // f32 pitch of the f32 output staging rows (64 d per pass)
constexpr int lds_bytes(int nw) { return 2 * STAGE > nw * 32 * OP * 2 ? 2 * STAGE : nw * 32 * OP * 2; }
constexpr float RESCALE_TH = 8.0f;    // log2 units

// K tile: key row r holds 16 B chunk c at slot c ^ (r % 16); V^T tile: d row
// holds 8-key chunk c at slot c ^ ((d / 2) % 8). A 16-lane phase of b128 reads
// (16 rows, one chunk) then covers all 64 banks once.
// Two waves per SIMD either way: one 8-wave or two 4-wave workgroups per CU.
// SMODE: 0 = the softmax reference is chosen in the kernel from the score
// bound (the prefix keys' norm is a device value); 1 = fixed reference, 2 =
// running maximum, both decided on the host. A kernel with one form has only
// that loop's registers to allocate.
template <int NW, bool PRE, bool MASKED, int SMODE, bool PAIR>
__global__ __launch_bounds__(64 * NW, 8 / NW) void attn_fast_kernel(const uint16_t *__restrict__ q, Seg s0, Seg s1,
                                                                    int64_t H, int64_t Sq, int64_t nq, int64_t B,
                                                                    float sl2, uint16_t *__restrict__ out,
                                                                    float *__restrict__ outf, KeyMask km,
                                                                    const int32_t *__restrict__ lim,
                                                                    ScoreBound sb, int q8) {
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(!PAIR || !MASKED, "the paired form is the cached step's");
    constexpr int QB = 32 * NW;  // queries per workgroup
    constexpr int DI = 16 / NW;  // DMA instructions per wave per 16 KB tile
    // operand stages / output staging; in the paired form then each query's
    // first-head maximum and its first dimension (2 words per query)
    __shared__ __attribute__((aligned(16))) uint8_t lds[lds_bytes(NW) + (PAIR ? QB * 8 : 0)];
    __shared__ int wlim[NW];
    // the wave index as a scalar (the DMA destinations then go to M0 without a lane read)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // XCD-aware order: workgroups are dealt round-robin over 8 XCDs; each XCD
    // gets a contiguous range of (batch, head, query tile) so the query tiles
    // of one head share that XCD's L2 copy of its K/V.
    // Under a key limit later query tiles see more keys: they are dispatched
    // first (query tile major in block order, from the last), so that the short
    // tiles fill the tail; workgroup b takes (batch, head) b % (B H), which
    // keeps a head on one XCD when B H is a multiple of 8.
    // The paired form takes heads 2 hp and 2 hp + 1 in turn (H / 2 head pairs).
    const int64_t HP = PAIR ? H / 2 : H;
    const int64_t total = nq * HP * B;
    int64_t L = blockIdx.x;
    int64_t qt, bhp;
    if (MASKED && lim) {
        qt = nq - 1 - L / (HP * B);
        bhp = L % (HP * B);
    } else {
        if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
        qt = L % nq;
        bhp = L / nq;
    }
    const int64_t bb = bhp / HP;
    const int64_t q0 = qt * QB + wave * 32;

    // one head (t: its index in the pair)
    auto head = [&](auto t_) __attribute__((always_inline)) {
        constexpr int t = decltype(t_)::value;
        const int64_t hh = PAIR ? 2 * (bhp % HP) + t : bhp % HP, bh = bb * H + hh;
        // in the paired form every lane-dependent value of a head derives from this
        // copy of the thread index, which the compiler cannot see through (nothing
        // of the second head is computed early and kept live across the first
        // head's loop); the mask keeps the lane's range known
        int lane = tid;
        if constexpr (PAIR) asm volatile("" : "+v"(lane));
        lane &= 63;
        const int g = lane >> 5, l32 = lane & 31;

        // Q^T fragments (B operand): lane holds query q0+l32, d = 16kk + 8g .. +8
        bf16x8 qf[8];
        {
            const int64_t qi = q0 + l32;
            const uint16_t *qr = q + (bh * Sq + (qi < Sq ? qi : 0)) * HD;
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                u32x4 v = *(const u32x4 *)(qr + kk * 16 + g * 8);
                if (qi >= Sq) v = u32x4{0u, 0u, 0u, 0u};
                qf[kk] = __builtin_bit_cast(bf16x8, v);
            }
        }

        const int len0 = (int)s0.len, len1 = (int)s1.len;
        const int nb0 = (len0 + KB - 1) / KB, nb1 = (len1 + KB - 1) / KB;
        int nblk = nb0 + nb1;

        // Mask state of the wave: its queries [q_lo, q_hi], the lane's query qi
        // and image id, the id range of the wave's queries; with a key limit the
        // workgroup's loop ends at the last key any of its queries may see (the
        // block-causal form has no prefix, so keys are the queries' sequence).
        int q_lo = 0, q_hi = 0, qid_min = -1, qid_max = -1;
        if constexpr (MASKED) {
            const int qi = (int)min(q0 + l32, Sq - 1);
            q_lo = (int)min(q0, Sq - 1);
            q_hi = (int)min(q0 + 31, Sq - 1);
            if (km.img) {
                const int idq = km.img[qi];
                qid_min = __builtin_amdgcn_readfirstlane(wave_min_i(idq));
                qid_max = __builtin_amdgcn_readfirstlane(wave_max_i(idq));
            }
            if (lim) {
                const int wl = __builtin_amdgcn_readfirstlane(wave_max_i(lim[qi]));
                if (lane == 0) wlim[wave] = wl;
                __syncthreads();
                int kmax = wlim[0];
#pragma unroll
                for (int i = 1; i < NW; i++) kmax = max(kmax, wlim[i]);
                nblk = min(nblk, (kmax + KB - 1) / KB);
            }
        }
        const char *kb0 = (const char *)(s0.k + bh * (int64_t)len0 * HD);
        const char *kb1 = (const char *)(s1.k + bh * (int64_t)len1 * HD);
        const char *vb0 = (const char *)(s0.vt + bh * (int64_t)HD * len0);
        const char *vb1 = (const char *)(s1.vt + bh * (int64_t)HD * len1);

        // DMA roles: instruction t = wave + NW i fills K rows 4t .. 4t+3 (lane at
        // row 4t + lane/16, slot lane%16) and V^T rows 8t .. 8t+7 (lane at row
        // 8t + lane/8, slot lane%8); lane l lands at LDS base + 16 l.
        uint32_t koff[DI], vrow[DI], vcol[DI];
#pragma unroll
        for (int i = 0; i < DI; i++) {
            const int r = 4 * (wave + NW * i) + (lane >> 4);
            koff[i] = (uint32_t)(r * 256 + (((lane & 15) ^ (r & 15)) << 4));
            const int d = 8 * (wave + NW * i) + (lane >> 3);
            vrow[i] = (uint32_t)d;
            vcol[i] = (uint32_t)(((lane & 7) ^ ((d >> 1) & 7)) << 4);
        }
        // Block j covers keys [start, start + 64) of its segment. The last block of
        // a segment of at least 64 keys slides back to end at len (window [kv0,
        // kv0 + 64), keys before `lo` already seen); a shorter segment clamps its
        // rows and masks keys from `hi` on. Every load stays inside the segment.
        struct Blk {
            const char *kb, *vb;
            int len, kv0, lo, hi, kbase;  // kbase: index of the segment's first key in [s0 ; s1]
        };
        auto blk_of = [&](int j) __attribute__((always_inline)) {
            Blk b;
            const bool first = j < nb0;
            b.kbase = first ? 0 : len0;
            b.len = first ? len0 : len1;
            b.kb = first ? kb0 : kb1;
            b.vb = first ? vb0 : vb1;
            const int start = (first ? j : j - nb0) * KB;
            if (b.len >= KB) {
                b.kv0 = min(start, b.len - KB);
                b.lo = start - b.kv0;
                b.hi = KB;
            } else {
                b.kv0 = 0;
                b.lo = 0;
                b.hi = b.len;
            }
            return b;
        };
        auto dma = [&](const Blk &b, int stage) __attribute__((always_inline)) {
            uint8_t *base = lds + stage * STAGE;
            if (b.len >= KB) {
                const char *kg = b.kb + (int64_t)b.kv0 * 256;
                const char *vg = b.vb + (int64_t)b.kv0 * 2;
#pragma unroll
                for (int i = 0; i < DI; i++)
                    __builtin_amdgcn_global_load_lds((const void *)(kg + koff[i]),
                                                     (lds_ptr_t)(base + (wave + NW * i) * 1024), 16, 0, 0);
#pragma unroll
                for (int i = 0; i < DI; i++)
                    __builtin_amdgcn_global_load_lds((const void *)(vg + (vrow[i] * (uint32_t)(2 * b.len) + vcol[i])),
                                                     (lds_ptr_t)(base + TILE + (wave + NW * i) * 1024), 16, 0, 0);
            } else {
#pragma unroll
                for (int i = 0; i < DI; i++) {
                    const int r = 4 * (wave + NW * i) + (lane >> 4);
                    const int gr = min(r, b.len - 1);
                    __builtin_amdgcn_global_load_lds((const void *)(b.kb + (koff[i] - r * 256) + gr * 256),
                                                     (lds_ptr_t)(base + (wave + NW * i) * 1024), 16, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < DI; i++) {
                    const int gc = min((int)vcol[i] >> 1, b.len - 8);
                    __builtin_amdgcn_global_load_lds((const void *)(b.vb + vrow[i] * (uint32_t)(2 * b.len) + 2 * gc),
                                                     (lds_ptr_t)(base + TILE + (wave + NW * i) * 1024), 16, 0, 0);
                }
            }
        };

        // S^T row m of a 32-key half is key pi(m) = m with bits 2 and 3 swapped,
        // so accumulator register r of lane (l32, g) is key 16 (r / 8) + 8 g + r % 8
        // and P^T register pairs map to consecutive keys. LDS read offsets are per
        // lane; stage, half and d-tile parts are immediates.
        const int krow = (l32 & ~12) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
        uint32_t kaddr[8], vaddr[2][2];
#pragma unroll
        for (int kk = 0; kk < 8; kk++) kaddr[kk] = (uint32_t)(krow * 256 + (((2 * kk + g) ^ (krow & 15)) << 4));
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int kk = 0; kk < 2; kk++)
                vaddr[h][kk] = (uint32_t)(TILE + l32 * 128 + (((4 * h + 2 * kk + g) ^ ((l32 >> 1) & 7)) << 4));

        f32x16 o[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[dt][r] = 0.f;
        // scores are kept relative to m_run (score units): the S accumulation
        // starts at -m_run
        float m_run = 0.f, l_run = 0.f;
        f32x16 negm;
#pragma unroll
        for (int r = 0; r < 16; r++) negm[r] = 0.f;
        bool first_half = true;
        bool fresh = true;  // MASKED: this lane's query has seen no visible key yet

        // kmask: visible keys of the window (bit kv), kid: lane kv holds the image
        // id of window key kv, kb0: index of the window's first key, partial: test
        // each score (MASKED only)
        auto half_step = [&](const uint8_t *stg, int h, int lo, int hi, uint64_t kmask, int kid, int kb0,
                             bool partial, auto stat) __attribute__((always_inline)) {
            constexpr bool STATIC = decltype(stat)::value;
            f32x16 st;
            if constexpr (STATIC) {
#pragma unroll
                for (int r = 0; r < 16; r++) st[r] = 0.f;
            } else {
                st = negm;
            }
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const bf16x8 a = *(const bf16x8 *)(stg + h * 32 * 256 + kaddr[kk]);
                st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], st, 0, 0, 0);
            }
            if (lo > h * 32 || hi < h * 32 + 32) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int kv = h * 32 + 16 * (r >> 3) + 8 * g + (r & 7);
                    if (kv < lo || kv >= hi) st[r] = -INFINITY;
                }
            }
            if constexpr (MASKED) {
                if (partial) {
                    // branch-free per-score test (bitwise, no short circuit): the
                    // key's validity bit and, with image ids, causal or same block.
                    // The lane's query and its image id are fetched here: only
                    // windows tested score by score need them.
                    const uint32_t kmw = h ? (uint32_t)(kmask >> 32) : (uint32_t)kmask;
                    if (km.img) {
                        const int qi = (int)min(q0 + l32, Sq - 1);
                        const int idq = km.img[qi];
                        const int qrel = qi - kb0 - h * 32;  // keys of this half at or before the query
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int kvh = 16 * (r >> 3) + 8 * g + (r & 7);
                            const int idk = __shfl(kid, h * 32 + kvh);
                            const int ok = (int)((kmw >> kvh) & 1u) & ((int)(qrel >= kvh) | ((int)(idq >= 0) & (int)(idk == idq)));
                            st[r] = ok ? st[r] : -INFINITY;
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int kvh = 16 * (r >> 3) + 8 * g + (r & 7);
                            st[r] = ((kmw >> kvh) & 1u) ? st[r] : -INFINITY;
                        }
                    }
                }
            }
            if constexpr (!STATIC) {
            float m0 = st[0], m1 = st[1];
#pragma unroll
            for (int r = 2; r < 16; r += 2) {
                m0 = fmaxf(m0, st[r]);
                m1 = fmaxf(m1, st[r + 1]);
            }
            float mx = xmax32(fmaxf(m0, m1));
            if (!PRE) mx *= sl2;  // log2 units
            bool rescale;
            if constexpr (MASKED) {
                // a lane's first visible key sets its reference point; a row with
                // none yet keeps 0 (its probabilities are exp2(-inf) = 0)
                const bool has = mx > -INFINITY;
                rescale = __builtin_amdgcn_ballot_w64(fresh ? has : mx > RESCALE_TH) != 0;
            } else {
                rescale = first_half || __builtin_amdgcn_ballot_w64(mx > RESCALE_TH);
            }
            if (rescale) {
                // move the reference point up by d (log2 units); the first half of
                // a row has at least one unmasked key, so d is finite there
                float d, alpha;
                if constexpr (MASKED) {
                    const bool has = mx > -INFINITY;
                    d = fresh ? (has ? mx : 0.f) : fmaxf(mx, 0.f);
                    alpha = fresh ? 0.f : __builtin_amdgcn_exp2f(-d);
                    fresh = fresh && !has;
                } else {
                    d = first_half ? mx : fmaxf(mx, 0.f);
                    alpha = first_half ? 0.f : __builtin_amdgcn_exp2f(-d);
                }
                first_half = false;
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < 4; dt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[dt][r] *= alpha;
                const float draw = PRE ? d : d / sl2;
                m_run += draw;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    st[r] -= draw;
                    negm[r] = -m_run;
                }
            }
            }  // !STATIC
            uint32_t pk[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float a = PRE ? st[2 * i] : st[2 * i] * sl2;
                const float b = PRE ? st[2 * i + 1] : st[2 * i + 1] * sl2;
                pk[i] = pack_bf16x2(__builtin_amdgcn_exp2f(a), __builtin_amdgcn_exp2f(b));
                l_run = dot2_ones(pk[i], l_run);
            }
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pk[4 * kk], pk[4 * kk + 1], pk[4 * kk + 2], pk[4 * kk + 3]});
#pragma unroll
                for (int dt = 0; dt < 4; dt++) {
                    const bf16x8 a = *(const bf16x8 *)(stg + dt * 32 * 128 + vaddr[h][kk]);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf, o[dt], 0, 0, 0);
                }
            }
        };

        // The fixed-reference form without a mask, split so that both halves'
        // scores come first: the exponentials of half 0 then issue while half 1's
        // QK MFMAs are still in the matrix pipe, and those of half 1 while half 0's
        // PV MFMAs run.
        auto qk_static = [&](const uint8_t *stg, int h) __attribute__((always_inline)) {
            f32x16 st;
#pragma unroll
            for (int r = 0; r < 16; r++) st[r] = 0.f;
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const bf16x8 a = *(const bf16x8 *)(stg + h * 32 * 256 + kaddr[kk]);
                st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], st, 0, 0, 0);
            }
            return st;
        };
        auto pv_static = [&](const uint8_t *stg, int h, f32x16 st, int lo, int hi) __attribute__((always_inline)) {
            if (lo > h * 32 || hi < h * 32 + 32) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int kv = h * 32 + 16 * (r >> 3) + 8 * g + (r & 7);
                    if (kv < lo || kv >= hi) st[r] = -INFINITY;
                }
            }
            uint32_t pk[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float a = PRE ? st[2 * i] : st[2 * i] * sl2;
                const float b = PRE ? st[2 * i + 1] : st[2 * i + 1] * sl2;
                pk[i] = pack_bf16x2(__builtin_amdgcn_exp2f(a), __builtin_amdgcn_exp2f(b));
                l_run = dot2_ones(pk[i], l_run);
            }
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pk[4 * kk], pk[4 * kk + 1], pk[4 * kk + 2], pk[4 * kk + 3]});
#pragma unroll
                for (int dt = 0; dt < 4; dt++) {
                    const bf16x8 a = *(const bf16x8 *)(stg + dt * 32 * 128 + vaddr[h][kk]);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf, o[dt], 0, 0, 0);
                }
            }
        };

        // MASKED: lane kv loads the image id of window key kv (0 without ids), or
        // KEY_OFF for a padded key, one block ahead; waited for with the tiles.
        constexpr int KEY_OFF = -0x7fffffff - 1;
        int mk = 0;
        auto mask_load = [&](const Blk &b) __attribute__((always_inline)) {
            const int kv = min(lane, b.len - 1 - b.kv0);
            const int64_t key = (int64_t)b.kbase + b.kv0 + kv;
            const bool valid = km.kvalid ? km.kvalid[bb * km.kv_len + key] != 0 : true;
            const int id = km.img ? km.img[key] : 0;
            mk = valid ? id : KEY_OFF;
        };

        // block j computes from stage cur while block j+1 streams into the other
        auto step = [&](int j, int cur, auto stat) __attribute__((always_inline)) {
            const Blk b = blk_of(j);
            int kid = 0, kb0 = 0;
            uint64_t kmask = 0;
            bool skip = false, partial = false;
            if constexpr (MASKED) {
                // classify the window for this wave's queries (wave-uniform)
                kid = mk;
                kb0 = b.kbase + b.kv0;
                const bool in = lane >= b.lo && lane < b.hi;
                const uint64_t inm = __builtin_amdgcn_ballot_w64(in);
                kmask = __builtin_amdgcn_ballot_w64(in && mk != KEY_OFF);
                const int k_lo = kb0 + b.lo, k_hi = kb0 + b.hi - 1;
                bool full = kmask == inm, empty = kmask == 0;
                if (km.img) {
                    const uint64_t same = __builtin_amdgcn_ballot_w64(in && mk == qid_min);
                    const bool one_block = qid_min == qid_max && qid_min >= 0;
                    full = full && (k_hi <= q_lo || (one_block && same == inm));
                    empty = empty || (k_lo > q_hi && (qid_max < 0 || (qid_min == qid_max && same == 0)));
                }
                skip = empty;
                partial = !full && !empty;
                if (j + 1 < nblk) mask_load(blk_of(j + 1));
            }
            if (j + 1 < nblk) dma(blk_of(j + 1), cur ^ 1);
            const uint8_t *stg = lds + cur * STAGE;
            if constexpr (decltype(stat)::value && !MASKED) {
                const f32x16 s0 = qk_static(stg, 0), s1 = qk_static(stg, 1);
                pv_static(stg, 0, s0, b.lo, b.hi);
                pv_static(stg, 1, s1, b.lo, b.hi);
            } else if (!skip) {
                half_step(stg, 0, b.lo, b.hi, kmask, kid, kb0, partial, stat);
                half_step(stg, 1, b.lo, b.hi, kmask, kid, kb0, partial, stat);
            }
            __builtin_amdgcn_s_waitcnt(WAIT_VM0);  // vmcnt(0): block j+1 landed
            __syncthreads();
        };

        if (nblk > 0) {
            if constexpr (MASKED) mask_load(blk_of(0));
            dma(blk_of(0), 0);
        }
        __builtin_amdgcn_s_waitcnt(WAIT_VM0);
        __syncthreads();
        // the fixed-reference form when the score bound allows it (wave-uniform)
        bool stat_ok = false;
        if (sb.q_norm > 0.f) {
            const float kn = sb.k_prefix ? fmaxf(sb.k_own, *sb.k_prefix) : sb.k_own;
            stat_ok = sb.q_norm * kn <= STATIC_MAX;
        }
        auto run = [&](auto stat) __attribute__((always_inline)) {
            int j = 0;
            for (; j + 1 < nblk; j += 2) {
                step(j, 0, stat);
                step(j + 1, 1, stat);
            }
            if (j < nblk) step(j, 0, stat);
        };
        if constexpr (SMODE == 1) {
            run(std::true_type{});
        } else if constexpr (SMODE == 2) {
            run(std::false_type{});
        } else {
            if (stat_ok)
                run(std::true_type{});
            else
                run(std::false_type{});
        }

        // normalize and stage O [32 q x 128 d] per wave through LDS for row stores
        const float l_tot = xsum32(l_run);
        const float inv = 1.0f / l_tot;
        const int64_t HDt = H * HD;
        uint16_t *os = (uint16_t *)lds + wave * 32 * OP;
        // the wave's staged bf16 rows to out at columns col0 ..
        auto store_rows = [&](int64_t col0) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int r = i * 4 + (lane >> 4);
                const int c = (lane & 15) * 8;
                const int64_t qi = q0 + r;
                if (qi < Sq)
                    *(u32x4 *)(out + (bb * Sq + qi) * HDt + col0 + c) = *(const u32x4 *)(os + r * OP + c);
            }
        };
        if constexpr (PAIR) {
            // Q8_K rounding over the head pair: the first head leaves its f32
            // output in outf (scratch) and each query's largest magnitude and
            // first column in LDS; the second combines them (the first head's
            // columns come first: it wins ties), reads the first head's values
            // back and stores both heads rounded (quant_act4<256>'s arithmetic)
            float a;
            int f;
            q8k_query_max(o, inv, g, 128 * t, a, f);
            float *pmax = (float *)(lds + lds_bytes(NW));
            int *pfirst = (int *)(pmax + QB);
            const int qslot = wave * 32 + l32;
            if constexpr (t == 0) {
                if (g == 0) {
                    pmax[qslot] = a;
                    pfirst[qslot] = f;
                }
                store_out_f32<OPF>((float *)lds + wave * 32 * OPF, o, inv, lane, outf, bb, Sq, HDt, hh * HD, q0);
                __syncthreads();  // staging reads done before the second head's stages land
            } else {
                if (!(a > pmax[qslot])) {
                    a = pmax[qslot];
                    f = pfirst[qslot];
                }
                float sc, dq;
                q8k_scales(a, (f & 1) ? -a : a, sc, dq);
                float va[4][16];
                load_back_f32<OPF>((float *)lds + wave * 32 * OPF, va, lane, outf, bb, Sq, HDt, (hh - 1) * HD, q0);
#pragma unroll
                for (int hd = 0; hd < 2; hd++) {
                    __syncthreads();
#pragma unroll
                    for (int dt = 0; dt < 4; dt++)
#pragma unroll
                        for (int rq = 0; rq < 4; rq++) {
                            f32x4 x;
#pragma unroll
                            for (int e = 0; e < 4; e++) x[e] = hd == 0 ? va[dt][4 * rq + e] : o[dt][4 * rq + e] * inv;
                            *(u32x2 *)(os + l32 * OP + dt * 32 + 8 * rq + 4 * g) = q8k_values4(x, sc, dq);
                        }
                    __syncthreads();
                    store_rows((hh - 1 + hd) * HD);
                }
            }
            return;
        }
        if (outf) {
            store_out_f32<OPF>((float *)lds + wave * 32 * OPF, o, inv, lane, outf, bb, Sq, HDt, hh * HD, q0);
            return;
        }
        stage_out_bf16<OP>(os, o, inv, lane, q8 != 0);
        __syncthreads();
        store_rows(hh * HD);
    };
    head(std::integral_constant<int, 0>{});
    if constexpr (PAIR) head(std::integral_constant<int, 1>{});
}

}  // namespace fast

namespace anylen {

constexpr int QB = 128;     // queries per workgroup
constexpr int KB = 64;      // keys per block
constexpr int HD = 128;     // head dim
constexpr int KP = 136;     // bf16 pitch of K tile rows (128 + 8)
constexpr int VP = 68;      // bf16 pitch of V^T tile rows (64 + 4): conflict-free 8 B reads
constexpr int KSTAGE = KB * KP;
constexpr int VSTAGE = HD * VP;
constexpr int STAGE = KSTAGE + VSTAGE;
constexpr int OP = 136;     // bf16 pitch of the output staging rows

// K and V^T tiles of 64 keys double-buffered in LDS through registers; the
// 16-key K-slots of the PV MFMA use the key order of the S^T accumulator
// layout, and V^T is read from LDS in the same order.
template <bool MASKED>
__global__ __launch_bounds__(256, 2) void attn_any_kernel(const uint16_t *__restrict__ q, Seg s0, Seg s1,
                                                      int64_t H, int64_t Sq, int64_t nq, int64_t B,
                                                      float sl2, uint16_t *__restrict__ out,
                                                      float *__restrict__ outf, KeyMask km, int q8) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;

    // XCD-aware order: the hardware deals workgroups round-robin over 8 XCDs;
    // give each XCD a contiguous range of (batch, head, query-tile) so the
    // query tiles of one head share that XCD's L2 copy of its K/V.
    const int64_t total = nq * H * B;
    int64_t L = blockIdx.x;
    if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
    const int64_t qt = L % nq, hh = (L / nq) % H, bb = L / (nq * H);
    const int64_t bh = bb * H + hh;
    const int64_t q0 = qt * QB + wave * 32;

    // Q^T fragments (B operand): lane holds query q0+l32, d = 16kk + 8g .. +8.
    bf16x8 qf[8];
    {
        const int64_t qi = q0 + l32;
        const uint16_t *qr = q + (bh * Sq + (qi < Sq ? qi : 0)) * HD;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            u32x4 v = *(const u32x4 *)(qr + kk * 16 + g * 8);
            if (qi >= Sq) v = u32x4{0u, 0u, 0u, 0u};
            qf[kk] = __builtin_bit_cast(bf16x8, v);
        }
    }

    const int64_t nb0 = (s0.len + KB - 1) / KB, nb1 = (s1.len + KB - 1) / KB;
    const int64_t nblk = nb0 + nb1;

    // loader roles
    const int k_row = tid >> 4, k_col = (tid & 15) * 8;  // 4 x (16 rows apart)
    const int v_row = tid >> 3, v_col = (tid & 7) * 8;   // 4 x (32 rows apart)
    u32x4 rk[4], rv[4];

    auto load_blk = [&](int64_t j) {
        const Seg &sg = j < nb0 ? s0 : s1;
        const int64_t kv0 = (j < nb0 ? j : j - nb0) * KB;
        const int64_t len = sg.len;
        const uint16_t *kb = sg.k + bh * len * HD;
        const uint16_t *vb = sg.vt + bh * HD * len;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t r = kv0 + k_row + 16 * i;
            rk[i] = r < len ? *(const u32x4 *)(kb + r * HD + k_col) : u32x4{0u, 0u, 0u, 0u};
        }
        const bool vec = (len & 7) == 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint16_t *vr = vb + (int64_t)(v_row + 32 * i) * len;
            const int64_t c = kv0 + v_col;
            if (vec) {
                rv[i] = c < len ? *(const u32x4 *)(vr + c) : u32x4{0u, 0u, 0u, 0u};
            } else {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint32_t lo = c + 2 * e < len ? vr[c + 2 * e] : 0u;
                    uint32_t hi = c + 2 * e + 1 < len ? vr[c + 2 * e + 1] : 0u;
                    w[e] = lo | (hi << 16);
                }
                rv[i] = u32x4{w[0], w[1], w[2], w[3]};
            }
        }
    };
    auto store_blk = [&](uint16_t *st) {
#pragma unroll
        for (int i = 0; i < 4; i++) *(u32x4 *)(st + (k_row + 16 * i) * KP + k_col) = rk[i];
        uint16_t *vs = st + KSTAGE;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint16_t *p = vs + (v_row + 32 * i) * VP + v_col;
            *(u32x2 *)p = u32x2{rv[i][0], rv[i][1]};
            *(u32x2 *)(p + 4) = u32x2{rv[i][2], rv[i][3]};
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    if (nblk > 0) {
        load_blk(0);
        store_blk(lds);
    }
    __syncthreads();

    for (int64_t j = 0; j < nblk; j++) {
        const int cur = (int)(j & 1);
        const bool more = j + 1 < nblk;
        if (more) load_blk(j + 1);
        const uint16_t *ks = lds + cur * STAGE;
        const uint16_t *vs = ks + KSTAGE;

        const Seg &sg = j < nb0 ? s0 : s1;
        const int64_t valid = sg.len - (j < nb0 ? j : j - nb0) * KB;  // keys of this block in range
        // The 64-key block is processed as two 32-key halves so only one
        // 32x32 S^T tile is live at a time.
#pragma unroll
        for (int half = 0; half < 2; half++) {
            // S^T (32 keys x 32 queries) = K_half Q^T
            f32x16 st;
#pragma unroll
            for (int r = 0; r < 16; r++) st[r] = 0.f;
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                bf16x8 a = *(const bf16x8 *)(ks + (half * 32 + l32) * KP + kk * 16 + g * 8);
                st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], st, 0, 0, 0);
            }
            // the prefetched tile goes to the other stage once its loads land,
            // ending the live range of the staging registers early
            if (half == 0 && more) store_blk(lds + (cur ^ 1) * STAGE);
            if (valid < (half + 1) * 32) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int kv = half * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (kv >= valid) st[r] = -INFINITY;
                }
            }
            if constexpr (MASKED) {
                // key index in the concatenated [prefix ; own] sequence
                const int64_t kb = (j < nb0 ? j * KB : s0.len + (j - nb0) * KB) + half * 32;
                const int64_t qi = min(q0 + l32, Sq - 1);
                const int32_t qimg = km.img ? km.img[qi] : -1;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int64_t kidx = kb + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (kidx >= km.kv_len) continue;  // beyond the keys: masked above
                    bool ok = km.kvalid ? km.kvalid[bb * km.kv_len + kidx] != 0 : true;
                    if (km.img) ok = ok && (qi >= kidx || (qimg >= 0 && km.img[kidx] == qimg));
                    if (!ok) st[r] = -INFINITY;
                }
            }
            // online softmax in the log2 domain
            float mx = st[0];
#pragma unroll
            for (int r = 1; r < 16; r++) mx = fmaxf(mx, st[r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m_run, mx * sl2);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
            float psum = 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[r], sl2, -m_use));
                st[r] = p;
                psum += p;
            }
            l_run = l_run * alpha + psum;
            m_run = m_new;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[dt][r] *= alpha;
            // P^T fragments: keys 32half + 16kk + {4g..4g+3, 8+4g..8+4g+3} are
            // accumulator registers st[8kk .. 8kk+8) of this lane.
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                u32x4 w{pack_bf16x2(st[8 * kk + 0], st[8 * kk + 1]), pack_bf16x2(st[8 * kk + 2], st[8 * kk + 3]),
                        pack_bf16x2(st[8 * kk + 4], st[8 * kk + 5]), pack_bf16x2(st[8 * kk + 6], st[8 * kk + 7])};
                const bf16x8 pf = __builtin_bit_cast(bf16x8, w);
                // O^T (128 d x 32 q) += V^T[:, keys] P^T[keys, :]
#pragma unroll
                for (int dt = 0; dt < 4; dt++) {
                    const uint16_t *vr = vs + (dt * 32 + l32) * VP + half * 32 + kk * 16 + 4 * g;
                    u32x2 lo = *(const u32x2 *)vr;
                    u32x2 hi = *(const u32x2 *)(vr + 8);
                    bf16x8 a = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf, o[dt], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    // normalize and stage O [32 q x 128 d] per wave through LDS for row stores
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = 1.0f / l_tot;
    if (outf) {
        store_out_f32<68>((float *)lds + wave * 32 * 68, o, inv, lane, outf, bb, Sq, H * HD, hh * HD, q0);
        return;
    }
    uint16_t *os = lds + wave * 32 * OP;
    stage_out_bf16<OP>(os, o, inv, lane, q8 != 0);
    __syncthreads();
    const int64_t HDt = H * HD;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = i * 4 + (lane >> 4);
        const int c = (lane & 15) * 8;
        const int64_t qi = q0 + r;
        if (qi < Sq)
            *(u32x4 *)(out + (bb * Sq + qi) * HDt + hh * HD + c) = *(const u32x4 *)(os + r * OP + c);
    }
}

}  // namespace anylen

template <int NW, bool PRE, bool MASKED, int SMODE = 0, bool PAIR = false>
void launch_fast(const uint16_t *q, Seg s0, Seg s1, int64_t h, int64_t sq, int64_t b, float sl2, uint16_t *out,
                 float *outf, const KeyMask &km, const int32_t *lim, const ScoreBound &sb, int q8,
                 hipStream_t stream) {
    const int64_t nq = (sq + 32 * NW - 1) / (32 * NW);
    fast::attn_fast_kernel<NW, PRE, MASKED, SMODE, PAIR>
        <<<dim3((unsigned)(nq * (PAIR ? h / 2 : h) * b)), dim3(64 * NW), 0, stream>>>(q, s0, s1, h, sq, nq, b, sl2,
                                                                                       out, outf, km, lim, sb, q8);
}

// The masked kernel with the softmax form decided on the host where the score
// bound needs no device value (no prefix keys).
template <bool PRE>
void launch_masked(const uint16_t *q, Seg s0, Seg s1, int64_t h, int64_t sq, int64_t b, float sl2, uint16_t *out,
                   float *outf, const KeyMask &km, const int32_t *lim, const ScoreBound &sb, int q8,
                   hipStream_t stream) {
    if (sb.q_norm <= 0.f)
        launch_fast<8, PRE, true, 2>(q, s0, s1, h, sq, b, sl2, out, outf, km, lim, sb, q8, stream);
    else if (sb.k_prefix)
        launch_fast<8, PRE, true, 0>(q, s0, s1, h, sq, b, sl2, out, outf, km, lim, sb, q8, stream);
    else if (sb.q_norm * sb.k_own <= STATIC_MAX)
        launch_fast<8, PRE, true, 1>(q, s0, s1, h, sq, b, sl2, out, outf, km, lim, sb, q8, stream);
    else
        launch_fast<8, PRE, true, 2>(q, s0, s1, h, sq, b, sl2, out, outf, km, lim, sb, q8, stream);
}

// Waves per workgroup of the unmasked fast kernel, from the rounds each form
// takes. An 8-wave workgroup holds a CU alone; a round of them costs 1. Two
// 4-wave workgroups share a CU and do the same work in 1.05 (one wave per
// SIMD each, twice the K/V tile traffic per query); a round with at most one
// 4-wave workgroup per CU, half the work, takes 0.84. Measured at 32 heads,
// 256 prefix keys on 256 CUs: 1024 queries 42.3 -> 35.7 us and 2304 queries
// 150 -> 133 us with 4 waves, 4096 queries 268 us with 8 against 282 with 4.
int fast_waves(int64_t bh, int64_t sq) {
    const int64_t cus = device_cu_count();
    if (cus <= 0) return 8;
    const int64_t n8 = (sq + 255) / 256 * bh, n4 = (sq + 127) / 128 * bh;
    const int64_t c8 = 100 * ((n8 + cus - 1) / cus);
    const int64_t r4 = n4 % (2 * cus);
    const int64_t c4 = 105 * (n4 / (2 * cus)) + (r4 == 0 ? 0 : r4 <= cus ? 84 : 105);
    return c4 < c8 ? 4 : 8;
}

// sl2 = softmax scale * log2(e) applied to raw scores, or 1 when q already
// carries it (PRE)
// The output rounding of the launchers (out_qblk): 0 none (bf16 to out, or f32
// to outf when it is set); 32 candle's Q8_0 blocks, rounded in the kernels'
// epilogue; 256 Q8_K blocks, which span two heads: the paired kernel rounds
// them where it runs (the cached step's 8-wave form, an even head count),
// else the output goes to outf in f32 and the rows quantizer rounds it. outf
// is the f32 scratch [B, Sq, H * 128] for 256.
bool out_qblk_ok(int out_qblk, const float *outf) {
    return out_qblk == 0 || out_qblk == 32 || (out_qblk == 256 && outf);
}
hipError_t finish_q8k(int out_qblk, bool rounded, const float *outf, int64_t b, int64_t h, int64_t sq,
                      uint16_t *out, hipStream_t stream) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || out_qblk != 256 || rounded) return e;
    return launch_quant_rows(outf, h * 128, b * sq, h * 128, 256, out, h * 128, stream);
}

template <bool PRE>
hipError_t launch(const uint16_t *q, const uint16_t *kp, const uint16_t *vtp, int64_t p, const uint16_t *ko,
                  const uint16_t *vto, int64_t so, int64_t b, int64_t h, int64_t sq, float sl2, uint16_t *out,
                  float *outf, const ScoreBound &sb, int out_qblk, hipStream_t stream) {
    if (sq <= 0 || b <= 0 || h <= 0) return hipSuccess;
    if (p < 0 || so < 0 || p + so <= 0 || !out_qblk_ok(out_qblk, outf)) return hipErrorInvalidValue;
    Seg s0{kp, vtp, p}, s1{ko, vto, so};
    if (p <= 0) {
        s0 = s1;
        s1 = Seg{ko, vto, 0};
    }
    const int q8 = out_qblk == 32;
    float *f32out = out_qblk == 32 ? nullptr : outf;  // f32 output (0 with outf, or 256 not paired)
    bool rounded = false;
    if ((p & 7) == 0 && (so & 7) == 0) {
        const KeyMask km{nullptr, nullptr, p + so};
        const int nw = fast_waves(b * h, sq);
        if (out_qblk == 256 && nw == 8 && h % 2 == 0) {
            launch_fast<8, PRE, false, 0, true>(q, s0, s1, h, sq, b, sl2, out, outf, km, nullptr, sb, 0, stream);
            rounded = true;
        } else if (nw == 4) {
            launch_fast<4, PRE, false>(q, s0, s1, h, sq, b, sl2, out, f32out, km, nullptr, sb, q8, stream);
        } else {
            launch_fast<8, PRE, false>(q, s0, s1, h, sq, b, sl2, out, f32out, km, nullptr, sb, q8, stream);
        }
    } else {
        const int64_t nq = (sq + anylen::QB - 1) / anylen::QB;
        anylen::attn_any_kernel<false><<<dim3((unsigned)(nq * h * b)), dim3(256), 0, stream>>>(
            q, s0, s1, h, sq, nq, b, sl2, out, f32out, KeyMask{nullptr, nullptr, p + so}, q8);
    }
    return finish_q8k(out_qblk, rounded, outf, b, h, sq, out, stream);
}

}  // namespace

hipError_t launch_attention(const uint16_t *q, const uint16_t *kp, const uint16_t *vtp, int64_t p,
                            const uint16_t *ko, const uint16_t *vto, int64_t so, int64_t b, int64_t h,
                            int64_t sq, float scale, uint16_t *out, hipStream_t stream, float *outf) {
    return launch<false>(q, kp, vtp, p, ko, vto, so, b, h, sq, scale * 1.4426950408889634f, out, outf,
                         ScoreBound{nullptr, 0.f, 0.f}, 0, stream);
}

hipError_t launch_attention_masked(const uint16_t *q, const uint16_t *kp, const uint16_t *vtp, int64_t p,
                                   const uint16_t *ko, const uint16_t *vto, int64_t so, int64_t b, int64_t h,
                                   int64_t sq, float sl2, const int32_t *img, const uint8_t *kvalid,
                                   int32_t *lim_scratch, uint16_t *out, hipStream_t stream, float *outf,
                                   const float *k_prefix_norm, float q_norm, float k_own_norm, int out_qblk) {
    if (sq <= 0 || b <= 0 || h <= 0) return hipSuccess;
    if (p < 0 || so < 0 || p + so <= 0 || !out_qblk_ok(out_qblk, outf)) return hipErrorInvalidValue;
    const int out_q8 = out_qblk == 32;
    if (out_qblk == 32) outf = nullptr;
    if (img && (p != 0 || so != sq)) return hipErrorInvalidValue;  // block-causal: one shared sequence
    Seg s0{kp, vtp, p}, s1{ko, vto, so};
    if (p <= 0) {
        s0 = s1;
        s1 = Seg{ko, vto, 0};
    }
    const KeyMask km{img, kvalid, p + so};
    if ((p & 7) == 0 && (so & 7) == 0 && (!img || (lim_scratch && sq <= LIMIT_MAX_S))) {
        if (img) {
            key_limit_kernel<<<dim3(1), dim3(1024), 0, stream>>>(img, (int)sq, lim_scratch);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        // the bound is on scores in log2 units: q's norm times sl2
        const ScoreBound sb{p > 0 ? k_prefix_norm : nullptr, q_norm * sl2, k_own_norm};
        // sl2 == 1: q already carries the scale (the block's q/k/v epilogue)
        if (sl2 == 1.0f)
            launch_masked<true>(q, s0, s1, h, sq, b, sl2, out, outf, km, img ? lim_scratch : nullptr, sb, out_q8,
                                stream);
        else
            launch_masked<false>(q, s0, s1, h, sq, b, sl2, out, outf, km, img ? lim_scratch : nullptr, sb, out_q8,
                                 stream);
        return finish_q8k(out_qblk, false, outf, b, h, sq, out, stream);
    }
    const int64_t nq = (sq + anylen::QB - 1) / anylen::QB;
    anylen::attn_any_kernel<true><<<dim3((unsigned)(nq * h * b)), dim3(256), 0, stream>>>(
        q, s0, s1, h, sq, nq, b, sl2, out, outf, km, out_q8);
    return finish_q8k(out_qblk, false, outf, b, h, sq, out, stream);
}

hipError_t launch_attention_log2(const uint16_t *q, const uint16_t *kp, const uint16_t *vtp, int64_t p,
                                 const uint16_t *ko, const uint16_t *vto, int64_t so, int64_t b, int64_t h,
                                 int64_t sq, uint16_t *out, hipStream_t stream, float *outf,
                                 const float *k_prefix_norm, float q_norm, float k_own_norm, int out_qblk) {
    return launch<true>(q, kp, vtp, p, ko, vto, so, b, h, sq, 1.0f, out, outf,
                        ScoreBound{p > 0 ? k_prefix_norm : nullptr, q_norm, k_own_norm}, out_qblk, stream);
}

}  // namespace qimm
