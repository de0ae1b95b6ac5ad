// Joint attention for gfx950: image-token queries over [cached prefix K/V ;
// own K/V], non-causal, head_dim 128, bf16 MFMA with f32 online softmax.
//
// Replaces the unmasked cached-step call of chunked_attention /
// flash_attention (src/transformer.rs:246-296) made from Attention::forward
// (src/quantized_transformer.rs:143-148). The two key segments are read in
// place (no concatenation copy, src/quantized_transformer.rs:143-146).
//
// Work split: one workgroup = 128 queries of one (batch, head), 4 waves x 32
// queries. Each wave computes S^T = K_blk Q^T (64 keys x 32 queries) with
// v_mfma_f32_32x32x16_bf16, so every lane owns one query column: the row max
// and row sum need only the lane and its partner lane^32. The probabilities
// stay in registers and are the B operand of O^T += V^T P^T; the 16-key
// K-slots of that MFMA use the permuted key order the S^T accumulator layout
// produces, and V^T is read from LDS in the same order. K and V^T tiles of 64
// keys are double-buffered in LDS.
#include "device_common.h"
#include "kernels.h"

namespace qimm {
namespace {

constexpr int QB = 128;     // queries per workgroup
constexpr int KB = 64;      // keys per block
constexpr int HD = 128;     // head dim
constexpr int KP = 136;     // bf16 pitch of K tile rows (128 + 8)
constexpr int VP = 68;      // bf16 pitch of V^T tile rows (64 + 4): conflict-free 8 B reads
constexpr int KSTAGE = KB * KP;
constexpr int VSTAGE = HD * VP;
constexpr int STAGE = KSTAGE + VSTAGE;
constexpr int OP = 136;     // bf16 pitch of the output staging rows

struct Seg {
    const uint16_t *k;   // [BH][len][128]
    const uint16_t *vt;  // [BH][128][len]
    int64_t len;
};

__global__ __launch_bounds__(256, 2) void attn_kernel(const uint16_t *__restrict__ q, Seg s0, Seg s1,
                                                      int64_t H, int64_t Sq, int64_t nq, int64_t B,
                                                      float sl2, uint16_t *__restrict__ out) {
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
    uint16_t *os = lds + wave * 32 * OP;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const int d = dt * 32 + 8 * rq + 4 * g;
            u32x2 w{pack_bf16x2(o[dt][4 * rq] * inv, o[dt][4 * rq + 1] * inv),
                    pack_bf16x2(o[dt][4 * rq + 2] * inv, o[dt][4 * rq + 3] * inv)};
            *(u32x2 *)(os + l32 * OP + d) = w;
        }
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

}  // namespace

hipError_t launch_attention(const uint16_t *q, const uint16_t *kp, const uint16_t *vtp, int64_t p,
                            const uint16_t *ko, const uint16_t *vto, int64_t so, int64_t b, int64_t h,
                            int64_t sq, float scale, uint16_t *out, hipStream_t stream) {
    if (sq <= 0 || b <= 0 || h <= 0) return hipSuccess;
    Seg s0{kp, vtp, p}, s1{ko, vto, so};
    if (p <= 0) {
        s0 = s1;
        s1 = Seg{ko, vto, 0};
    }
    const int64_t nq = (sq + QB - 1) / QB;
    const float sl2 = scale * 1.4426950408889634f;
    attn_kernel<<<dim3((unsigned)(nq * h * b)), dim3(256), 0, stream>>>(q, s0, s1, h, sq, nq, b, sl2, out);
    return hipGetLastError();
}

}  // namespace qimm
