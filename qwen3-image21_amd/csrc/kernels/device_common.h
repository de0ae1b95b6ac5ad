// Device-side helpers shared by the gfx950 kernels: vector types for the
// bf16 MFMA operands, GGML f16 decoding, bf16 packing and wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qimm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// IEEE binary16 -> f32 by bit manipulation (exact for every input, subnormals
// included), so dequantized values never depend on the FP16 denormal mode.
// Branch-free (selects, no divergent control flow in the GEMM loops that
// decode block scales every k step).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    const uint32_t sub = __float_as_uint((float)m * 5.9604644775390625e-08f) | sign;  // m * 2^-24, exact
    const uint32_t norm = sign | ((e + 112u) << 23) | (m << 13);
    const uint32_t inf = sign | 0x7f800000u | (m << 13);
    return __uint_as_float(e == 0 ? sub : (e == 31 ? inf : norm));
}

// The same by the hardware convert (v_cvt_f32_f16): exact for every finite
// input, subnormals included, because HIP kernels run with f16 denormals
// preserved (FLOAT_DENORM_MODE_16_64 = 3 in every kernel descriptor here). A
// single instruction, so the GEMM loops that decode block scales every k step
// keep one basic block.
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}

// Round-to-nearest-even f32 -> bf16 (lowers to v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 r;
    r[0] = (__bf16)lo;
    r[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, r);
}

// Q4_K device layout: the 144 B GGUF blocks of 16 consecutive rows are
// interleaved per super-block, so one super-block column of a 16-row group is
// 2304 contiguous bytes: block (n, sb) at ((n / 16) * sbs + sb) * 16 + n % 16.
__device__ __forceinline__ const uint8_t *q4k_block(const uint8_t *q, int64_t n, int64_t sb, int64_t sbs) {
    return q + (((n >> 4) * sbs + sb) * 16 + (n & 15)) * 144;
}

// Q6_K device layout, the same interleave with blocks padded to 224 B.
__device__ __forceinline__ const uint8_t *q6k_block(const uint8_t *q, int64_t n, int64_t sb, int64_t sbs) {
    return q + (((n >> 4) * sbs + sb) * 16 + (n & 15)) * 224;
}

// f32 fma with src0 read as f16 from the low / high half of x: a code q held
// as the f16 subnormal q * 2^-24 (exact) times a scale pre-multiplied by 2^24
// gives q*scale + off with a single rounding, no separate integer convert.
__device__ __forceinline__ float mix_lo(uint32_t x, float s, float c) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(s), "v"(c));
    return r;
}
__device__ __forceinline__ float mix_hi(uint32_t x, float s, float c) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x), "v"(s), "v"(c));
    return r;
}

// MFMA operand tiles in LDS: dense 128 B rows (64 bf16 of a k step), 16 B
// chunk c of row r at slot c ^ key(r), key = (r & 7) ^ ((r >> 3) & 1).
// Measured on gfx950: 16 B reads are served 16 lanes (256 B) per cycle and are
// conflict free when the 16 rows of a group cover all 16 slots of a 256 B
// window (same-parity rows need distinct keys); 16 B writes are served 8 lanes
// (128 B) per cycle and need distinct keys on each aligned group of 8 rows.
// This key satisfies both.
__device__ __forceinline__ int swz_key(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ swz_key(r)) << 4); }

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// s_waitcnt immediates for __builtin_amdgcn_s_waitcnt (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt in 6:4, lgkmcnt in 11:8; an all-ones field does
// not wait on that counter).
constexpr unsigned WAIT_VM0 = 0x0f70;        // vmcnt(0)
constexpr unsigned WAIT_LGKM0 = 0xc07f;      // lgkmcnt(0)
constexpr unsigned WAIT_VM0_LGKM0 = 0x0070;  // vmcnt(0) lgkmcnt(0)

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
    return __uint_as_float(b << 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float group_sum(float v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// An f32 whose rounding to bf16 (nearest even, as pack_bf16x2 rounds) is that
// of the exact product d * q, for an integer code q (|q| <= 128: the product
// has at most 32 significant bits). p = fma(d, q, +0) is the product rounded
// once to f32, and +0 for q = 0 whatever the signs. The bf16 rounding of p is
// the exact product's unless p lies exactly halfway between two bf16 values
// (low half 0x8000) while the product is not p: then p moves one f32 ulp
// toward the product (its error e = dq - p by one fma gives the side), off the
// halfway point. That case is rare and sits behind a branch.
__device__ __forceinline__ float product_for_bf16(float d, float q) {
    const float p = __builtin_fmaf(d, q, 0.f);
    const uint32_t b = __float_as_uint(p);
    if (__builtin_expect((b & 0xffffu) == 0x8000u, 0)) {
        const float e = __builtin_fmaf(d, q, -p);
        // same signs: the product is larger in magnitude, so is the next pattern
        if (e != 0.f) return __uint_as_float(((__float_as_uint(e) ^ b) >> 31) ? b - 1u : b + 1u);
    }
    return p;
}

// Rounding half away from zero for |x| < 2^22: x plus the largest float below
// 1/2 with x's sign, truncated. The sum reaches the next integer exactly when
// x's fraction is at least 1/2: below that it stays short of the integer by
// more than half an ulp of the sum, so its own rounding does not reach it.
__device__ __forceinline__ float round_half_away(float x) {
    return __builtin_truncf(x + __builtin_copysignf(0.49999997f, x));
}

// round_half_away(v * s) with the product rounded to f32 first, as candle
// computes iscale * x. Contraction is off here: HIP device code contracts by
// default, and v * s fused into the add above rounds once, which differs
// where v s lies within half an f32 ulp of k + 1/2 (2.4999999 rounds to the
// float 2.5 and then to 3, but 2.4999999 + 0.49999997 rounds to 2.9999998).
__device__ __forceinline__ float round_half_away_product(float v, float s) {
#pragma clang fp contract(off)
    const float x = v * s;
    return __builtin_truncf(x + __builtin_copysignf(0.49999997f, x));
}

// max over each aligned group of 8 lanes (a >= 0 or any floats): DPP moves
// within quads (xor 1, xor 2), then the half-row mirror (lane i <-> 7 - i)
template <int CTRL>
__device__ __forceinline__ float dpp_fmax(float a) {
    return fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), CTRL, 0xf, 0xf, false)));
}
__device__ __forceinline__ float max8_lanes(float a) {
    a = dpp_fmax<0xb1>(a);      // quad_perm [1,0,3,2]
    a = dpp_fmax<0x4e>(a);      // quad_perm [2,3,0,1]
    return dpp_fmax<0x141>(a);  // row_half_mirror
}
// max over the wave, the same value in every lane: 8-lane groups, the row
// mirror (16 lanes), then the four rows' values read as scalars
__device__ __forceinline__ float max_wave(float a) {
    a = dpp_fmax<0x140>(max8_lanes(a));  // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Q8_K block rounding from the block's largest magnitude a and the signed value
// xmax at its first occurrence: iscale s = -128 / xmax and d = 1 / s (both 0
// for an all-zero block); one value's operand is bf16(d * min(127, round(v s)))
// (q8k_values4).
__device__ __forceinline__ void q8k_scales(float a, float xmax, float &s, float &d) {
    s = a == 0.f ? 0.f : -128.f / xmax;
    d = a == 0.f ? 0.f : 1.f / s;
}
// Q8_0 block rounding from the block's largest magnitude a: q = round(v s) with
// s = 1 / (a / 127) (0 for an all-zero block), the value d q with d = a / 127
// kept as f16 (q8_0_values4).
__device__ __forceinline__ void q8_0_scales(float a, float &s, float &d) {
    const float d32 = a / 127.f;
    s = d32 != 0.f ? 1.f / d32 : 0.f;
    d = (float)(_Float16)d32;
}

// Four bf16 operands bf16(d * q_e), packed, each as product_for_bf16 gives it:
// the products rounded once to f32, the rare halfway test made once for the
// four (one branch instead of four), and the exact form taken for all four
// when any of them sits on a bf16 halfway point.
__device__ __forceinline__ u32x2 products4_bf16(float d, f32x4 q) {
    float p[4];
    bool half = false;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        p[e] = __builtin_fmaf(d, q[e], 0.f);
        half |= (__float_as_uint(p[e]) & 0xffffu) == 0x8000u;
    }
    if (__builtin_expect(half, 0)) {
#pragma unroll
        for (int e = 0; e < 4; e++) p[e] = product_for_bf16(d, q[e]);
    }
    return u32x2{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
}
// four values' Q8_K operands bf16(d * min(127, round(v s))) / Q8_0 operands
// bf16(d * round(v s)), packed
__device__ __forceinline__ u32x2 q8k_values4(f32x4 v, float s, float d) {
    f32x4 q;
#pragma unroll
    for (int e = 0; e < 4; e++) q[e] = fminf(round_half_away_product(v[e], s), 127.f);
    return products4_bf16(d, q);
}
__device__ __forceinline__ u32x2 q8_0_values4(f32x4 v, float s, float d) {
    f32x4 q;
#pragma unroll
    for (int e = 0; e < 4; e++) q[e] = round_half_away_product(v[e], s);
    return products4_bf16(d, q);
}

// Magnitudes (non-negative floats) compared as their bit patterns, whose
// unsigned order is theirs, so each DPP move folds into one integer max (and
// the wave's four row maxima combine on the scalar unit): the largest over
// each aligned group of 8 lanes, and over the wave. The same values as
// max8_lanes / max_wave for inputs without NaN.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t a) {
    return max(a, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a, CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float mag_max8_lanes(float a) {
    uint32_t u = __float_as_uint(a);
    u = dpp_umax<0xb1>(u);   // quad_perm [1,0,3,2]
    u = dpp_umax<0x4e>(u);   // quad_perm [2,3,0,1]
    u = dpp_umax<0x141>(u);  // row_half_mirror
    return __uint_as_float(u);
}
__device__ __forceinline__ float mag_max_wave(float a) {
    const uint32_t u = dpp_umax<0x140>(__float_as_uint(mag_max8_lanes(a)));  // row_mirror
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)u, 0);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)u, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)u, 32);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)u, 48);
    return __uint_as_float(max(max(r0, r1), max(r2, r3)));
}

// The activation rounding of candle's CPU QMatMul (candle-core 0.11
// quantized/k_quants.rs, the vec-dot type of the weight): each lane holds four
// consecutive values of a row, consecutive lanes continue the row.
//  QBLK 256, BlockQ8K::from_float: the wave's 256 values are one block; x_max is
//    the first value (in row order) of largest magnitude, iscale = -128/x_max,
//    q = min(127, round(iscale * x)) (round half away from zero), d = 1/iscale.
//  QBLK 32, BlockQ8_0::from_float: each aligned group of 8 lanes is one block;
//    d = amax/127, q = round(x / d) computed as x * (1/d), and the block keeps d
//    as f16 (round to nearest even).
// Returns the four bf16 operands bf16(d * q) (product_for_bf16), packed in
// pairs. Every lane of the block must take part (whole waves for 256, whole
// 8-lane groups for 32); all-zero blocks give zeros, as candle's d = 0 does.
// quant_act4 rounds one chunk of four values per lane; quant_act4_n rounds N
// chunks at once (chunk i its own Q8_K block, or its own eight Q8_0 blocks),
// each step taken for all chunks before the next, without branches but the one
// rare halfway test for all N x 4 products, so the chunks' reduction chains
// interleave.
template <int QBLK, int N>
__device__ __forceinline__ void quant_act4_n(const f32x4 (&v)[N], u32x2 (&out)[N]) {
    static_assert(QBLK == 32 || QBLK == 256, "Q8_0 or Q8_K blocks");
    float a[N], s[N], d[N];  // value = d * q, q from x * s
#pragma unroll
    for (int i = 0; i < N; i++)
        a[i] = fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3])));
    if constexpr (QBLK == 256) {
#pragma unroll
        for (int i = 0; i < N; i++) a[i] = mag_max_wave(a[i]);
#pragma unroll
        for (int i = 0; i < N; i++) {
            // the lane's first value of the largest magnitude, then the first lane holding one
            float mine = v[i][3];
            bool hit = fabsf(v[i][3]) == a[i];
#pragma unroll
            for (int e = 2; e >= 0; e--) {
                const bool h = fabsf(v[i][e]) == a[i];
                mine = h ? v[i][e] : mine;
                hit = hit || h;
            }
            const uint64_t lanes = __ballot(hit);
            const int first = lanes ? (int)__builtin_ctzll(lanes) : 0;
            const float xmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), first));
            q8k_scales(a[i], xmax, s[i], d[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; i++) q8_0_scales(mag_max8_lanes(a[i]), s[i], d[i]);
    }
    float q[N][4], p[N][4];
    bool half = false;
#pragma unroll
    for (int i = 0; i < N; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float r = round_half_away_product(v[i][e], s[i]);
            q[i][e] = QBLK == 256 ? fminf(r, 127.f) : r;
            p[i][e] = __builtin_fmaf(d[i], q[i][e], 0.f);
            half |= (__float_as_uint(p[i][e]) & 0xffffu) == 0x8000u;
        }
    if (__builtin_expect(half, 0)) {
#pragma unroll
        for (int i = 0; i < N; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) p[i][e] = product_for_bf16(d[i], q[i][e]);
    }
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = u32x2{pack_bf16x2(p[i][0], p[i][1]), pack_bf16x2(p[i][2], p[i][3])};
}

template <int QBLK>
__device__ __forceinline__ u32x2 quant_act4(f32x4 v) {
    const f32x4 c[1] = {v};
    u32x2 o[1];
    quant_act4_n<QBLK, 1>(c, o);
    return o[0];
}

}  // namespace qimm
