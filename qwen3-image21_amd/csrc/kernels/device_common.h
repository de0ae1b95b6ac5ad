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

}  // namespace qimm
