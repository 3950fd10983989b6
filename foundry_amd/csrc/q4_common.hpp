// Device-side helpers shared by the q4 kernels: the bf16 codec and the q4
// nibble layout.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fh {

// Group size the kernels implement (elements of K sharing one scale/bias).
constexpr int kGroup = 64;

// bf16 -> f32 is exact: the bf16 bits are the top half of the f32 bits
// (src/metal/kernels/common.metal:29-31).
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// f32 -> bf16, round to nearest with ties to even; a NaN keeps its top bits
// and is made quiet (src/metal/kernels/common.metal:37-43). The same rule as
// the reference so every materialised value, NaN included, is bit-identical.
// gfx950's v_cvt_pk_bf16_f32 implements exactly this rule (checked on the
// GPU against (b + 0x7FFF + ((b >> 16) & 1)) >> 16, with NaN -> (b >> 16) |
// 0x40, for 4.2M inputs: every tie pattern of every upper half, denormals,
// the largest finite values, infinities and NaN payloads), so the conversion
// is one instruction.
typedef __attribute__((ext_vector_type(2))) __bf16 fh_bf16x2_t;

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}

// Two values in one conversion: lo in bits 0..15, hi in 16..31.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_rne(float lo, float hi) {
    const fh_bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// Dequantised weight in fp32: the product, rounded, then the sum, rounded.
// s*q is exact whenever it is finite (8-bit significand times a 4-bit
// integer), so this equals fmaf(s, q, b) except when s*q overflows fp32
// (|s| > 2^124), where the product becomes an infinity as in the reference's
// mul-then-add order. Contraction is switched off here so the two roundings
// stay two instructions.
__device__ __forceinline__ float q4_dequant(float s, uint32_t q, float b) {
#pragma clang fp contract(off)
    const float prod = s * static_cast<float>(q);
    return prod + b;
}

// Same value through one fma, for the GEMM's register dequantisation; equal
// to q4_dequant whenever s*q is finite in fp32.
__device__ __forceinline__ float q4_dequant_fma(float s, uint32_t q, float b) {
    return fmaf(s, static_cast<float>(q), b);
}

// Loads of bytes a launch reads once (the weights a decode GEMV streams):
// the nontemporal hint (`nt`) marks them as streaming for the caches.
// Measured: the cold 14.2 MB one-row GEMV 5.40 -> 5.26 us (weights and its
// scale/bias table), the batch-1 decode step 1.010 -> 0.964 ms, the batch-8
// step 2.819 -> 2.805 ms (the matrix-core GEMV's weights only: on its
// scale/bias table the hint cost 3.5%, and on the decode attention's K/V
// reads it was no faster).
typedef __attribute__((ext_vector_type(4))) uint32_t stream_u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t stream_u32x2_t;

__device__ __forceinline__ uint4 load_stream16(const uint4 *p) {
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const stream_u32x4_t *>(p)));
}

__device__ __forceinline__ uint2 load_stream8(const uint2 *p) {
    return __builtin_bit_cast(uint2, __builtin_nontemporal_load(reinterpret_cast<const stream_u32x2_t *>(p)));
}

}  // namespace fh
