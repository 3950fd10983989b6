// Device helpers shared by the decoder-step kernels: bf16 rounding in the
// reference's convention, 8-value bf16 unpacking, wavefront reductions and
// the RoPE rotation of an 8-dim piece.
#pragma once

#include <initializer_list>

#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

__device__ __forceinline__ uint16_t rne(float v) { return static_cast<uint16_t>(f32_to_bf16_rne(v)); }
__device__ __forceinline__ float bf(uint16_t b) { return bf16_to_f32(b); }

// act(g) * u of LlamaMlp (src/models/llama/mlp.rs:49-58) on bf16 g and u:
// RNE(RNE(g / (1 + exp(-g))) * u), the rounding of the reference's separate
// silu and mul ops. Every kernel that forms the activation uses this.
__device__ __forceinline__ uint16_t silu_mul1(uint16_t gb, uint16_t ub) {
    const float g = bf(gb), u = bf(ub);
    const float den = expf(-g) + 1.0f;
    return rne(bf(rne(g / den)) * u);
}

// Elements i .. i + 7 of a GEMM split over K (f32 partials [splits][...],
// `stride` elements apart, i a multiple of 4): each the RNE to bf16 of its
// partials added in split order, the sum gemm_split_reduce_kernel forms;
// packed two per word. Every split's loads are issued before any add.
__device__ __forceinline__ uint4 split_sum8(const float *__restrict__ part, uint32_t splits, uint64_t stride,
                                            uint64_t i) {
    float4 lo[kMaxGemmSplits], hi[kMaxGemmSplits];
#pragma unroll
    for (uint32_t sp = 0; sp < kMaxGemmSplits; ++sp) {
        const float *p = part + static_cast<uint64_t>(sp < splits ? sp : splits - 1) * stride + i;
        lo[sp] = *reinterpret_cast<const float4 *>(p);
        hi[sp] = *reinterpret_cast<const float4 *>(p + 4);
    }
    float4 a = lo[0], b = hi[0];
#pragma unroll
    for (uint32_t sp = 1; sp < kMaxGemmSplits; ++sp)
        if (sp < splits) {
            a.x += lo[sp].x, a.y += lo[sp].y, a.z += lo[sp].z, a.w += lo[sp].w;
            b.x += hi[sp].x, b.y += hi[sp].y, b.z += hi[sp].z, b.w += hi[sp].w;
        }
    return make_uint4(rne(a.x) | static_cast<uint32_t>(rne(a.y)) << 16, rne(a.z) | static_cast<uint32_t>(rne(a.w)) << 16,
                      rne(b.x) | static_cast<uint32_t>(rne(b.y)) << 16, rne(b.z) | static_cast<uint32_t>(rne(b.w)) << 16);
}

__device__ __forceinline__ void unpack8(const uint4 v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[2 * e] = bf(w[e] & 0xFFFFu);
        f[2 * e + 1] = bf(w[e] >> 16);
    }
}

// The K cache of one (sequence, KV head) holds max_len keys of head_dim in
// groups of 16 keys: group g (keys 16 g .. 16 g + n_g - 1, n_g = min(16,
// max_len - 16 g)) is n_g * head_dim contiguous elements laid out
// [head_dim / 32][n_g][32], so dims d .. d + 7 (d a multiple of 8) of key j
// start at 16 g * head_dim + (d / 32) * n_g * 32 + (j - 16 g) * 32 + d % 32.
// One matrix-core B fragment (16 keys x 32 dims, 16 bytes per lane) is then a
// single 1 KB run instead of 16 runs of 64 bytes. The V cache stays
// [max_len][head_dim].
struct KTile {
    uint64_t base;    // element offset of key j's group and row within it
    uint32_t stride;  // elements between its 32-dim blocks (n_g * 32)
};
__host__ __device__ __forceinline__ KTile k_tile(uint32_t j, uint32_t max_len, uint32_t head_dim) {
    const uint32_t g = j >> 4, left = max_len - (g << 4);
    const uint32_t n_g = left < 16u ? left : 16u;
    return KTile{static_cast<uint64_t>(g) * 16u * head_dim + (j & 15u) * 32u, n_g * 32u};
}
__host__ __device__ __forceinline__ uint64_t k_offset(uint32_t j, uint32_t d, uint32_t max_len, uint32_t head_dim) {
    const KTile t = k_tile(j, max_len, head_dim);
    return t.base + (d >> 5) * t.stride + (d & 31u);
}

// Lane value of a DPP permutation within 16-lane rows (CDNA DPP controls:
// 0xB1 quad_perm [1,0,3,2], 0x4E quad_perm [2,3,0,1], 0x141 row_half_mirror,
// 0x140 row_mirror).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N = 8, 16 or 32), the total in every
// lane of the group. Within a row the steps are DPP moves (no LDS traffic);
// every lane of a group computes the same additions in the same order, so
// all hold bit-identical totals.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 8 || N == 16 || N == 32, "group of 8, 16 or 32 lanes");
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    if constexpr (N >= 16) v += dpp_mov<0x140>(v);
    if constexpr (N == 32) v += __shfl_xor(v, 16, 64);
    return v;
}

// Maximum over aligned groups of N lanes, as group_sum.
template <int N>
__device__ __forceinline__ float group_max(float v) {
    static_assert(N == 8 || N == 16 || N == 32, "group of 8, 16 or 32 lanes");
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    if constexpr (N >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
    if constexpr (N == 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Wavefront sum and maximum: DPP within each 16-lane row, then the four row
// results read out and combined in a fixed order (uniform result, no LDS
// round trips).
__device__ __forceinline__ float wave_sum(float v) {
    v = group_sum<16>(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = group_max<16>(v);
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// RoPE (src/models/llama/rotary_emb.rs:62-85) of dims p*8 .. p*8+7 of one
// head: x' = RNE(RNE(x * cos) + RNE(rot * sin)), rot = cat(-x2, x1); the
// partner piece is the matching 8 dims of the other half (hp pieces per
// half). head: the head's row; c, s: the position's table rows.
// The rotation of one piece from its loaded values: x (the piece), r (its
// partner piece), c and s (the table rows' matching pieces); first_half:
// rot = -partner.
__device__ __forceinline__ uint4 rope_apply(const uint4 x4, const uint4 r4, const uint4 c4, const uint4 s4,
                                            bool first_half) {
    const float sign = first_half ? -1.0f : 1.0f;
    float xv[8], rv[8], cv[8], sv[8];
    unpack8(x4, xv);
    unpack8(r4, rv);
    unpack8(c4, cv);
    unpack8(s4, sv);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t lo = rne(bf(rne(xv[2 * e] * cv[2 * e])) + bf(rne(sign * rv[2 * e] * sv[2 * e])));
        const uint32_t hi = rne(bf(rne(xv[2 * e + 1] * cv[2 * e + 1])) + bf(rne(sign * rv[2 * e + 1] * sv[2 * e + 1])));
        o[e] = lo | (hi << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ uint4 rope_piece(const uint16_t *head, const uint16_t *c, const uint16_t *s,
                                            uint32_t p, uint32_t hp) {
    const uint32_t partner = p < hp ? p + hp : p - hp;
    return rope_apply(*reinterpret_cast<const uint4 *>(head + p * 8), *reinterpret_cast<const uint4 *>(head + partner * 8),
                      *reinterpret_cast<const uint4 *>(c + p * 8), *reinterpret_cast<const uint4 *>(s + p * 8), p < hp);
}

}  // namespace fh

// Host-side check shared by the decoder entry points: sizes are
// non-negative and fit 32-bit kernel arguments.
inline int fh_check_dims(const char *fn, std::initializer_list<int64_t> dims) {
    for (int64_t d : dims)
        if (d < 0 || d > 0x7FFFFFFFll)
            return fh::fail(FH_ERR_INVALID_ARGUMENT, "%s: dimension %lld out of range", fn, (long long)d);
    return FH_OK;
}
