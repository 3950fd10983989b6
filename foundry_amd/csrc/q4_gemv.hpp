// q4 decode GEMV: y[m, r] = sum_j x[m, j] * (s[r, j/64] * q[r, j] + b[r, j/64])
// for m < 8 rows of x. Replaces the M=1..8 use of matmul_tiled
// (src/metal/kernels/matmul.metal:29-65) behind Linear::forward
// (src/nn/linear.rs:22-35), where 15 of 16 thread rows idle at M=1.
//
// HBM-bound: per weight 0.5 byte of nibbles plus 4 bytes of scale+bias per 64.
// Design for CDNA4:
// - A lane owns 16-byte chunks (32 weights, half a group) of one weight row;
//   L lanes share a row, chunk c = sub + L*i, so each load instruction of an
//   L-lane row group reads 16*L contiguous bytes. A wavefront covers 64/L
//   rows at once (a "row group").
// - Blocks are persistent: the grid is sized to the chip (8 blocks of 4
//   wavefronts per CU), each block stages x once and its wavefronts walk row
//   groups with a stride. A lane issues all CPL chunk loads of a row group at
//   once, and the next row group's loads before the current one's reduction;
//   latency is hidden by occupancy (one register buffer keeps VGPRs low).
// - x is staged into LDS, permuted so that the bf16 pair for nibbles
//   (e, e+4) of a word is one dword, and laid out [m][word-in-chunk][chunk]
//   so neighbouring lanes read neighbouring 16 bytes (no bank conflicts).
//   Per-chunk sums of x are staged beside it.
// - Dequantisation in registers without conversions: (w >> 4t) & 0x000F000F
//   | 0x43004300 is a bf16 pair (128 + q_t, 128 + q_{t+4}), exact since q < 16;
//   v_dot2_f32_bf16 multiplies it with the x pair and accumulates in fp32.
//   Per chunk: sum_j x_j (s q_j + b) = s * d + (b - 128 s) * X, with
//   d = sum_j x_j (128 + q_j) and X = sum_j x_j.
// - Partial sums are reduced across the L lanes of a row with cross-lane
//   shuffles; one lane writes each output (bf16 RNE or fp32).
#pragma once

#include "decoder_common.hpp"
#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

#ifndef FH_GEMV_THREADS
#define FH_GEMV_THREADS 256
#endif
constexpr int kGemvThreads = FH_GEMV_THREADS;
constexpr int kGemvWaves = kGemvThreads / 64;
// Dynamic LDS one block may use for staged x (bytes).
constexpr uint32_t kGemvLdsLimit = 64 * 1024;
// Persistent blocks per CU.
constexpr uint32_t kGemvBlocksPerCu = 8;

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Bytes of LDS the kernel needs for `m` rows of x with k columns (plus the
// staged norm weight with the RMSNorm prologue).
__host__ __device__ constexpr uint32_t gemv_lds_bytes(uint32_t m, uint32_t k, bool norm = false) {
    return m * (k / 32) * (4 * 16 + 4) + (norm ? k * 2 : 0);
}

// Decode-step fusions (the reference runs these as separate ops):
//   PRO kProRmsNorm: the product's input is RmsNorm (src/nn/norm.rs:32-50) of
//     h = x (+ res): h_j = RNE(x_j + res_j), x'_j = RNE(RNE(h_j * scale) *
//     w_j), scale = 1 / sqrt(sum h^2 * (1/k) + eps); block 0 writes h to
//     res_out. Work items are 8-value pieces spread over the whole block, and
//     x, res and w are requested before the weights, so the prologue costs
//     one block reduction on the block's critical path.
//   EPI kEpiSiluMul: act(gate) * up of LlamaMlp (src/models/llama/mlp.rs:
//     49-58) on the rows [gate (f) | up (f)] of the weight: a wavefront's row
//     group holds gate rows in its first half and the matching up rows in its
//     second, so after the reduction one shuffle brings u to g's lane, which
//     writes RNE(RNE(g / (exp(-g) + 1)) * u) with g, u the bf16 outputs. The
//     output has f columns (bf16).
enum GemvPro { kProNone = 0, kProRmsNorm = 1 };
enum GemvEpi { kEpiNone = 0, kEpiSiluMul = 1 };

struct GemvFusion {
    const uint16_t *res;  // kProRmsNorm: residual rows (stride k), or null
    uint16_t *res_out;    // kProRmsNorm: h rows (stride k), or null; no overlap with x or res
    const uint16_t *w;    // kProRmsNorm: norm weight [k]
    float eps, dim_inv;
};

// A 16-byte piece (x0..x7) as the staged layout holds it: dwords (x0,x4)
// (x1,x5) (x2,x6) (x3,x7), the bf16 pairs that nibbles (e, e+4) of a word meet.
__device__ __forceinline__ uint4 gemv_permute(const uint4 v) {
    uint4 p;
    p.x = (v.x & 0xFFFFu) | (v.z << 16);
    p.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
    p.z = (v.y & 0xFFFFu) | (v.w << 16);
    p.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
    return p;
}

// f applied to matching bf16 values of two pieces, RNE'd back into a.
template <typename F>
__device__ __forceinline__ uint4 gemv_pairwise(const uint4 a, const uint4 b, F f) {
    const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        o[e] = f32x2_to_bf16x2_rne(f(bf16_to_f32(av[e] & 0xFFFFu), bf16_to_f32(bv[e] & 0xFFFFu)),
                                   f(bf16_to_f32(av[e] >> 16), bf16_to_f32(bv[e] >> 16)));
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// One lane's chunks of one row group: packed words and the group scale/bias.
template <int CPL>
struct GemvChunks {
    uint4 w[CPL];
    uint32_t s[CPL], b[CPL];
};

// FULL: every lane's CPL chunks exist (k is a multiple of 32*CPL*L), so the
// loads need no per-chunk guard and share one address with immediate offsets.
// SB: a chunk's scale and bias come from sbi, the table interleaved per group
// pair (dword 2p of a row: scales of groups 2p, 2p + 1; dword 2p + 1: their
// biases), one 8-byte load instead of two 2-byte loads.
template <int M, int L, int CPL, bool FULL, int PRO, int EPI, bool SB>
__global__ __launch_bounds__(kGemvThreads) void q4_gemv_kernel(
    const uint16_t *__restrict__ x, uint32_t x_ld, const uint32_t *__restrict__ wq,
    const uint16_t *__restrict__ scales, const uint16_t *__restrict__ biases, const uint32_t *__restrict__ sbi,
    uint32_t n, uint32_t k, void *__restrict__ y, uint32_t y_ld, int y_is_f32, GemvFusion fu) {
    constexpr uint32_t kRowsPerWave = 64 / L;
    static_assert(EPI == kEpiNone || kRowsPerWave >= 2, "the SiLU epilogue pairs rows within a wavefront");
    // rows of one wavefront that produce outputs: with kEpiSiluMul, gate rows
    // (the other half are their up rows)
    constexpr uint32_t kOutRowsPerWave = EPI == kEpiSiluMul ? kRowsPerWave / 2 : kRowsPerWave;
    extern __shared__ uint4 lds[];
    const uint32_t chunks = k / 32;
    uint4 *xs = lds;                                                // [M][4][chunks]
    float *xsum = reinterpret_cast<float *>(lds + M * 4 * chunks);  // [M][chunks]

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t sub = lane % L;
    const uint32_t seg_chunks = CPL * L;
    const uint32_t segs = FULL ? chunks / seg_chunks : (chunks == 0 ? 1 : (chunks + seg_chunks - 1) / seg_chunks);
    const uint32_t n_out = EPI == kEpiSiluMul ? n / 2 : n;  // output columns
    const uint32_t groups_total = (n_out + kOutRowsPerWave - 1) / kOutRowsPerWave;
    const uint32_t group_first = blockIdx.x * kGemvWaves + wave;
    const uint32_t group_stride = gridDim.x * kGemvWaves;
    // output column of this lane's row in a row group, and its weight row
    const uint32_t rl = lane / L;
    auto out_col = [&](uint32_t group) {
        return group * kOutRowsPerWave + (EPI == kEpiSiluMul ? rl % kOutRowsPerWave : rl);
    };
    auto weight_row = [&](uint32_t group) {
        const uint32_t col = out_col(group);
        return EPI == kEpiSiluMul && rl >= kOutRowsPerWave ? col + n_out : col;
    };
    const bool out_lane = EPI == kEpiSiluMul ? rl < kOutRowsPerWave : true;

    auto load = [&](uint32_t group, uint32_t seg, GemvChunks<CPL> &buf) {
        const uint32_t row = weight_row(group);
        const bool in = out_col(group) < n_out;
        const uint64_t row_c = in ? row : n - 1;  // clamped rows load, never store
        const uint32_t c0 = seg * seg_chunks + sub;
        const uint4 *wrow = reinterpret_cast<const uint4 *>(wq + row_c * (k / 8)) + c0;
        const uint16_t *srow = scales + row_c * (k / kGroup);
        const uint16_t *brow = biases + row_c * (k / kGroup);
        const uint2 *irow = reinterpret_cast<const uint2 *>(sbi + row_c * (k / kGroup));
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const uint32_t c = c0 + u * L;
            if (FULL || c < chunks) {
                buf.w[u] = load_stream16(wrow + u * L);
                if constexpr (SB) {
                    // group c / 2 is half (c / 2) & 1 of pair c / 4 (the bf16
                    // conversion takes the low half)
                    const uint2 v = load_stream8(irow + c / 4);
                    const uint32_t sh = (c & 2u) * 8u;
                    buf.s[u] = v.x >> sh;
                    buf.b[u] = v.y >> sh;
                } else {
                    buf.s[u] = srow[c / 2];
                    buf.b[u] = brow[c / 2];
                }
            }
        }
    };

    // Stage x: one thread per (m, chunk): four 16-byte loads, permute, sum.
    // The first item's x loads go out before the weight loads so that waiting
    // for x (in-order load counters) does not wait for the weights; chunk 0 of
    // the weights is then computed while later chunks are still arriving.
    auto stage = [&](uint32_t t, const uint4 (&v)[4]) {
        const uint32_t m = t / chunks, c = t % chunks;
        float sum = 0.f;
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {  // v[wi] = (x0,x1) (x2,x3) (x4,x5) (x6,x7)
            uint4 p;
            p.x = (v[wi].x & 0xFFFFu) | (v[wi].z << 16);      // (x0, x4)
            p.y = (v[wi].x >> 16) | (v[wi].z & 0xFFFF0000u);  // (x1, x5)
            p.z = (v[wi].y & 0xFFFFu) | (v[wi].w << 16);      // (x2, x6)
            p.w = (v[wi].y >> 16) | (v[wi].w & 0xFFFF0000u);  // (x3, x7)
            xs[(m * 4 + wi) * chunks + c] = p;
            // pair sums as dot products with (1, 1): one instruction per pair
            sum = dot2_bf16(v[wi].x, 0x3F803F80u, sum);
            sum = dot2_bf16(v[wi].y, 0x3F803F80u, sum);
            sum = dot2_bf16(v[wi].z, 0x3F803F80u, sum);
            sum = dot2_bf16(v[wi].w, 0x3F803F80u, sum);
        }
        xsum[m * chunks + c] = sum;
    };
    auto load_x = [&](uint32_t t, uint4 (&v)[4]) {
        const uint32_t m = t / chunks, c = t % chunks;
        const uint4 *src = reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(m) * x_ld + c * 32);
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) v[wi] = src[wi];
    };

    GemvChunks<CPL> buf;
    if constexpr (PRO == kProRmsNorm) {
        // Pieces of 8 values, piece t = (m * chunks + c) * 4 + wi: 4 adjacent
        // lanes hold a chunk. Pass 1: h = x (+ res) staged (permuted) and sum
        // of squares per row; the norm weight staged beside it. Reduction.
        // Pass 2 in LDS: x' = RNE(RNE(h * scale) * w) and the chunk sums.
        uint4 *wsh = reinterpret_cast<uint4 *>(xsum + M * chunks);  // [4][chunks] norm weight
        __shared__ float red[kGemvWaves][M];
        const uint32_t pieces = M * chunks * 4;
        auto xoff = [&](uint32_t t) {
            const uint32_t m = t / (chunks * 4), r = t % (chunks * 4);
            return static_cast<uint64_t>(m) * k + r * 8;
        };
        float ss[M];
#pragma unroll
        for (int m = 0; m < M; ++m) ss[m] = 0.f;
        // a round's pieces load while the previous round is processed; past
        // the end, addresses are clamped to piece 0 and the values unused
        auto load_round = [&](uint32_t t0, uint4 &xv, uint4 &rv, uint4 &wv) {
            const uint32_t t = t0 + threadIdx.x;
            const uint64_t o = xoff(t < pieces ? t : 0);
            xv = *reinterpret_cast<const uint4 *>(x + o);
            rv = fu.res ? *reinterpret_cast<const uint4 *>(fu.res + o) : make_uint4(0u, 0u, 0u, 0u);
            wv = *reinterpret_cast<const uint4 *>(fu.w + (t < chunks * 4 ? t : 0) * 8);
        };
        // The first two rounds (every piece when M * k <= 4096) and the first
        // row group's weights are requested in straight-line code, with
        // clamped indices instead of guards, so each wait for a round counts
        // exactly the loads issued after it (a guarded load makes the
        // compiler wait for all of them, weights included).
        auto process = [&](uint32_t t0, uint4 xv, uint4 rv, uint4 wv) {
            const uint32_t t = t0 + threadIdx.x;
            const bool live = t < pieces;
            const uint64_t o = xoff(live ? t : 0);
            const bool wpiece = t < chunks * 4;
            if (fu.res) {
                xv = gemv_pairwise(xv, rv, [](float a, float b) { return a + b; });
                if (blockIdx.x == 0 && fu.res_out && live) *reinterpret_cast<uint4 *>(fu.res_out + o) = xv;
            }
            if (live) {
                const uint32_t hv[4] = {xv.x, xv.y, xv.z, xv.w};
                float sq = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = bf16_to_f32(hv[e] & 0xFFFFu), hi = bf16_to_f32(hv[e] >> 16);
                    sq += lo * lo;
                    sq += hi * hi;
                }
                const uint32_t m = t / (chunks * 4), c = (t / 4) % chunks, wi = t % 4;
#pragma unroll
                for (int mm = 0; mm < M; ++mm)
                    if (mm == static_cast<int>(m)) ss[mm] += sq;
                xs[(m * 4 + wi) * chunks + c] = gemv_permute(xv);
                if (wpiece) wsh[wi * chunks + c] = gemv_permute(wv);
            }
        };
        // the sum-of-squares reduction, then pass 2 (every thread calls it)
        auto finish = [&]() {
            {
                const uint32_t lane_x = threadIdx.x & 63, wave_x = threadIdx.x >> 6;
    #pragma unroll
                for (int m = 0; m < M; ++m) {
                    float v = ss[m];
    #pragma unroll
                    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
                    if (lane_x == 0) red[wave_x][m] = v;
                }
            }
            __syncthreads();
            for (uint32_t t0 = 0; t0 < pieces; t0 += kGemvThreads) {
                const uint32_t t = t0 + threadIdx.x;
                const bool live = t < pieces;
                const uint32_t m = live ? t / (chunks * 4) : 0, c = (t / 4) % chunks, wi = t % 4;
                float tot = 0.f;
    #pragma unroll
                for (int w = 0; w < kGemvWaves; ++w) tot += red[w][m];
                const float scale = 1.0f / sqrtf(tot * fu.dim_inv + fu.eps);
                float psum = 0.f;
                if (live) {
                    const uint4 p = gemv_pairwise(xs[(m * 4 + wi) * chunks + c], wsh[wi * chunks + c],
                                                  [scale](float h, float g) {
                                                      return bf16_to_f32(f32_to_bf16_rne(h * scale)) * g;
                                                  });
                    xs[(m * 4 + wi) * chunks + c] = p;
                    // (x0+x1) + (x2+x3) + (x4+x5) + (x6+x7) of the piece
                    psum = ((bf16_to_f32(p.x & 0xFFFFu) + bf16_to_f32(p.y & 0xFFFFu)) +
                            (bf16_to_f32(p.z & 0xFFFFu) + bf16_to_f32(p.w & 0xFFFFu))) +
                           ((bf16_to_f32(p.x >> 16) + bf16_to_f32(p.y >> 16)) +
                            (bf16_to_f32(p.z >> 16) + bf16_to_f32(p.w >> 16)));
                }
                psum += dpp_mov<0xB1>(psum);  // lane ^ 1
                psum += dpp_mov<0x4E>(psum);  // lane ^ 2
                if (live && wi == 0) xsum[m * chunks + c] = psum;
            }
        };
        // Two code paths with their own tails: a join between the weight
        // loads and the reduction would make the compiler wait for the
        // weights there.
        if (pieces <= 2 * kGemvThreads) {
            // every piece stays in its thread's registers between the two
            // passes (h and its norm weight), so pass 2 reads no LDS and pass
            // 1 writes none; the arithmetic is finish()'s
            uint4 x0, r0, w0, x1, r1, w1;
            auto load_round_w = [&](uint32_t t0, uint4 &xv, uint4 &rv, uint4 &wv) {
                const uint32_t t = t0 + threadIdx.x;
                const uint64_t o = xoff(t < pieces ? t : 0);
                xv = *reinterpret_cast<const uint4 *>(x + o);
                rv = fu.res ? *reinterpret_cast<const uint4 *>(fu.res + o) : make_uint4(0u, 0u, 0u, 0u);
                wv = *reinterpret_cast<const uint4 *>(fu.w + ((t < pieces ? t : 0) % (chunks * 4)) * 8);
            };
            load_round_w(0, x0, r0, w0);
            load_round_w(kGemvThreads, x1, r1, w1);
            __builtin_amdgcn_sched_barrier(0);  // keep these ahead of the weight loads
            load(group_first < groups_total ? group_first : groups_total - 1, 0, buf);
            // both rounds are handled unconditionally (dead pieces are masked
            // inside), so their loads cannot sink below the weights'
            auto sum_round = [&](uint32_t t0, uint4 &xv, const uint4 rv) {
                const uint32_t t = t0 + threadIdx.x;
                const bool live = t < pieces;
                if (fu.res) {
                    xv = gemv_pairwise(xv, rv, [](float a, float b) { return a + b; });
                    if (blockIdx.x == 0 && fu.res_out && live)
                        *reinterpret_cast<uint4 *>(fu.res_out + xoff(t)) = xv;
                }
                if (live) {
                    const uint32_t hv[4] = {xv.x, xv.y, xv.z, xv.w};
                    float sq = 0.f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float lo = bf16_to_f32(hv[e] & 0xFFFFu), hi = bf16_to_f32(hv[e] >> 16);
                        sq += lo * lo;
                        sq += hi * hi;
                    }
                    const uint32_t m = t / (chunks * 4);
#pragma unroll
                    for (int mm = 0; mm < M; ++mm)
                        if (mm == static_cast<int>(m)) ss[mm] += sq;
                }
            };
            sum_round(0, x0, r0);
            sum_round(kGemvThreads, x1, r1);
            {
                const uint32_t lane_x = threadIdx.x & 63, wave_x = threadIdx.x >> 6;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float v = ss[m];
#pragma unroll
                    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
                    if (lane_x == 0) red[wave_x][m] = v;
                }
            }
            __syncthreads();
            auto norm_round = [&](uint32_t t0, const uint4 hv, const uint4 wv) {
                const uint32_t t = t0 + threadIdx.x;
                const bool live = t < pieces;
                const uint32_t m = live ? t / (chunks * 4) : 0, c = (t / 4) % chunks, wi = t % 4;
                float tot = 0.f;
#pragma unroll
                for (int w = 0; w < kGemvWaves; ++w) tot += red[w][m];
                const float scale = 1.0f / sqrtf(tot * fu.dim_inv + fu.eps);
                float psum = 0.f;
                if (live) {
                    const uint4 p = gemv_permute(gemv_pairwise(hv, wv, [scale](float h, float g) {
                        return bf16_to_f32(f32_to_bf16_rne(h * scale)) * g;
                    }));
                    xs[(m * 4 + wi) * chunks + c] = p;
                    psum = ((bf16_to_f32(p.x & 0xFFFFu) + bf16_to_f32(p.y & 0xFFFFu)) +
                            (bf16_to_f32(p.z & 0xFFFFu) + bf16_to_f32(p.w & 0xFFFFu))) +
                           ((bf16_to_f32(p.x >> 16) + bf16_to_f32(p.y >> 16)) +
                            (bf16_to_f32(p.z >> 16) + bf16_to_f32(p.w >> 16)));
                }
                psum += dpp_mov<0xB1>(psum);  // lane ^ 1
                psum += dpp_mov<0x4E>(psum);  // lane ^ 2
                if (live && wi == 0) xsum[m * chunks + c] = psum;
            };
            norm_round(0, x0, w0);
            norm_round(kGemvThreads, x1, w1);
        } else {
            load(group_first < groups_total ? group_first : groups_total - 1, 0, buf);
            for (uint32_t t0 = 0; t0 < pieces; t0 += kGemvThreads) {
                uint4 xv, rv, wv;
                load_round(t0, xv, rv, wv);
                process(t0, xv, rv, wv);
            }
            finish();
        }
    } else {
        // x and the first row group's weights are requested unconditionally
        // (clamped indices; see the RMSNorm path) so that staging x waits
        // only for x. Threads past the last item stage a copy of item 0:
        // the same values to the same place, and no guarded use under which
        // the compiler could sink the x loads below the weight loads.
        const uint32_t items_x = M * chunks;
        uint4 xv[4];
        const uint32_t t_first = threadIdx.x < items_x ? threadIdx.x : 0;
        load_x(t_first, xv);
        __builtin_amdgcn_sched_barrier(0);
        load(group_first < groups_total ? group_first : groups_total - 1, 0, buf);
        stage(t_first, xv);
        for (uint32_t t = threadIdx.x + kGemvThreads; t < items_x; t += kGemvThreads) {
            load_x(t, xv);
            stage(t, xv);
        }
    }
    __syncthreads();

    // The bf16 exponent constant lives in a VGPR so that mask-and-or is one
    // v_and_or_b32 (a VOP3 on gfx9 takes no literal and at most one SGPR).
    uint32_t magic = 0x43004300u;
    asm volatile("" : "+v"(magic));

    for (uint32_t group = group_first; group < groups_total; group += group_stride) {
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.f;
        for (uint32_t seg = 0; seg < segs; ++seg) {
            if (seg > 0) load(group, seg, buf);
            const uint32_t c0 = seg * seg_chunks + sub;
#pragma unroll
            for (int u = 0; u < CPL; ++u) {
                const uint32_t c = c0 + u * L;
                if (FULL || c < chunks) {
                    const float s = bf16_to_f32(buf.s[u]);
                    const float bc = fmaf(-128.f, s, bf16_to_f32(buf.b[u]));
                    const uint32_t words[4] = {buf.w[u].x, buf.w[u].y, buf.w[u].z, buf.w[u].w};
                    uint32_t pr[4][4];
#pragma unroll
                    for (int wi = 0; wi < 4; ++wi)
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            pr[wi][t] = ((words[wi] >> (4 * t)) & 0x000F000Fu) | magic;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float d0 = 0.f, d1 = 0.f;
#pragma unroll
                        for (int wi = 0; wi < 4; ++wi) {
                            const uint4 xp = xs[(m * 4 + wi) * chunks + c];
                            d0 = dot2_bf16(pr[wi][0], xp.x, d0);
                            d1 = dot2_bf16(pr[wi][1], xp.y, d1);
                            d0 = dot2_bf16(pr[wi][2], xp.z, d0);
                            d1 = dot2_bf16(pr[wi][3], xp.w, d1);
                        }
                        acc[m] = fmaf(s, d0 + d1, acc[m]);
                        acc[m] = fmaf(bc, xsum[m * chunks + c], acc[m]);
                    }
                }
            }
        }
        // next row group's loads go out before this one's reduction
        const uint32_t next = group + group_stride;
        if (next < groups_total) load(next, 0, buf);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float v = acc[m];
#pragma unroll
            for (int off = L / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
            acc[m] = v;
        }
        if constexpr (EPI == kEpiSiluMul) {
            // the up row's sum, from the lane kOutRowsPerWave rows further on
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float u = __shfl_down(acc[m], kOutRowsPerWave * L, 64);
                const float g = bf16_to_f32(f32_to_bf16_rne(acc[m]));
                const float ub = bf16_to_f32(f32_to_bf16_rne(u));
                acc[m] = bf16_to_f32(f32_to_bf16_rne(g / (expf(-g) + 1.0f))) * ub;
            }
        }
        const uint32_t col = out_col(group);
        if (out_lane && col < n_out && sub == 0) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint64_t o = static_cast<uint64_t>(m) * y_ld + col;
                if (y_is_f32)
                    static_cast<float *>(y)[o] = acc[m];
                else
                    static_cast<uint16_t *>(y)[o] = static_cast<uint16_t>(f32_to_bf16_rne(acc[m]));
            }
        }
    }
}

// Blocks of `kernel` that stay resident on one CU with `lds` bytes each,
// capped at kGemvBlocksPerCu; a persistent grid larger than this would leave
// the excess blocks to run after the others, as a tail.
template <typename Kernel>
inline uint32_t resident_blocks(Kernel kernel, uint32_t lds) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kGemvThreads, lds) != hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    return per_cu < static_cast<int>(kGemvBlocksPerCu) ? per_cu : kGemvBlocksPerCu;
}

// Everything one GEMV launch needs besides its template shape.
struct GemvArgs {
    const uint16_t *x;
    uint32_t x_ld;
    const uint32_t *wq;
    const uint16_t *s, *b;
    uint32_t n, k;  // weight rows (with kEpiSiluMul: 2f), columns
    void *y;
    uint32_t y_ld;
    int y_is_f32;
    int pro, epi;
    GemvFusion fu;
    // matrix-core GEMV over K ranges: k is one range's length, the weight
    // rows hold kranges of them (0 or 1: k is the whole row); y then takes
    // f32 partial sums [kranges][rows][y_ld]
    uint32_t kranges = 0;
    // the scales and biases interleaved per group pair (fh_q4_interleave),
    // or null; read by the matrix-core GEMV where it has a form for them
    const uint32_t *sb = nullptr;
    // the words tiled in the matrix-core GEMV's task order (fh_q4_tile;
    // [gate; up] weights with the SiLU pairing), or null; read together with
    // sb by the matrix-core GEMV
    const uint32_t *wt = nullptr;
};

template <int M, int L, int CPL, bool FULL, int PRO, int EPI, bool SB>
inline void launch_gemv_full(hipStream_t stream, uint32_t cus, const GemvArgs &a) {
    constexpr uint32_t kRowsPerWave = 64 / L;
    constexpr uint32_t kOutRows = EPI == kEpiSiluMul ? kRowsPerWave / 2 : kRowsPerWave;
    auto kernel = q4_gemv_kernel<M, L, CPL, FULL, PRO, EPI, SB>;
    const uint32_t lds = gemv_lds_bytes(M, a.k, PRO == kProRmsNorm);
    const uint32_t n_out = EPI == kEpiSiluMul ? a.n / 2 : a.n;
    const uint32_t groups = (n_out + kOutRows - 1) / kOutRows;
    const uint32_t need = (groups + kGemvWaves - 1) / kGemvWaves;
    const uint32_t cap = cus * resident_blocks(kernel, lds);
    const uint32_t blocks = need < cap ? need : cap;
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kGemvThreads), lds, stream, a.x, a.x_ld, a.wq, a.s, a.b, a.sb,
                       a.n, a.k, a.y, a.y_ld, a.y_is_f32, a.fu);
}

// The interleaved scale/bias table (a.sb) is read by the one-row
// single-segment kernels, the decoder's batch-1 step.
template <int M, int L, int CPL, int PRO, int EPI>
inline void launch_gemv_fused(hipStream_t stream, uint32_t cus, const GemvArgs &a) {
    const uint32_t chunks = a.k / 32;
    if (chunks > 0 && chunks % (CPL * L) == 0) {
        if constexpr (M == 1) {
            if (a.sb != nullptr && (reinterpret_cast<uintptr_t>(a.sb) & 7u) == 0 && a.k % (2 * kGroup) == 0) {
                launch_gemv_full<M, L, CPL, true, PRO, EPI, true>(stream, cus, a);
                return;
            }
        }
        launch_gemv_full<M, L, CPL, true, PRO, EPI, false>(stream, cus, a);
    } else {
        launch_gemv_full<M, L, CPL, false, PRO, EPI, false>(stream, cus, a);
    }
}

template <int M, int L, int CPL>
inline void launch_gemv_mlc(hipStream_t stream, uint32_t cus, const GemvArgs &a) {
    if constexpr (L <= 32) {  // the SiLU epilogue needs two rows per wavefront
        if (a.epi == kEpiSiluMul) {
            if (a.pro == kProRmsNorm)
                launch_gemv_fused<M, L, CPL, kProRmsNorm, kEpiSiluMul>(stream, cus, a);
            else
                launch_gemv_fused<M, L, CPL, kProNone, kEpiSiluMul>(stream, cus, a);
            return;
        }
    }
    if (a.pro == kProRmsNorm)
        launch_gemv_fused<M, L, CPL, kProRmsNorm, kEpiNone>(stream, cus, a);
    else
        launch_gemv_fused<M, L, CPL, kProNone, kEpiNone>(stream, cus, a);
}

// (lanes per row, chunks per lane) shapes the kernels are built for; X lists
// them for the per-row-count translation units and the dispatcher.
#define FH_GEMV_SHAPES(X) \
    X(16, 2) X(16, 4) X(16, 6) X(16, 8) X(32, 3) X(32, 4) X(32, 8) X(64, 2) X(64, 4) X(64, 7) X(64, 8)

// Defined in q4_gemv_m<M>.hip: launches the M-row GEMV with the given shape.
template <int M>
void launch_gemv_m(uint32_t lanes, uint32_t cpl, hipStream_t stream, uint32_t cus, const GemvArgs &a);

}  // namespace fh
