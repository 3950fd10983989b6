// q4 decode GEMV: y[m, r] = sum_j x[m, j] * (s[r, j/64] * q[r, j] + b[r, j/64])
// for m < 8 rows of x. Replaces the M=1..8 use of matmul_tiled
// (src/metal/kernels/matmul.metal:29-65) behind Linear::forward
// (src/nn/linear.rs:22-35), where 15 of 16 thread rows idle at M=1.
//
// HBM-bound: per weight 0.5 byte of nibbles plus 4 bytes of scale+bias per 64.
// Design for CDNA4:
// - A lane owns 16-byte chunks (32 weights, half a group) of one weight row;
//   L lanes share a row, chunk c = sub + L*i, so each load instruction of an
//   L-lane row group reads 16*L contiguous bytes. Loads are software-pipelined
//   one batch of kBatch chunks ahead.
// - x is staged once per block into LDS, permuted so that the bf16 pair for
//   nibbles (e, e+4) of a word is one dword, and laid out [m][word-in-chunk]
//   [chunk] so neighbouring lanes read neighbouring 16 bytes (no bank
//   conflicts). Per-chunk sums of x are staged beside it.
// - Dequantisation in registers without conversions: (w >> 4t) & 0x000F000F
//   | 0x43004300 is a bf16 pair (128 + q_t, 128 + q_{t+4}), exact since q < 16;
//   v_dot2_f32_bf16 multiplies it with the x pair and accumulates in fp32.
//   Per chunk: sum_j x_j (s q_j + b) = s * d + (b - 128 s) * X, with
//   d = sum_j x_j (128 + q_j) and X = sum_j x_j.
// - Partial sums are reduced across the L lanes of a row with cross-lane
//   shuffles; one lane writes each output (bf16 RNE or fp32).
#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

constexpr int kGemvThreads = 256;
constexpr int kBatch = 4;
// Dynamic LDS one block may use for staged x (bytes).
constexpr uint32_t kGemvLdsLimit = 64 * 1024;

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Bytes of LDS the kernel needs for `m` rows of x with k columns.
__host__ __device__ constexpr uint32_t gemv_lds_bytes(uint32_t m, uint32_t k) {
    return m * (k / 32) * (4 * 16 + 4);
}

template <int M, int L>
__global__ __launch_bounds__(kGemvThreads) void q4_gemv_kernel(
    const uint16_t *__restrict__ x, uint32_t x_ld, const uint32_t *__restrict__ wq,
    const uint16_t *__restrict__ scales, const uint16_t *__restrict__ biases, uint32_t n,
    uint32_t k, void *__restrict__ y, uint32_t y_ld, int y_is_f32) {
    constexpr int kRowsPerWave = 64 / L;
    constexpr int kRowsPerBlock = (kGemvThreads / 64) * kRowsPerWave;
    extern __shared__ uint4 lds[];
    const uint32_t chunks = k / 32;
    uint4 *xs = lds;                                                // [M][4][chunks]
    float *xsum = reinterpret_cast<float *>(lds + M * 4 * chunks);  // [M][chunks]

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t sub = lane % L;
    const uint32_t row = blockIdx.x * kRowsPerBlock + wave * kRowsPerWave + lane / L;
    const bool valid = row < n;
    const uint32_t row_c = valid ? row : 0;  // clamped: invalid lanes load row 0, discard
    const uint4 *wrow = reinterpret_cast<const uint4 *>(wq + static_cast<uint64_t>(row_c) * (k / 8));
    const uint16_t *srow = scales + static_cast<uint64_t>(row_c) * (k / kGroup);
    const uint16_t *brow = biases + static_cast<uint64_t>(row_c) * (k / kGroup);

    // first batch of weights goes out before x is staged
    uint4 wv[kBatch];
    uint32_t sv[kBatch], bv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
        const uint32_t c = sub + u * L;
        if (c < chunks) {
            wv[u] = wrow[c];
            sv[u] = srow[c / 2];
            bv[u] = brow[c / 2];
        }
    }

    // stage x: one thread per (m, chunk): four 16-byte loads, permute, sum
    for (uint32_t t = threadIdx.x; t < M * chunks; t += kGemvThreads) {
        const uint32_t m = t / chunks, c = t % chunks;
        const uint4 *src = reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(m) * x_ld + c * 32);
        float sum = 0.f;
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
            const uint4 v = src[wi];  // (x0,x1) (x2,x3) (x4,x5) (x6,x7)
            uint4 p;
            p.x = (v.x & 0xFFFFu) | (v.z << 16);          // (x0, x4)
            p.y = (v.x >> 16) | (v.z & 0xFFFF0000u);      // (x1, x5)
            p.z = (v.y & 0xFFFFu) | (v.w << 16);          // (x2, x6)
            p.w = (v.y >> 16) | (v.w & 0xFFFF0000u);      // (x3, x7)
            xs[(m * 4 + wi) * chunks + c] = p;
            sum += bf16_to_f32(v.x & 0xFFFFu) + bf16_to_f32(v.x >> 16);
            sum += bf16_to_f32(v.y & 0xFFFFu) + bf16_to_f32(v.y >> 16);
            sum += bf16_to_f32(v.z & 0xFFFFu) + bf16_to_f32(v.z >> 16);
            sum += bf16_to_f32(v.w & 0xFFFFu) + bf16_to_f32(v.w >> 16);
        }
        xsum[m * chunks + c] = sum;
    }
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.f;

    for (uint32_t c0 = sub; c0 < chunks; c0 += kBatch * L) {
        // prefetch the next batch while this one is computed
        uint4 nw[kBatch];
        uint32_t ns[kBatch], nb[kBatch];
        const uint32_t c1 = c0 + kBatch * L;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const uint32_t c = c1 + u * L;
            if (c < chunks) {
                nw[u] = wrow[c];
                ns[u] = srow[c / 2];
                nb[u] = brow[c / 2];
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const uint32_t c = c0 + u * L;
            if (c < chunks) {
                const float s = bf16_to_f32(sv[u]);
                const float bc = fmaf(-128.f, s, bf16_to_f32(bv[u]));
                const uint32_t words[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
                uint32_t pr[4][4];
#pragma unroll
                for (int wi = 0; wi < 4; ++wi)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        pr[wi][t] = ((words[wi] >> (4 * t)) & 0x000F000Fu) | 0x43004300u;
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
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            wv[u] = nw[u];
            sv[u] = ns[u];
            bv[u] = nb[u];
        }
    }

#pragma unroll
    for (int m = 0; m < M; ++m) {
        float v = acc[m];
#pragma unroll
        for (int off = L / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        acc[m] = v;
    }
    if (valid && sub == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const uint64_t o = static_cast<uint64_t>(m) * y_ld + row;
            if (y_is_f32)
                static_cast<float *>(y)[o] = acc[m];
            else
                static_cast<uint16_t *>(y)[o] = static_cast<uint16_t>(f32_to_bf16_rne(acc[m]));
        }
    }
}

template <int M, int L>
static void launch_gemv_ml(hipStream_t stream, const uint16_t *x, uint32_t x_ld,
                           const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t n,
                           uint32_t k, void *y, uint32_t y_ld, int y_is_f32) {
    constexpr int kRowsPerBlock = (kGemvThreads / 64) * (64 / L);
    const uint32_t blocks = (n + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL((q4_gemv_kernel<M, L>), dim3(blocks), dim3(kGemvThreads),
                       gemv_lds_bytes(M, k), stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32);
}

template <int L>
static void launch_gemv_l(int m, hipStream_t stream, const uint16_t *x, uint32_t x_ld,
                          const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t n,
                          uint32_t k, void *y, uint32_t y_ld, int y_is_f32) {
    switch (m) {
        case 1: launch_gemv_ml<1, L>(stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); break;
        case 2: launch_gemv_ml<2, L>(stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); break;
        case 3: launch_gemv_ml<3, L>(stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); break;
        case 4: launch_gemv_ml<4, L>(stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); break;
        case 5: launch_gemv_ml<5, L>(stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); break;
        case 6: launch_gemv_ml<6, L>(stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); break;
        case 7: launch_gemv_ml<7, L>(stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); break;
        default: launch_gemv_ml<8, L>(stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); break;
    }
}

// Largest count of x rows whose staged copy fits the LDS budget at this k.
uint32_t gemv_rows_per_launch(uint32_t k) {
    const uint32_t per_row = gemv_lds_bytes(1, k);
    if (per_row == 0) return 8;
    uint32_t r = kGemvLdsLimit / per_row;
    return r > 8 ? 8 : r;
}

// Launches the GEMV for m in [1, 8] rows of x whose staged copy fits LDS;
// the caller splits larger m (see gemv_rows_per_launch).
void launch_q4_gemv(hipStream_t stream, int m, const uint16_t *x, uint32_t x_ld,
                    const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t n,
                    uint32_t k, void *y, uint32_t y_ld, int y_is_f32) {
    const uint32_t chunks = k / 32;
    if (chunks <= 128)
        launch_gemv_l<16>(m, stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32);
    else if (chunks <= 256)
        launch_gemv_l<32>(m, stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32);
    else
        launch_gemv_l<64>(m, stream, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32);
}

}  // namespace fh
