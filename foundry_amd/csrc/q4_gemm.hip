// q4 prefill GEMM: Y[m, r] = sum_j X[m, j] * RNE_bf16(s[r, j/64] * q[r, j] + b[r, j/64])
// Replaces matmul_tiled (src/metal/kernels/matmul.metal:29-65) behind
// Linear::forward (src/nn/linear.rs:22-35) for prompt-length row counts.
//
// Compute-bound (about 1700 FLOP per HBM byte at the Llama-3.2-3B MLP shape).
// Design for CDNA4:
// - Block tile 128 (rows of X) x 128 (weight rows), K step 64 = one
//   quantisation group, 256 threads = 4 wavefronts in a 2 x 2 arrangement,
//   each owning a 64 x 64 output tile computed with 2 x 2
//   v_mfma_f32_32x32x16_bf16 tiles (fp32 accumulation).
// - Each K step the block loads the X tile (16-byte loads) and the packed
//   weight tile (one 16-byte load of 32 nibbles per thread), dequantises the
//   weights in registers to bf16 (v_cvt_pk_bf16_f32, round to nearest even,
//   the same value fh_q4_dequant materialises) and writes both to LDS with a
//   row pitch of 72 bf16 so the 16-byte fragment reads are conflict-free.
// - Global loads for step i+1 are issued before the MFMAs of step i.
#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

constexpr int kGemmThreads = 256;
constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;  // bf16 elements per LDS row

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// 8 weights of one packed word -> 4 dwords of bf16 pairs, natural order.
__device__ __forceinline__ void dequant_word(uint32_t w, float s, float b, uint32_t out[4]) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const float lo = q4_dequant_fma(s, (w >> (8 * p)) & 0xFu, b);
        const float hi = q4_dequant_fma(s, (w >> (8 * p + 4)) & 0xFu, b);
        out[p] = pack_bf16x2(lo, hi);
    }
}

__global__ __launch_bounds__(kGemmThreads) void q4_gemm_kernel(
    const uint16_t *__restrict__ x, uint32_t x_ld, const uint32_t *__restrict__ wq,
    const uint16_t *__restrict__ scales, const uint16_t *__restrict__ biases, uint32_t m,
    uint32_t n, uint32_t k, void *__restrict__ y, int y_is_f32) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[kBM * kPitch];
    __shared__ __attribute__((aligned(16))) uint16_t ws[kBN * kPitch];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = blockIdx.y * kBM;
    const uint32_t n0 = blockIdx.x * kBN;
    const uint32_t kw = k / 8;         // words per weight row
    const uint32_t kg = k / kGroup;    // groups per weight row

    // X tile: 128 rows x 8 sixteen-byte pieces; thread t loads pieces t + 256 i
    uint4 xr[4];
    // W tile: 128 rows x 2 sixteen-byte pieces; thread t loads one
    const uint32_t w_row = tid >> 1, w_half = tid & 1;
    const bool w_valid = n0 + w_row < n;
    const uint64_t w_row_g = w_valid ? n0 + w_row : 0;
    uint4 wr;
    uint32_t sr, br;

    auto load_tiles = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t idx = tid + kGemmThreads * i;
            const uint32_t r = idx >> 3, piece = idx & 7;
            if (m0 + r < m)
                xr[i] = *reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(m0 + r) * x_ld + k0 + piece * 8);
            else
                xr[i] = make_uint4(0u, 0u, 0u, 0u);
        }
        wr = *reinterpret_cast<const uint4 *>(wq + w_row_g * kw + k0 / 8 + w_half * 4);
        sr = scales[w_row_g * kg + k0 / kGroup];
        br = biases[w_row_g * kg + k0 / kGroup];
    };

    auto store_tiles = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t idx = tid + kGemmThreads * i;
            const uint32_t r = idx >> 3, piece = idx & 7;
            *reinterpret_cast<uint4 *>(&xs[r * kPitch + piece * 8]) = xr[i];
        }
        uint4 *dst = reinterpret_cast<uint4 *>(&ws[w_row * kPitch + w_half * 32]);
        if (w_valid) {
            const float s = bf16_to_f32(sr), b = bf16_to_f32(br);
            const uint32_t words[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) {
                uint32_t o[4];
                dequant_word(words[wi], s, b, o);
                dst[wi] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        } else {
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) dst[wi] = make_uint4(0u, 0u, 0u, 0u);
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const uint32_t frag_row = lane & 31;
    const uint32_t frag_k = (lane >> 5) * 8;

    if (k > 0) load_tiles(0);
    for (uint32_t k0 = 0; k0 < k; k0 += kBK) {
        __syncthreads();  // previous step's fragment reads are done
        store_tiles();
        __syncthreads();
        if (k0 + kBK < k) load_tiles(k0 + kBK);
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            bf16x8_t a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const bf16x8_t *>(
                    &xs[(wm * 64 + i * 32 + frag_row) * kPitch + kk + frag_k]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const bf16x8_t *>(
                    &ws[(wn * 64 + j * 32 + frag_row) * kPitch + kk + frag_k]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }

    // 32x32 accumulator layout: register r of lane l holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t col = n0 + wn * 64 + j * 32 + (lane & 31);
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                if (row >= m) continue;
                const uint64_t o = static_cast<uint64_t>(row) * n + col;
                if (y_is_f32)
                    static_cast<float *>(y)[o] = acc[i][j][r];
                else
                    static_cast<uint16_t *>(y)[o] = static_cast<uint16_t>(f32_to_bf16_rne(acc[i][j][r]));
            }
        }
}

void launch_q4_gemm(hipStream_t stream, const uint16_t *x, uint32_t x_ld, const uint32_t *wq,
                    const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n, uint32_t k,
                    void *y, int y_is_f32) {
    dim3 grid((n + kBN - 1) / kBN, (m + kBM - 1) / kBM);
    hipLaunchKernelGGL(q4_gemm_kernel, grid, dim3(kGemmThreads), 0, stream, x, x_ld, wq, s, b, m,
                       n, k, y, y_is_f32);
}

}  // namespace fh
