// q4 prefill GEMM: Y[m, r] = sum_j X[m, j] * RNE_bf16(s[r, j/64] * q[r, j] + b[r, j/64])
// Replaces matmul_tiled (src/metal/kernels/matmul.metal:29-65) behind
// Linear::forward (src/nn/linear.rs:22-35) for prompt-length row counts.
//
// Compute-bound (about 1700 FLOP per HBM byte at the Llama-3.2-3B MLP shape).
// Design for CDNA4:
// - Block tile 256 (rows of X) x 256 (weight rows), or 256 x 128 when the
//   larger tile would leave CUs idle; K step 64 = one quantisation group;
//   512 threads = 8 wavefronts (two per SIMD, so one wavefront's
//   dequantisation overlaps the other's MFMAs), 2 x 4 of 128 x 64 tiles
//   (4 x 2 accumulators of v_mfma_f32_32x32x16_bf16, fp32, 128 registers per
//   lane) or 4 x 2 of 64 x 64.
// - LDS holds two stages of both tiles (X and dequantised W, bf16, row pitch
//   72 so 16-byte fragment reads and writes are conflict-free): 144 KiB of the
//   CU's 160 KiB at 256 x 256. One barrier per K step: while step i is
//   computed from one stage, step i+1's global loads are in flight and then
//   written to the other.
// - Weights are dequantised in registers on the way to LDS: each thread owns
//   32 nibbles of one weight row for the step (inside one group: one scale and
//   bias), converts each nibble exactly (v_cvt_f32_ubyte), forms s*q + b with
//   one fma (equal to the materialised dequant whenever s*q is finite) and
//   rounds pairs to bf16 with v_cvt_pk_bf16_f32 (nearest even).
// - X rows past m load as zeros; W rows past n read weight row 0. Either
//   way they only feed outputs that are never stored. (A branch-free clamp
//   of the row index measured 35% slower: the select and 64-bit multiply sit
//   on every load's address.)
#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;  // bf16 elements per LDS row

// Block tile BM x BN, WM x WN wavefronts each owning (BM/WM) x (BN/WN).
template <int BM, int BN, int WM, int WN>
struct GemmTile {
    static constexpr int kThreads = 64 * WM * WN;
    static constexpr int kXElems = BM * kPitch, kWElems = BN * kPitch;  // one stage
    static constexpr uint32_t kLds = 2u * (kXElems + kWElems) * 2u;      // 2 stages, bytes
    static constexpr int TI = BM / WM / 32, TJ = BN / WN / 32;           // 32x32 MFMA tiles per wavefront
    static constexpr int kXPieces = BM * kBK / 8 / kThreads;             // 16-byte X pieces per thread
    // 16-byte W pieces per thread; with fewer pieces than threads, the first
    // BN * 2 threads (whole wavefronts) stage one each
    static constexpr int kWPieces = BN * 2 >= kThreads ? BN * 2 / kThreads : 1;
    static constexpr int kWThreads = BN * 2 >= kThreads ? kThreads : BN * 2;
    static_assert(kXPieces >= 1 && BM * kBK / 8 % kThreads == 0 && BN * 2 % kWThreads == 0 && kWThreads % 64 == 0,
                  "every staging thread stages whole pieces");
};

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// Byte i of v as a float (one v_cvt_f32_ubyte<i>).
template <int I>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
    return static_cast<float>((v >> (8 * I)) & 0xFFu);
}

// 8 weights of one packed word -> 4 dwords of bf16 pairs, natural order.
__device__ __forceinline__ uint4 dequant_word(uint32_t w, float s, float b) {
    const uint32_t lo = w & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6 in bytes 0..3
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
    uint4 o;
    o.x = pack_bf16x2(fmaf(s, ubyte_f32<0>(lo), b), fmaf(s, ubyte_f32<0>(hi), b));
    o.y = pack_bf16x2(fmaf(s, ubyte_f32<1>(lo), b), fmaf(s, ubyte_f32<1>(hi), b));
    o.z = pack_bf16x2(fmaf(s, ubyte_f32<2>(lo), b), fmaf(s, ubyte_f32<2>(hi), b));
    o.w = pack_bf16x2(fmaf(s, ubyte_f32<3>(lo), b), fmaf(s, ubyte_f32<3>(hi), b));
    return o;
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void q4_gemm_kernel(
    const uint16_t *__restrict__ x, uint32_t x_ld, const uint32_t *__restrict__ wq,
    const uint16_t *__restrict__ scales, const uint16_t *__restrict__ biases, uint32_t m,
    uint32_t n, uint32_t k, void *__restrict__ y, int y_is_f32) {
    using T = GemmTile<BM, BN, WM, WN>;
    constexpr int kGemmThreads = T::kThreads, TI = T::TI, TJ = T::TJ;
    constexpr int kXPieces = T::kXPieces, kWPieces = T::kWPieces;
    constexpr int kBM = BM, kBN = BN;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    uint16_t *const xs0 = smem;
    uint16_t *const ws0 = smem + T::kXElems;
    uint16_t *const xs1 = smem + T::kXElems + T::kWElems;
    uint16_t *const ws1 = smem + 2 * T::kXElems + T::kWElems;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = tid >> 6;
    const uint32_t wm = wave / WN, wn = wave % WN;
    const uint32_t m0 = blockIdx.y * kBM;
    const uint32_t n0 = blockIdx.x * kBN;
    const uint32_t kw = k / 8;       // words per weight row
    const uint32_t kg = k / kGroup;  // groups per weight row
    // K split blockIdx.z of gridDim.z: K steps [st0, st0 + steps); y then
    // takes this split's f32 partial tile at [blockIdx.z][m][n]
    const uint32_t steps_all = k / kBK;
    const uint32_t per_split = (steps_all + gridDim.z - 1) / gridDim.z;
    const uint32_t st0 = blockIdx.z * per_split < steps_all ? blockIdx.z * per_split : steps_all;
    const uint32_t steps = st0 + per_split < steps_all ? per_split : steps_all - st0;
    if (gridDim.z > 1) y = static_cast<float *>(y) + static_cast<uint64_t>(blockIdx.z) * m * n;

    // One K step in registers: X pieces (256 rows x 8 sixteen-byte pieces;
    // thread t holds pieces t + 512 i) and W pieces (256 rows x 2 sixteen-byte
    // pieces of 32 nibbles; thread t holds piece t) with the row's scale, bias.
    uint4 xr[kXPieces];
    uint4 wr[kWPieces];
    uint32_t sr[kWPieces], br[kWPieces];

    auto load_tiles = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < kXPieces; ++i) {
            const uint32_t idx = tid + kGemmThreads * i;
            const uint32_t r = idx >> 3, piece = idx & 7;
            if (m0 + r < m)
                xr[i] = *reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(m0 + r) * x_ld + k0 + piece * 8);
            else
                xr[i] = make_uint4(0u, 0u, 0u, 0u);
        }
        if (tid >= T::kWThreads) return;  // whole wavefronts
#pragma unroll
        for (int i = 0; i < kWPieces; ++i) {
            const uint32_t idx = tid + T::kWThreads * i;
            const uint32_t r = idx >> 1, half = idx & 1;
            const uint64_t row = n0 + r < n ? n0 + r : 0;
            wr[i] = reinterpret_cast<const uint4 *>(wq + row * kw + k0 / 8)[half];
            sr[i] = scales[row * kg + k0 / kGroup];
            br[i] = biases[row * kg + k0 / kGroup];
        }
    };

    auto store_tiles = [&](uint16_t *xs, uint16_t *ws) {
#pragma unroll
        for (int i = 0; i < kXPieces; ++i) {
            const uint32_t idx = tid + kGemmThreads * i;
            const uint32_t r = idx >> 3, piece = idx & 7;
            *reinterpret_cast<uint4 *>(&xs[r * kPitch + piece * 8]) = xr[i];
        }
        if (tid >= T::kWThreads) return;
#pragma unroll
        for (int i = 0; i < kWPieces; ++i) {
            const uint32_t idx = tid + T::kWThreads * i;
            const uint32_t r = idx >> 1, half = idx & 1;
            uint4 *dst = reinterpret_cast<uint4 *>(&ws[r * kPitch + half * 32]);
            const float s = bf16_to_f32(sr[i]), b = bf16_to_f32(br[i]);
            dst[0] = dequant_word(wr[i].x, s, b);
            dst[1] = dequant_word(wr[i].y, s, b);
            dst[2] = dequant_word(wr[i].z, s, b);
            dst[3] = dequant_word(wr[i].w, s, b);
        }
    };

    f32x16_t acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Fragment of lane l: row l%32 of a 32-row tile, k = kk + 8*(l/32) .. +8.
    const uint32_t frag_row = lane & 31;
    const uint32_t frag_k = (lane >> 5) * 8;

    auto compute = [&](const uint16_t *xs, const uint16_t *ws) {
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            bf16x8_t a[TI], b[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i)
                a[i] = *reinterpret_cast<const bf16x8_t *>(
                    &xs[(wm * TI * 32 + i * 32 + frag_row) * kPitch + kk + frag_k]);
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                b[j] = *reinterpret_cast<const bf16x8_t *>(
                    &ws[(wn * TJ * 32 + j * 32 + frag_row) * kPitch + kk + frag_k]);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    // Two LDS stages, one barrier per step.
    if (steps > 0) {
        load_tiles(st0 * kBK);
        store_tiles(xs0, ws0);
        __syncthreads();
    }
    for (uint32_t st = 0; st < steps; ++st) {
        const bool odd = st & 1;
        const bool more = st + 1 < steps;
        if (more) load_tiles((st0 + st + 1) * kBK);
        compute(odd ? xs1 : xs0, odd ? ws1 : ws0);
        if (more) store_tiles(odd ? xs0 : xs1, odd ? ws0 : ws1);
        __syncthreads();
    }

    // 32x32 accumulator layout: register r of lane l holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const uint32_t col = n0 + wn * TJ * 32 + j * 32 + (lane & 31);
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * TI * 32 + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                if (row >= m) continue;
                const uint64_t o = static_cast<uint64_t>(row) * n + col;
                if (y_is_f32)
                    static_cast<float *>(y)[o] = acc[i][j][r];
                else
                    static_cast<uint16_t *>(y)[o] = static_cast<uint16_t>(f32_to_bf16_rne(acc[i][j][r]));
            }
        }
}

template <int BM, int BN, int WM, int WN>
static void launch_gemm_tile(hipStream_t stream, const uint16_t *x, uint32_t x_ld, const uint32_t *wq,
                             const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n, uint32_t k, void *y,
                             int y_is_f32, uint32_t splits) {
    using T = GemmTile<BM, BN, WM, WN>;
    static bool lds_opt_in = false;
    if (!lds_opt_in) {
        // more than 64 KiB of dynamic LDS needs the kernel's opt-in
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(q4_gemm_kernel<BM, BN, WM, WN>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, T::kLds);
        lds_opt_in = true;
    }
    dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM, splits);
    hipLaunchKernelGGL((q4_gemm_kernel<BM, BN, WM, WN>), grid, dim3(T::kThreads), T::kLds, stream, x, x_ld, wq, s, b,
                       m, n, k, y, y_is_f32);
}

// Adds the f32 partials of a GEMM split over K in split order: y[i] =
// RNE(sum_s part[s][i]) (or the f32 sum). Each thread takes 4 consecutive
// outputs; its kMaxGemmSplits loads are issued before any add (clamped to
// the last split, whose extra values are not added).

__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float *__restrict__ part, uint32_t splits,
                                                                 uint64_t count, void *__restrict__ y,
                                                                 int y_is_f32) {
    const uint64_t i0 = (static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i0 >= count) return;
    if (count % 4 == 0) {  // every split's partial is then 16-byte aligned
        float4 v[kMaxGemmSplits];
#pragma unroll
        for (uint32_t sp = 0; sp < kMaxGemmSplits; ++sp)
            v[sp] = *reinterpret_cast<const float4 *>(part + static_cast<uint64_t>(sp < splits ? sp : splits - 1) * count + i0);
        float4 o = v[0];
#pragma unroll
        for (uint32_t sp = 1; sp < kMaxGemmSplits; ++sp)
            if (sp < splits) {
                o.x += v[sp].x;
                o.y += v[sp].y;
                o.z += v[sp].z;
                o.w += v[sp].w;
            }
        if (y_is_f32) {
            float *yf = static_cast<float *>(y) + i0;
            yf[0] = o.x;
            yf[1] = o.y;
            yf[2] = o.z;
            yf[3] = o.w;
        } else {
            uint16_t *yb = static_cast<uint16_t *>(y) + i0;
            yb[0] = static_cast<uint16_t>(f32_to_bf16_rne(o.x));
            yb[1] = static_cast<uint16_t>(f32_to_bf16_rne(o.y));
            yb[2] = static_cast<uint16_t>(f32_to_bf16_rne(o.z));
            yb[3] = static_cast<uint16_t>(f32_to_bf16_rne(o.w));
        }
        return;
    }
    for (uint64_t i = i0; i < i0 + 4 && i < count; ++i) {
        float o = part[i];
        for (uint32_t sp = 1; sp < splits; ++sp) o += part[static_cast<uint64_t>(sp) * count + i];
        if (y_is_f32)
            static_cast<float *>(y)[i] = o;
        else
            static_cast<uint16_t *>(y)[i] = static_cast<uint16_t>(f32_to_bf16_rne(o));
    }
}

// 256 x 256 tiles, or 256 x 128 when the larger tile leaves CUs idle: each
// weight element is still dequantised once per 256 rows of X, and the
// down-projection shape (2048 x 3072 x 8192) gets 192 blocks instead of 96
// (249 -> 186 us; the 2048 x 8192 x 3072 shape stays at 256 x 256, 139 us
// against 164). When even the small tiles leave more than half the CUs idle
// (prompt-length m such as 512 against n = 3072 or 5120), K is split over
// up to kMaxGemmSplits ranges so that tiles x splits about fills the chip;
// the splits' f32 partials go to `area` (kPartialAreaBytes) and
// gemm_split_reduce_kernel adds them in order. launch_q4_gemm_deferred stops
// before that add and returns the split count (1: y was written), so that a
// consumer of y can add the partials itself, in the same order.
uint32_t launch_q4_gemm_direct(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld,
                               const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n,
                               uint32_t k, void *y, int y_is_f32, void *area);

uint32_t launch_q4_gemm_deferred(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld,
                                 const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n,
                                 uint32_t k, void *y, int y_is_f32, void *area) {
    const uint64_t big = static_cast<uint64_t>((n + 255) / 256) * ((m + 255) / 256);
    // 256 x 256 tiles fill the chip, or 3/4 of it over two K ranges: weights
    // straight to the matrix cores (q4_gemm_direct.hip)
    if (const uint32_t d = launch_q4_gemm_direct(stream, cus, x, x_ld, wq, s, b, m, n, k, y, y_is_f32, area)) return d;
    if (big >= cus) {
        launch_gemm_tile<256, 256, 2, 4>(stream, x, x_ld, wq, s, b, m, n, k, y, y_is_f32, 1);
        return 1;
    }
    const uint64_t tiles = static_cast<uint64_t>((n + 127) / 128) * ((m + 255) / 256);
    const uint64_t steps = k / kBK;
    uint64_t splits = 1;
    if (area != nullptr && 2 * tiles <= cus) {
        splits = cus / tiles;
        if (splits > kMaxGemmSplits) splits = kMaxGemmSplits;
        if (splits > steps / 4) splits = steps / 4;  // at least 4 K steps per split
        while (splits > 1 && splits * m * n * 4 > kPartialAreaBytes) --splits;
        if (splits < 1) splits = 1;
    }
    if (splits == 1) {
        launch_gemm_tile<256, 128, 4, 2>(stream, x, x_ld, wq, s, b, m, n, k, y, y_is_f32, 1);
        return 1;
    }
    launch_gemm_tile<256, 128, 4, 2>(stream, x, x_ld, wq, s, b, m, n, k, area, 1, static_cast<uint32_t>(splits));
    return static_cast<uint32_t>(splits);
}

void launch_q4_gemm(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld, const uint32_t *wq,
                    const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n, uint32_t k, void *y,
                    int y_is_f32, void *area) {
    const uint32_t splits = launch_q4_gemm_deferred(stream, cus, x, x_ld, wq, s, b, m, n, k, y, y_is_f32, area);
    if (splits == 1) return;
    const uint64_t count = static_cast<uint64_t>(m) * n;
    const uint64_t blocks = (count + 1023) / 1024;
    hipLaunchKernelGGL(gemm_split_reduce_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream,
                       static_cast<const float *>(area), splits, count, y, y_is_f32);
}

}  // namespace fh
