// q4 embedding gather and materialised dequantisation.
//
// Replaces index_select_rows (src/metal/kernels/index_select.metal:11-29),
// which Embedding::forward (src/nn/linear.rs:53-69) reaches through
// Op::IndexSelect, for a q4 table: each selected row is unpacked and
// dequantised to bf16; an id >= rows writes a zero row, as the reference does.
//
// The work is HBM-bound and write-dominated (per 8 elements: 4 bytes of
// nibbles in, 16 bytes of bf16 out). One thread handles one packed word: a
// 4-byte load and a 16-byte store, both coalesced across the wavefront, so
// a wave reads 256 contiguous bytes of a table row and writes 1 KiB of
// contiguous output.
#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

constexpr int kEmbedThreads = 256;

// grid.x covers the words of a row, grid.y strides over the selected rows.
// ids == nullptr selects row i for output row i (materialised dequant).
__global__ __launch_bounds__(kEmbedThreads) void q4_rows_kernel(
    const uint32_t *__restrict__ wq, const uint16_t *__restrict__ scales,
    const uint16_t *__restrict__ biases, uint32_t rows, uint32_t words_per_row,
    uint32_t groups_per_row, const uint32_t *__restrict__ ids, uint32_t n_out,
    uint4 *__restrict__ out) {
    const uint32_t j = blockIdx.x * kEmbedThreads + threadIdx.x;  // word in row
    if (j >= words_per_row) return;
    const uint32_t g = j / (kGroup / 8);
    for (uint32_t i = blockIdx.y; i < n_out; i += gridDim.y) {
        const uint32_t id = ids ? ids[i] : i;
        uint4 o = make_uint4(0u, 0u, 0u, 0u);
        if (id < rows) {
            const uint64_t row = id;
            const uint32_t w = wq[row * words_per_row + j];
            const float s = bf16_to_f32(scales[row * groups_per_row + g]);
            const float b = bf16_to_f32(biases[row * groups_per_row + g]);
            uint32_t h[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = f32_to_bf16_rne(q4_dequant(s, (w >> (4 * e)) & 0xFu, b));
            o.x = h[0] | (h[1] << 16);
            o.y = h[2] | (h[3] << 16);
            o.z = h[4] | (h[5] << 16);
            o.w = h[6] | (h[7] << 16);
        }
        out[static_cast<uint64_t>(i) * words_per_row + j] = o;
    }
}

// Rows of 64 * U words (k = 512 U: 3072 and 4096 for the BASELINE tables)
// when there are enough of them to give every CU a block: one wavefront per
// output row. Lane l takes words u * 64 + l (u < U), so each load reads 256
// contiguous bytes of the row and each store writes 1 KiB of output, and
// every load of the row (the id first, then words, scales and biases) is
// issued before any arithmetic: a wavefront waits for memory once, instead
// of once per word as in q4_rows_kernel, whose many short waves pay the load
// latency round after round (config 2, B = 4096: 9.5 -> 7.3 us). The rows
// are stored with the nontemporal hint, as a stream the caches need not keep
// (B = 4096: 7.06 -> 6.47 us cold, 6.56 -> 5.39 us warm; the same hint on
// the loads was slower). An id >= rows reads row 0 and writes zeros.
constexpr int kEmbedWaves = kEmbedThreads / 64;

template <int U>
__global__ __launch_bounds__(kEmbedThreads) void q4_rows_wave_kernel(
    const uint32_t *__restrict__ wq, const uint16_t *__restrict__ scales, const uint16_t *__restrict__ biases,
    uint32_t rows, const uint32_t *__restrict__ ids, uint32_t n_out, uint4 *__restrict__ out) {
    constexpr uint32_t W = U * 64, G = U * 8;  // words and groups per row
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t i = blockIdx.x * kEmbedWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (i >= n_out) return;  // uniform across the wavefront
    const uint32_t id = ids ? ids[i] : i;
    const bool live = id < rows;
    const uint64_t row = live ? id : 0u;
    uint32_t w[U], sv[U], bv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        w[u] = wq[row * W + u * 64 + lane];
        sv[u] = scales[row * G + u * 8 + lane / 8];
        bv[u] = biases[row * G + u * 8 + lane / 8];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const float s = bf16_to_f32(sv[u]), b = bf16_to_f32(bv[u]);
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            h[e] = f32x2_to_bf16x2_rne(q4_dequant(s, (w[u] >> (8 * e)) & 0xFu, b),
                                      q4_dequant(s, (w[u] >> (8 * e + 4)) & 0xFu, b));
        const stream_u32x4_t ov = live ? stream_u32x4_t{h[0], h[1], h[2], h[3]} : stream_u32x4_t{0u, 0u, 0u, 0u};
        __builtin_nontemporal_store(ov, reinterpret_cast<stream_u32x4_t *>(out + static_cast<uint64_t>(i) * W + u * 64 + lane));
    }
}

// Shared validation of the q4 table arguments.
int check_q4_table(const fh_device *dev, const char *fn, const uint32_t *wq,
                   const uint16_t *scales, const uint16_t *biases, int64_t rows, int64_t k,
                   int64_t group) {
    if (rows < 0 || k < 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: negative shape rows=%lld k=%lld", fn,
                    (long long)rows, (long long)k);
    if (group != kGroup)
        return fail(FH_ERR_UNSUPPORTED, "%s: group %lld; the kernels implement group 64", fn,
                    (long long)group);
    if (k % kGroup != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: k=%lld is not a multiple of the group (64)",
                    fn, (long long)k);
    if (rows > 0x7FFFFFFFll || k > 0x7FFFFFFFll)
        return fail(FH_ERR_INDEX_TOO_LARGE, "%s: rows or k exceeds 2^31-1", fn);
    if (reinterpret_cast<uintptr_t>(wq) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: wq must be 16-byte aligned", fn);
    const uint64_t words = static_cast<uint64_t>(rows) * (k / 8);
    const uint64_t groups = static_cast<uint64_t>(rows) * (k / kGroup);
    if (int rc = check_range(dev, wq, words * 4, fn, "wq")) return rc;
    if (int rc = check_range(dev, scales, groups * 2, fn, "scales")) return rc;
    if (int rc = check_range(dev, biases, groups * 2, fn, "biases")) return rc;
    return FH_OK;
}

static int launch_rows(fh_device *dev, const char *fn, const uint32_t *wq,
                       const uint16_t *scales, const uint16_t *biases, int64_t rows, int64_t k,
                       const uint32_t *ids, int64_t n_out, uint16_t *out) {
    if (n_out == 0 || k == 0) return FH_OK;
    const uint32_t words = static_cast<uint32_t>(k / 8);
    // fewer rows than CUs x 4 (B = 64: 16 blocks) keep q4_rows_kernel's wider
    // grid: 2.75 against 2.89 us at B = 64. An empty table (rows == 0) also
    // takes q4_rows_kernel, which loads nothing for an id >= rows: the wave
    // kernel reads row 0 for such ids, and an empty table has no row 0.
    if (rows > 0 && words % 64 == 0 && (words / 64 == 6 || words / 64 == 8) &&
        n_out >= static_cast<int64_t>(kEmbedWaves) * dev->compute_units) {
        const uint32_t blocks = static_cast<uint32_t>((n_out + kEmbedWaves - 1) / kEmbedWaves);
        return dispatch(dev, fn, [&] {
            auto kernel = words / 64 == 6 ? q4_rows_wave_kernel<6> : q4_rows_wave_kernel<8>;
            hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kEmbedThreads), 0, dev->stream, wq, scales, biases,
                               static_cast<uint32_t>(rows), ids, static_cast<uint32_t>(n_out),
                               reinterpret_cast<uint4 *>(out));
        });
    }
    dim3 grid((words + kEmbedThreads - 1) / kEmbedThreads,
              static_cast<uint32_t>(n_out < 65535 ? n_out : 65535));
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(q4_rows_kernel, grid, dim3(kEmbedThreads), 0, dev->stream, wq, scales,
                           biases, static_cast<uint32_t>(rows), words,
                           static_cast<uint32_t>(k / kGroup), ids,
                           static_cast<uint32_t>(n_out), reinterpret_cast<uint4 *>(out));
    });
}

}  // namespace fh

using namespace fh;

extern "C" int fh_q4_embed(fh_device *dev, const uint32_t *wq, const uint16_t *scales,
                           const uint16_t *biases, int64_t rows, int64_t k, int64_t group,
                           const uint32_t *ids, int64_t n_ids, uint16_t *out) {
    const char *fn = "fh_q4_embed";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = check_q4_table(dev, fn, wq, scales, biases, rows, k, group)) return rc;
    if (n_ids < 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: n_ids=%lld", fn, (long long)n_ids);
    if (n_ids > 0x7FFFFFFFll) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: n_ids >= 2^31", fn);
    if (int rc = check_range(dev, ids, static_cast<uint64_t>(n_ids) * 4, fn, "ids")) return rc;
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: out must be 16-byte aligned", fn);
    if (int rc = check_range(dev, out, static_cast<uint64_t>(n_ids) * k * 2, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return launch_rows(dev, fn, wq, scales, biases, rows, k, ids, n_ids, out);
}

extern "C" int fh_q4_dequant(fh_device *dev, const uint32_t *wq, const uint16_t *scales,
                             const uint16_t *biases, int64_t rows, int64_t k, int64_t group,
                             uint16_t *out) {
    const char *fn = "fh_q4_dequant";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = check_q4_table(dev, fn, wq, scales, biases, rows, k, group)) return rc;
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: out must be 16-byte aligned", fn);
    if (int rc = check_range(dev, out, static_cast<uint64_t>(rows) * k * 2, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return launch_rows(dev, fn, wq, scales, biases, rows, k, nullptr, rows, out);
}
