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
