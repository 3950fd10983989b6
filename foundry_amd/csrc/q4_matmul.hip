// fh_q4_matmul: validation and dispatch of the q4 Linear.
//
// Mirrors MetalDevice::matmul (src/metal/mod.rs:434-481): check the operands
// (src/nn/primitive.rs:234-256 for the shape rule), then pick the kernel. The
// reference has one tiled kernel for every shape; here m <= 8 goes to the
// decode GEMV and larger m to the MFMA GEMM.
#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

int check_q4_table(const fh_device *dev, const char *fn, const uint32_t *wq,
                   const uint16_t *scales, const uint16_t *biases, int64_t rows, int64_t k,
                   int64_t group);
void launch_q4_gemv(hipStream_t stream, uint32_t cus, int m, const uint16_t *x, uint32_t x_ld,
                    const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t n,
                    uint32_t k, void *y, uint32_t y_ld, int y_is_f32);
uint32_t gemv_rows_per_launch(uint32_t k);
void launch_q4_gemm(hipStream_t stream, const uint16_t *x, uint32_t x_ld, const uint32_t *wq,
                    const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n, uint32_t k,
                    void *y, int y_is_f32);

// Row counts up to this go to the GEMV.
constexpr int64_t kGemvMaxRows = 8;

}  // namespace fh

using namespace fh;

extern "C" int fh_q4_matmul(fh_device *dev, const uint16_t *x, int64_t m, int64_t k,
                            int64_t x_ld, const uint32_t *wq, const uint16_t *scales,
                            const uint16_t *biases, int64_t n, int64_t group, void *y,
                            int y_dtype) {
    const char *fn = "fh_q4_matmul";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = check_q4_table(dev, fn, wq, scales, biases, n, k, group)) return rc;
    if (m < 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: m=%lld", fn, (long long)m);
    if (m > 65535ll * 128) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: m > 65535*128 rows", fn);
    if (y_dtype != FH_BF16 && y_dtype != FH_F32)
        return fail(FH_ERR_DTYPE, "%s: y_dtype must be FH_BF16 or FH_F32", fn);
    if (x_ld < k)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: x_ld=%lld < k=%lld", fn, (long long)x_ld,
                    (long long)k);
    if (x_ld % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT,
                    "%s: x must be 16-byte aligned with a row stride that is a multiple of 8", fn);
    if (x_ld > 0x7FFFFFFFll) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: x_ld >= 2^31", fn);
    const int y_is_f32 = y_dtype == FH_F32;
    if (reinterpret_cast<uintptr_t>(y) % (y_is_f32 ? 4 : 2) != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: y is misaligned for its dtype", fn);
    if (m == 0 || n == 0) return FH_OK;
    const uint64_t x_bytes = (static_cast<uint64_t>(m - 1) * x_ld + k) * 2;
    if (int rc = check_range(dev, x, x_bytes, fn, "x")) return rc;
    const uint64_t y_bytes = static_cast<uint64_t>(m) * n * (y_is_f32 ? 4 : 2);
    if (int rc = check_range(dev, y, y_bytes, fn, "y")) return rc;
    if (int rc = set_current(dev, fn)) return rc;

    const uint32_t k32 = static_cast<uint32_t>(k), n32 = static_cast<uint32_t>(n);
    const uint32_t ld32 = static_cast<uint32_t>(x_ld);
    if (m <= kGemvMaxRows) {
        // x rows whose staged copy fits LDS go in one launch; the rest follow
        const int64_t per = gemv_rows_per_launch(k32);
        if (per < 1)
            return fail(FH_ERR_UNSUPPORTED, "%s: k=%lld is too large for the GEMV's LDS stage", fn,
                        (long long)k);
        for (int64_t r0 = 0; r0 < m; r0 += per) {
            const int rows = static_cast<int>(m - r0 < per ? m - r0 : per);
            const uint16_t *xr = x + r0 * x_ld;
            void *yr = y_is_f32 ? static_cast<void *>(static_cast<float *>(y) + r0 * n)
                                : static_cast<void *>(static_cast<uint16_t *>(y) + r0 * n);
            int rc = dispatch(dev, fn, [&] {
                launch_q4_gemv(dev->stream, dev->compute_units, rows, xr, ld32, wq, scales, biases, n32, k32, yr, n32,
                               y_is_f32);
            });
            if (rc) return rc;
        }
        return FH_OK;
    }
    return dispatch(dev, fn, [&] {
        launch_q4_gemm(dev->stream, x, ld32, wq, scales, biases, static_cast<uint32_t>(m), n32,
                       k32, y, y_is_f32);
    });
}
