// fh_q4_matmul: validation and dispatch of the q4 Linear.
//
// Mirrors MetalDevice::matmul (src/metal/mod.rs:434-481): check the operands
// (src/nn/primitive.rs:234-256 for the shape rule), then pick the kernel. The
// reference has one tiled kernel for every shape; here m <= 8 goes to the
// decode GEMV and larger m to the MFMA GEMM.
#include "q4_gemv_mfma.hpp"

namespace fh {

int check_q4_table(const fh_device *dev, const char *fn, const uint32_t *wq,
                   const uint16_t *scales, const uint16_t *biases, int64_t rows, int64_t k,
                   int64_t group);
void launch_q4_gemv(hipStream_t stream, uint32_t cus, int m, const GemvArgs &a);
void launch_q4_gemv_mfma(hipStream_t stream, uint32_t cus, int m, const GemvArgs &a);
void launch_mf_pack(hipStream_t stream, int m, const GemvArgs &a, void *area, const float *part = nullptr,
                    uint32_t ranges = 0);
uint32_t gemv_rows_per_launch(uint32_t k, bool norm);
void launch_q4_gemm(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld, const uint32_t *wq,
                    const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n, uint32_t k,
                    void *y, int y_is_f32, void *area);
bool launch_q4_gemm_direct_silu(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld,
                                const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t f,
                                uint32_t k, uint16_t *act);

// Row counts up to this go to the GEMV.
constexpr int64_t kGemvMaxRows = 8;

// Launches the GEMV over m rows in groups whose staged x fits LDS (every
// prologue and epilogue is row-independent): the matrix-core kernel for
// groups of 2..8 rows where it takes the shape (after the pack kernel for
// RMSNorm rows), else the dot2 kernel; x, res, res_out and y advance by their
// row strides. y_cols: columns of y per row.
// Ranges of K a matrix-core GEMV may be split into (partial sums per range).
// x bytes per block the range count aims at (each block stages its range of
// every x row).
constexpr uint32_t kMfRangeXBytes = 32 * 1024;

// Adds the K-range partial sums [ranges][rows][n] of a split GEMV in range
// order (4 outputs per thread, every range's load issued first) and writes y
// (RNE to bf16, or f32).
__global__ __launch_bounds__(256) void mf_combine_kernel(const float *__restrict__ part, uint32_t ranges,
                                                         uint32_t rows, uint32_t n, void *__restrict__ y,
                                                         uint32_t y_ld, int y_is_f32) {
    const uint32_t i = (blockIdx.x * 256 + threadIdx.x) * 4;
    const uint32_t ic = i < rows * n ? i : 0u;
    const uint32_t m = ic / n, c = ic % n;
    float4 q[kMfMaxRanges];
#pragma unroll
    for (uint32_t r = 0; r < kMfMaxRanges; ++r)
        q[r] = *reinterpret_cast<const float4 *>(part + (static_cast<uint64_t>(r < ranges ? r : 0u) * rows + m) * n + c);
    float4 v = q[0];
#pragma unroll
    for (uint32_t r = 1; r < kMfMaxRanges; ++r)
        if (r < ranges) v = make_float4(v.x + q[r].x, v.y + q[r].y, v.z + q[r].z, v.w + q[r].w);
    if (i >= rows * n) return;
    const uint64_t o = static_cast<uint64_t>(m) * y_ld + c;
    if (y_is_f32) {
        float *yo = static_cast<float *>(y) + o;
        yo[0] = v.x, yo[1] = v.y, yo[2] = v.z, yo[3] = v.w;
    } else {
        uint16_t *yo = static_cast<uint16_t *>(y) + o;
        yo[0] = static_cast<uint16_t>(f32_to_bf16_rne(v.x));
        yo[1] = static_cast<uint16_t>(f32_to_bf16_rne(v.y));
        yo[2] = static_cast<uint16_t>(f32_to_bf16_rne(v.z));
        yo[3] = static_cast<uint16_t>(f32_to_bf16_rne(v.w));
    }
}

// K ranges for m plain rows whose x does not fit LDS over the whole row:
// ranges of a multiple of 512 values (every range's scale and bias rows
// start 16-byte aligned) that hold all m rows, preferring the fewest whose
// staged x is at most kMfRangeXBytes, else the fewest that fit; 0 if none.
static uint32_t mf_k_ranges(fh_device *dev, int64_t m, const GemvArgs &a) {
    if (a.pro != kProNone || a.epi != kEpiNone || a.n % 4 != 0) return 0;
    for (int pass = 0; pass < 2; ++pass) {
        for (uint32_t r = 2; r <= kMfMaxRanges; ++r) {
            if (a.k % (r * 512) != 0) continue;
            const uint32_t kp = a.k / r;
            if (pass == 0 && static_cast<uint64_t>(kp) * m * 2 > kMfRangeXBytes) continue;
            if (static_cast<uint64_t>(r) * m * a.n * 4 > kPartialAreaBytes) continue;
            const uint32_t cus = dev->compute_units / r > 0 ? dev->compute_units / r : 1;
            if (mf_rows_per_launch(kp) >= m && pick_mf_split(a.n / 16, kp / kGroup, cus) != 0) return r;
        }
    }
    return 0;
}

int launch_gemv_rows(fh_device *dev, const char *fn, int64_t m, const GemvArgs &base, int64_t y_cols) {
    const bool mf = m >= 2 && mf_eligible(static_cast<uint32_t>(m), base);
    const int64_t per = mf ? mf_rows_per_launch(base.k)
                           : gemv_rows_per_launch(base.k, base.pro == kProRmsNorm);
    if (mf && per < m) {
        // all rows over K ranges instead of row groups over all of K: the
        // weights are read once, each block stages one range of x, and the
        // combine kernel adds the ranges' f32 sums (the device's partial area)
        if (const uint32_t ranges = mf_k_ranges(dev, m, base)) {
            GemvArgs a = base;
            a.k = base.k / ranges;
            a.kranges = ranges;
            a.y = dev->partial_area;
            a.y_is_f32 = 1;
            a.y_ld = base.n;
            if (int rc = dispatch(dev, fn, [&] {
                    launch_q4_gemv_mfma(dev->stream, dev->compute_units, static_cast<int>(m), a);
                }))
                return rc;
            const uint32_t outs = static_cast<uint32_t>(m) * base.n;
            return dispatch(dev, fn, [&] {
                hipLaunchKernelGGL(mf_combine_kernel, dim3((outs / 4 + 255) / 256), dim3(256), 0, dev->stream,
                                   static_cast<const float *>(dev->partial_area), ranges, static_cast<uint32_t>(m),
                                   base.n, base.y, static_cast<uint32_t>(y_cols), base.y_is_f32);
            });
        }
    }
    for (int64_t r0 = 0; r0 < m; r0 += per) {
        const int rows = static_cast<int>(m - r0 < per ? m - r0 : per);
        GemvArgs a = base;
        a.x += r0 * base.x_ld;
        if (a.fu.res) a.fu.res += r0 * base.k;
        if (a.fu.res_out) a.fu.res_out += r0 * base.k;
        a.y = base.y_is_f32 ? static_cast<void *>(static_cast<float *>(base.y) + r0 * y_cols)
                            : static_cast<void *>(static_cast<uint16_t *>(base.y) + r0 * y_cols);
        if (mf && rows >= 2 && a.pro == kProRmsNorm) {
            // RMSNorm rows: normalised once into the pack area, which the
            // matrix-core GEMV then takes as its x
            if (int rc = dispatch(dev, fn, [&] { launch_mf_pack(dev->stream, rows, a, dev->pack_area); })) return rc;
            a.x = static_cast<const uint16_t *>(dev->pack_area);
        }
        int rc = dispatch(dev, fn, [&] {
            if (mf && rows >= 2)
                launch_q4_gemv_mfma(dev->stream, dev->compute_units, rows, a);
            else
                launch_q4_gemv(dev->stream, dev->compute_units, rows, a);
        });
        if (rc) return rc;
    }
    return FH_OK;
}

// The batched decode step's down projection and the next RMSNorm'd GEMV's
// pack as one launch less: y = x W^T runs over K ranges into the partial
// area as fh_q4_matmul would run it, and the pack kernel then forms each row
// of y from the ranges' sums itself (no combine launch, no y in memory),
// adds the residual (h to res_out), normalises it with norm_weight and
// writes the image the next GEMV (next_n rows of w.n columns) reads, the
// same values fh_q4_matmul followed by fh_q4_matmul_rmsnorm's pack produce.
// *packed = false (nothing launched) when the shapes do not take that route:
// m outside 2..8, the down projection not split into K ranges, or the next
// GEMV not taking all m rows from one image.
int q4_down_pack(fh_device *dev, const char *fn, const uint16_t *x, int64_t m, int64_t x_ld, const uint32_t *wq,
                 const uint16_t *scales, const uint16_t *biases, const uint32_t *sb, const uint32_t *wt, int64_t n,
                 int64_t k, const uint16_t *res, uint16_t *res_out, const uint16_t *norm_weight, float eps,
                 const uint32_t *next_wq, const uint16_t *next_scales, const uint16_t *next_biases,
                 const uint32_t *next_sb, const uint32_t *next_wt, int64_t next_n, bool *packed) {
    *packed = false;
    if (m < 2 || m > 8 || k <= 0 || n <= 0 || n > kMfPackMaxK || x_ld > 0x7FFFFFFFll) return FH_OK;
    GemvArgs down{x, static_cast<uint32_t>(x_ld), wq, scales, biases, static_cast<uint32_t>(n),
                  static_cast<uint32_t>(k), nullptr, static_cast<uint32_t>(n), 1, kProNone, kEpiNone,
                  GemvFusion{}};
    down.sb = sb;
    down.wt = wt;
    if (!mf_eligible(static_cast<uint32_t>(m), down) || mf_rows_per_launch(down.k) >= m) return FH_OK;
    const uint32_t ranges = mf_k_ranges(dev, m, down);
    if (ranges == 0) return FH_OK;
    GemvArgs next{nullptr, static_cast<uint32_t>(n), next_wq, next_scales, next_biases, static_cast<uint32_t>(next_n),
                  static_cast<uint32_t>(n), nullptr, static_cast<uint32_t>(next_n), 0, kProRmsNorm, kEpiNone,
                  GemvFusion{}};
    next.sb = next_sb;
    next.wt = next_wt;
    if (!mf_eligible(static_cast<uint32_t>(m), next) || mf_rows_per_launch(next.k) < m) return FH_OK;
    for (const void *p : {static_cast<const void *>(x), static_cast<const void *>(res),
                          static_cast<const void *>(res_out), static_cast<const void *>(norm_weight)})
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return FH_OK;
    if (!norm_weight || (res_out && !res)) return FH_OK;
    const uint64_t row_bytes = static_cast<uint64_t>(m) * n * 2;
    if (int rc = check_range(dev, x, (static_cast<uint64_t>(m - 1) * x_ld + k) * 2, fn, "x")) return rc;
    if (res)
        if (int rc = check_range(dev, res, row_bytes, fn, "residual")) return rc;
    if (res_out)
        if (int rc = check_range(dev, res_out, row_bytes, fn, "residual_out")) return rc;
    if (int rc = check_range(dev, norm_weight, static_cast<uint64_t>(n) * 2, fn, "norm_weight")) return rc;
    GemvArgs a = down;
    a.k = down.k / ranges;
    a.kranges = ranges;
    a.y = dev->partial_area;
    a.y_is_f32 = 1;
    a.y_ld = down.n;
    if (int rc = dispatch(dev, fn, [&] { launch_q4_gemv_mfma(dev->stream, dev->compute_units, static_cast<int>(m), a); }))
        return rc;
    GemvArgs p{};
    p.k = static_cast<uint32_t>(n);
    p.fu = GemvFusion{res, res_out, norm_weight, eps, 1.0f / static_cast<float>(n)};
    if (int rc = dispatch(dev, fn, [&] {
            launch_mf_pack(dev->stream, static_cast<int>(m), p, dev->pack_area,
                           static_cast<const float *>(dev->partial_area), ranges);
        }))
        return rc;
    *packed = true;
    return FH_OK;
}

// The RMSNorm'd GEMV of m rows on the image q4_down_pack left in the pack
// area (weight [n, k], k the image's row length).
// Whether q4_gemv_packed takes m rows (2..8) of this weight from an image
// in the pack area: the matrix-core GEMV with the image prologue applies.
bool gemv_packed_applies(int64_t m, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                         const uint32_t *sb, const uint32_t *wt, int64_t n, int64_t k) {
    if (m < 2 || m > 8 || n <= 0 || k <= 0 || n > 0x7FFFFFFFll || k > kMfPackMaxK) return false;
    GemvArgs a{nullptr, static_cast<uint32_t>(k), wq, scales, biases, static_cast<uint32_t>(n),
               static_cast<uint32_t>(k), nullptr, static_cast<uint32_t>(n), 0, kProRmsNorm, kEpiNone, GemvFusion{}};
    a.sb = sb;
    a.wt = wt;
    return mf_eligible(static_cast<uint32_t>(m), a) && mf_rows_per_launch(a.k) >= m;
}

int q4_gemv_packed(fh_device *dev, const char *fn, int64_t m, const uint32_t *wq, const uint16_t *scales,
                   const uint16_t *biases, const uint32_t *sb, const uint32_t *wt, int64_t n, int64_t k, void *y,
                   int y_is_f32) {
    GemvArgs a{static_cast<const uint16_t *>(dev->pack_area), static_cast<uint32_t>(k), wq, scales, biases,
               static_cast<uint32_t>(n), static_cast<uint32_t>(k), y, static_cast<uint32_t>(n), y_is_f32,
               kProRmsNorm, kEpiNone, GemvFusion{}};
    a.sb = sb;
    a.wt = wt;
    if (int rc = check_range(dev, y, static_cast<uint64_t>(m) * n * (y_is_f32 ? 4 : 2), fn, "y")) return rc;
    return dispatch(dev, fn, [&] { launch_q4_gemv_mfma(dev->stream, dev->compute_units, static_cast<int>(m), a); });
}

// The interleaved scale/bias table of an n x k weight (fh_q4_interleave):
// null, or 16-byte aligned n * k / 64 dwords with k a multiple of 128.
int check_sb(fh_device *dev, const char *fn, const uint32_t *sb, int64_t n, int64_t k) {
    if (sb == nullptr) return FH_OK;
    if (k % (2 * kGroup) != 0 || reinterpret_cast<uintptr_t>(sb) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT,
                    "%s: an interleaved scale/bias table needs k %% 128 == 0 (k=%lld) and 16-byte alignment", fn,
                    (long long)k);
    return check_range(dev, sb, static_cast<uint64_t>(n) * (k / kGroup) * 4, fn, "interleaved scale/bias");
}

// The tiled words of an n x k weight (fh_q4_tile): null, or 16-byte aligned
// n * k / 8 words, n a multiple of 16 and k of 128; only with an
// interleaved scale/bias table.
int check_wt(fh_device *dev, const char *fn, const uint32_t *wt, const uint32_t *sb, int64_t n, int64_t k) {
    if (wt == nullptr) return FH_OK;
    if (sb == nullptr)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: tiled words need the interleaved scale/bias table too", fn);
    if (n % 16 != 0 || k % (2 * kGroup) != 0 || reinterpret_cast<uintptr_t>(wt) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT,
                    "%s: tiled words need n %% 16 == 0 (n=%lld), k %% 128 == 0 (k=%lld) and 16-byte alignment", fn,
                    (long long)n, (long long)k);
    return check_range(dev, wt, static_cast<uint64_t>(n) * (k / 8) * 4, fn, "tiled words");
}

// fh_q4_matmul with the weight's optional interleaved scale/bias table and
// tiled words (the words in plain row order).
int q4_matmul(fh_device *dev, const uint16_t *x, int64_t m, int64_t k, int64_t x_ld, const uint32_t *wq,
              const uint16_t *scales, const uint16_t *biases, const uint32_t *sb, const uint32_t *wt, int64_t n,
              int64_t group, void *y, int y_dtype) {
    const char *fn = "fh_q4_matmul";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = check_q4_table(dev, fn, wq, scales, biases, n, k, group)) return rc;
    if (int rc = check_sb(dev, fn, sb, n, k)) return rc;
    if (int rc = check_wt(dev, fn, wt, sb, n, k)) return rc;
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
    // an empty sum: every output is RNE(0) = 0, and no kernel may read x or W
    if (k == 0) return zero_fill(dev, fn, y, y_bytes);

    const uint32_t k32 = static_cast<uint32_t>(k), n32 = static_cast<uint32_t>(n);
    const uint32_t ld32 = static_cast<uint32_t>(x_ld);
    if (m <= kGemvMaxRows) {
        if (gemv_rows_per_launch(k32, false) < 1)
            return fail(FH_ERR_UNSUPPORTED, "%s: k=%lld is too large for the GEMV's LDS stage", fn,
                        (long long)k);
        GemvArgs a{x, ld32, wq, scales, biases, n32, k32, y, n32, y_is_f32, kProNone, kEpiNone, GemvFusion{}};
        a.sb = sb;
        a.wt = wt;
        return launch_gemv_rows(dev, fn, m, a, n);
    }
    return dispatch(dev, fn, [&] {
        launch_q4_gemm(dev->stream, dev->compute_units, x, ld32, wq, scales, biases, static_cast<uint32_t>(m), n32,
                       k32, y, y_is_f32, dev->partial_area);
    });
}

}  // namespace fh

using namespace fh;

extern "C" int fh_q4_matmul(fh_device *dev, const uint16_t *x, int64_t m, int64_t k,
                            int64_t x_ld, const uint32_t *wq, const uint16_t *scales,
                            const uint16_t *biases, int64_t n, int64_t group, void *y,
                            int y_dtype) {
    return q4_matmul(dev, x, m, k, x_ld, wq, scales, biases, nullptr, nullptr, n, group, y, y_dtype);
}

namespace {

// Checks shared by the fused decode entry points: the q4 table, at most
// kGemvMaxRows rows, y's dtype, alignment and range (y_cols columns).
int check_fused(fh_device *dev, const char *fn, int64_t m, int64_t k, const uint32_t *wq, const uint16_t *scales,
                const uint16_t *biases, int64_t n, int64_t group, void *y, int y_dtype, int64_t y_cols, bool norm) {
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = check_q4_table(dev, fn, wq, scales, biases, n, k, group)) return rc;
    if (m < 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: m=%lld", fn, (long long)m);
    if (m > kGemvMaxRows)
        return fail(FH_ERR_UNSUPPORTED, "%s: %lld rows; the fused GEMV takes at most %lld, use the unfused ops", fn,
                    (long long)m, (long long)kGemvMaxRows);
    if (gemv_rows_per_launch(static_cast<uint32_t>(k), norm) < 1)
        return fail(FH_ERR_UNSUPPORTED, "%s: k=%lld is too large for the GEMV's LDS stage", fn, (long long)k);
    if (y_dtype != FH_BF16 && y_dtype != FH_F32)
        return fail(FH_ERR_DTYPE, "%s: y_dtype must be FH_BF16 or FH_F32", fn);
    if (reinterpret_cast<uintptr_t>(y) % (y_dtype == FH_F32 ? 4 : 2) != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: y is misaligned for its dtype", fn);
    if (m == 0 || y_cols == 0) return FH_OK;
    return check_range(dev, y, static_cast<uint64_t>(m) * y_cols * (y_dtype == FH_F32 ? 4 : 2), fn, "y");
}

bool overlaps(const void *a, uint64_t na, const void *b, uint64_t nb) {
    const auto pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return a && b && pa < pb + nb && pb < pa + na;
}

}  // namespace

namespace {

// Validates the RMSNorm prologue's operands (norm_weight null: no norm).
int check_norm_operands(fh_device *dev, const char *fn, const uint16_t *x, const uint16_t *residual,
                        const uint16_t *residual_out, const uint16_t *norm_weight, int64_t m, int64_t k) {
    if (!norm_weight && (residual || residual_out))
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: a residual without a norm weight", fn);
    if (residual_out && !residual)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: residual_out without residual", fn);
    for (const void *p : {static_cast<const void *>(x), static_cast<const void *>(residual),
                          static_cast<const void *>(residual_out), static_cast<const void *>(norm_weight)})
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
            return fail(FH_ERR_INVALID_ARGUMENT, "%s: x, residual, residual_out and the weight must be 16-byte aligned",
                        fn);
    if (m == 0) return FH_OK;
    const uint64_t rows_bytes = static_cast<uint64_t>(m) * k * 2;
    if (int rc = check_range(dev, x, rows_bytes, fn, "x")) return rc;
    if (norm_weight) {
        if (int rc = check_range(dev, norm_weight, static_cast<uint64_t>(k) * 2, fn, "norm_weight")) return rc;
    }
    if (residual) {
        if (int rc = check_range(dev, residual, rows_bytes, fn, "residual")) return rc;
    }
    if (residual_out) {
        if (int rc = check_range(dev, residual_out, rows_bytes, fn, "residual_out")) return rc;
        // block 0 writes h while every block reads x and the residual
        if (overlaps(residual_out, rows_bytes, x, rows_bytes) || overlaps(residual_out, rows_bytes, residual, rows_bytes))
            return fail(FH_ERR_INVALID_ARGUMENT, "%s: residual_out overlaps x or residual", fn);
    }
    return FH_OK;
}

}  // namespace

namespace fh {

// fh_q4_matmul_rmsnorm with the weight's optional interleaved scale/bias
// table and tiled words (plain row order).
int q4_matmul_rmsnorm(fh_device *dev, const uint16_t *x, const uint16_t *residual, uint16_t *residual_out,
                      const uint16_t *norm_weight, float eps, int64_t m, int64_t k, const uint32_t *wq,
                      const uint16_t *scales, const uint16_t *biases, const uint32_t *sb, const uint32_t *wt,
                      int64_t n, int64_t group, void *y, int y_dtype) {
    const char *fn = "fh_q4_matmul_rmsnorm";
    if (int rc = check_fused(dev, fn, m, k, wq, scales, biases, n, group, y, y_dtype, n, true)) return rc;
    if (int rc = check_sb(dev, fn, sb, n, k)) return rc;
    if (int rc = check_wt(dev, fn, wt, sb, n, k)) return rc;
    if (!norm_weight) return fail(FH_ERR_INVALID_ARGUMENT, "%s: null norm weight", fn);
    if (int rc = check_norm_operands(dev, fn, x, residual, residual_out, norm_weight, m, k)) return rc;
    if (m == 0 || n == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    // empty rows: h and the normalised x are empty, y = x' W^T is zeros
    if (k == 0) return zero_fill(dev, fn, y, static_cast<uint64_t>(m) * n * (y_dtype == FH_F32 ? 4 : 2));
    const uint32_t k32 = static_cast<uint32_t>(k), n32 = static_cast<uint32_t>(n);
    GemvArgs a{x, k32, wq, scales, biases, n32, k32, y, n32, y_dtype == FH_F32, kProRmsNorm, kEpiNone,
               GemvFusion{residual, residual_out, norm_weight, eps, 1.0f / static_cast<float>(k)}};
    a.sb = sb;
    a.wt = wt;
    return launch_gemv_rows(dev, fn, m, a, n);
}

// fh_q4_gate_up_silu with the weight's optional interleaved scale/bias table
// and tiled words (in the SiLU pairing: fh_q4_tile with silu_pairs = 1).
// Prompt-length rows: the [gate; up] GEMM with the activation in its
// epilogue (launch_q4_gemm_direct_silu), where that kernel applies.
int gate_up_silu_gemm(fh_device *dev, const char *fn, const uint16_t *x, int64_t m, int64_t k, const uint32_t *wq,
                      const uint16_t *scales, const uint16_t *biases, int64_t n, int64_t group, uint16_t *act) {
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = check_q4_table(dev, fn, wq, scales, biases, n, k, group)) return rc;
    if (m > 65535ll * 128) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: m > 65535*128 rows", fn);
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(act) % 16 != 0 || k % 8 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: above %lld rows x and act must be 16-byte aligned and k %% 8 == 0",
                    fn, (long long)kGemvMaxRows);
    const uint64_t x_bytes = static_cast<uint64_t>(m) * k * 2, act_bytes = static_cast<uint64_t>(m) * (n / 2) * 2;
    if (int rc = check_range(dev, x, x_bytes, fn, "x")) return rc;
    if (int rc = check_range(dev, act, act_bytes, fn, "act")) return rc;
    if (overlaps(x, x_bytes, act, act_bytes)) return fail(FH_ERR_INVALID_ARGUMENT, "%s: act overlaps x", fn);
    if (int rc = set_current(dev, fn)) return rc;
    bool done = false;
    if (int rc = dispatch(dev, fn, [&] {
            done = launch_q4_gemm_direct_silu(dev->stream, dev->compute_units, x, static_cast<uint32_t>(k), wq, scales,
                                              biases, static_cast<uint32_t>(m), static_cast<uint32_t>(n / 2),
                                              static_cast<uint32_t>(k), act);
        }))
        return rc;
    if (!done)
        return fail(FH_ERR_UNSUPPORTED,
                    "%s: %lld rows x f=%lld x k=%lld: the fused GEMM needs tiles of 256 rows x 128 pairs that fill "
                    "the chip, f %% 128 == 0 and k %% 512 == 0; use the unfused ops",
                    fn, (long long)m, (long long)(n / 2), (long long)k);
    return FH_OK;
}

int q4_gate_up_silu(fh_device *dev, const uint16_t *x, const uint16_t *residual, uint16_t *residual_out,
                    const uint16_t *norm_weight, float eps, int64_t m, int64_t k, const uint32_t *wq,
                    const uint16_t *scales, const uint16_t *biases, const uint32_t *sb, const uint32_t *wt,
                    int64_t n, int64_t group, uint16_t *act) {
    const char *fn = "fh_q4_gate_up_silu";
    if (n % 2 != 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: n=%lld is not [gate; up] rows", fn, (long long)n);
    const bool norm = norm_weight != nullptr;
    if (m > kGemvMaxRows && !norm && residual == nullptr && residual_out == nullptr)
        return gate_up_silu_gemm(dev, fn, x, m, k, wq, scales, biases, n, group, act);
    if (int rc = check_fused(dev, fn, m, k, wq, scales, biases, n, group, act, FH_BF16, n / 2, norm)) return rc;
    if (int rc = check_sb(dev, fn, sb, n, k)) return rc;
    if (int rc = check_wt(dev, fn, wt, sb, n, k)) return rc;
    if (wt != nullptr && n % 32 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: tiled [gate; up] words need n %% 32 == 0 (n=%lld)", fn,
                    (long long)n);
    if (int rc = check_norm_operands(dev, fn, x, residual, residual_out, norm_weight, m, k)) return rc;
    if (m == 0 || n == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    // empty rows: gate and up are zeros, and RNE(RNE(silu(0)) * 0) = 0
    if (k == 0) return zero_fill(dev, fn, act, static_cast<uint64_t>(m) * (n / 2) * 2);
    const uint32_t k32 = static_cast<uint32_t>(k), n32 = static_cast<uint32_t>(n);
    GemvArgs a{x, k32, wq, scales, biases, n32, k32, act, n32 / 2, 0, norm ? kProRmsNorm : kProNone,
               kEpiSiluMul, GemvFusion{residual, residual_out, norm_weight, eps, 1.0f / static_cast<float>(k)}};
    a.sb = sb;
    a.wt = wt;
    return launch_gemv_rows(dev, fn, m, a, n / 2);
}

// Tiled words: uint4 d of wt is words 4 (d % 4) .. + 3 of group pair p of
// weight row r, for d = ((t * pairs + p) * 16 + c) * 4 + d % 4 and r the
// row of column c in task tile t (c < 8 with the SiLU pairing: gate row
// 8 t + c, else up row n / 2 + 8 t + c - 8; plain: 16 t + c).
__global__ __launch_bounds__(256) void q4_tile_kernel(const uint4 *__restrict__ wq, uint32_t n, uint32_t pairs,
                                                      int silu_pairs, uint4 *__restrict__ wt) {
    const uint64_t total = static_cast<uint64_t>(n) * pairs * 4;
    for (uint64_t d = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; d < total;
         d += static_cast<uint64_t>(gridDim.x) * 256) {
        const uint32_t q = d % 4, c = (d / 4) % 16;
        const uint64_t tp = d / 64;
        const uint32_t p = tp % pairs;
        const uint32_t t = static_cast<uint32_t>(tp / pairs);
        const uint32_t r = silu_pairs ? (c < 8 ? 8 * t + c : n / 2 + 8 * t + c - 8) : 16 * t + c;
        wt[d] = wq[(static_cast<uint64_t>(r) * pairs + p) * 4 + q];
    }
}

// Writes sb[r][2p] = the scales of groups 2p, 2p + 1 of row r (low half:
// group 2p) and sb[r][2p + 1] = their biases, i.e. dword i of the scales
// and of the biases (viewed as dword arrays) go to dwords 2i and 2i + 1.
__global__ __launch_bounds__(256) void q4_interleave_kernel(const uint32_t *__restrict__ s,
                                                            const uint32_t *__restrict__ b, uint64_t pairs,
                                                            uint2 *__restrict__ sb) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x; i < pairs;
         i += static_cast<uint64_t>(gridDim.x) * 256)
        sb[i] = make_uint2(s[i], b[i]);
}

}  // namespace fh

extern "C" int fh_q4_matmul_rmsnorm(fh_device *dev, const uint16_t *x, const uint16_t *residual,
                                    uint16_t *residual_out, const uint16_t *norm_weight, float eps, int64_t m,
                                    int64_t k, const uint32_t *wq, const uint16_t *scales,
                                    const uint16_t *biases, int64_t n, int64_t group, void *y, int y_dtype) {
    return q4_matmul_rmsnorm(dev, x, residual, residual_out, norm_weight, eps, m, k, wq, scales, biases, nullptr,
                             nullptr, n, group, y, y_dtype);
}

extern "C" int fh_q4_gate_up_silu(fh_device *dev, const uint16_t *x, const uint16_t *residual,
                                  uint16_t *residual_out, const uint16_t *norm_weight, float eps, int64_t m,
                                  int64_t k, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                                  int64_t n, int64_t group, uint16_t *act) {
    return q4_gate_up_silu(dev, x, residual, residual_out, norm_weight, eps, m, k, wq, scales, biases, nullptr,
                           nullptr, n, group, act);
}

extern "C" int fh_q4_interleave(fh_device *dev, const uint16_t *scales, const uint16_t *biases, int64_t n,
                                int64_t k, int64_t group, uint32_t *sb) {
    const char *fn = "fh_q4_interleave";
    if (int rc = check_usable(dev, fn)) return rc;
    if (n < 0 || k < 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: negative shape n=%lld k=%lld", fn, (long long)n,
                                    (long long)k);
    if (group != kGroup)
        return fail(FH_ERR_UNSUPPORTED, "%s: group %lld; the kernels implement group 64", fn, (long long)group);
    if (k % (2 * kGroup) != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: k=%lld is not a multiple of two groups (128)", fn, (long long)k);
    if ((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(biases)) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(sb) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: scales and biases must be 4-byte aligned, sb 16-byte aligned", fn);
    const uint64_t pairs = static_cast<uint64_t>(n) * (k / kGroup) / 2;
    if (pairs == 0) return FH_OK;
    if (int rc = check_range(dev, scales, pairs * 4, fn, "scales")) return rc;
    if (int rc = check_range(dev, biases, pairs * 4, fn, "biases")) return rc;
    if (int rc = check_range(dev, sb, pairs * 8, fn, "sb")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    const uint64_t blocks = (pairs + 255) / 256;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(q4_interleave_kernel, dim3(blocks < 65536 ? blocks : 65536), dim3(256), 0, dev->stream,
                           reinterpret_cast<const uint32_t *>(scales), reinterpret_cast<const uint32_t *>(biases),
                           pairs, reinterpret_cast<uint2 *>(sb));
    });
}

extern "C" int fh_q4_tile(fh_device *dev, const uint32_t *wq, int64_t n, int64_t k, int64_t group, int silu_pairs,
                          uint32_t *wt) {
    const char *fn = "fh_q4_tile";
    if (int rc = check_usable(dev, fn)) return rc;
    if (n < 0 || k < 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: negative shape n=%lld k=%lld", fn, (long long)n, (long long)k);
    if (group != kGroup)
        return fail(FH_ERR_UNSUPPORTED, "%s: group %lld; the kernels implement group 64", fn, (long long)group);
    if (n % (silu_pairs ? 32 : 16) != 0 || k % (2 * kGroup) != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: n=%lld must be a multiple of %d and k=%lld of 128", fn, (long long)n,
                    silu_pairs ? 32 : 16, (long long)k);
    if (n > 0x7FFFFFFFll || k > 0x7FFFFFFFll) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: n or k exceeds 2^31-1", fn);
    if ((reinterpret_cast<uintptr_t>(wq) | reinterpret_cast<uintptr_t>(wt)) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: wq and wt must be 16-byte aligned", fn);
    const uint64_t bytes = static_cast<uint64_t>(n) * (k / 8) * 4;
    if (bytes == 0) return FH_OK;
    if (int rc = check_range(dev, wq, bytes, fn, "wq")) return rc;
    if (int rc = check_range(dev, wt, bytes, fn, "wt")) return rc;
    if (overlaps(wq, bytes, wt, bytes)) return fail(FH_ERR_INVALID_ARGUMENT, "%s: wt overlaps wq", fn);
    if (int rc = set_current(dev, fn)) return rc;
    const uint64_t blocks = (bytes / 16 + 255) / 256;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(q4_tile_kernel, dim3(blocks < 65536 ? blocks : 65536), dim3(256), 0, dev->stream,
                           reinterpret_cast<const uint4 *>(wq), static_cast<uint32_t>(n),
                           static_cast<uint32_t>(k / kGroup / 2), silu_pairs, reinterpret_cast<uint4 *>(wt));
    });
}
