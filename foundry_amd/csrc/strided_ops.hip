// Strided entry points for the reference's non-quantized Ops
// (src/nn/primitive.rs:48-68), the rest of what Device::run and
// Device::run_in_place need (src/metal/mod.rs:639-725): copy, dtype
// conversion, unary and binary elementwise ops, row reductions, matmul,
// index_select, cat and slice_scatter, each over strided views.
//
// These are plain kernels, one output element per thread (one block per
// output element for the reductions), with the Metal kernels' arithmetic:
// values decoded to fp32, the op in fp32, one rounding on the way out
// (src/metal/kernels/common.metal:29-43). They serve the model code that
// runs op by op; the decoder's hot path has its own fused kernels.
#include "device.hpp"
#include "q4_common.hpp"

namespace fh {
namespace {

constexpr int kRank = 4;
constexpr uint32_t kThreads = 256;
// src/nn/shape.rs:13: a shape holds at most 2^31 - 1 elements, so a linear
// element index fits 32 bits.
constexpr int64_t kMaxNumel = 0x7FFFFFFF;

// fh_view as the kernels take it (by value), dims past ndim padded with 1.
struct View {
    int64_t offset;
    int64_t strides[kRank];
    uint32_t dims[kRank];
    int32_t ndim;
};

// Element index of the view's linear (row-major) element `i`, the
// decomposition StridedArgs describes (src/metal/kernels/common.metal:13-21).
__device__ __forceinline__ int64_t at(uint32_t i, const View &v) {
    int64_t idx = v.offset;
#pragma unroll
    for (int d = kRank - 1; d >= 0; --d) {
        if (d >= v.ndim) continue;
        const uint32_t size = v.dims[d];
        idx += static_cast<int64_t>(i % size) * v.strides[d];
        i /= size;
    }
    return idx;
}

__device__ __forceinline__ uint32_t gid() { return blockIdx.x * kThreads + threadIdx.x; }

// Float element access by fh_dtype: F32 as is, BF16 decoded exactly and
// written with the reference's RNE.
template <int DT>
struct Float;
template <>
struct Float<FH_F32> {
    using T = float;
    __device__ static float get(const T *p, int64_t i) { return p[i]; }
    __device__ static void put(T *p, int64_t i, float v) { p[i] = v; }
};
template <>
struct Float<FH_BF16> {
    using T = uint16_t;
    __device__ static float get(const T *p, int64_t i) { return bf16_to_f32(p[i]); }
    __device__ static void put(T *p, int64_t i, float v) { p[i] = static_cast<uint16_t>(f32_to_bf16_rne(v)); }
};

template <typename T>
__global__ __launch_bounds__(kThreads) void copy_kernel(const T *__restrict__ src, View v, T *__restrict__ dst,
                                                        uint32_t n) {
    const uint32_t i = gid();
    if (i < n) dst[i] = src[at(i, v)];
}

template <int IN, int OUT>
__global__ __launch_bounds__(kThreads) void convert_kernel(const typename Float<IN>::T *__restrict__ src, View v,
                                                           typename Float<OUT>::T *__restrict__ dst, uint32_t n) {
    const uint32_t i = gid();
    if (i < n) Float<OUT>::put(dst, i, Float<IN>::get(src, at(i, v)));
}

__device__ __forceinline__ float unary(int op, float x) {
    switch (op) {
        case FH_NEG: return -x;
        case FH_EXP: return expf(x);
        case FH_SQRT: return sqrtf(x);
        default: return 1.0f / x;
    }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void unary_kernel(const typename Float<DT>::T *__restrict__ src, View v,
                                                         typename Float<DT>::T *__restrict__ dst, uint32_t n, int op) {
    const uint32_t i = gid();
    if (i < n) Float<DT>::put(dst, i, unary(op, Float<DT>::get(src, at(i, v))));
}

__device__ __forceinline__ float binary(int op, float a, float b) {
    switch (op) {
        case FH_ADD: return a + b;
        case FH_SUB: return a - b;
        case FH_MUL: return a * b;
        default: return a / b;
    }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void binary_kernel(const typename Float<DT>::T *__restrict__ lhs, View lv,
                                                          const typename Float<DT>::T *__restrict__ rhs, View rv,
                                                          typename Float<DT>::T *__restrict__ dst, uint32_t n, int op) {
    const uint32_t i = gid();
    if (i < n) Float<DT>::put(dst, i, binary(op, Float<DT>::get(lhs, at(i, lv)), Float<DT>::get(rhs, at(i, rv))));
}

// One block per output element. Thread t folds elements t, t + 256, ... of
// the reduced dim in order, then the 256 partials meet in a halving tree
// (width 128, 64, ..., 1), the order reduce_rows uses
// (src/metal/kernels/reduce.metal:17-40), so sums round as the reference's do.
template <int DT, bool AMAX>
__global__ __launch_bounds__(kThreads) void reduce_kernel(const typename Float<DT>::T *__restrict__ src, View rows,
                                                          uint32_t dim_size, int64_t dim_stride,
                                                          typename Float<DT>::T *__restrict__ dst,
                                                          uint32_t n_rows) {
    __shared__ float part[kThreads];
    const uint32_t t = threadIdx.x;
    // blocks stride over the output rows: the grid is capped so that its
    // work-item count stays below 2^32 however many rows there are
    for (uint32_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
        const int64_t base = at(row, rows);
        float acc = AMAX ? -INFINITY : 0.0f;
        for (uint32_t k = t; k < dim_size; k += kThreads) {
            const float x = Float<DT>::get(src, base + static_cast<int64_t>(k) * dim_stride);
            acc = AMAX ? fmaxf(acc, x) : acc + x;
        }
        __syncthreads();  // the previous row's tree has read part[]
        part[t] = acc;
        __syncthreads();
        for (uint32_t w = kThreads / 2; w > 0; w /= 2) {
            if (t < w) part[t] = AMAX ? fmaxf(part[t], part[t + w]) : part[t] + part[t + w];
            __syncthreads();
        }
        if (t == 0) Float<DT>::put(dst, row, part[0]);
    }
}

// argmax_rows (src/metal/kernels/reduce.metal:42-78): a thread keeps its
// first strict maximum; the tree prefers the larger value, then the lower
// index. A NaN never wins; a row with no larger value than -inf gives 0.
template <int DT>
__global__ __launch_bounds__(kThreads) void argmax_kernel(const typename Float<DT>::T *__restrict__ src, View rows,
                                                          uint32_t dim_size, int64_t dim_stride,
                                                          uint32_t *__restrict__ dst, uint32_t n_rows) {
    __shared__ float val[kThreads];
    __shared__ uint32_t idx[kThreads];
    const uint32_t t = threadIdx.x;
    for (uint32_t row = blockIdx.x; row < n_rows; row += gridDim.x) {  // as reduce_kernel
        const int64_t base = at(row, rows);
        float best = -INFINITY;
        uint32_t best_i = 0;
        for (uint32_t k = t; k < dim_size; k += kThreads) {
            const float x = Float<DT>::get(src, base + static_cast<int64_t>(k) * dim_stride);
            if (x > best) best = x, best_i = k;
        }
        __syncthreads();  // the previous row's tree has read val[], idx[]
        val[t] = best;
        idx[t] = best_i;
        __syncthreads();
        for (uint32_t w = kThreads / 2; w > 0; w /= 2) {
            if (t < w) {
                const float o = val[t + w];
                const uint32_t oi = idx[t + w];
                if (o > val[t] || (o == val[t] && oi < idx[t])) val[t] = o, idx[t] = oi;
            }
            __syncthreads();
        }
        if (t == 0) dst[row] = idx[0];
    }
}

// Batched matmul over strided operands. A block owns a 32 x 32 output tile
// of one batch entry; 256 threads each hold 2 x 2 sums. Operand tiles of 16
// along k go through LDS as fp32; every sum runs over k in order (one fma per
// step), as matmul_tiled accumulates (src/metal/kernels/matmul.metal:42-64).
struct MatmulShape {
    uint32_t m, n, k, batch_ndim;
    uint32_t batch_dims[2];
    int64_t l_off, l_rs, l_cs, l_bs[2];
    int64_t r_off, r_rs, r_cs, r_bs[2];
};

constexpr uint32_t kMmTile = 32;
constexpr uint32_t kMmK = 16;

template <int DT>
__global__ __launch_bounds__(kThreads) void matmul_kernel(const typename Float<DT>::T *__restrict__ lhs,
                                                          const typename Float<DT>::T *__restrict__ rhs, MatmulShape s,
                                                          typename Float<DT>::T *__restrict__ dst) {
    __shared__ float lt[kMmTile][kMmK + 1];
    __shared__ float rt[kMmK][kMmTile + 1];
    const uint32_t t = threadIdx.x;
    const uint32_t row0 = blockIdx.y * kMmTile, col0 = blockIdx.x * kMmTile;
    // batch entry -> each operand's base offset (batch dims row-major)
    int64_t lb = s.l_off, rb = s.r_off;
    uint32_t b = blockIdx.z;
    for (int d = static_cast<int>(s.batch_ndim) - 1; d >= 0; --d) {
        const uint32_t size = s.batch_dims[d];
        lb += static_cast<int64_t>(b % size) * s.l_bs[d];
        rb += static_cast<int64_t>(b % size) * s.r_bs[d];
        b /= size;
    }
    const uint32_t tr = (t / 16) * 2, tc = (t % 16) * 2;  // this thread's 2 x 2 sums
    float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
    for (uint32_t k0 = 0; k0 < s.k; k0 += kMmK) {
        // 32 x 16 of lhs and 16 x 32 of rhs: two loads per thread each
        for (uint32_t e = t; e < kMmTile * kMmK; e += kThreads) {
            const uint32_t r = e / kMmK, kk = e % kMmK;
            const uint32_t gr = row0 + r, gk = k0 + kk;
            lt[r][kk] = (gr < s.m && gk < s.k) ? Float<DT>::get(lhs, lb + gr * s.l_rs + gk * s.l_cs) : 0.0f;
            const uint32_t kr = e / kMmTile, c = e % kMmTile;
            const uint32_t rk = k0 + kr, gc = col0 + c;
            rt[kr][c] = (rk < s.k && gc < s.n) ? Float<DT>::get(rhs, rb + rk * s.r_rs + gc * s.r_cs) : 0.0f;
        }
        __syncthreads();
        const uint32_t steps = s.k - k0 < kMmK ? s.k - k0 : kMmK;
        for (uint32_t kk = 0; kk < steps; ++kk) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = fmaf(lt[tr + i][kk], rt[kk][tc + j], acc[i][j]);
        }
        __syncthreads();
    }
    const uint64_t out_base = static_cast<uint64_t>(blockIdx.z) * s.m * s.n;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t r = row0 + tr + i, c = col0 + tc + j;
            if (r < s.m && c < s.n) Float<DT>::put(dst, static_cast<int64_t>(out_base + static_cast<uint64_t>(r) * s.n + c),
                                                 acc[i][j]);
        }
}

// index_select_rows (src/metal/kernels/index_select.metal:11-29): an id at
// or past the table's rows gives a zero row.
template <typename T>
__global__ __launch_bounds__(kThreads) void index_select_kernel(const T *__restrict__ table, int64_t t_off,
                                                                int64_t t_rs, int64_t t_cs, uint32_t rows,
                                                                uint32_t cols, const uint32_t *__restrict__ ids,
                                                                View iv, T *__restrict__ dst, uint32_t n) {
    const uint32_t i = gid();
    if (i >= n) return;
    const uint32_t r = i / cols, c = i % cols;
    const uint32_t id = ids[at(r, iv)];
    dst[i] = id < rows ? table[t_off + static_cast<int64_t>(id) * t_rs + static_cast<int64_t>(c) * t_cs] : T(0);
}

// slice_scatter_strided (src/metal/kernels/slice_scatter.metal:1-15): the
// i-th element of the source view goes to the i-th element of the window.
template <typename T>
__global__ __launch_bounds__(kThreads) void scatter_kernel(const T *__restrict__ src, View sv, T *__restrict__ dst,
                                                           View wv, uint32_t n) {
    const uint32_t i = gid();
    if (i < n) dst[at(i, wv)] = src[at(i, sv)];
}

// ---- host side ----

int itemsize(int dtype) { return dtype == FH_BF16 ? 2 : 4; }

bool valid_dtype(int dtype) { return dtype == FH_F32 || dtype == FH_BF16 || dtype == FH_U32; }

int require_float(const char *fn, int dtype) {
    if (dtype != FH_F32 && dtype != FH_BF16)
        return fail(FH_ERR_DTYPE, "%s: dtype %d is not a float dtype (TensorError::DTypeNotFloat)", fn, dtype);
    return FH_OK;
}

int64_t numel_of(const fh_view &v) {
    int64_t n = 1;
    for (int d = 0; d < v.ndim; ++d) n *= v.dims[d];
    return n;
}

// Checks a view (rank, sizes, strides, element count) and that every element
// it addresses lies inside one live allocation; fills the kernel's View.
int check_view(const fh_device *dev, const char *fn, const char *what, const void *base, const fh_view *v, int dtype,
               View *out) {
    if (!v) return fail(FH_ERR_INVALID_ARGUMENT, "%s: %s view is null", fn, what);
    if (v->ndim < 0 || v->ndim > kRank)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: %s has rank %d (TensorError::RankTooLarge)", fn, what, v->ndim);
    if (v->offset < 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: %s has a negative offset", fn, what);
    unsigned __int128 numel = 1, last = static_cast<unsigned __int128>(v->offset);
    for (int d = 0; d < v->ndim; ++d) {
        if (v->dims[d] < 0 || v->dims[d] > kMaxNumel || v->strides[d] < 0)
            return fail(FH_ERR_INVALID_ARGUMENT, "%s: %s dim %d has size %lld, stride %lld", fn, what, d,
                        (long long)v->dims[d], (long long)v->strides[d]);
        numel *= static_cast<uint64_t>(v->dims[d]);
        if (v->dims[d] > 0) last += static_cast<unsigned __int128>(v->dims[d] - 1) * static_cast<uint64_t>(v->strides[d]);
    }
    if (numel > static_cast<unsigned __int128>(kMaxNumel))
        return fail(FH_ERR_INDEX_TOO_LARGE, "%s: %s has more than 2^31 - 1 elements (TensorError::NumelOverflow)", fn,
                    what);
    const int size = itemsize(dtype);
    if (reinterpret_cast<uintptr_t>(base) % size != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: %s is misaligned for its dtype", fn, what);
    if (numel > 0) {
        const unsigned __int128 bytes = (last + 1) * static_cast<unsigned>(size);
        if (bytes > static_cast<unsigned __int128>(UINT64_MAX >> 1))
            return fail(FH_ERR_OUT_OF_BOUNDS, "%s: %s addresses past any allocation", fn, what);
        if (int rc = check_range(dev, base, static_cast<uint64_t>(bytes), fn, what)) return rc;
    }
    out->offset = v->offset;
    out->ndim = v->ndim;
    for (int d = 0; d < kRank; ++d) {
        out->dims[d] = d < v->ndim ? static_cast<uint32_t>(v->dims[d]) : 1u;
        out->strides[d] = d < v->ndim ? v->strides[d] : 0;
    }
    return FH_OK;
}

int check_out(const fh_device *dev, const char *fn, void *dst, int64_t numel, int dtype) {
    if (reinterpret_cast<uintptr_t>(dst) % itemsize(dtype) != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: dst is misaligned for its dtype", fn);
    return check_range(dev, dst, static_cast<uint64_t>(numel) * itemsize(dtype), fn, "dst");
}

int begin(fh_device *dev, const char *fn) {
    if (int rc = check_usable(dev, fn)) return rc;
    return FH_OK;
}

uint32_t blocks_for(int64_t n) { return static_cast<uint32_t>((n + kThreads - 1) / kThreads); }

// A contiguous view of `dims` at `offset` (the layout of a fresh output).
View contiguous(const int64_t *dims, int ndim, int64_t offset) {
    View v{};
    v.offset = offset;
    v.ndim = ndim;
    int64_t stride = 1;
    for (int d = kRank - 1; d >= 0; --d) {
        v.dims[d] = d < ndim ? static_cast<uint32_t>(dims[d]) : 1u;
        v.strides[d] = d < ndim ? stride : 0;
        if (d < ndim) stride *= dims[d];
    }
    return v;
}

// Launches the scatter of every element of src (view sv, n elements) into
// the window wv of dst.
int scatter(fh_device *dev, const char *fn, int dtype, const void *src, const View &sv, void *dst, const View &wv,
            int64_t n) {
    if (n == 0) return FH_OK;
    return dispatch(dev, fn, [&] {
        if (dtype == FH_BF16)
            hipLaunchKernelGGL(scatter_kernel<uint16_t>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint16_t *>(src), sv, static_cast<uint16_t *>(dst), wv,
                               static_cast<uint32_t>(n));
        else
            hipLaunchKernelGGL(scatter_kernel<uint32_t>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint32_t *>(src), sv, static_cast<uint32_t *>(dst), wv,
                               static_cast<uint32_t>(n));
    });
}

// dims equal except at `dim` (src/nn/primitive.rs:356-367)
bool dims_equal_except(const fh_view &a, const fh_view &b, int dim) {
    if (a.ndim != b.ndim) return false;
    for (int d = 0; d < a.ndim; ++d)
        if (d != dim && a.dims[d] != b.dims[d]) return false;
    return true;
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int fh_copy_strided(fh_device *dev, int dtype, const void *src, const fh_view *view, void *dst) {
    const char *fn = "fh_copy_strided";
    if (int rc = begin(dev, fn)) return rc;
    if (!valid_dtype(dtype)) return fail(FH_ERR_DTYPE, "%s: unknown dtype %d", fn, dtype);
    View v;
    if (int rc = check_view(dev, fn, "src", src, view, dtype, &v)) return rc;
    const int64_t n = numel_of(*view);
    if (int rc = check_out(dev, fn, dst, n, dtype)) return rc;
    if (n == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        if (dtype == FH_BF16)
            hipLaunchKernelGGL(copy_kernel<uint16_t>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint16_t *>(src), v, static_cast<uint16_t *>(dst),
                               static_cast<uint32_t>(n));
        else
            hipLaunchKernelGGL(copy_kernel<uint32_t>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint32_t *>(src), v, static_cast<uint32_t *>(dst),
                               static_cast<uint32_t>(n));
    });
}

extern "C" int fh_to_dtype(fh_device *dev, int from, const void *src, const fh_view *view, int to, void *dst) {
    const char *fn = "fh_to_dtype";
    if (int rc = begin(dev, fn)) return rc;
    if (int rc = require_float(fn, from)) return rc;
    if (int rc = require_float(fn, to)) return rc;
    if (from == to) return fh_copy_strided(dev, from, src, view, dst);
    View v;
    if (int rc = check_view(dev, fn, "src", src, view, from, &v)) return rc;
    const int64_t n = numel_of(*view);
    if (int rc = check_out(dev, fn, dst, n, to)) return rc;
    if (n == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        if (from == FH_F32)
            hipLaunchKernelGGL((convert_kernel<FH_F32, FH_BF16>), dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const float *>(src), v, static_cast<uint16_t *>(dst),
                               static_cast<uint32_t>(n));
        else
            hipLaunchKernelGGL((convert_kernel<FH_BF16, FH_F32>), dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint16_t *>(src), v, static_cast<float *>(dst),
                               static_cast<uint32_t>(n));
    });
}

extern "C" int fh_unary(fh_device *dev, int op, int dtype, const void *src, const fh_view *view, void *dst) {
    const char *fn = "fh_unary";
    if (int rc = begin(dev, fn)) return rc;
    if (op < FH_NEG || op > FH_RECIPROCAL) return fail(FH_ERR_INVALID_ARGUMENT, "%s: unknown unary op %d", fn, op);
    if (int rc = require_float(fn, dtype)) return rc;
    View v;
    if (int rc = check_view(dev, fn, "src", src, view, dtype, &v)) return rc;
    const int64_t n = numel_of(*view);
    if (int rc = check_out(dev, fn, dst, n, dtype)) return rc;
    if (n == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        if (dtype == FH_F32)
            hipLaunchKernelGGL(unary_kernel<FH_F32>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const float *>(src), v, static_cast<float *>(dst),
                               static_cast<uint32_t>(n), op);
        else
            hipLaunchKernelGGL(unary_kernel<FH_BF16>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint16_t *>(src), v, static_cast<uint16_t *>(dst),
                               static_cast<uint32_t>(n), op);
    });
}

extern "C" int fh_binary(fh_device *dev, int op, int dtype, const void *lhs, const fh_view *lhs_view,
                         const void *rhs, const fh_view *rhs_view, void *dst) {
    const char *fn = "fh_binary";
    if (int rc = begin(dev, fn)) return rc;
    if (op < FH_ADD || op > FH_DIV) return fail(FH_ERR_INVALID_ARGUMENT, "%s: unknown binary op %d", fn, op);
    if (int rc = require_float(fn, dtype)) return rc;
    View lv, rv;
    if (int rc = check_view(dev, fn, "lhs", lhs, lhs_view, dtype, &lv)) return rc;
    if (int rc = check_view(dev, fn, "rhs", rhs, rhs_view, dtype, &rv)) return rc;
    if (!dims_equal_except(*lhs_view, *rhs_view, -1))
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: lhs and rhs views must have the output's dims (broadcast first)",
                    fn);
    const int64_t n = numel_of(*lhs_view);
    if (int rc = check_out(dev, fn, dst, n, dtype)) return rc;
    if (n == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        if (dtype == FH_F32)
            hipLaunchKernelGGL(binary_kernel<FH_F32>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const float *>(lhs), lv, static_cast<const float *>(rhs), rv,
                               static_cast<float *>(dst), static_cast<uint32_t>(n), op);
        else
            hipLaunchKernelGGL(binary_kernel<FH_BF16>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint16_t *>(lhs), lv, static_cast<const uint16_t *>(rhs), rv,
                               static_cast<uint16_t *>(dst), static_cast<uint32_t>(n), op);
    });
}

extern "C" int fh_reduce(fh_device *dev, int op, int dtype, const void *src, const fh_view *view, int32_t dim,
                         void *dst) {
    const char *fn = "fh_reduce";
    if (int rc = begin(dev, fn)) return rc;
    if (op < FH_SUM || op > FH_ARGMAX) return fail(FH_ERR_INVALID_ARGUMENT, "%s: unknown reduce op %d", fn, op);
    if (int rc = require_float(fn, dtype)) return rc;
    View v;
    if (int rc = check_view(dev, fn, "src", src, view, dtype, &v)) return rc;
    if (dim < 0 || dim >= view->ndim)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: dim %d of a rank-%d view (TensorError::DimOutOfRange)", fn, dim,
                    view->ndim);
    const int64_t dim_size = view->dims[dim];
    if (op != FH_SUM && dim_size == 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: reduction over an empty dim (TensorError::EmptyReduction)", fn);
    int64_t rows = 1;
    for (int d = 0; d < view->ndim; ++d) rows *= d == dim ? 1 : view->dims[d];
    const int out_dtype = op == FH_ARGMAX ? FH_U32 : dtype;
    if (int rc = check_out(dev, fn, dst, rows, out_dtype)) return rc;
    if (rows == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    View rv = v;  // the input's strides over the output's dims
    rv.dims[dim] = 1;
    const int64_t stride = view->strides[dim];
    const uint32_t size = static_cast<uint32_t>(dim_size);
    return dispatch(dev, fn, [&] {
        // at most 2^20 blocks (2^28 work-items); the kernels stride over the rest
        const uint32_t n_rows = static_cast<uint32_t>(rows);
        const dim3 grid(n_rows < (1u << 20) ? n_rows : (1u << 20)), block(kThreads);
        if (dtype == FH_F32) {
            auto *s = static_cast<const float *>(src);
            if (op == FH_SUM)
                hipLaunchKernelGGL((reduce_kernel<FH_F32, false>), grid, block, 0, dev->stream, s, rv, size, stride,
                                   static_cast<float *>(dst), n_rows);
            else if (op == FH_AMAX)
                hipLaunchKernelGGL((reduce_kernel<FH_F32, true>), grid, block, 0, dev->stream, s, rv, size, stride,
                                   static_cast<float *>(dst), n_rows);
            else
                hipLaunchKernelGGL(argmax_kernel<FH_F32>, grid, block, 0, dev->stream, s, rv, size, stride,
                                   static_cast<uint32_t *>(dst), n_rows);
        } else {
            auto *s = static_cast<const uint16_t *>(src);
            if (op == FH_SUM)
                hipLaunchKernelGGL((reduce_kernel<FH_BF16, false>), grid, block, 0, dev->stream, s, rv, size, stride,
                                   static_cast<uint16_t *>(dst), n_rows);
            else if (op == FH_AMAX)
                hipLaunchKernelGGL((reduce_kernel<FH_BF16, true>), grid, block, 0, dev->stream, s, rv, size, stride,
                                   static_cast<uint16_t *>(dst), n_rows);
            else
                hipLaunchKernelGGL(argmax_kernel<FH_BF16>, grid, block, 0, dev->stream, s, rv, size, stride,
                                   static_cast<uint32_t *>(dst), n_rows);
        }
    });
}

extern "C" int fh_matmul(fh_device *dev, int dtype, const void *lhs, const fh_view *lhs_view, const void *rhs,
                         const fh_view *rhs_view, void *dst) {
    const char *fn = "fh_matmul";
    if (int rc = begin(dev, fn)) return rc;
    if (int rc = require_float(fn, dtype)) return rc;
    View lv, rv;
    if (int rc = check_view(dev, fn, "lhs", lhs, lhs_view, dtype, &lv)) return rc;
    if (int rc = check_view(dev, fn, "rhs", rhs, rhs_view, dtype, &rv)) return rc;
    // src/nn/primitive.rs:209-233: [..., m, k] x [..., k, n], equal batch dims
    const int nd = lhs_view->ndim;
    if (nd < 2 || rhs_view->ndim != nd || lhs_view->dims[nd - 1] != rhs_view->dims[nd - 2])
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: shapes cannot be multiplied (TensorError::MatmulIncompatible)", fn);
    for (int d = 0; d < nd - 2; ++d)
        if (lhs_view->dims[d] != rhs_view->dims[d])
            return fail(FH_ERR_INVALID_ARGUMENT, "%s: batch dims differ (TensorError::MatmulIncompatible)", fn);
    MatmulShape s{};
    s.m = static_cast<uint32_t>(lhs_view->dims[nd - 2]);
    s.k = static_cast<uint32_t>(lhs_view->dims[nd - 1]);
    s.n = static_cast<uint32_t>(rhs_view->dims[nd - 1]);
    s.batch_ndim = static_cast<uint32_t>(nd - 2);
    int64_t batch = 1;
    for (int d = 0; d < nd - 2; ++d) {
        s.batch_dims[d] = static_cast<uint32_t>(lhs_view->dims[d]);
        s.l_bs[d] = lhs_view->strides[d];
        s.r_bs[d] = rhs_view->strides[d];
        batch *= lhs_view->dims[d];
    }
    s.l_off = lhs_view->offset, s.l_rs = lhs_view->strides[nd - 2], s.l_cs = lhs_view->strides[nd - 1];
    s.r_off = rhs_view->offset, s.r_rs = rhs_view->strides[nd - 2], s.r_cs = rhs_view->strides[nd - 1];
    const int64_t out = batch * s.m * s.n;
    if (out > kMaxNumel) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: output exceeds 2^31 - 1 elements", fn);
    if (int rc = check_out(dev, fn, dst, out, dtype)) return rc;
    if (out == 0) return FH_OK;
    if (batch > 65535) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: %lld batch entries exceed the grid", fn,
                                   (long long)batch);
    if (int rc = set_current(dev, fn)) return rc;
    const dim3 grid((s.n + kMmTile - 1) / kMmTile, (s.m + kMmTile - 1) / kMmTile, static_cast<uint32_t>(batch));
    if (grid.y > 65535) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: m=%u exceeds the grid", fn, s.m);
    // grid.x * 256 work-items must stay below 2^32
    if (static_cast<uint64_t>(grid.x) * kThreads > 0xFFFFFFFFull)
        return fail(FH_ERR_INDEX_TOO_LARGE, "%s: n=%u exceeds the grid", fn, s.n);
    return dispatch(dev, fn, [&] {
        if (dtype == FH_F32)
            hipLaunchKernelGGL(matmul_kernel<FH_F32>, grid, dim3(kThreads), 0, dev->stream,
                               static_cast<const float *>(lhs), static_cast<const float *>(rhs), s,
                               static_cast<float *>(dst));
        else
            hipLaunchKernelGGL(matmul_kernel<FH_BF16>, grid, dim3(kThreads), 0, dev->stream,
                               static_cast<const uint16_t *>(lhs), static_cast<const uint16_t *>(rhs), s,
                               static_cast<uint16_t *>(dst));
    });
}

extern "C" int fh_index_select(fh_device *dev, int dtype, const void *table, const fh_view *table_view,
                               const uint32_t *ids, const fh_view *ids_view, void *dst) {
    const char *fn = "fh_index_select";
    if (int rc = begin(dev, fn)) return rc;
    if (int rc = require_float(fn, dtype)) return rc;
    View tv, iv;
    if (int rc = check_view(dev, fn, "table", table, table_view, dtype, &tv)) return rc;
    if (int rc = check_view(dev, fn, "ids", ids, ids_view, FH_U32, &iv)) return rc;
    if (table_view->ndim != 2 || ids_view->ndim != 1)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: a 2-D table and 1-D ids (TensorError::IndexSelectIncompatible)",
                    fn);
    const int64_t rows = table_view->dims[0], cols = table_view->dims[1], count = ids_view->dims[0];
    const int64_t n = count * cols;
    if (n > kMaxNumel) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: output exceeds 2^31 - 1 elements", fn);
    if (int rc = check_out(dev, fn, dst, n, dtype)) return rc;
    if (n == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        if (dtype == FH_BF16)
            hipLaunchKernelGGL(index_select_kernel<uint16_t>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint16_t *>(table), tv.offset, tv.strides[0], tv.strides[1],
                               static_cast<uint32_t>(rows), static_cast<uint32_t>(cols), ids, iv,
                               static_cast<uint16_t *>(dst), static_cast<uint32_t>(n));
        else
            hipLaunchKernelGGL(index_select_kernel<uint32_t>, dim3(blocks_for(n)), dim3(kThreads), 0, dev->stream,
                               static_cast<const uint32_t *>(table), tv.offset, tv.strides[0], tv.strides[1],
                               static_cast<uint32_t>(rows), static_cast<uint32_t>(cols), ids, iv,
                               static_cast<uint32_t *>(dst), static_cast<uint32_t>(n));
    });
}

extern "C" int fh_cat(fh_device *dev, int dtype, int32_t dim, const void *lhs, const fh_view *lhs_view,
                      const void *rhs, const fh_view *rhs_view, void *dst) {
    const char *fn = "fh_cat";
    if (int rc = begin(dev, fn)) return rc;
    if (int rc = require_float(fn, dtype)) return rc;
    View lv, rv;
    if (int rc = check_view(dev, fn, "lhs", lhs, lhs_view, dtype, &lv)) return rc;
    if (int rc = check_view(dev, fn, "rhs", rhs, rhs_view, dtype, &rv)) return rc;
    if (dim < 0 || dim >= lhs_view->ndim)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: dim %d (TensorError::DimOutOfRange)", fn, dim);
    if (!dims_equal_except(*lhs_view, *rhs_view, dim))
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: shapes cannot be concatenated (TensorError::CatIncompatible)", fn);
    int64_t dims[kRank];
    for (int d = 0; d < lhs_view->ndim; ++d) dims[d] = lhs_view->dims[d];
    dims[dim] = lhs_view->dims[dim] + rhs_view->dims[dim];
    if (dims[dim] > kMaxNumel) return fail(FH_ERR_INVALID_ARGUMENT, "%s: dim %d overflows", fn, dim);
    const int64_t nl = numel_of(*lhs_view), nr = numel_of(*rhs_view);
    if (nl + nr > kMaxNumel) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: output exceeds 2^31 - 1 elements", fn);
    if (int rc = check_out(dev, fn, dst, nl + nr, dtype)) return rc;
    if (nl + nr == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    // MetalDevice::cat: both inputs scatter into windows of the contiguous
    // output, rhs from lhs.dims[dim] along dim
    const View out = contiguous(dims, lhs_view->ndim, 0);
    View lw = out, rw = out;
    for (int d = 0; d < lhs_view->ndim; ++d) lw.dims[d] = static_cast<uint32_t>(lhs_view->dims[d]);
    for (int d = 0; d < lhs_view->ndim; ++d) rw.dims[d] = static_cast<uint32_t>(rhs_view->dims[d]);
    rw.offset = lhs_view->dims[dim] * out.strides[dim];
    if (int rc = scatter(dev, fn, dtype, lhs, lv, dst, lw, nl)) return rc;
    return scatter(dev, fn, dtype, rhs, rv, dst, rw, nr);
}

extern "C" int fh_slice_scatter(fh_device *dev, int dtype, int32_t dim, int64_t start, void *target,
                                const fh_view *target_view, const void *src, const fh_view *src_view) {
    const char *fn = "fh_slice_scatter";
    if (int rc = begin(dev, fn)) return rc;
    if (int rc = require_float(fn, dtype)) return rc;
    View tv, sv;
    if (int rc = check_view(dev, fn, "target", target, target_view, dtype, &tv)) return rc;
    if (int rc = check_view(dev, fn, "src", src, src_view, dtype, &sv)) return rc;
    if (dim < 0 || dim >= target_view->ndim)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: dim %d (TensorError::DimOutOfRange)", fn, dim);
    // src/nn/primitive.rs:314-335: src fits the target from start along dim
    if (start < 0 || !dims_equal_except(*target_view, *src_view, dim) ||
        start + src_view->dims[dim] > target_view->dims[dim])
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: slice does not fit the target (TensorError::SliceScatterOutOfBounds)",
                    fn);
    const View want = contiguous(target_view->dims, target_view->ndim, target_view->offset);
    for (int d = 0; d < target_view->ndim; ++d)
        if (target_view->dims[d] != 1 && target_view->strides[d] != want.strides[d])
            return fail(FH_ERR_INVALID_ARGUMENT,
                        "%s: the target must be contiguous (TensorError::SliceScatterNonContiguous)", fn);
    const int64_t n = numel_of(*src_view);
    if (n == 0) return FH_OK;
    if (int rc = set_current(dev, fn)) return rc;
    View window = tv;  // the target's strides over src's dims, from start along dim
    for (int d = 0; d < target_view->ndim; ++d) window.dims[d] = static_cast<uint32_t>(src_view->dims[d]);
    window.offset = target_view->offset + start * target_view->strides[dim];
    return scatter(dev, fn, dtype, src, sv, target, window, n);
}
