// Decoder-step ops around the q4 linears (attention is in attention.hip):
// residual add + RMSNorm, RoPE with the KV-cache write, SiLU-and-multiply,
// argmax and the device-side position counter. They are the HIP counterparts
// of the reference's RmsNorm (src/nn/norm.rs:32-50), apply_rotary_pos_emb
// (src/models/llama/rotary_emb.rs:62-85), StaticCache::update
// (src/nn/kv_cache.rs:41-80), Silu (src/nn/activation.rs:19-28) and the
// greedy argmax (src/generate/mod.rs:192-204; src/metal/kernels/reduce.metal:42-78).
//
// Each keeps the reference's bf16 rounding points (its tensors are bf16, and
// every op rounds its output): e.g. RMSNorm rounds x*scale to bf16 before the
// weight multiply, RoPE rounds x*cos and rot*sin before adding. Where the
// reference runs several dispatches (about ten for RMSNorm, six for SiLU)
// these are one kernel each.
//
// The decode step is captured once as a HIP graph and replayed: the token id
// and position live in device memory (argmax writes the next id that the
// embedding gather reads; fh_advance_positions bumps the position), so no
// kernel argument changes between steps.
#include "decoder_common.hpp"

namespace fh {

// Sum across a 256-thread block (every thread gets the result).
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) t += red[w];
    return t;
}

__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) t = fmaxf(t, red[w]);
    return t;
}

// One block per row, the row held in registers (16-byte loads, up to
// kNormChunks pieces of 8 per thread). With `res`, h = RNE(x + res) is formed
// first (the residual add, src/models/llama/model.rs:254-279) and written to
// res_out. y = RNE(RNE(h * scale) * w), scale = 1 / sqrt(sum(h^2) * (1/dim) + eps).
// With PART, x is not read: each x value is formed from the f32 partials of
// the GEMM that produced it (split_sum8, the value gemm_split_reduce_kernel
// would have stored), so the norm stands in for that reduce.
constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;  // dim <= 256 * 8 * 4 = 8192

template <bool PART>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const uint16_t *__restrict__ x,
                                                                const uint16_t *__restrict__ res,
                                                                uint16_t *__restrict__ res_out,
                                                                const uint16_t *__restrict__ w,
                                                                uint32_t dim, float eps, float dim_inv,
                                                                uint16_t *__restrict__ y,
                                                                const float *__restrict__ part, uint32_t splits,
                                                                uint64_t part_stride) {
    __shared__ float red[kNormThreads / 64];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * dim;
    const uint32_t pieces = dim / 8;
    float h[kNormChunks][8];
    uint4 wv[kNormChunks];  // the weight loads go out with x's, before the reduction
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
        const uint32_t piece = threadIdx.x + c * kNormThreads;
        if (piece < pieces) wv[c] = *reinterpret_cast<const uint4 *>(w + piece * 8);
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
        const uint32_t piece = threadIdx.x + c * kNormThreads;
        if (piece < pieces) {
            const uint4 xv = PART ? split_sum8(part, splits, part_stride, base + piece * 8)
                                  : *reinterpret_cast<const uint4 *>(x + base + piece * 8);
            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
            uint32_t hw[4];
            if (res) {
                const uint4 rv = *reinterpret_cast<const uint4 *>(res + base + piece * 8);
                const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t lo = rne(bf(xw[e] & 0xFFFFu) + bf(rw[e] & 0xFFFFu));
                    const uint32_t hi = rne(bf(xw[e] >> 16) + bf(rw[e] >> 16));
                    hw[e] = lo | (hi << 16);
                }
                *reinterpret_cast<uint4 *>(res_out + base + piece * 8) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) hw[e] = xw[e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h[c][2 * e] = bf(hw[e] & 0xFFFFu);
                h[c][2 * e + 1] = bf(hw[e] >> 16);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += h[c][e] * h[c][e];
        }
    }
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss * dim_inv + eps);
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
        const uint32_t piece = threadIdx.x + c * kNormThreads;
        if (piece < pieces) {
            const uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = rne(bf(rne(h[c][2 * e] * scale)) * bf(ww[e] & 0xFFFFu));
                const uint32_t hi = rne(bf(rne(h[c][2 * e + 1] * scale)) * bf(ww[e] >> 16));
                o[e] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4 *>(y + base + piece * 8) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// RoPE on q and k of one token (block), then k and v into the cache at the
// token's position. qkv row: [q heads | k heads | v heads] * head_dim.
// x' = RNE(RNE(x * cos) + RNE(rot * sin)), rot = cat(-x2, x1). A thread
// handles 8 consecutive dims (16-byte loads); its rotation partner is the
// matching 8 dims of the other half (head_dim is a multiple of 16).
// With part, the qkv values are formed from the f32 partials of the q/k/v
// GEMM (split_sum8; row t at part + t * width), which stands in for its reduce.
__device__ __forceinline__ uint4 qkv_piece(const uint16_t *row, const float *part, uint32_t splits, uint64_t stride,
                                           uint64_t row0, uint32_t e) {
    return part ? split_sum8(part, splits, stride, row0 + e) : *reinterpret_cast<const uint4 *>(row + e);
}

__global__ __launch_bounds__(256) void rope_kv_kernel(
    const uint16_t *__restrict__ qkv, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim,
    const uint16_t *__restrict__ cos_tab, const uint16_t *__restrict__ sin_tab, uint32_t table_len,
    const uint32_t *__restrict__ positions, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, uint32_t max_len, uint16_t *__restrict__ q_out,
    const float *__restrict__ part, uint32_t splits, uint64_t part_stride, uint32_t seq_tokens, uint64_t seq_cache) {
    const uint32_t t = blockIdx.x;
    const uint32_t pos = positions[t];
    // token t belongs to sequence t / seq_tokens, whose caches start seq_cache
    // elements after the previous sequence's
    k_cache += (t / seq_tokens) * seq_cache;
    v_cache += (t / seq_tokens) * seq_cache;
    // positions are device data the host cannot check: a position outside the
    // cache or the tables writes nothing
    if (pos >= max_len || pos >= table_len) return;
    const uint32_t width = (n_heads + 2 * n_kv) * head_dim;
    const uint16_t *row = qkv + static_cast<uint64_t>(t) * width;
    const uint16_t *c = cos_tab + static_cast<uint64_t>(pos) * head_dim;
    const uint16_t *s = sin_tab + static_cast<uint64_t>(pos) * head_dim;
    const uint32_t ppw = head_dim / 8, hp = ppw / 2;  // pieces per head, per half
    const uint32_t rot_pieces = (n_heads + n_kv) * ppw;
    const uint64_t row0 = static_cast<uint64_t>(t) * width;
    for (uint32_t i = threadIdx.x; i < rot_pieces; i += blockDim.x) {
        const uint32_t h = i / ppw, p = i % ppw;
        const uint32_t partner = p < hp ? p + hp : p - hp;
        const uint4 ov = part ? rope_apply(qkv_piece(row, part, splits, part_stride, row0, h * head_dim + p * 8),
                                           qkv_piece(row, part, splits, part_stride, row0, h * head_dim + partner * 8),
                                           *reinterpret_cast<const uint4 *>(c + p * 8),
                                           *reinterpret_cast<const uint4 *>(s + p * 8), p < hp)
                              : rope_piece(row + h * head_dim, c, s, p, hp);
        if (h < n_heads)
            *reinterpret_cast<uint4 *>(q_out + (static_cast<uint64_t>(t) * n_heads + h) * head_dim + p * 8) = ov;
        else
            *reinterpret_cast<uint4 *>(k_cache + static_cast<uint64_t>(h - n_heads) * max_len * head_dim +
                                       k_offset(pos, p * 8, max_len, head_dim)) = ov;
    }
    const uint16_t *vrow = row + rot_pieces * 8;
    for (uint32_t i = threadIdx.x; i < n_kv * ppw; i += blockDim.x) {
        const uint32_t kh = i / ppw, p = i % ppw;
        *reinterpret_cast<uint4 *>(v_cache + (static_cast<uint64_t>(kh) * max_len + pos) * head_dim + p * 8) =
            qkv_piece(vrow, part, splits, part_stride, row0 + rot_pieces * 8, i * 8);
    }
}

// out = RNE(RNE(g / (1 + exp(-g))) * u) (silu_mul1), gu row = [g (F) | u (F)].
// Block (256 pieces of 8 outputs, row): with vec (f % 8 == 0, operands
// 16-byte aligned) a thread reads 16 bytes of g and of u and writes 16
// bytes; otherwise it walks its 8 outputs one at a time. Rows past the grid's
// y extent (65535) loop.

// With part (vec only), g and u are formed from the f32 partials of the
// gate/up GEMM (split_sum8), which stands in for its reduce.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ gu, uint32_t f, uint32_t rows,
                                                       int vec, uint16_t *__restrict__ out,
                                                       const float *__restrict__ part, uint32_t splits,
                                                       uint64_t part_stride) {
    const uint32_t c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (c0 >= f) return;
    for (uint32_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const uint16_t *g = gu + static_cast<uint64_t>(r) * 2 * f;
        const uint16_t *u = g + f;
        uint16_t *o = out + static_cast<uint64_t>(r) * f;
        if (vec) {
            const uint64_t gi = static_cast<uint64_t>(r) * 2 * f + c0;
            const uint4 gv = part ? split_sum8(part, splits, part_stride, gi) : *reinterpret_cast<const uint4 *>(g + c0);
            const uint4 uv = part ? split_sum8(part, splits, part_stride, gi + f) : *reinterpret_cast<const uint4 *>(u + c0);
            const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
            uint32_t ow[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ow[e] = silu_mul1(gw[e] & 0xFFFFu, uw[e] & 0xFFFFu) |
                        (static_cast<uint32_t>(silu_mul1(gw[e] >> 16, uw[e] >> 16)) << 16);
            *reinterpret_cast<uint4 *>(o + c0) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
        } else {
            for (uint32_t c = c0; c < c0 + 8 && c < f; ++c) o[c] = silu_mul1(g[c], u[c]);
        }
    }
}

// Row argmax of bf16 values; ties go to the lowest index. One block of 1024
// threads per row, 16-byte loads (8 values) per thread per step.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ void take_max(float &best, uint32_t &idx, float v, uint32_t i) {
    if (v > best || (v == best && i < idx)) {
        best = v;
        idx = i;
    }
}

// Per thread, kArgmaxBatch 16-byte loads are issued together before any is
// compared, so a row costs one or two memory round trips instead of one per
// load. The loads are unconditional (indices past the row are clamped to its
// last piece and ignored): a guarded load sits in its own basic block, where
// the compiler drains every outstanding load before issuing it. Lanes then
// wavefronts reduce with the same (max, lowest index) rule.
constexpr int kArgmaxBatch = 16;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const uint16_t *__restrict__ x, uint32_t n,
                                                                uint32_t *__restrict__ out) {
    __shared__ float bv[kArgmaxThreads / 64];
    __shared__ uint32_t bi[kArgmaxThreads / 64];
    const uint16_t *row = x + static_cast<uint64_t>(blockIdx.x) * n;
    float best = -INFINITY;
    uint32_t idx = 0xFFFFFFFFu;
    const bool aligned = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
    const uint32_t pieces = aligned ? n / 8 : 0;
    for (uint32_t p0 = 0; p0 < pieces; p0 += kArgmaxThreads * kArgmaxBatch) {
        uint4 v[kArgmaxBatch];
#pragma unroll
        for (int u = 0; u < kArgmaxBatch; ++u) {
            const uint32_t p = min(p0 + u * kArgmaxThreads + threadIdx.x, pieces - 1);
            v[u] = *reinterpret_cast<const uint4 *>(row + static_cast<uint64_t>(p) * 8);
        }
#pragma unroll
        for (int u = 0; u < kArgmaxBatch; ++u) {
            const uint32_t p = p0 + u * kArgmaxThreads + threadIdx.x;
            if (p < pieces) {
                const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    take_max(best, idx, bf(w[e] & 0xFFFFu), p * 8 + 2 * e);
                    take_max(best, idx, bf(w[e] >> 16), p * 8 + 2 * e + 1);
                }
            }
        }
    }
    for (uint32_t i = pieces * 8 + threadIdx.x; i < n; i += kArgmaxThreads) take_max(best, idx, bf(row[i]), i);
    if (idx == 0xFFFFFFFFu) best = -INFINITY;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const uint32_t oi = __shfl_xor(idx, off, 64);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    const uint32_t wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) {
                best = bv[w];
                idx = bi[w];
            }
        out[blockIdx.x] = idx == 0xFFFFFFFFu ? 0u : idx;
    }
}

// log[position - base] = token when that index is below capacity.
__global__ void append_token_kernel(const uint32_t *__restrict__ token, uint32_t rows,
                                    uint32_t *__restrict__ log, const uint32_t *__restrict__ position,
                                    uint32_t base, uint32_t capacity) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint32_t p = position[r], idx = p - base;
    if (p >= base && idx < capacity) log[static_cast<uint64_t>(r) * capacity + idx] = token[r];
}

__global__ void advance_kernel(uint32_t *__restrict__ p, uint32_t n, uint32_t by) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] += by;
}

// append_token_kernel, then position += by, in one launch: thread r reads its
// token and position before it writes the advanced position, so the two may
// share memory (no __restrict__ on them).
__global__ void append_advance_kernel(const uint32_t *token, uint32_t rows, uint32_t *__restrict__ log,
                                      uint32_t *position, uint32_t base, uint32_t capacity, uint32_t by) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint32_t p = position[r], t = token[r], idx = p - base;
    if (p >= base && idx < capacity) log[static_cast<uint64_t>(r) * capacity + idx] = t;
    position[r] = p + by;
}

// Long aligned rows take two passes: kArgmaxSegs blocks per row each reduce
// one segment to (value bits, index) in the device's partial area, then one
// wavefront per row picks the winner among the segments. (max, lowest index)
// orders all non-NaN values totally, so the winner is the one-block kernel's;
// NaN is never taken, and a row of NaN gives index 0 in both.
constexpr uint32_t kArgmaxSegs = 64;
constexpr int kArgmaxSegThreads = 256;
constexpr uint32_t kArgmaxTwoPassMinN = 16384;

__global__ __launch_bounds__(kArgmaxSegThreads) void argmax_seg_kernel(const uint16_t *__restrict__ x, uint32_t n,
                                                                       uint32_t seg_pieces, uint2 *__restrict__ part) {
    __shared__ float bv[kArgmaxSegThreads / 64];
    __shared__ uint32_t bi[kArgmaxSegThreads / 64];
    const uint16_t *row = x + static_cast<uint64_t>(blockIdx.y) * n;
    const uint32_t pieces = n / 8, p0 = blockIdx.x * seg_pieces;
    const uint32_t p1 = p0 + seg_pieces < pieces ? p0 + seg_pieces : pieces;
    float best = -INFINITY;
    uint32_t idx = 0xFFFFFFFFu;
    for (uint32_t p = p0 + threadIdx.x; p < p1; p += kArgmaxSegThreads) {
        const uint4 v = *reinterpret_cast<const uint4 *>(row + static_cast<uint64_t>(p) * 8);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            take_max(best, idx, bf(w[e] & 0xFFFFu), p * 8 + 2 * e);
            take_max(best, idx, bf(w[e] >> 16), p * 8 + 2 * e + 1);
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const uint32_t oi = __shfl_xor(idx, off, 64);
        take_max(best, idx, ov, oi);
    }
    const uint32_t wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxSegThreads / 64; ++w) take_max(best, idx, bv[w], bi[w]);
        if (idx == 0xFFFFFFFFu) best = -INFINITY;
        part[static_cast<uint64_t>(blockIdx.y) * gridDim.x + blockIdx.x] = make_uint2(__float_as_uint(best), idx);
    }
}

__global__ __launch_bounds__(64) void argmax_join_kernel(const uint2 *__restrict__ part, uint32_t segs,
                                                         uint32_t *__restrict__ out) {
    float best = -INFINITY;
    uint32_t idx = 0xFFFFFFFFu;
    for (uint32_t sg = threadIdx.x; sg < segs; sg += 64) {
        const uint2 p = part[static_cast<uint64_t>(blockIdx.x) * segs + sg];
        take_max(best, idx, __uint_as_float(p.x), p.y);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const uint32_t oi = __shfl_xor(idx, off, 64);
        take_max(best, idx, ov, oi);
    }
    if (threadIdx.x == 0) out[blockIdx.x] = idx == 0xFFFFFFFFu ? 0u : idx;
}

// Launches for a consumer that stands in for a split GEMM's reduce (part:
// [splits][rows][width] f32, the operands checked by the caller).
void launch_rms_norm_partials(hipStream_t stream, const float *part, uint32_t splits, const uint16_t *res,
                              uint16_t *res_out, const uint16_t *w, uint32_t rows, uint32_t dim, float eps,
                              uint16_t *y) {
    hipLaunchKernelGGL(rms_norm_kernel<true>, dim3(rows), dim3(kNormThreads), 0, stream, nullptr, res, res_out, w,
                       dim, eps, 1.0f / static_cast<float>(dim), y, part, splits, static_cast<uint64_t>(rows) * dim);
}

void launch_silu_mul_partials(hipStream_t stream, const float *part, uint32_t splits, uint32_t rows, uint32_t f,
                              uint16_t *out) {
    const dim3 grid((f + 2047) / 2048, rows < 65535 ? rows : 65535);
    hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(256), 0, stream, nullptr, f, rows, 1, out, part, splits,
                       static_cast<uint64_t>(rows) * 2 * f);
}

}  // namespace fh

using namespace fh;

extern "C" int fh_rms_norm(fh_device *dev, const uint16_t *x, const uint16_t *residual,
                           uint16_t *residual_out, const uint16_t *weight, int64_t rows,
                           int64_t dim, float eps, uint16_t *y) {
    const char *fn = "fh_rms_norm";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {rows, dim})) return rc;
    if (rows == 0 || dim == 0) return FH_OK;
    if ((residual == nullptr) != (residual_out == nullptr))
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: residual and residual_out go together", fn);
    if (dim % 8 != 0 || dim > 8 * kNormThreads * kNormChunks)
        return fail(FH_ERR_UNSUPPORTED, "%s: dim %lld must be a multiple of 8 and at most %d", fn,
                    (long long)dim, 8 * kNormThreads * kNormChunks);
    for (const void *p : {static_cast<const void *>(x), static_cast<const void *>(residual),
                          static_cast<const void *>(residual_out), static_cast<const void *>(weight),
                          static_cast<const void *>(y)})
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
            return fail(FH_ERR_INVALID_ARGUMENT, "%s: operands must be 16-byte aligned", fn);
    const uint64_t bytes = static_cast<uint64_t>(rows) * dim * 2;
    if (int rc = check_range(dev, x, bytes, fn, "x")) return rc;
    if (residual) {
        if (int rc = check_range(dev, residual, bytes, fn, "residual")) return rc;
        if (int rc = check_range(dev, residual_out, bytes, fn, "residual_out")) return rc;
    }
    if (int rc = check_range(dev, weight, static_cast<uint64_t>(dim) * 2, fn, "weight")) return rc;
    if (int rc = check_range(dev, y, bytes, fn, "y")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    const float dim_inv = 1.0f / static_cast<float>(dim);
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(rms_norm_kernel<false>, dim3(static_cast<uint32_t>(rows)), dim3(kNormThreads), 0,
                           dev->stream, x, residual, residual_out, weight,
                           static_cast<uint32_t>(dim), eps, dim_inv, y, nullptr, 1u, uint64_t{0});
    });
}

namespace fh {

// fh_rope_kv, its qkv either bf16 (part null) or the f32 partials of a GEMM
// split over K: `splits` slices [tokens][width] that are part_stride floats
// apart inside the device's partial area.
int rope_kv(fh_device *dev, const char *fn, const uint16_t *qkv, const float *part, uint32_t splits,
            uint64_t part_stride, int64_t seq_tokens, int64_t n_heads, int64_t n_kv, int64_t head_dim,
            const uint16_t *cos_tab, const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
            uint16_t *k_cache, uint16_t *v_cache, int64_t max_len, uint16_t *q_out, int64_t batch) {
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {seq_tokens, n_heads, n_kv, head_dim, table_len, max_len, batch})) return rc;
    const int64_t tokens = seq_tokens * batch;  // batch sequences' rows, one after another
    if (tokens == 0) return FH_OK;
    if (tokens > 0x7FFFFFFFll) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: %lld rows", fn, (long long)tokens);
    if (n_kv == 0 || n_heads % n_kv != 0 || head_dim % 16 != 0 || head_dim == 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: heads %lld/%lld, head_dim %lld", fn,
                    (long long)n_heads, (long long)n_kv, (long long)head_dim);
    for (const void *p : {static_cast<const void *>(qkv), static_cast<const void *>(cos_tab),
                          static_cast<const void *>(sin_tab), static_cast<const void *>(k_cache),
                          static_cast<const void *>(v_cache), static_cast<const void *>(q_out)})
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
            return fail(FH_ERR_INVALID_ARGUMENT, "%s: operands must be 16-byte aligned", fn);
    const uint64_t width = static_cast<uint64_t>(n_heads + 2 * n_kv) * head_dim;
    if (part == nullptr) {
        if (int rc = check_range(dev, qkv, tokens * width * 2, fn, "qkv")) return rc;
    } else {
        const uintptr_t area = reinterpret_cast<uintptr_t>(dev->partial_area), at = reinterpret_cast<uintptr_t>(part);
        if (splits < 2 || splits > kMaxGemmSplits || part_stride < tokens * width || at < area || at % 16 != 0 ||
            (at - area) / 4 + (splits - 1) * part_stride + tokens * width > kPartialAreaBytes / 4)
            return fail(FH_ERR_INVALID_ARGUMENT, "%s: split partials outside the device's partial area", fn);
    }
    if (int rc = check_range(dev, cos_tab, static_cast<uint64_t>(table_len) * head_dim * 2, fn, "cos")) return rc;
    if (int rc = check_range(dev, sin_tab, static_cast<uint64_t>(table_len) * head_dim * 2, fn, "sin")) return rc;
    if (int rc = check_range(dev, positions, static_cast<uint64_t>(tokens) * 4, fn, "positions")) return rc;
    const uint64_t seq_cache = static_cast<uint64_t>(n_kv) * max_len * head_dim;  // elements per sequence
    if (int rc = check_range(dev, k_cache, batch * seq_cache * 2, fn, "k_cache")) return rc;
    if (int rc = check_range(dev, v_cache, batch * seq_cache * 2, fn, "v_cache")) return rc;
    if (int rc = check_range(dev, q_out, static_cast<uint64_t>(tokens) * n_heads * head_dim * 2, fn, "q_out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(rope_kv_kernel, dim3(static_cast<uint32_t>(tokens)), dim3(256), 0,
                           dev->stream, qkv, static_cast<uint32_t>(n_heads),
                           static_cast<uint32_t>(n_kv), static_cast<uint32_t>(head_dim), cos_tab,
                           sin_tab, static_cast<uint32_t>(table_len), positions, k_cache, v_cache,
                           static_cast<uint32_t>(max_len), q_out, part, splits, part_stride,
                           static_cast<uint32_t>(seq_tokens), seq_cache);
    });
}

}  // namespace fh

extern "C" int fh_rope_kv(fh_device *dev, const uint16_t *qkv, int64_t tokens, int64_t n_heads,
                          int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab,
                          const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
                          uint16_t *k_cache, uint16_t *v_cache, int64_t max_len,
                          uint16_t *q_out) {
    return fh::rope_kv(dev, "fh_rope_kv", qkv, nullptr, 1u, 0u, tokens, n_heads, n_kv, head_dim, cos_tab, sin_tab,
                       table_len, positions, k_cache, v_cache, max_len, q_out, 1);
}

extern "C" int fh_silu_mul(fh_device *dev, const uint16_t *gate_up, int64_t rows, int64_t f,
                           uint16_t *out) {
    const char *fn = "fh_silu_mul";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {rows, f})) return rc;
    if (rows == 0 || f == 0) return FH_OK;
    const uint64_t total = static_cast<uint64_t>(rows) * f;
    if (int rc = check_range(dev, gate_up, total * 4, fn, "gate_up")) return rc;
    if (int rc = check_range(dev, out, total * 2, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    const int vec = f % 8 == 0 && ((reinterpret_cast<uintptr_t>(gate_up) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
    const dim3 grid(static_cast<uint32_t>((f + 2047) / 2048), static_cast<uint32_t>(rows < 65535 ? rows : 65535));
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(256), 0, dev->stream, gate_up, static_cast<uint32_t>(f),
                           static_cast<uint32_t>(rows), vec, out, nullptr, 1u, uint64_t{0});
    });
}

extern "C" int fh_argmax(fh_device *dev, const uint16_t *x, int64_t rows, int64_t n, uint32_t *out) {
    const char *fn = "fh_argmax";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {rows, n})) return rc;
    if (rows == 0) return FH_OK;
    if (n == 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: argmax over an empty row", fn);
    if (int rc = check_range(dev, x, static_cast<uint64_t>(rows) * n * 2, fn, "x")) return rc;
    if (int rc = check_range(dev, out, static_cast<uint64_t>(rows) * 4, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    const bool two_pass = n >= kArgmaxTwoPassMinN && n % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                          rows <= 65535 && dev->partial_area != nullptr &&
                          static_cast<uint64_t>(rows) * kArgmaxSegs * sizeof(uint2) <= kPartialAreaBytes;
    if (two_pass) {
        const uint32_t pieces = static_cast<uint32_t>(n / 8);
        const uint32_t seg_pieces = (pieces + kArgmaxSegs - 1) / kArgmaxSegs;
        uint2 *part = static_cast<uint2 *>(dev->partial_area);
        return dispatch(dev, fn, [&] {
            hipLaunchKernelGGL(argmax_seg_kernel, dim3(kArgmaxSegs, static_cast<uint32_t>(rows)),
                               dim3(kArgmaxSegThreads), 0, dev->stream, x, static_cast<uint32_t>(n), seg_pieces, part);
            hipLaunchKernelGGL(argmax_join_kernel, dim3(static_cast<uint32_t>(rows)), dim3(64), 0, dev->stream,
                               static_cast<const uint2 *>(part), kArgmaxSegs, out);
        });
    }
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(argmax_kernel, dim3(static_cast<uint32_t>(rows)), dim3(kArgmaxThreads), 0,
                           dev->stream, x, static_cast<uint32_t>(n), out);
    });
}

extern "C" int fh_advance_positions(fh_device *dev, uint32_t *positions, int64_t n, int64_t by) {
    const char *fn = "fh_advance_positions";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {n, by})) return rc;
    if (n == 0) return FH_OK;
    if (int rc = check_range(dev, positions, static_cast<uint64_t>(n) * 4, fn, "positions")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(advance_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256),
                           0, dev->stream, positions, static_cast<uint32_t>(n),
                           static_cast<uint32_t>(by));
    });
}

extern "C" int fh_append_token(fh_device *dev, const uint32_t *token, int64_t rows, uint32_t *log,
                               const uint32_t *position, int64_t base, int64_t capacity) {
    const char *fn = "fh_append_token";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {rows, base, capacity})) return rc;
    if (rows == 0 || capacity == 0) return FH_OK;
    if (static_cast<uint64_t>(rows) * static_cast<uint64_t>(capacity) > 0xFFFFFFFFull)
        return fail(FH_ERR_UNSUPPORTED, "%s: rows * capacity must fit in 32 bits", fn);
    if (int rc = check_range(dev, token, static_cast<uint64_t>(rows) * 4, fn, "token")) return rc;
    if (int rc = check_range(dev, position, static_cast<uint64_t>(rows) * 4, fn, "position")) return rc;
    if (int rc = check_range(dev, log, static_cast<uint64_t>(rows) * capacity * 4, fn, "log")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(append_token_kernel, dim3(static_cast<uint32_t>((rows + 63) / 64)), dim3(64), 0,
                           dev->stream, token, static_cast<uint32_t>(rows), log, position,
                           static_cast<uint32_t>(base), static_cast<uint32_t>(capacity));
    });
}

extern "C" int fh_append_token_advance(fh_device *dev, const uint32_t *token, int64_t rows, uint32_t *log,
                                       uint32_t *position, int64_t base, int64_t capacity, int64_t by) {
    const char *fn = "fh_append_token_advance";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {rows, base, capacity, by})) return rc;
    if (rows == 0) return FH_OK;
    if (static_cast<uint64_t>(rows) * static_cast<uint64_t>(capacity) > 0xFFFFFFFFull)
        return fail(FH_ERR_UNSUPPORTED, "%s: rows * capacity must fit in 32 bits", fn);
    if (int rc = check_range(dev, token, static_cast<uint64_t>(rows) * 4, fn, "token")) return rc;
    if (int rc = check_range(dev, position, static_cast<uint64_t>(rows) * 4, fn, "position")) return rc;
    if (capacity > 0)
        if (int rc = check_range(dev, log, static_cast<uint64_t>(rows) * capacity * 4, fn, "log")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(append_advance_kernel, dim3(static_cast<uint32_t>((rows + 63) / 64)), dim3(64), 0,
                           dev->stream, token, static_cast<uint32_t>(rows), log, position,
                           static_cast<uint32_t>(base), static_cast<uint32_t>(capacity),
                           static_cast<uint32_t>(by));
    });
}
