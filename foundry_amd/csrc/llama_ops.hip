// Decoder-step ops around the q4 linears: residual add + RMSNorm, RoPE with
// the KV-cache write, attention, SiLU-and-multiply, argmax and the device-side
// position counter. They are the HIP counterparts of the reference's
// RmsNorm (src/nn/norm.rs:32-50), apply_rotary_pos_emb
// (src/models/llama/rotary_emb.rs:62-85), StaticCache::update
// (src/nn/kv_cache.rs:41-80), scaled_dot_product_attention
// (src/nn/attention.rs:23-60), Silu (src/nn/activation.rs:19-28) and the
// greedy argmax (src/generate/mod.rs:192-204; src/metal/kernels/reduce.metal:42-78).
//
// Each keeps the reference's bf16 rounding points (its tensors are bf16, and
// every op rounds its output): e.g. RMSNorm rounds x*scale to bf16 before the
// weight multiply, RoPE rounds x*cos and rot*sin before adding, attention
// rounds the scores and the probabilities to bf16. Where the reference runs
// several dispatches (about ten for RMSNorm, six for SiLU, twelve for SDPA)
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
constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;  // dim <= 256 * 8 * 4 = 8192

__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const uint16_t *__restrict__ x,
                                                                const uint16_t *__restrict__ res,
                                                                uint16_t *__restrict__ res_out,
                                                                const uint16_t *__restrict__ w,
                                                                uint32_t dim, float eps, float dim_inv,
                                                                uint16_t *__restrict__ y) {
    __shared__ float red[kNormThreads / 64];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * dim;
    const uint32_t pieces = dim / 8;
    float h[kNormChunks][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
        const uint32_t piece = threadIdx.x + c * kNormThreads;
        if (piece < pieces) {
            const uint4 xv = *reinterpret_cast<const uint4 *>(x + base + piece * 8);
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
            const uint4 wv = *reinterpret_cast<const uint4 *>(w + piece * 8);
            const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
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
__global__ __launch_bounds__(256) void rope_kv_kernel(
    const uint16_t *__restrict__ qkv, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim,
    const uint16_t *__restrict__ cos_tab, const uint16_t *__restrict__ sin_tab, uint32_t table_len,
    const uint32_t *__restrict__ positions, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, uint32_t max_len, uint16_t *__restrict__ q_out) {
    const uint32_t t = blockIdx.x;
    const uint32_t pos = positions[t];
    // positions are device data the host cannot check: a position outside the
    // cache or the tables writes nothing
    if (pos >= max_len || pos >= table_len) return;
    const uint32_t width = (n_heads + 2 * n_kv) * head_dim;
    const uint16_t *row = qkv + static_cast<uint64_t>(t) * width;
    const uint16_t *c = cos_tab + static_cast<uint64_t>(pos) * head_dim;
    const uint16_t *s = sin_tab + static_cast<uint64_t>(pos) * head_dim;
    const uint32_t ppw = head_dim / 8, hp = ppw / 2;  // pieces per head, per half
    const uint32_t rot_pieces = (n_heads + n_kv) * ppw;
    for (uint32_t i = threadIdx.x; i < rot_pieces; i += blockDim.x) {
        const uint32_t h = i / ppw, p = i % ppw;
        const uint4 ov = rope_piece(row + h * head_dim, c, s, p, hp);
        if (h < n_heads)
            *reinterpret_cast<uint4 *>(q_out + (static_cast<uint64_t>(t) * n_heads + h) * head_dim + p * 8) = ov;
        else
            *reinterpret_cast<uint4 *>(k_cache + (static_cast<uint64_t>(h - n_heads) * max_len + pos) * head_dim + p * 8) = ov;
    }
    const uint16_t *vrow = row + rot_pieces * 8;
    for (uint32_t i = threadIdx.x; i < n_kv * ppw; i += blockDim.x) {
        const uint32_t kh = i / ppw, p = i % ppw;
        *reinterpret_cast<uint4 *>(v_cache + (static_cast<uint64_t>(kh) * max_len + pos) * head_dim + p * 8) =
            *reinterpret_cast<const uint4 *>(vrow + i * 8);
    }
}

// Split-context attention. The keys 0..ctx-1 of a (token, KV head) are cut
// into chunks of kAttnChunk keys, dealt round-robin to `splits` blocks; block
// (KV head, split, token) serves all G = n_heads / n_kv query heads of its KV
// head, so a K or V row is read once per chunk for the whole group. splits
// is chosen so that tokens * n_kv * splits is about kAttnTargetBlocks: decode
// (one token) spreads its context over many blocks, prefill (many tokens)
// keeps one block per (token, KV head) and needs no cross-block combine.
// Two kernels, because the reference rounds each probability to bf16 from
// the GLOBAL max and sum of its row:
//   attn_scores_kernel: s_j = RNE(q.k_j) * scale, written to the workspace
//     with each chunk's (m_c = max s_j, l_c = sum exp(s_j - m_c)).
//   attn_pv_kernel: M = max m_c, S = sum l_c exp(m_c - M), p_j =
//     RNE(exp(s_j - M) / S) as the reference forms them, and the block's
//     partial sum_j p_j v_j over its chunks. With one active split the block
//     writes RNE of it; otherwise the last block of the (token, KV head) to
//     finish (a completion counter in the workspace) adds the partials in
//     split order, writes RNE(sum) and re-arms the counter at zero, so the
//     result does not depend on block timing.
// A key row of HD bf16 is read by HD/8 lanes with 16-byte loads: one
// wavefront load covers 64/(HD/8) whole keys.
constexpr int kAttnChunk = 128;
constexpr int kAttnMaxGroup = 8;
constexpr int kAttnThreads = 256;
constexpr uint64_t kAttnTargetBlocks = 512;

struct AttnLayout {
    uint64_t nck, splits, stats, scores, partial, total;  // byte offsets; counters at 0
};

static AttnLayout attn_layout(uint64_t tokens, uint64_t n_heads, uint64_t n_kv, uint64_t head_dim,
                              uint64_t max_len) {
    auto round_up = [](uint64_t b) { return (b + 255) & ~static_cast<uint64_t>(255); };
    AttnLayout a;
    a.nck = (max_len + kAttnChunk - 1) / kAttnChunk;
    const uint64_t rows = tokens * n_kv;
    const uint64_t want = rows ? (kAttnTargetBlocks + rows - 1) / rows : 1;
    a.splits = want < a.nck ? want : a.nck;
    if (a.splits == 0) a.splits = 1;
    a.stats = round_up(tokens * n_kv * 4);
    a.scores = a.stats + round_up(tokens * n_heads * a.nck * 8);
    a.partial = a.scores + round_up(tokens * n_heads * max_len * 4);
    a.total = a.partial + (a.splits > 1 ? round_up(tokens * n_heads * a.splits * head_dim * 4) : 0);
    return a;
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k_cache,
    const uint32_t *__restrict__ positions, uint32_t n_heads, uint32_t n_kv, uint32_t max_len,
    uint32_t nck, uint32_t splits, float scale, float *__restrict__ scores, float2 *__restrict__ stats) {
    constexpr int LPK = HD / 8, KPI = 64 / LPK, IT = kAttnChunk / 4 / KPI;
    __shared__ float sc[kAttnMaxGroup][kAttnChunk];
    const uint32_t t = blockIdx.y, kvh = blockIdx.x / splits, split = blockIdx.x % splits;
    // keys 0..pos, never past the cache (positions are unchecked device data)
    const uint32_t ctx = positions[t] < max_len ? positions[t] + 1 : max_len;
    const uint32_t nact = (ctx + kAttnChunk - 1) / kAttnChunk;
    if (split >= nact) return;
    const uint32_t G = n_heads / n_kv, h0 = kvh * G;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t ks = lane / LPK, li = lane % LPK;
    const uint16_t *kb = k_cache + static_cast<uint64_t>(kvh) * max_len * HD + li * 8;
    float qf[kAttnMaxGroup][8];
#pragma unroll
    for (int g = 0; g < kAttnMaxGroup; ++g)
        if (g < static_cast<int>(G))
            unpack8(*reinterpret_cast<const uint4 *>(q + (static_cast<uint64_t>(t) * n_heads + h0 + g) * HD + li * 8),
                    qf[g]);
    for (uint32_t c = split; c < nact; c += splits) {
        const uint32_t j0 = c * kAttnChunk;
        const uint32_t jw = j0 + wave * (kAttnChunk / 4) + ks;
        uint4 kr[IT];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const uint32_t j = jw + it * KPI;
            kr[it] = j < ctx ? *reinterpret_cast<const uint4 *>(kb + static_cast<uint64_t>(j) * HD)
                             : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            float kf[8];
            unpack8(kr[it], kf);
            const uint32_t j = jw + it * KPI;
#pragma unroll
            for (int g = 0; g < kAttnMaxGroup; ++g) {
                if (g < static_cast<int>(G)) {
                    float d = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d += qf[g][e] * kf[e];
#pragma unroll
                    for (int off = 1; off < LPK; off <<= 1) d += __shfl_xor(d, off, 64);
                    if (li == 0) sc[g][j - j0] = j < ctx ? bf(rne(d)) * scale : -INFINITY;
                }
            }
        }
        __syncthreads();
        static_assert(kAttnChunk == 128, "statistics pass assumes two scores per lane");
        for (uint32_t g = wave; g < G; g += 4) {
            const float a = sc[g][lane], b = sc[g][lane + 64];
            const float m = wave_max(fmaxf(a, b));
            const float l = wave_sum(expf(a - m) + expf(b - m));
            if (lane == 0) stats[(static_cast<uint64_t>(t) * n_heads + h0 + g) * nck + c] = make_float2(m, l);
        }
        const uint32_t valid = min(ctx - j0, static_cast<uint32_t>(kAttnChunk));
        for (uint32_t i = threadIdx.x; i < G * kAttnChunk; i += kAttnThreads) {
            const uint32_t g = i / kAttnChunk, jj = i % kAttnChunk;
            if (jj < valid) scores[(static_cast<uint64_t>(t) * n_heads + h0 + g) * max_len + j0 + jj] = sc[g][jj];
        }
        __syncthreads();  // sc is rewritten by the next chunk
    }
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_pv_kernel(
    const uint16_t *__restrict__ v_cache, const uint32_t *__restrict__ positions, uint32_t n_heads,
    uint32_t n_kv, uint32_t max_len, uint32_t nck, uint32_t splits, const float *__restrict__ scores,
    const float2 *__restrict__ stats, float *__restrict__ partial, uint32_t *__restrict__ counters,
    uint16_t *__restrict__ out) {
    constexpr int LPK = HD / 8, KPI = 64 / LPK, IT = kAttnChunk / 4 / KPI;
    __shared__ float p[kAttnMaxGroup][kAttnChunk];
    __shared__ float wsum[4][kAttnMaxGroup * HD];
    __shared__ float mg[kAttnMaxGroup], sg[kAttnMaxGroup];
    __shared__ uint32_t is_last;
    const uint32_t t = blockIdx.y, kvh = blockIdx.x / splits, split = blockIdx.x % splits;
    const uint32_t ctx = positions[t] < max_len ? positions[t] + 1 : max_len;
    const uint32_t nact = (ctx + kAttnChunk - 1) / kAttnChunk;
    if (split >= nact) return;
    const uint32_t nsp = min(splits, nact);  // splits holding at least one chunk
    const uint32_t G = n_heads / n_kv, h0 = kvh * G;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t ks = lane / LPK, li = lane % LPK;
    const uint16_t *vb = v_cache + static_cast<uint64_t>(kvh) * max_len * HD + li * 8;
    for (uint32_t g = wave; g < G; g += 4) {
        const float2 *st = stats + (static_cast<uint64_t>(t) * n_heads + h0 + g) * nck;
        float m = -INFINITY;
        for (uint32_t cc = lane; cc < nact; cc += 64) m = fmaxf(m, st[cc].x);
        m = wave_max(m);
        float s = 0.f;
        for (uint32_t cc = lane; cc < nact; cc += 64) {
            const float2 v = st[cc];
            s += v.y * expf(v.x - m);
        }
        s = wave_sum(s);
        if (lane == 0) {
            mg[g] = m;
            sg[g] = s;
        }
    }
    float acc[kAttnMaxGroup][8];
#pragma unroll
    for (int g = 0; g < kAttnMaxGroup; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    for (uint32_t c = split; c < nact; c += splits) {
        const uint32_t j0 = c * kAttnChunk;
        // V rows first: they do not depend on the probabilities
        const uint32_t jw = j0 + wave * (kAttnChunk / 4) + ks;
        uint4 vr[IT];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const uint32_t j = jw + it * KPI;
            vr[it] = j < ctx ? *reinterpret_cast<const uint4 *>(vb + static_cast<uint64_t>(j) * HD)
                             : make_uint4(0u, 0u, 0u, 0u);
        }
        __syncthreads();  // mg/sg written; p free from the previous chunk
        const uint32_t valid = min(ctx - j0, static_cast<uint32_t>(kAttnChunk));
        for (uint32_t i = threadIdx.x; i < G * kAttnChunk; i += kAttnThreads) {
            const uint32_t g = i / kAttnChunk, jj = i % kAttnChunk;
            float v = 0.f;
            if (jj < valid)
                v = bf(rne(expf(scores[(static_cast<uint64_t>(t) * n_heads + h0 + g) * max_len + j0 + jj] - mg[g]) /
                           sg[g]));
            p[g][jj] = v;
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            float vf[8];
            unpack8(vr[it], vf);
            const uint32_t jj = wave * (kAttnChunk / 4) + it * KPI + ks;
#pragma unroll
            for (int g = 0; g < kAttnMaxGroup; ++g) {
                if (g < static_cast<int>(G)) {
                    const float pg = p[g][jj];
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[g][e] += pg * vf[e];
                }
            }
        }
    }
    // sum over the key slots of the wavefront, then over the four wavefronts
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1)
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g)
            if (g < static_cast<int>(G))
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[g][e] += __shfl_xor(acc[g][e], off, 64);
    if (ks == 0) {
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g)
            if (g < static_cast<int>(G))
#pragma unroll
                for (int e = 0; e < 8; ++e) wsum[wave][g * HD + li * 8 + e] = acc[g][e];
    }
    __syncthreads();
    uint16_t *orow = out + (static_cast<uint64_t>(t) * n_heads + h0) * HD;
    float *part = partial + (static_cast<uint64_t>(t) * n_kv + kvh) * splits * G * HD;
    for (uint32_t i = threadIdx.x; i < G * HD; i += kAttnThreads) {
        const float v = wsum[0][i] + wsum[1][i] + wsum[2][i] + wsum[3][i];
        if (nsp == 1)
            orow[i] = rne(v);
        else
            part[static_cast<uint64_t>(split) * G * HD + i] = v;
    }
    if (nsp == 1) return;
    // publish this split's partial, then count it; the last split to arrive
    // combines
    __threadfence();
    __syncthreads();
    uint32_t *counter = counters + static_cast<uint64_t>(t) * n_kv + kvh;
    if (threadIdx.x == 0)
        is_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == nsp - 1;
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (uint32_t i = threadIdx.x; i < G * HD; i += kAttnThreads) {
        float s = 0.f;
        for (uint32_t sp = 0; sp < nsp; ++sp) s += part[static_cast<uint64_t>(sp) * G * HD + i];
        orow[i] = rne(s);
    }
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// out = RNE(RNE(g / (1 + exp(-g))) * u), gu row = [g (F) | u (F)].
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ gu, uint32_t f,
                                                       uint64_t total, uint16_t *__restrict__ out) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const uint64_t r = i / f, c = i % f;
    const float g = bf(gu[r * 2 * f + c]);
    const float u = bf(gu[r * 2 * f + f + c]);
    const float den = expf(-g) + 1.0f;
    out[i] = rne(bf(rne(g / den)) * u);
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

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const uint16_t *__restrict__ x, uint32_t n,
                                                                uint32_t *__restrict__ out) {
    __shared__ float bv[kArgmaxThreads];
    __shared__ uint32_t bi[kArgmaxThreads];
    const uint16_t *row = x + static_cast<uint64_t>(blockIdx.x) * n;
    float best = -INFINITY;
    uint32_t idx = 0xFFFFFFFFu;
    const uint32_t pieces = n / 8;
    const bool aligned = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
    if (aligned) {
        for (uint32_t p = threadIdx.x; p < pieces; p += kArgmaxThreads) {
            const uint4 v = *reinterpret_cast<const uint4 *>(row + p * 8);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                take_max(best, idx, bf(w[e] & 0xFFFFu), p * 8 + 2 * e);
                take_max(best, idx, bf(w[e] >> 16), p * 8 + 2 * e + 1);
            }
        }
    }
    for (uint32_t i = (aligned ? pieces * 8 : 0) + threadIdx.x; i < n; i += kArgmaxThreads)
        take_max(best, idx, bf(row[i]), i);
    if (idx == 0xFFFFFFFFu) best = -INFINITY;
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (uint32_t off = kArgmaxThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) {
            const float ov = bv[threadIdx.x + off];
            const uint32_t oi = bi[threadIdx.x + off];
            if (ov > bv[threadIdx.x] || (ov == bv[threadIdx.x] && oi < bi[threadIdx.x])) {
                bv[threadIdx.x] = ov;
                bi[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = bi[0] == 0xFFFFFFFFu ? 0u : bi[0];
}

// log[position - base] = token when that index is below capacity.
__global__ void append_token_kernel(const uint32_t *__restrict__ token, uint32_t *__restrict__ log,
                                    const uint32_t *__restrict__ position, uint32_t base,
                                    uint32_t capacity) {
    const uint32_t idx = position[0] - base;
    if (position[0] >= base && idx < capacity) log[idx] = token[0];
}

__global__ void advance_kernel(uint32_t *__restrict__ p, uint32_t n, uint32_t by) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] += by;
}

}  // namespace fh

using namespace fh;

namespace {

// The workspace holds at most tokens * n_heads * (3 max_len + head_dim)
// floats (scores, chunk partials); refuse sizes whose byte counts would not
// fit comfortably in 64 bits.
int check_attn_size(const char *fn, int64_t tokens, int64_t n_heads, int64_t head_dim, int64_t max_len) {
    const long double floats = static_cast<long double>(tokens) * n_heads * (3.0L * max_len + head_dim);
    if (floats > 0x1p56L)
        return fail(FH_ERR_INDEX_TOO_LARGE, "%s: attention workspace for %lld tokens x %lld heads x %lld "
                    "keys is too large", fn, (long long)tokens, (long long)n_heads, (long long)max_len);
    return FH_OK;
}

}  // namespace

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
        hipLaunchKernelGGL(rms_norm_kernel, dim3(static_cast<uint32_t>(rows)), dim3(kNormThreads), 0,
                           dev->stream, x, residual, residual_out, weight,
                           static_cast<uint32_t>(dim), eps, dim_inv, y);
    });
}

extern "C" int fh_rope_kv(fh_device *dev, const uint16_t *qkv, int64_t tokens, int64_t n_heads,
                          int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab,
                          const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
                          uint16_t *k_cache, uint16_t *v_cache, int64_t max_len,
                          uint16_t *q_out) {
    const char *fn = "fh_rope_kv";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {tokens, n_heads, n_kv, head_dim, table_len, max_len})) return rc;
    if (tokens == 0) return FH_OK;
    if (n_kv == 0 || n_heads % n_kv != 0 || head_dim % 16 != 0 || head_dim == 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: heads %lld/%lld, head_dim %lld", fn,
                    (long long)n_heads, (long long)n_kv, (long long)head_dim);
    for (const void *p : {static_cast<const void *>(qkv), static_cast<const void *>(cos_tab),
                          static_cast<const void *>(sin_tab), static_cast<const void *>(k_cache),
                          static_cast<const void *>(v_cache), static_cast<const void *>(q_out)})
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
            return fail(FH_ERR_INVALID_ARGUMENT, "%s: operands must be 16-byte aligned", fn);
    const uint64_t width = static_cast<uint64_t>(n_heads + 2 * n_kv) * head_dim;
    if (int rc = check_range(dev, qkv, tokens * width * 2, fn, "qkv")) return rc;
    if (int rc = check_range(dev, cos_tab, static_cast<uint64_t>(table_len) * head_dim * 2, fn, "cos")) return rc;
    if (int rc = check_range(dev, sin_tab, static_cast<uint64_t>(table_len) * head_dim * 2, fn, "sin")) return rc;
    if (int rc = check_range(dev, positions, static_cast<uint64_t>(tokens) * 4, fn, "positions")) return rc;
    const uint64_t cache = static_cast<uint64_t>(n_kv) * max_len * head_dim * 2;
    if (int rc = check_range(dev, k_cache, cache, fn, "k_cache")) return rc;
    if (int rc = check_range(dev, v_cache, cache, fn, "v_cache")) return rc;
    if (int rc = check_range(dev, q_out, static_cast<uint64_t>(tokens) * n_heads * head_dim * 2, fn, "q_out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(rope_kv_kernel, dim3(static_cast<uint32_t>(tokens)), dim3(256), 0,
                           dev->stream, qkv, static_cast<uint32_t>(n_heads),
                           static_cast<uint32_t>(n_kv), static_cast<uint32_t>(head_dim), cos_tab,
                           sin_tab, static_cast<uint32_t>(table_len), positions, k_cache, v_cache,
                           static_cast<uint32_t>(max_len), q_out);
    });
}

extern "C" int fh_attention_workspace(int64_t tokens, int64_t n_heads, int64_t n_kv, int64_t head_dim,
                                      int64_t max_len, uint64_t *bytes) {
    const char *fn = "fh_attention_workspace";
    if (!bytes) return fail(FH_ERR_INVALID_ARGUMENT, "%s: null output", fn);
    if (int rc = fh_check_dims(fn, {tokens, n_heads, n_kv, head_dim, max_len})) return rc;
    if (int rc = check_attn_size(fn, tokens, n_heads, head_dim, max_len)) return rc;
    *bytes = attn_layout(tokens, n_heads, n_kv, head_dim, max_len).total;
    return FH_OK;
}

template <int HD>
static void launch_attention(hipStream_t stream, dim3 grid, const uint16_t *q, const uint16_t *k_cache,
                             const uint16_t *v_cache, const uint32_t *positions, uint32_t n_heads,
                             uint32_t n_kv, uint32_t max_len, uint32_t nck, float scale, char *ws,
                             const AttnLayout &a, uint16_t *out) {
    auto *counters = reinterpret_cast<uint32_t *>(ws);
    auto *stats = reinterpret_cast<float2 *>(ws + a.stats);
    auto *scores = reinterpret_cast<float *>(ws + a.scores);
    auto *partial = reinterpret_cast<float *>(ws + a.partial);
    const uint32_t splits = static_cast<uint32_t>(a.splits);
    hipLaunchKernelGGL(attn_scores_kernel<HD>, grid, dim3(kAttnThreads), 0, stream, q, k_cache, positions,
                       n_heads, n_kv, max_len, nck, splits, scale, scores, stats);
    hipLaunchKernelGGL(attn_pv_kernel<HD>, grid, dim3(kAttnThreads), 0, stream, v_cache, positions, n_heads,
                       n_kv, max_len, nck, splits, scores, stats, partial, counters, out);
}

extern "C" int fh_attention(fh_device *dev, const uint16_t *q, const uint16_t *k_cache,
                            const uint16_t *v_cache, const uint32_t *positions, int64_t tokens,
                            int64_t n_heads, int64_t n_kv, int64_t head_dim, int64_t max_len,
                            float scale, void *workspace, uint64_t workspace_bytes, uint16_t *out) {
    const char *fn = "fh_attention";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {tokens, n_heads, n_kv, head_dim, max_len})) return rc;
    if (tokens == 0) return FH_OK;
    if (n_kv == 0 || n_heads % n_kv != 0 || n_heads / n_kv > kAttnMaxGroup ||
        (head_dim != 64 && head_dim != 128 && head_dim != 256))
        return fail(FH_ERR_UNSUPPORTED, "%s: heads %lld/%lld, head_dim %lld", fn, (long long)n_heads,
                    (long long)n_kv, (long long)head_dim);
    if (max_len == 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: empty KV cache", fn);
    if (int rc = check_attn_size(fn, tokens, n_heads, head_dim, max_len)) return rc;
    const AttnLayout a = attn_layout(tokens, n_heads, n_kv, head_dim, max_len);
    if (tokens > 65535 || static_cast<uint64_t>(n_kv) * a.splits > 0x7FFFFFFFu)
        return fail(FH_ERR_INDEX_TOO_LARGE, "%s: %lld tokens x %llu splits exceed the grid", fn,
                    (long long)tokens, (unsigned long long)(n_kv * a.splits));
    if (workspace_bytes < a.total)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: workspace of %llu bytes, %llu needed", fn,
                    (unsigned long long)workspace_bytes, (unsigned long long)a.total);
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
         reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(workspace)) & 15u)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: q, caches and workspace must be 16-byte aligned", fn);
    const uint64_t cache = static_cast<uint64_t>(n_kv) * max_len * head_dim * 2;
    if (int rc = check_range(dev, q, static_cast<uint64_t>(tokens) * n_heads * head_dim * 2, fn, "q")) return rc;
    if (int rc = check_range(dev, k_cache, cache, fn, "k_cache")) return rc;
    if (int rc = check_range(dev, v_cache, cache, fn, "v_cache")) return rc;
    if (int rc = check_range(dev, positions, static_cast<uint64_t>(tokens) * 4, fn, "positions")) return rc;
    if (int rc = check_range(dev, workspace, a.total, fn, "workspace")) return rc;
    if (int rc = check_range(dev, out, static_cast<uint64_t>(tokens) * n_heads * head_dim * 2, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    const dim3 grid(static_cast<uint32_t>(n_kv * a.splits), static_cast<uint32_t>(tokens));
    const uint32_t nh = static_cast<uint32_t>(n_heads), nk = static_cast<uint32_t>(n_kv),
                   ml = static_cast<uint32_t>(max_len), nck = static_cast<uint32_t>(a.nck);
    char *ws = static_cast<char *>(workspace);
    return dispatch(dev, fn, [&] {
        if (head_dim == 64)
            launch_attention<64>(dev->stream, grid, q, k_cache, v_cache, positions, nh, nk, ml, nck, scale, ws, a, out);
        else if (head_dim == 128)
            launch_attention<128>(dev->stream, grid, q, k_cache, v_cache, positions, nh, nk, ml, nck, scale, ws, a, out);
        else
            launch_attention<256>(dev->stream, grid, q, k_cache, v_cache, positions, nh, nk, ml, nck, scale, ws, a, out);
    });
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
    const uint32_t blocks = static_cast<uint32_t>((total + 255) / 256);
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(256), 0, dev->stream, gate_up,
                           static_cast<uint32_t>(f), total, out);
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

extern "C" int fh_append_token(fh_device *dev, const uint32_t *token, uint32_t *log,
                               const uint32_t *position, int64_t base, int64_t capacity) {
    const char *fn = "fh_append_token";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {base, capacity})) return rc;
    if (capacity == 0) return FH_OK;
    if (int rc = check_range(dev, token, 4, fn, "token")) return rc;
    if (int rc = check_range(dev, position, 4, fn, "position")) return rc;
    if (int rc = check_range(dev, log, static_cast<uint64_t>(capacity) * 4, fn, "log")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(append_token_kernel, dim3(1), dim3(1), 0, dev->stream, token, log, position,
                           static_cast<uint32_t>(base), static_cast<uint32_t>(capacity));
    });
}
