// Attention with the causal mask, split over the context: the HIP
// counterpart of scaled_dot_product_attention (src/nn/attention.rs:23-60,
// mask src/nn/masking.rs:11-32) with the reference's rounding points --
// scores RNE(q.k) (fp32 sums) times scale in fp32, fp32 softmax,
// probabilities RNE to bf16 from the row's GLOBAL max and sum, out =
// RNE(sum p v). Two entry points share the kernels:
//   fh_attention: the tokens of one sequence (prefill) over a shared cache,
//     after fh_rope_kv wrote their keys and values;
//   fh_decode_attention: a batch of sequences that each add one token, each
//     with its own cache; RoPE (src/models/llama/rotary_emb.rs:62-85) of the
//     token's q and k and its cache write (StaticCache::update,
//     src/nn/kv_cache.rs:41-80) happen inside the scores kernel.
//
// A row (a token, or a sequence) attends keys 0..ctx-1 of its KV head. Two
// kernels, because each probability is rounded from the row's global max and
// sum; neither combines across blocks (a device-scope fence per block costs
// an L2 write-back on this part), and every block serves the G = n_heads /
// n_kv query heads of its KV head, so a K or V row is read once for the group:
//   attn_scores_kernel, block (KV head, split, row): chunks of kAttnChunk keys
//     dealt round-robin to `splits` blocks; s_j = RNE(q.k_j) * scale to the
//     workspace with each chunk's (m_c = max s_j, l_c = sum exp(s_j - m_c)).
//     A key row of HD bf16 is read by HD/8 lanes with 16-byte loads (one
//     wavefront load covers 64 / (HD/8) whole keys); the lane partials are
//     summed with DPP moves.
//   attn_pv_kernel, block (KV head, slice, row): M = max m_c, S = sum l_c
//     exp(m_c - M) (the same in every block), p_j = RNE(exp(s_j - M) / S), and
//     sum_j p_j v_j over all keys for head_dim / slices of the dims, so each
//     output element comes from one block in a fixed order.
// splits and slices make rows * n_kv * splits about kAttnTargetBlocks: decode
// spreads one row over many CUs, prefill keeps one block per (row, KV head).
#include "decoder_common.hpp"

namespace fh {

constexpr int kAttnChunk = 64;
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kAttnMaxGroup = 8;
constexpr uint64_t kAttnTargetBlocks = 1024;

// Workspace: per-chunk softmax statistics [rows][n_heads][nck] float2, then
// the scores [rows][n_heads][max_len] f32. splits: blocks per (row, KV head)
// of the scores kernel; slices: blocks per (row, KV head) of the P.V kernel,
// each over head_dim / slices dims (at least 16).
struct AttnLayout {
    uint64_t nck, splits, slices, scores, total;  // stats at byte 0
};

static AttnLayout attn_layout(uint64_t rows, uint64_t n_heads, uint64_t n_kv, uint64_t head_dim,
                              uint64_t max_len) {
    auto round_up = [](uint64_t b) { return (b + 255) & ~static_cast<uint64_t>(255); };
    AttnLayout a;
    a.nck = (max_len + kAttnChunk - 1) / kAttnChunk;
    const uint64_t blocks = rows * n_kv;
    const uint64_t want = blocks ? (kAttnTargetBlocks + blocks - 1) / blocks : 1;
    a.splits = want < a.nck ? want : a.nck;
    if (a.splits == 0) a.splits = 1;
    a.slices = 1;
    while (a.slices * 2 <= want && head_dim / (a.slices * 2) >= 16) a.slices *= 2;
    a.scores = round_up(rows * n_heads * a.nck * 8);
    a.total = a.scores + round_up(rows * n_heads * max_len * 4);
    return a;
}

// ROPE: q_src is the qkv rows, the block rotates its q heads and the row's
// key, and the block owning key `pos` writes the key and value to the cache.
// Otherwise q_src is the rotated q [rows, n_heads * HD] and the cache is
// complete. Rows whose position is >= pos_limit are skipped (the PV kernel
// writes their zero output).
template <int HD, int G, bool ROPE>
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(
    const uint16_t *__restrict__ q_src, const uint16_t *__restrict__ cos_tab, const uint16_t *__restrict__ sin_tab,
    const uint32_t *__restrict__ positions, uint32_t pos_limit, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, uint64_t row_stride, uint32_t n_heads, uint32_t n_kv, uint32_t max_len,
    uint32_t nck, uint32_t splits, float scale, float *__restrict__ scores, float2 *__restrict__ stats) {
    constexpr int LPK = HD / 8, KPI = 64 / LPK, IT = kAttnChunk / kAttnWaves / KPI;
    constexpr uint32_t PPH = HD / 8;  // 8-dim pieces per head
    __shared__ float sc[G][kAttnChunk];
    __shared__ float qs[ROPE ? G : 1][ROPE ? HD : 1];
    __shared__ __align__(16) uint16_t knew[ROPE ? HD : 8];
    const uint32_t tid = threadIdx.x, r = blockIdx.y, kvh = blockIdx.x / splits, split = blockIdx.x % splits;
    const uint32_t pos = positions[r];
    if (pos >= pos_limit) return;
    const uint32_t ctx = pos < max_len ? pos + 1 : max_len;
    const uint32_t nact = (ctx + kAttnChunk - 1) / kAttnChunk;
    if (split >= nact) return;
    const uint32_t h0 = kvh * G;
    const uint32_t wave = tid >> 6, lane = tid & 63, ks = lane / LPK, li = lane % LPK;
    const uint64_t cache = static_cast<uint64_t>(r) * row_stride + static_cast<uint64_t>(kvh) * max_len * HD;
    // keys below kmax come from the cache; with ROPE key pos is the new one
    // (from LDS, substituted when the chunk is scored)
    const uint32_t kmax = ROPE ? pos : ctx;
    const uint16_t *kb = k_cache + cache + li * 8;
    auto load_chunk = [&](uint32_t c, uint4 (&kr)[IT]) {
        const uint32_t jw = c * kAttnChunk + wave * (kAttnChunk / kAttnWaves) + ks;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const uint32_t j = jw + it * KPI;
            kr[it] = j < kmax ? *reinterpret_cast<const uint4 *>(kb + static_cast<uint64_t>(j) * HD)
                              : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    uint4 kr[IT];
    load_chunk(split, kr);  // in flight during the q set-up
    float qf[G][8];
    uint4 kn = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (ROPE) {
        const uint16_t *row = q_src + static_cast<uint64_t>(r) * (n_heads + 2 * n_kv) * HD;
        const uint16_t *c = cos_tab + static_cast<uint64_t>(pos) * HD;
        const uint16_t *s = sin_tab + static_cast<uint64_t>(pos) * HD;
        const bool owner = (pos / kAttnChunk) % splits == split;
        if (tid < (G + 1) * PPH) {
            const uint32_t hh = tid / PPH, p = tid % PPH;  // hh < G: query head h0 + hh; hh == G: the key
            const uint16_t *head = row + static_cast<uint64_t>(hh < G ? h0 + hh : n_heads + kvh) * HD;
            const uint4 ov = rope_piece(head, c, s, p, PPH / 2);
            if (hh < G) {
                float f[8];
                unpack8(ov, f);
#pragma unroll
                for (int e = 0; e < 8; ++e) qs[hh][p * 8 + e] = f[e];
            } else {
                *reinterpret_cast<uint4 *>(knew + p * 8) = ov;
                if (owner) *reinterpret_cast<uint4 *>(k_cache + cache + static_cast<uint64_t>(pos) * HD + p * 8) = ov;
            }
        } else if (owner && tid < (G + 2) * PPH) {
            const uint32_t p = tid - (G + 1) * PPH;
            *reinterpret_cast<uint4 *>(v_cache + cache + static_cast<uint64_t>(pos) * HD + p * 8) =
                *reinterpret_cast<const uint4 *>(row + static_cast<uint64_t>(n_heads + n_kv + kvh) * HD + p * 8);
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[g][e] = qs[g][li * 8 + e];
        kn = *reinterpret_cast<const uint4 *>(knew + li * 8);
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g)
            unpack8(*reinterpret_cast<const uint4 *>(q_src + (static_cast<uint64_t>(r) * n_heads + h0 + g) * HD + li * 8),
                    qf[g]);
    }
    for (uint32_t c = split; c < nact; c += splits) {
        const uint32_t j0 = c * kAttnChunk;
        const uint32_t jw = j0 + wave * (kAttnChunk / kAttnWaves) + ks;
        uint4 next[IT];
        const bool more = c + splits < nact;
        if (more) load_chunk(c + splits, next);  // the next chunk's keys load while this one is scored
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const uint32_t j = jw + it * KPI;
            float kf[8];
            unpack8(ROPE && j == pos ? kn : kr[it], kf);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d += qf[g][e] * kf[e];
                d = group_sum<LPK>(d);
                if (li == 0) sc[g][j - j0] = j < ctx ? bf(rne(d)) * scale : -INFINITY;
            }
        }
        __syncthreads();
        static_assert(kAttnChunk == 64, "statistics pass assumes one score per lane");
        for (uint32_t g = wave; g < G; g += kAttnWaves) {
            const float x = sc[g][lane];
            const float m = wave_max(x);
            const float l = wave_sum(expf(x - m));
            if (lane == 0) stats[(static_cast<uint64_t>(r) * n_heads + h0 + g) * nck + c] = make_float2(m, l);
        }
        const uint32_t valid = min(ctx - j0, static_cast<uint32_t>(kAttnChunk));
        for (uint32_t i = tid; i < G * kAttnChunk; i += kAttnThreads) {
            const uint32_t g = i / kAttnChunk, jj = i % kAttnChunk;
            if (jj < valid) scores[(static_cast<uint64_t>(r) * n_heads + h0 + g) * max_len + j0 + jj] = sc[g][jj];
        }
        __syncthreads();  // sc is rewritten by the next chunk
        if (more)
#pragma unroll
            for (int it = 0; it < IT; ++it) kr[it] = next[it];
    }
}

// P.V over a slice of 2P dims of head_dim for all keys of the row: block
// (KV head, slice, row). Thread (pair q, key slot s) owns dims d0 + 2q, +1 and
// keys j = s, s + S, ... (S = 256 / P slots); tiles of T keys are staged as
// probabilities in LDS, then the slots' partial sums are added in slot order.
template <int P>
struct PvShape {
    static constexpr int kSlots = kAttnThreads / P;
    static constexpr int kLoads = P >= 32 ? 32 : P;  // loads per thread per tile
    static constexpr int kTile = kSlots * kLoads;    // keys per tile
};

template <int G, int P>
__global__ __launch_bounds__(kAttnThreads) void attn_pv_kernel(
    const uint16_t *__restrict__ v_cache, uint64_t row_stride, const uint32_t *__restrict__ positions,
    uint32_t pos_limit, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t max_len, uint32_t nck,
    uint32_t slices, const float *__restrict__ scores, const float2 *__restrict__ stats,
    uint16_t *__restrict__ out) {
    using S = PvShape<P>;
    __shared__ float p[G][S::kTile];
    __shared__ float red[kAttnThreads][G * 2];
    __shared__ float mg[G], sg[G];
    const uint32_t tid = threadIdx.x, r = blockIdx.y, kvh = blockIdx.x / slices, slice = blockIdx.x % slices;
    const uint32_t h0 = kvh * G, d0 = slice * 2 * P;
    uint16_t *orow = out + (static_cast<uint64_t>(r) * n_heads + h0) * head_dim + d0;
    const uint32_t pos = positions[r];
    if (pos >= pos_limit) {  // a position the cache or the tables cannot hold: zero output
        for (uint32_t i = tid; i < G * 2 * P; i += kAttnThreads) orow[(i / (2 * P)) * head_dim + i % (2 * P)] = 0;
        return;
    }
    const uint32_t ctx = pos < max_len ? pos + 1 : max_len;
    const uint32_t nact = (ctx + kAttnChunk - 1) / kAttnChunk;
    const uint32_t wave = tid >> 6, lane = tid & 63, q = tid % P, s = tid / P;
    const uint16_t *vb = v_cache + static_cast<uint64_t>(r) * row_stride + static_cast<uint64_t>(kvh) * max_len * head_dim +
                         d0 + 2 * q;
    const float *srow = scores + (static_cast<uint64_t>(r) * n_heads + h0) * max_len;
    // A tile: V of keys t0 + s + k * slots (this thread's dims) and the raw
    // scores of entries i = tid + n * 256 of the tile's [G][kTile] block.
    constexpr int NS = (G * S::kTile + kAttnThreads - 1) / kAttnThreads;
    auto load_tile = [&](uint32_t t0, uint32_t (&vr)[S::kLoads], float (&sr)[NS]) {
#pragma unroll
        for (int k = 0; k < S::kLoads; ++k) {
            const uint32_t j = t0 + s + k * S::kSlots;
            vr[k] = j < ctx ? *reinterpret_cast<const uint32_t *>(vb + static_cast<uint64_t>(j) * head_dim) : 0u;
        }
#pragma unroll
        for (int n = 0; n < NS; ++n) {
            const uint32_t i = tid + n * kAttnThreads, g = i / S::kTile, j = t0 + i % S::kTile;
            sr[n] = i < G * S::kTile && j < ctx ? srow[static_cast<uint64_t>(g) * max_len + j] : 0.f;
        }
    };
    uint32_t vr[S::kLoads];
    float sr[NS];
    load_tile(0, vr, sr);  // independent of the softmax statistics
    for (uint32_t g = wave; g < G; g += kAttnWaves) {
        const float2 *st = stats + (static_cast<uint64_t>(r) * n_heads + h0 + g) * nck;
        float m = -INFINITY;
        for (uint32_t cc = lane; cc < nact; cc += 64) m = fmaxf(m, st[cc].x);
        m = wave_max(m);
        float sum = 0.f;
        for (uint32_t cc = lane; cc < nact; cc += 64) {
            const float2 v = st[cc];
            sum += v.y * expf(v.x - m);
        }
        sum = wave_sum(sum);
        if (lane == 0) {
            mg[g] = m;
            sg[g] = sum;
        }
    }
    float acc[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;
    for (uint32_t t0 = 0; t0 < ctx; t0 += S::kTile) {
        uint32_t vnext[S::kLoads];
        float snext[NS];
        const bool more = t0 + S::kTile < ctx;
        if (more) load_tile(t0 + S::kTile, vnext, snext);  // in flight while this tile is used
        __syncthreads();  // mg/sg written; p free from the previous tile
#pragma unroll
        for (int n = 0; n < NS; ++n) {
            const uint32_t i = tid + n * kAttnThreads, g = i / S::kTile, jj = i % S::kTile;
            if (i < G * S::kTile) p[g][jj] = t0 + jj < ctx ? bf(rne(expf(sr[n] - mg[g]) / sg[g])) : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < S::kLoads; ++k) {
            const uint32_t jj = s + k * S::kSlots;
            const float v0 = bf(vr[k] & 0xFFFFu), v1 = bf(vr[k] >> 16);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                acc[g][0] += p[g][jj] * v0;
                acc[g][1] += p[g][jj] * v1;
            }
        }
        if (more) {
#pragma unroll
            for (int k = 0; k < S::kLoads; ++k) vr[k] = vnext[k];
#pragma unroll
            for (int n = 0; n < NS; ++n) sr[n] = snext[n];
        }
    }
    // slots of one dim pair inside a wavefront are P lanes apart: add them
    // with shuffles first, so LDS holds one partial per wavefront (and the
    // final sums read a few values instead of kSlots)
    constexpr int SW = P < 64 ? 64 / P : 1;  // slots per wavefront
#pragma unroll
    for (int off = P; off < 64; off <<= 1)
#pragma unroll
        for (int g = 0; g < G; ++g) {
            acc[g][0] += __shfl_xor(acc[g][0], off, 64);
            acc[g][1] += __shfl_xor(acc[g][1], off, 64);
        }
    if (s % SW == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            red[tid][2 * g] = acc[g][0];
            red[tid][2 * g + 1] = acc[g][1];
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < G * 2 * P; i += kAttnThreads) {
        const uint32_t g = i / (2 * P), dd = i % (2 * P), qq = dd / 2, e = dd % 2;
        float o = 0.f;
        for (int ss = 0; ss < S::kSlots; ss += SW) o += red[ss * P + qq][2 * g + e];
        orow[g * head_dim + dd] = rne(o);
    }
}

struct AttnArgs {
    const uint16_t *q_src, *cos_tab, *sin_tab;
    const uint32_t *positions;
    uint32_t pos_limit;
    uint16_t *k_cache, *v_cache;
    uint64_t row_stride;
    uint32_t n_heads, n_kv, max_len;
    float scale;
    char *ws;
    uint16_t *out;
};

template <int G, int P>
static void launch_pv(hipStream_t stream, uint32_t rows, const AttnLayout &a, const AttnArgs &x, uint32_t head_dim,
                      const float *scores, const float2 *stats) {
    const dim3 grid(static_cast<uint32_t>(x.n_kv * a.slices), rows);
    hipLaunchKernelGGL((attn_pv_kernel<G, P>), grid, dim3(kAttnThreads), 0, stream, x.v_cache, x.row_stride,
                       x.positions, x.pos_limit, x.n_heads, x.n_kv, head_dim, x.max_len,
                       static_cast<uint32_t>(a.nck), static_cast<uint32_t>(a.slices), scores, stats, x.out);
}

template <int HD, int G, bool ROPE>
static void launch_attention(hipStream_t stream, uint32_t rows, const AttnLayout &a, const AttnArgs &x) {
    auto *stats = reinterpret_cast<float2 *>(x.ws);
    auto *scores = reinterpret_cast<float *>(x.ws + a.scores);
    const dim3 grid(static_cast<uint32_t>(x.n_kv * a.splits), rows);
    hipLaunchKernelGGL((attn_scores_kernel<HD, G, ROPE>), grid, dim3(kAttnThreads), 0, stream, x.q_src, x.cos_tab,
                       x.sin_tab, x.positions, x.pos_limit, x.k_cache, x.v_cache, x.row_stride, x.n_heads, x.n_kv,
                       x.max_len, static_cast<uint32_t>(a.nck), static_cast<uint32_t>(a.splits), x.scale, scores,
                       stats);
    switch (HD / a.slices / 2) {  // dim pairs per P.V block
        case 8: return launch_pv<G, 8>(stream, rows, a, x, HD, scores, stats);
        case 16: return launch_pv<G, 16>(stream, rows, a, x, HD, scores, stats);
        case 32: return launch_pv<G, 32>(stream, rows, a, x, HD, scores, stats);
        case 64: return launch_pv<G, 64>(stream, rows, a, x, HD, scores, stats);
        default: return launch_pv<G, 128>(stream, rows, a, x, HD, scores, stats);
    }
}

template <bool ROPE>
static bool launch_attention_shape(int64_t head_dim, int64_t g, hipStream_t stream, uint32_t rows,
                                   const AttnLayout &a, const AttnArgs &x) {
#define FH_ATTN_G(HD, GG)                                          \
    case GG:                                                       \
        launch_attention<HD, GG, ROPE>(stream, rows, a, x);        \
        return true;
#define FH_ATTN_HD(HD)                                             \
    if (head_dim == HD) switch (g) {                               \
            FH_ATTN_G(HD, 1)                                       \
            FH_ATTN_G(HD, 2)                                       \
            FH_ATTN_G(HD, 3)                                       \
            FH_ATTN_G(HD, 4)                                       \
            FH_ATTN_G(HD, 5)                                       \
            FH_ATTN_G(HD, 6)                                       \
            FH_ATTN_G(HD, 7)                                       \
            FH_ATTN_G(HD, 8)                                       \
        }
    FH_ATTN_HD(64)
    FH_ATTN_HD(128)
    FH_ATTN_HD(256)
#undef FH_ATTN_HD
#undef FH_ATTN_G
    return false;
}

}  // namespace fh

using namespace fh;

namespace {

int check_heads(const char *fn, int64_t n_heads, int64_t n_kv, int64_t head_dim) {
    if (n_kv == 0 || n_heads == 0 || n_heads % n_kv != 0 || n_heads / n_kv > kAttnMaxGroup ||
        (head_dim != 64 && head_dim != 128 && head_dim != 256))
        return fail(FH_ERR_UNSUPPORTED, "%s: heads %lld/%lld, head_dim %lld", fn, (long long)n_heads,
                    (long long)n_kv, (long long)head_dim);
    return FH_OK;
}

// The workspace holds rows * n_heads * (max_len + 2 * chunks) floats (scores,
// statistics); refuse sizes whose byte counts would not fit comfortably in 64
// bits.
int check_attn_size(const char *fn, int64_t rows, int64_t n_heads, int64_t head_dim, int64_t max_len) {
    const long double floats = static_cast<long double>(rows) * n_heads * (3.0L * max_len + head_dim);
    if (floats > 0x1p56L)
        return fail(FH_ERR_INDEX_TOO_LARGE, "%s: attention workspace for %lld rows x %lld heads x %lld keys is too large",
                    fn, (long long)rows, (long long)n_heads, (long long)max_len);
    return FH_OK;
}

int workspace_bytes(const char *fn, int64_t rows, int64_t n_heads, int64_t n_kv, int64_t head_dim, int64_t max_len,
                    uint64_t *bytes) {
    if (!bytes) return fail(FH_ERR_INVALID_ARGUMENT, "%s: null output", fn);
    if (int rc = fh_check_dims(fn, {rows, n_heads, n_kv, head_dim, max_len})) return rc;
    if (int rc = check_attn_size(fn, rows, n_heads, head_dim, max_len)) return rc;
    *bytes = attn_layout(rows, n_heads, n_kv, head_dim, max_len).total;
    return FH_OK;
}

// Shared validation of both entry points; fills the layout.
int check_attention(const char *fn, fh_device *dev, int64_t rows, int64_t n_heads, int64_t n_kv, int64_t head_dim,
                    int64_t max_len, void *workspace, uint64_t workspace_bytes, AttnLayout *a) {
    if (int rc = check_heads(fn, n_heads, n_kv, head_dim)) return rc;
    if (max_len == 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: empty KV cache", fn);
    if (int rc = check_attn_size(fn, rows, n_heads, head_dim, max_len)) return rc;
    *a = attn_layout(rows, n_heads, n_kv, head_dim, max_len);
    if (rows > 65535 || static_cast<uint64_t>(n_kv) * (a->splits + a->slices) > 0x7FFFFFFFu)
        return fail(FH_ERR_INDEX_TOO_LARGE, "%s: %lld rows x %llu splits exceed the grid", fn, (long long)rows,
                    (unsigned long long)(n_kv * a->splits));
    if (workspace_bytes < a->total)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: workspace of %llu bytes, %llu needed", fn,
                    (unsigned long long)workspace_bytes, (unsigned long long)a->total);
    if (reinterpret_cast<uintptr_t>(workspace) & 15u)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: workspace must be 16-byte aligned", fn);
    return check_range(dev, workspace, a->total, fn, "workspace");
}

}  // namespace

extern "C" int fh_attention_workspace(int64_t tokens, int64_t n_heads, int64_t n_kv, int64_t head_dim,
                                      int64_t max_len, uint64_t *bytes) {
    return workspace_bytes("fh_attention_workspace", tokens, n_heads, n_kv, head_dim, max_len, bytes);
}

extern "C" int fh_attention(fh_device *dev, const uint16_t *q, const uint16_t *k_cache,
                            const uint16_t *v_cache, const uint32_t *positions, int64_t tokens,
                            int64_t n_heads, int64_t n_kv, int64_t head_dim, int64_t max_len,
                            float scale, void *workspace, uint64_t workspace_bytes, uint16_t *out) {
    const char *fn = "fh_attention";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {tokens, n_heads, n_kv, head_dim, max_len})) return rc;
    if (tokens == 0) return FH_OK;
    AttnLayout a;
    if (int rc = check_attention(fn, dev, tokens, n_heads, n_kv, head_dim, max_len, workspace, workspace_bytes, &a))
        return rc;
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
         reinterpret_cast<uintptr_t>(v_cache)) & 15u)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: q and caches must be 16-byte aligned", fn);
    const uint64_t cache = static_cast<uint64_t>(n_kv) * max_len * head_dim * 2;
    if (int rc = check_range(dev, q, static_cast<uint64_t>(tokens) * n_heads * head_dim * 2, fn, "q")) return rc;
    if (int rc = check_range(dev, k_cache, cache, fn, "k_cache")) return rc;
    if (int rc = check_range(dev, v_cache, cache, fn, "v_cache")) return rc;
    if (int rc = check_range(dev, positions, static_cast<uint64_t>(tokens) * 4, fn, "positions")) return rc;
    if (int rc = check_range(dev, out, static_cast<uint64_t>(tokens) * n_heads * head_dim * 2, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    // the tokens share one cache (row stride 0); positions past the cache
    // attend the whole cache, as fh_rope_kv wrote nothing for them
    const AttnArgs x{q, nullptr, nullptr, positions, 0xFFFFFFFFu, const_cast<uint16_t *>(k_cache),
                     const_cast<uint16_t *>(v_cache), 0, static_cast<uint32_t>(n_heads),
                     static_cast<uint32_t>(n_kv), static_cast<uint32_t>(max_len), scale,
                     static_cast<char *>(workspace), out};
    return dispatch(dev, fn, [&] {
        launch_attention_shape<false>(head_dim, n_heads / n_kv, dev->stream, static_cast<uint32_t>(tokens), a, x);
    });
}

extern "C" int fh_decode_attention_workspace(int64_t batch, int64_t n_heads, int64_t n_kv, int64_t head_dim,
                                             int64_t max_len, uint64_t *bytes) {
    return workspace_bytes("fh_decode_attention_workspace", batch, n_heads, n_kv, head_dim, max_len, bytes);
}

extern "C" int fh_decode_attention(fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads,
                                   int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab,
                                   const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
                                   uint16_t *k_cache, uint16_t *v_cache, int64_t max_len, float scale,
                                   void *workspace, uint64_t workspace_bytes, uint16_t *out) {
    const char *fn = "fh_decode_attention";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {batch, n_heads, n_kv, head_dim, table_len, max_len})) return rc;
    if (batch == 0) return FH_OK;
    AttnLayout a;
    if (int rc = check_attention(fn, dev, batch, n_heads, n_kv, head_dim, max_len, workspace, workspace_bytes, &a))
        return rc;
    if ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(cos_tab) |
         reinterpret_cast<uintptr_t>(sin_tab) | reinterpret_cast<uintptr_t>(k_cache) |
         reinterpret_cast<uintptr_t>(v_cache)) & 15u)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: operands must be 16-byte aligned", fn);
    const uint64_t width = static_cast<uint64_t>(n_heads + 2 * n_kv) * head_dim;
    const uint64_t row_stride = static_cast<uint64_t>(n_kv) * max_len * head_dim;
    if (int rc = check_range(dev, qkv, batch * width * 2, fn, "qkv")) return rc;
    if (int rc = check_range(dev, cos_tab, static_cast<uint64_t>(table_len) * head_dim * 2, fn, "cos")) return rc;
    if (int rc = check_range(dev, sin_tab, static_cast<uint64_t>(table_len) * head_dim * 2, fn, "sin")) return rc;
    if (int rc = check_range(dev, positions, static_cast<uint64_t>(batch) * 4, fn, "positions")) return rc;
    if (int rc = check_range(dev, k_cache, batch * row_stride * 2, fn, "k_cache")) return rc;
    if (int rc = check_range(dev, v_cache, batch * row_stride * 2, fn, "v_cache")) return rc;
    if (int rc = check_range(dev, out, static_cast<uint64_t>(batch) * n_heads * head_dim * 2, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    const uint32_t limit = static_cast<uint32_t>(max_len < table_len ? max_len : table_len);
    const AttnArgs x{qkv, cos_tab, sin_tab, positions, limit, k_cache, v_cache, row_stride,
                     static_cast<uint32_t>(n_heads), static_cast<uint32_t>(n_kv), static_cast<uint32_t>(max_len),
                     scale, static_cast<char *>(workspace), out};
    return dispatch(dev, fn, [&] {
        launch_attention_shape<true>(head_dim, n_heads / n_kv, dev->stream, static_cast<uint32_t>(batch), a, x);
    });
}
