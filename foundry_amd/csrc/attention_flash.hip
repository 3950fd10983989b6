// Prefill attention in one pass per query tile, with the reference's
// rounding points: the counterpart of scaled_dot_product_attention
// (src/nn/attention.rs:23-60) under the causal mask (src/nn/masking.rs:11-32)
// for head_dim 128. Scores s_j = RNE(q.k_j) * scale (fp32 dot products, bf16
// rounding, fp32 scale), M = max_j s_j, S = sum_j exp(s_j - M), probabilities
// p_j = RNE(exp(s_j - M) / S) -- from the row's GLOBAL max and sum, as the
// reference rounds them before P.V -- and out = RNE(sum_j p_j v_j).
//
// Design for CDNA4: block (KV head, tile of 256 / G query rows), 8 wavefronts;
// the tile's (row, head) pairs are the columns of the score tiles, 32 per
// wavefront. The keys are walked twice, 64 at a time through LDS:
//   pass 1: S^T = K Q^T on the matrix cores (v_mfma_f32_32x32x16_bf16, the
//     keys as A rows, the pairs' q as B columns held in registers for the
//     whole block), so a lane holds 16 keys of ONE pair: the running max and
//     sum of exp need no cross-lane work until the two half-wavefronts that
//     share a pair combine them once, at the end;
//   pass 2: the same scores again, p_j rounded from the final M and S, and
//     P.V on the matrix cores: the lane's 16 probabilities of a 32-key tile
//     are already an A fragment pair (keys in the order the score layout
//     gives them), and V is staged transposed in LDS with its keys in that
//     same order, so each B fragment is one 16-byte read.
// No scores or statistics leave the CU (the two-kernel path writes both
// through a workspace), and every key and value is read from L2 once per
// 256 (row, head) pairs. Every sum runs in a fixed order, so results do not
// change from run to run.
#include <type_traits>

#include "decoder_common.hpp"

namespace fh {

namespace {

constexpr int kFlHd = 128;
constexpr int kFlThreads = 512;
constexpr int kFlWaves = kFlThreads / 64;
constexpr int kFlKeys = 64;                       // keys per LDS block
constexpr uint32_t kFlKBlock = kFlKeys * kFlHd;   // bf16 per K or V block

typedef __attribute__((ext_vector_type(8))) __bf16 fl_bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float fl_f32x16_t;

__device__ __forceinline__ fl_f32x16_t fl_mfma(const uint4 a, const uint4 b, const fl_f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(fl_bf16x8_t, a), __builtin_bit_cast(fl_bf16x8_t, b),
                                                   c, 0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t fl_rsrc(const void *p, uint64_t bytes) {
    const uint32_t records = bytes < 0xFFFFFFFFull ? static_cast<uint32_t>(bytes) : 0xFFFFFFFFu;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), static_cast<short>(0), static_cast<int>(records),
                                             0x00020000);
}

// Slot of key k (0..63 of a block) in a V^T row: within each 16-key group,
// keys 0-3 and 8-11 (the first half-wavefront's keys of an MFMA k step) fill
// slots 0-7, keys 4-7 and 12-15 slots 8-15.
__device__ __forceinline__ uint32_t fl_slot(uint32_t k) {
    const uint32_t o = k & 15u;
    return (k & ~15u) + 8u * ((o >> 2) & 1u) + (o & 3u) + 4u * (o >> 3);
}

// exp of the softmax arguments, and each probability from it and the sum.
// The reference compiles its Metal kernels with the default options
// (src/metal/mod.rs:109-128: no MTLCompileOptions), under which Metal's fast
// math is on: its exp (unary.metal:6) and divide (binary.metal:14) are not
// the correctly rounded functions. Here exp(s - m) is v_exp_f32 of one fma,
// b * (scale log2 e) - mb * (scale log2 e) for s = b * scale (b = RNE(q.k))
// and m = mb * scale, and p = e * (1 / S): the same class of approximation.
// With expf of s - m and a true division the one-pass kernel takes 1.8x as
// long (the VALU work per score bounds it). FH_FLASH_EXP2=0 / FH_FLASH_RCP=0
// select those.
#ifndef FH_FLASH_EXP2
#define FH_FLASH_EXP2 1
#endif
#ifndef FH_FLASH_RCP
#define FH_FLASH_RCP 1
#endif
// exp(b * scale - mb * scale) as ex(b, ex.base(mb)); b may be -inf, mb
// is finite
struct FlExp {
    float scale, c1;  // c1 = scale * log2(e)
    __device__ float base(float mb) const {
#if FH_FLASH_EXP2
        return -(mb * c1);
#else
        return __fmul_rn(mb, scale);
#endif
    }
    __device__ float operator()(float b, float base_) const {
#if FH_FLASH_EXP2
        return __builtin_amdgcn_exp2f(fmaf(b, c1, base_));
#else
        return expf(__fmul_rn(b, scale) - base_);
#endif
    }
};

}  // namespace

// Block (KV head, sequence, query tile): rows r0 .. r0 + 256 / G - 1 of
// sequence blockIdx.y (`rows` rows each, its cache seq_cache elements after
// the previous one's; K tiled in groups of 16 keys, k_tile; V [max_len][128])
// over its cache. positions[r]: the row's position; it attends keys 0 ..
// min(pos, max_len - 1). Tiles go out last first: a prompt's later rows
// attend more keys, and the longest blocks then start first.
template <int G>
__global__ __launch_bounds__(kFlThreads) void attn_flash_kernel(
    const uint16_t *__restrict__ q, const uint32_t *__restrict__ positions, uint32_t rows,
    const uint16_t *__restrict__ k_cache, const uint16_t *__restrict__ v_cache, uint64_t seq_cache, uint32_t n_heads,
    uint32_t max_len, float scale, uint16_t *__restrict__ out) {
    constexpr uint32_t QT = 256 / G;   // query rows per block
    constexpr uint32_t LIVE = QT * G;  // (row, head) pairs of the block
    // K blocks: [key][16 pieces of 8 dims], piece slot s of key k holding
    // piece s ^ (k % 16); V^T blocks: [dim][64 key slots], 16-byte piece slot
    // s of dim d holding piece s ^ ((d / 2) % 8). Both are conflict-free for
    // the fragment reads below.
    __shared__ __align__(16) uint16_t kls[2][kFlKBlock];
    __shared__ __align__(16) uint16_t vls[2][kFlKBlock];
    // the wavefronts' longest contexts, read before V^T buffer 1 is first written
    uint32_t *const wmax = reinterpret_cast<uint32_t *>(&vls[1][0]);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
    const uint32_t kvh = blockIdx.x, sq = blockIdx.y, r0 = (gridDim.z - 1 - blockIdx.z) * QT, h0 = kvh * G;
    {
        const uint64_t rows0 = static_cast<uint64_t>(sq) * rows;  // the sequence's first row
        q += rows0 * n_heads * kFlHd;
        out += rows0 * n_heads * kFlHd;
        positions += rows0;
        k_cache += sq * seq_cache;
        v_cache += sq * seq_cache;
    }
    const uint16_t *const kc = k_cache + static_cast<uint64_t>(kvh) * max_len * kFlHd;
    const uint16_t *const vc = v_cache + static_cast<uint64_t>(kvh) * max_len * kFlHd;

    // this lane's pair: column l % 32 of its wavefront's score tiles
    const uint32_t p = wave * 32 + (lane & 31);
    const bool alive = p < LIVE && r0 + p / G < rows;
    const uint32_t prow = alive ? r0 + p / G : 0, phead = h0 + (alive ? p % G : 0);
    const uint32_t pos = alive ? positions[prow] : 0u;
    const uint32_t ctx = alive ? (pos < max_len ? pos + 1 : max_len) : 0u;
    // the block's longest and shortest live contexts: key blocks below the
    // shortest need no mask
    {
        const float mx = wave_max(static_cast<float>(ctx));
        const float mn = -wave_max(alive ? -static_cast<float>(ctx) : -static_cast<float>(max_len));
        if (lane == 0) wmax[wave] = static_cast<uint32_t>(mx), wmax[kFlWaves + wave] = static_cast<uint32_t>(mn);
    }
    // q of the pair as B fragments: dims 16 s + 8 h .. + 7
    uint4 qf[8];
    {
        const uint16_t *qp = q + (static_cast<uint64_t>(prow) * n_heads + phead) * kFlHd + 8 * h;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint4 v = *reinterpret_cast<const uint4 *>(qp + 16 * s);
            qf[s] = alive ? v : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    __syncthreads();
    uint32_t kmax = 0, kmin = max_len;
#pragma unroll
    for (int w = 0; w < kFlWaves; ++w) {
        kmax = wmax[w] > kmax ? wmax[w] : kmax;
        kmin = wmax[kFlWaves + w] < kmin ? wmax[kFlWaves + w] : kmin;
    }
    if (kmax == 0) return;  // no live row (uniform over the block)
    const uint32_t nkb = (kmax + kFlKeys - 1) / kFlKeys;

    // K block kb into LDS by DMA: wavefront w brings keys 8 w .. 8 w + 7 as
    // two 1 KiB pieces (4 keys x 16 slots each); keys past the block's
    // longest context read key kmax - 1 (valid, never used)
    const __amdgpu_buffer_rsrc_t rk = fl_rsrc(kc, static_cast<uint64_t>(max_len) * kFlHd * 2);
    auto stage_k = [&](uint32_t kb, uint32_t buf) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint32_t kl = 8 * wave + 4 * c + (lane >> 4);  // key within the block
            uint32_t key = kb * kFlKeys + kl;
            key = key < kmax ? key : kmax - 1;
            const uint32_t piece = (lane & 15) ^ (kl & 15);
            const uint32_t off = static_cast<uint32_t>(k_offset(key, 8 * piece, max_len, kFlHd)) * 2;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rk, (__attribute__((address_space(3))) void *)(&kls[buf][(8 * wave + 4 * c) * kFlHd]), 16,
                static_cast<int>(off), 0, 0, 0);
        }
    };
    // V block kb: thread (key pair i = tid % 32, dim piece c = tid / 32)
    // loads keys 2 i, 2 i + 1 of dims 8 c .. 8 c + 7, then writes dword
    // (v[2i][d], v[2i+1][d]) of each dim d to V^T
    auto load_v = [&](uint32_t kb, uint4 (&v)[2]) {
        const uint32_t i = tid & 31, c = tid >> 5;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            uint32_t key = kb * kFlKeys + 2 * i + e;
            key = key < kmax ? key : kmax - 1;
            v[e] = *reinterpret_cast<const uint4 *>(vc + static_cast<uint64_t>(key) * kFlHd + 8 * c);
        }
    };
    auto store_v = [&](const uint4 (&v)[2], uint32_t buf) {
        const uint32_t i = tid & 31, c = tid >> 5;
        const uint32_t slot = fl_slot(2 * i);  // even; key 2 i + 1 is the next slot
        const uint32_t a[4] = {v[0].x, v[0].y, v[0].z, v[0].w}, b[4] = {v[1].x, v[1].y, v[1].z, v[1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t d = 8 * c + e;
            const uint32_t lo = (a[e / 2] >> (16 * (e % 2))) & 0xFFFFu, hi = (b[e / 2] >> (16 * (e % 2))) & 0xFFFFu;
            const uint32_t at = d * kFlKeys + (((slot >> 3) ^ ((d >> 1) & 7u)) << 3) + (slot & 7u);
            *reinterpret_cast<uint32_t *>(&vls[buf][at]) = lo | (hi << 16);
        }
    };
    // S^T of 32-key tile t of a staged block: rows = keys 32 t + 8 (r / 4) +
    // 4 h + r % 4, column = this lane's pair
    auto scores = [&](uint32_t buf, int t) {
        const uint32_t kl = 32 * t + (lane & 31);
        const uint16_t *kr = &kls[buf][kl * kFlHd];
        fl_f32x16_t d;
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint4 a = *reinterpret_cast<const uint4 *>(kr + (((2 * s + h) ^ (kl & 15)) << 3));
            d = fl_mfma(a, qf[s], d);
        }
        return d;
    };
    // b_j = RNE(q.k_j) (the score is s_j = b_j * scale; the scale is applied
    // inside the exp argument, and the max over b is the max over s), or -inf
    // past the pair's context (MASK: the block reaches past some live pair's
    // context)
    const FlExp ex{scale, scale * 1.44269504088896341f};
    auto score_of = [&](const fl_f32x16_t &d, uint32_t kb, int t, int r, auto mask) {
        const float sv = bf(rne(d[r]));
        if constexpr (decltype(mask)::value) {
            const uint32_t j = kb * kFlKeys + 32 * t + 8 * (r / 4) + 4 * h + (r % 4);
            return j < ctx ? sv : -INFINITY;
        }
        return sv;
    };
    using Masked = std::integral_constant<bool, true>;
    using Unmasked = std::integral_constant<bool, false>;

    // Pass 1: running (max of b, sum of exp(s - m)) over this lane's keys of the pair
    float m = -INFINITY, l = 0.f;
    stage_k(0, 0);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();
    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const uint32_t buf = kb & 1;
        if (kb + 1 < nkb) stage_k(kb + 1, buf ^ 1);
        auto stats = [&](auto mask) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const fl_f32x16_t d = scores(buf, t);
                float sv[16], mt = -INFINITY;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    sv[r] = score_of(d, kb, t, r, mask);
                    mt = fmaxf(mt, sv[r]);
                }
                const float mn = fmaxf(m, mt);
                if (mn != -INFINITY) {
                    const float o = ex.base(mn);
                    float sum = 0.f;
#pragma unroll
                    for (int r = 0; r < 16; ++r) sum += ex(sv[r], o);
                    l = l * ex(m, o) + sum;
                    m = mn;
                }
            }
        };
        if ((kb + 1) * kFlKeys <= kmin)
            stats(Unmasked{});
        else
            stats(Masked{});
        __builtin_amdgcn_s_waitcnt(0x0f70);  // the next block's DMA has landed
        __syncthreads();
    }
    // the pair's two halves (lanes l and l ^ 32) combined, the h = 0 half first
    float M, S;
    {
        const float mo = __shfl_xor(m, 32, 64), lo = __shfl_xor(l, 32, 64);
        const float m0 = h ? mo : m, l0 = h ? lo : l, m1 = h ? m : mo, l1 = h ? l : lo;
        M = fmaxf(m0, m1);
        const float o = M == -INFINITY ? 0.f : ex.base(M);
        S = M == -INFINITY ? 1.f : (m0 == -INFINITY ? 0.f : l0 * ex(m0, o)) + (m1 == -INFINITY ? 0.f : l1 * ex(m1, o));
    }
    // a pair with no key (a dead lane) gets exp(-inf) = 0 everywhere, not NaN
    const float oM = M == -INFINITY ? 0.f : ex.base(M);
#if FH_FLASH_RCP
    const float rS = 1.f / S;
#endif

    // Pass 2: p_j = RNE(exp(s_j - M) / S) (masked keys: exp(-inf) = 0), acc +=
    // P V over 4 tiles of 32 dims
    fl_f32x16_t acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
    {
        uint4 vr[2];
        stage_k(0, 0);
        load_v(0, vr);
        store_v(vr, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    fl_f32x16_t dsc;  // the current score tile
    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const uint32_t buf = kb & 1;
        uint4 vr[2];
        const bool next = kb + 1 < nkb;
        if (next) {
            stage_k(kb + 1, buf ^ 1);
            load_v(kb + 1, vr);
        }
        auto probs = [&](int t, uint32_t (&pw)[8], auto mask) {
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const fl_f32x16_t &d = dsc;
                const float s0 = score_of(d, kb, t, r, mask), s1 = score_of(d, kb, t, r + 1, mask);
#if FH_FLASH_RCP
                const float p0 = ex(s0, oM) * rS, p1 = ex(s1, oM) * rS;
#else
                const float p0 = ex(s0, oM) / S, p1 = ex(s1, oM) / S;
#endif
                pw[r / 2] = f32x2_to_bf16x2_rne(p0, p1);
            }
        };
        const bool full = (kb + 1) * kFlKeys <= kmin;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            dsc = scores(buf, t);
            uint32_t pw[8];  // probabilities as bf16 pairs, in register order
            if (full)
                probs(t, pw, Unmasked{});
            else
                probs(t, pw, Masked{});
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const uint4 a = make_uint4(pw[4 * ks], pw[4 * ks + 1], pw[4 * ks + 2], pw[4 * ks + 3]);
                const uint32_t piece = 2 * (2 * t + ks) + h;  // slots 16 (2 t + ks) + 8 h .. + 7
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const uint32_t dd = 32 * dt + (lane & 31);
                    const uint4 b = *reinterpret_cast<const uint4 *>(
                        &vls[buf][dd * kFlKeys + ((piece ^ ((dd >> 1) & 7u)) << 3)]);
                    acc[dt] = fl_mfma(a, b, acc[dt]);
                }
            }
        }
        if (next) store_v(vr, buf ^ 1);  // buffer buf ^ 1 was last read before the previous barrier
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();
    }

    // out[row][head][dim]: lane holds dim 32 dt + l % 32 of pairs 8 (r / 4) + 4 h + r % 4
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t pp = wave * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        if (pp >= LIVE || r0 + pp / G >= rows) continue;
        uint16_t *orow = out + (static_cast<uint64_t>(r0 + pp / G) * n_heads + h0 + pp % G) * kFlHd + (lane & 31);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) orow[32 * dt] = rne(acc[dt][r]);
    }
}

// Whether the one-pass kernel takes `rows` prompt rows of one sequence:
// head_dim 128, G = n_heads / n_kv of 1 .. 8, and its blocks (n_kv per query
// tile) fill at least half the CUs.
bool attention_flash_applies(uint32_t cus, uint32_t rows, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim) {
    if (head_dim != kFlHd || n_kv == 0 || n_heads % n_kv != 0) return false;
    const uint32_t g = n_heads / n_kv;
    if (g < 1 || g > 8) return false;
    const uint64_t tiles = (rows + 256 / g - 1) / (256 / g);
    return tiles * n_kv * 2 >= cus && tiles <= 65535;
}

// Launches the one-pass kernel over `batch` sequences of `rows` rows (q, out
// and positions consecutive per sequence, caches seq_cache elements apart)
// when attention_flash_applies to one sequence; returns false otherwise (the
// caller takes the two-kernel path). Every block is the one a launch per
// sequence would run, so the outputs are those of per-sequence launches.
bool launch_attention_flash(hipStream_t stream, uint32_t cus, const uint16_t *q, const uint32_t *positions,
                            uint32_t rows, const uint16_t *k_cache, const uint16_t *v_cache, uint32_t n_heads,
                            uint32_t n_kv, uint32_t head_dim, uint32_t max_len, float scale, uint16_t *out,
                            uint32_t batch, uint64_t seq_cache) {
    if (batch == 0 || batch > 65535 || !attention_flash_applies(cus, rows, n_heads, n_kv, head_dim)) return false;
    const uint32_t g = n_heads / n_kv;
    const uint32_t tiles = (rows + 256 / g - 1) / (256 / g);
    const dim3 grid(n_kv, batch, tiles);
#define FH_FLASH_G(GG)                                                                                          \
    case GG:                                                                                                    \
        hipLaunchKernelGGL(attn_flash_kernel<GG>, grid, dim3(kFlThreads), 0, stream, q, positions, rows, k_cache, \
                           v_cache, seq_cache, n_heads, max_len, scale, out);                                   \
        return true;
    switch (g) {
        FH_FLASH_G(1)
        FH_FLASH_G(2)
        FH_FLASH_G(3)
        FH_FLASH_G(4)
        FH_FLASH_G(5)
        FH_FLASH_G(6)
        FH_FLASH_G(7)
        FH_FLASH_G(8)
    }
#undef FH_FLASH_G
    return false;
}

}  // namespace fh
