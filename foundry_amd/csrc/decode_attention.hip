// Fused decode attention: for each sequence of a batch adding one token,
// RoPE on the token's q and k, the k/v write into the sequence's cache at its
// position, and attention over keys 0..position -- in one kernel, with the
// scores kept in LDS. It is the decode-step composition of
// apply_rotary_pos_emb (src/models/llama/rotary_emb.rs:62-85),
// StaticCache::update (src/nn/kv_cache.rs:41-80) and
// scaled_dot_product_attention (src/nn/attention.rs:23-60) with the reference's
// rounding points: rotated q/k RNE to bf16, scores RNE(q.k) * scale in fp32,
// fp32 softmax, probabilities RNE to bf16 from the row's max and sum, out =
// RNE(sum p v).
//
// One block per (KV head, sequence) serves the G = n_heads / n_kv query heads
// of that KV head, so each K and V row is read once for the group:
//   - scores: a key row of HD bf16 is read by HD/8 lanes with 16-byte loads
//     (one wavefront load covers 64 / (HD/8) whole keys) and the partial dot
//     products are summed by DPP within the lane group;
//   - softmax: max and sum over the row in one block reduction per pass, for
//     all G heads at once; the sum runs in a fixed order, so it is
//     deterministic;
//   - P.V: lanes over dims (2 or 4 per lane), wavefronts over keys, partial
//     vectors summed across wavefronts through LDS in wavefront order.
// The new token's key and value enter from LDS, so the block never reads
// back what it just wrote to the cache.
#include "decoder_common.hpp"

namespace fh {

constexpr int kDecThreads = 512;
constexpr int kDecWaves = kDecThreads / 64;
constexpr int kDecMaxGroup = 8;
// dynamic LDS per block: a gfx950 CU has 160 KiB; 1 KiB is left for the
// kernel's static reduction buffer
constexpr uint64_t kDecLdsLimit = 159 * 1024;

// LDS plan (bytes): scores [G][max_len] f32, reused for the [waves][G*HD]
// P.V partials; rotated q [G][HD] f32; new k and v bits [HD] u16 each.
struct DecLds {
    uint64_t sc_floats, bytes;
};

static DecLds dec_lds(uint64_t g, uint64_t hd, uint64_t max_len) {
    DecLds d;
    const uint64_t scores = g * max_len, partials = static_cast<uint64_t>(kDecWaves) * g * hd;
    // rounded up to 4 floats, so that what follows stays 16-byte aligned
    d.sc_floats = ((scores > partials ? scores : partials) + 3) & ~static_cast<uint64_t>(3);
    d.bytes = d.sc_floats * 4 + g * hd * 4 + 2 * hd * 2;
    return d;
}

template <int G>
__device__ __forceinline__ void block_reduce(float (&v)[G], float (&red)[kDecWaves][kDecMaxGroup], bool is_max) {
#pragma unroll
    for (int g = 0; g < G; ++g) v[g] = is_max ? wave_max(v[g]) : wave_sum(v[g]);
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();  // red free from any earlier reduction
    if (lane == 0)
#pragma unroll
        for (int g = 0; g < G; ++g) red[wave][g] = v[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float t = red[0][g];
        for (int w = 1; w < kDecWaves; ++w) t = is_max ? fmaxf(t, red[w][g]) : t + red[w][g];
        v[g] = t;
    }
}

template <int HD, int G>
__global__ __launch_bounds__(kDecThreads) void decode_attention_kernel(
    const uint16_t *__restrict__ qkv, uint32_t n_heads, uint32_t n_kv, const uint16_t *__restrict__ cos_tab,
    const uint16_t *__restrict__ sin_tab, uint32_t table_len, const uint32_t *__restrict__ positions,
    uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache, uint32_t max_len, uint32_t sc_floats,
    float scale, uint16_t *__restrict__ out) {
    extern __shared__ float lds[];
    float *sc = lds;                // [G][max_len] scores, then probabilities
    float *qs = lds + sc_floats;    // [G][HD] rotated q
    auto *knew = reinterpret_cast<uint16_t *>(qs + G * HD);  // [HD] rotated k (bf16 bits)
    uint16_t *vnew = knew + HD;                              // [HD] v (bf16 bits)
    __shared__ float red[kDecWaves][kDecMaxGroup];
    const uint32_t tid = threadIdx.x, b = blockIdx.y, kvh = blockIdx.x, h0 = kvh * G;
    const uint32_t pos = positions[b];
    uint16_t *orow = out + (static_cast<uint64_t>(b) * n_heads + h0) * HD;
    // positions are device data the host cannot check: outside the cache or
    // the tables, nothing is written to the cache and the output is zero
    if (pos >= max_len || pos >= table_len) {
        for (uint32_t i = tid; i < G * HD; i += kDecThreads) orow[i] = 0;
        return;
    }
    const uint16_t *row = qkv + static_cast<uint64_t>(b) * (n_heads + 2 * n_kv) * HD;
    const uint64_t cache = (static_cast<uint64_t>(b) * n_kv + kvh) * max_len * HD;
    constexpr uint32_t PPH = HD / 8;  // 8-dim pieces per head
    {
        const uint16_t *c = cos_tab + static_cast<uint64_t>(pos) * HD;
        const uint16_t *s = sin_tab + static_cast<uint64_t>(pos) * HD;
        if (tid < (G + 1) * PPH) {
            const uint32_t hh = tid / PPH, p = tid % PPH;  // hh < G: query head h0 + hh; hh == G: the key
            const uint16_t *head = row + static_cast<uint64_t>(hh < G ? h0 + hh : n_heads + kvh) * HD;
            const uint4 ov = rope_piece(head, c, s, p, PPH / 2);
            if (hh < G) {
                float f[8];
                unpack8(ov, f);
#pragma unroll
                for (int e = 0; e < 8; ++e) qs[hh * HD + p * 8 + e] = f[e];
            } else {
                *reinterpret_cast<uint4 *>(knew + p * 8) = ov;
                *reinterpret_cast<uint4 *>(k_cache + cache + static_cast<uint64_t>(pos) * HD + p * 8) = ov;
            }
        } else if (tid < (G + 2) * PPH) {
            const uint32_t p = tid - (G + 1) * PPH;
            const uint4 v = *reinterpret_cast<const uint4 *>(row + static_cast<uint64_t>(n_heads + n_kv + kvh) * HD + p * 8);
            *reinterpret_cast<uint4 *>(vnew + p * 8) = v;
            *reinterpret_cast<uint4 *>(v_cache + cache + static_cast<uint64_t>(pos) * HD + p * 8) = v;
        }
    }
    __syncthreads();
    const uint32_t n = pos + 1;  // keys 0..pos; key pos is the new one
    const uint32_t wave = tid >> 6, lane = tid & 63;
    {
        constexpr int LPK = HD / 8, KPI = 64 / LPK, U = HD == 256 ? 4 : 8;
        const uint32_t ks = lane / LPK, li = lane % LPK;
        float qf[G][8];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[g][e] = qs[g * HD + li * 8 + e];
        const uint16_t *kb = k_cache + cache + li * 8;
        const uint4 kn = *reinterpret_cast<const uint4 *>(knew + li * 8);
        for (uint32_t jb = 0; jb < n; jb += kDecWaves * KPI * U) {
            uint4 kr[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t j = jb + (u * kDecWaves + wave) * KPI + ks;
                kr[u] = j < pos ? *reinterpret_cast<const uint4 *>(kb + static_cast<uint64_t>(j) * HD)
                                : (j == pos ? kn : make_uint4(0u, 0u, 0u, 0u));
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t j = jb + (u * kDecWaves + wave) * KPI + ks;
                float kf[8];
                unpack8(kr[u], kf);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float d = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d += qf[g][e] * kf[e];
                    d = group_sum<LPK>(d);
                    if (li == 0 && j < n) sc[g * max_len + j] = bf(rne(d)) * scale;
                }
            }
        }
    }
    __syncthreads();
    {
        float m[G], s[G];
#pragma unroll
        for (int g = 0; g < G; ++g) m[g] = -INFINITY;
        for (uint32_t j = tid; j < n; j += kDecThreads)
#pragma unroll
            for (int g = 0; g < G; ++g) m[g] = fmaxf(m[g], sc[g * max_len + j]);
        block_reduce<G>(m, red, true);
#pragma unroll
        for (int g = 0; g < G; ++g) s[g] = 0.f;
        for (uint32_t j = tid; j < n; j += kDecThreads)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float e = expf(sc[g * max_len + j] - m[g]);
                sc[g * max_len + j] = e;
                s[g] += e;
            }
        block_reduce<G>(s, red, false);
        for (uint32_t j = tid; j < n; j += kDecThreads)
#pragma unroll
            for (int g = 0; g < G; ++g) sc[g * max_len + j] = bf(rne(sc[g * max_len + j] / s[g]));
    }
    __syncthreads();
    {
        constexpr int VW = HD == 256 ? 4 : 2, LPV = HD / VW, KPV = 64 / LPV, U = 16;
        const uint32_t kslot = lane / LPV, dl = lane % LPV;
        float acc[G][VW];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < VW; ++e) acc[g][e] = 0.f;
        const uint16_t *vb = v_cache + cache + dl * VW;
        uint2 vn;
        if constexpr (VW == 4)
            vn = *reinterpret_cast<const uint2 *>(vnew + dl * VW);
        else
            vn = make_uint2(*reinterpret_cast<const uint32_t *>(vnew + dl * VW), 0u);
        for (uint32_t jb = 0; jb < n; jb += kDecWaves * KPV * U) {
            uint2 vr[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t j = jb + (u * kDecWaves + wave) * KPV + kslot;
                if (j < pos) {
                    const uint16_t *src = vb + static_cast<uint64_t>(j) * HD;
                    if constexpr (VW == 4)
                        vr[u] = *reinterpret_cast<const uint2 *>(src);
                    else
                        vr[u] = make_uint2(*reinterpret_cast<const uint32_t *>(src), 0u);
                } else {
                    vr[u] = j == pos ? vn : make_uint2(0u, 0u);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t j = jb + (u * kDecWaves + wave) * KPV + kslot;
                const float v0 = bf(vr[u].x & 0xFFFFu), v1 = bf(vr[u].x >> 16);
                const float v2 = bf(vr[u].y & 0xFFFFu), v3 = bf(vr[u].y >> 16);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = j < n ? sc[g * max_len + j] : 0.f;
                    acc[g][0] += p * v0;
                    acc[g][1] += p * v1;
                    if constexpr (VW == 4) {
                        acc[g][2] += p * v2;
                        acc[g][3] += p * v3;
                    }
                }
            }
        }
        if constexpr (KPV == 2)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < VW; ++e) acc[g][e] += __shfl_xor(acc[g][e], 32, 64);
        __syncthreads();  // every wavefront is done with the probabilities
        float *wsum = sc;  // [waves][G * HD]
        if (kslot == 0)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < VW; ++e) wsum[wave * G * HD + g * HD + dl * VW + e] = acc[g][e];
        __syncthreads();
        for (uint32_t i = tid; i < G * HD; i += kDecThreads) {
            float o = wsum[i];
            for (int w = 1; w < kDecWaves; ++w) o += wsum[w * G * HD + i];
            orow[i] = rne(o);
        }
    }
}

template <int HD, int G>
static int launch_decode(fh_device *dev, const char *fn, dim3 grid, const DecLds &l, const uint16_t *qkv,
                         uint32_t n_heads, uint32_t n_kv, const uint16_t *cos_tab, const uint16_t *sin_tab,
                         uint32_t table_len, const uint32_t *positions, uint16_t *k_cache, uint16_t *v_cache,
                         uint32_t max_len, float scale, uint16_t *out) {
    auto kernel = decode_attention_kernel<HD, G>;
    if (l.bytes > 64 * 1024) {
        // opt in to more than 64 KiB of dynamic LDS (once per instantiation)
        static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                                           static_cast<int>(kDecLdsLimit));
        if (attr != hipSuccess)
            return fail(FH_ERR_LAUNCH, "%s: LDS opt-in failed: %s", fn, hipGetErrorString(attr));
    }
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(kernel, grid, dim3(kDecThreads), static_cast<uint32_t>(l.bytes), dev->stream, qkv,
                           n_heads, n_kv, cos_tab, sin_tab, table_len, positions, k_cache, v_cache, max_len,
                           static_cast<uint32_t>(l.sc_floats), scale, out);
    });
}

template <int HD>
static int launch_decode_hd(int g, fh_device *dev, const char *fn, dim3 grid, const DecLds &l, const uint16_t *qkv,
                            uint32_t n_heads, uint32_t n_kv, const uint16_t *cos_tab, const uint16_t *sin_tab,
                            uint32_t table_len, const uint32_t *positions, uint16_t *k_cache, uint16_t *v_cache,
                            uint32_t max_len, float scale, uint16_t *out) {
#define FH_DEC_CASE(GG)                                                                                      \
    case GG:                                                                                                 \
        return launch_decode<HD, GG>(dev, fn, grid, l, qkv, n_heads, n_kv, cos_tab, sin_tab, table_len,     \
                                     positions, k_cache, v_cache, max_len, scale, out);
    switch (g) {
        FH_DEC_CASE(1)
        FH_DEC_CASE(2)
        FH_DEC_CASE(3)
        FH_DEC_CASE(4)
        FH_DEC_CASE(5)
        FH_DEC_CASE(6)
        FH_DEC_CASE(7)
        FH_DEC_CASE(8)
    }
#undef FH_DEC_CASE
    return fail(FH_ERR_UNSUPPORTED, "%s: group of %d query heads per KV head", fn, g);
}

}  // namespace fh

using namespace fh;

extern "C" int fh_decode_attention_max_len(int64_t n_heads, int64_t n_kv, int64_t head_dim, int64_t *max_len) {
    const char *fn = "fh_decode_attention_max_len";
    if (!max_len) return fail(FH_ERR_INVALID_ARGUMENT, "%s: null output", fn);
    if (int rc = fh_check_dims(fn, {n_heads, n_kv, head_dim})) return rc;
    if (n_kv == 0 || n_heads % n_kv != 0 || n_heads / n_kv > kDecMaxGroup || n_heads == 0 ||
        (head_dim != 64 && head_dim != 128 && head_dim != 256))
        return fail(FH_ERR_UNSUPPORTED, "%s: heads %lld/%lld, head_dim %lld", fn, (long long)n_heads,
                    (long long)n_kv, (long long)head_dim);
    const uint64_t g = static_cast<uint64_t>(n_heads / n_kv);
    // largest max_len whose LDS plan fits
    const uint64_t fixed = dec_lds(g, head_dim, 0).bytes - dec_lds(g, head_dim, 0).sc_floats * 4;
    const uint64_t ml = (kDecLdsLimit - fixed) / (4 * g) & ~static_cast<uint64_t>(3);
    *max_len = static_cast<int64_t>(dec_lds(g, head_dim, ml).bytes <= kDecLdsLimit ? ml : ml - 4);
    return FH_OK;
}

extern "C" int fh_decode_attention(fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads,
                                   int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab,
                                   const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
                                   uint16_t *k_cache, uint16_t *v_cache, int64_t max_len, float scale,
                                   uint16_t *out) {
    const char *fn = "fh_decode_attention";
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {batch, n_heads, n_kv, head_dim, table_len, max_len})) return rc;
    if (batch == 0) return FH_OK;
    if (n_kv == 0 || n_heads % n_kv != 0 || n_heads / n_kv > kDecMaxGroup || n_heads == 0 ||
        (head_dim != 64 && head_dim != 128 && head_dim != 256))
        return fail(FH_ERR_UNSUPPORTED, "%s: heads %lld/%lld, head_dim %lld", fn, (long long)n_heads,
                    (long long)n_kv, (long long)head_dim);
    if (max_len == 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: empty KV cache", fn);
    if (batch > 65535) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: batch of %lld sequences", fn, (long long)batch);
    const uint64_t g = static_cast<uint64_t>(n_heads / n_kv);
    const DecLds l = dec_lds(g, head_dim, max_len);
    if (l.bytes > kDecLdsLimit)
        return fail(FH_ERR_UNSUPPORTED,
                    "%s: max_len %lld needs %llu bytes of LDS for the scores (limit %llu); use fh_rope_kv + "
                    "fh_attention",
                    fn, (long long)max_len, (unsigned long long)l.bytes, (unsigned long long)kDecLdsLimit);
    if ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(cos_tab) |
         reinterpret_cast<uintptr_t>(sin_tab) | reinterpret_cast<uintptr_t>(k_cache) |
         reinterpret_cast<uintptr_t>(v_cache)) & 15u)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: operands must be 16-byte aligned", fn);
    const uint64_t width = static_cast<uint64_t>(n_heads + 2 * n_kv) * head_dim;
    const uint64_t cache = static_cast<uint64_t>(batch) * n_kv * max_len * head_dim * 2;
    if (int rc = check_range(dev, qkv, batch * width * 2, fn, "qkv")) return rc;
    if (int rc = check_range(dev, cos_tab, static_cast<uint64_t>(table_len) * head_dim * 2, fn, "cos")) return rc;
    if (int rc = check_range(dev, sin_tab, static_cast<uint64_t>(table_len) * head_dim * 2, fn, "sin")) return rc;
    if (int rc = check_range(dev, positions, static_cast<uint64_t>(batch) * 4, fn, "positions")) return rc;
    if (int rc = check_range(dev, k_cache, cache, fn, "k_cache")) return rc;
    if (int rc = check_range(dev, v_cache, cache, fn, "v_cache")) return rc;
    if (int rc = check_range(dev, out, static_cast<uint64_t>(batch) * n_heads * head_dim * 2, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    const dim3 grid(static_cast<uint32_t>(n_kv), static_cast<uint32_t>(batch));
    const uint32_t nh = static_cast<uint32_t>(n_heads), nk = static_cast<uint32_t>(n_kv),
                   tl = static_cast<uint32_t>(table_len), ml = static_cast<uint32_t>(max_len);
    if (head_dim == 64)
        return launch_decode_hd<64>(static_cast<int>(g), dev, fn, grid, l, qkv, nh, nk, cos_tab, sin_tab, tl,
                                    positions, k_cache, v_cache, ml, scale, out);
    if (head_dim == 128)
        return launch_decode_hd<128>(static_cast<int>(g), dev, fn, grid, l, qkv, nh, nk, cos_tab, sin_tab, tl,
                                     positions, k_cache, v_cache, ml, scale, out);
    return launch_decode_hd<256>(static_cast<int>(g), dev, fn, grid, l, qkv, nh, nk, cos_tab, sin_tab, tl,
                                 positions, k_cache, v_cache, ml, scale, out);
}
