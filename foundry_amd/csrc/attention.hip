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
// A row (a token, or a sequence) attends keys 0..ctx-1 of its KV head. The
// scores and the P.V are separate launches, because each probability is
// rounded from the row's global max and sum; no kernel waits on another
// block (a device-scope fence per block costs an L2 write-back on this part),
// and every block serves the G = n_heads / n_kv query heads of its KV head,
// so a K or V row is read once for the group:
//   attn_scores_kernel, block (KV head, split, row): chunks of kAttnChunk keys
//     dealt round-robin to the split blocks and their wavefronts;
//     s_j = RNE(q.k_j) * scale from matrix-core dot products; RNE(q.k_j)
//     goes to the workspace (bf16) with each chunk's (m_c = max s_j, l_c =
//     sum exp(s_j - m_c)).
//     Decode uses it; fh_attention uses attn_scores_tile_kernel, the same
//     per row but with a block serving a tile of 16 / G query rows, so that
//     every key it loads serves the whole tile.
//   P.V, from M = max m_c and S = sum l_c exp(m_c - M) (the same in every
//     block) and p_j = RNE(exp(s_j - M) / S), one of two ways:
//     attn_pv_kernel, block (KV head, slice, row): all keys for head_dim /
//       slices of the dims -- few, short rows;
//     attn_pv_chunk_kernel, block (KV head, chunk, row): a chunk of keys for
//       all dims, then attn_combine_kernel adds the chunks -- long or many
//       rows.
//   fh_attention with head_dim 128 uses attn_pv_tile_kernel instead: the
//   query-row tiles of the scores, P.V on the matrix cores (M and S combined
//   over each row's chunks in another fixed order). A prompt-length call
//   whose 256-pair query tiles fill half the device takes one launch of
//   attn_flash_kernel instead (attention_flash.hip): both passes over the
//   keys in one block per tile, no workspace.
//   Every output element is a sum in a fixed order, so results do not
//   change from run to run.
// splits and slices make rows * n_kv * (blocks per pair) about
// kAttnTargetBlocks, chunks about kPvTargetBlocks: decode spreads one row
// over many CUs, prefill keeps one block per (row, KV head).
// Decode over a cache of at most 1024 positions (head_dim 64 or 128) runs
// instead as ONE launch, attn_decode_short_kernel: each block scores all of
// its KV head's keys itself (16 wavefronts, a chunk each), meets the chunks'
// statistics at block barriers and sums P.V for a 16-dim slice of V. Its
// cost is the keys every block pulls through one CU (about 34 GB/s per CU
// in the matrix-core fragment pattern), so it only pays for short caches.
#include "decoder_common.hpp"
#include "q4_gemv_mfma.hpp"

#ifndef FH_PV_CHUNKED_MIN_KEYS
#define FH_PV_CHUNKED_MIN_KEYS 16384
#endif

namespace fh {

// The one-pass prefill kernel (attention_flash.hip); false when it does not
// apply to the shape.
bool launch_attention_flash(hipStream_t stream, uint32_t cus, const uint16_t *q, const uint32_t *positions,
                            uint32_t rows, const uint16_t *k_cache, const uint16_t *v_cache, uint32_t n_heads,
                            uint32_t n_kv, uint32_t head_dim, uint32_t max_len, float scale, uint16_t *out,
                            uint32_t batch, uint64_t seq_cache);

constexpr int kAttnChunk = 64;
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kAttnMaxGroup = 8;
#ifndef FH_ATTN_TARGET_BLOCKS
#define FH_ATTN_TARGET_BLOCKS 1024
#endif
constexpr uint64_t kAttnTargetBlocks = FH_ATTN_TARGET_BLOCKS;
// The chunked P.V aims at fewer, longer blocks: each block first gathers
// the row's softmax statistics, and its partials are added by the combine
// pass (config-5 decode attention 37.3 -> 36.1 us per call against 1024).
#ifndef FH_PV_TARGET_BLOCKS
#define FH_PV_TARGET_BLOCKS 512
#endif
constexpr uint64_t kPvTargetBlocks = FH_PV_TARGET_BLOCKS;

// Workspace: per-chunk softmax statistics [rows][n_heads][nck] float2, then
// the scores [rows][n_heads][max_len] as bf16 RNE(q.k) (score_of forms
// RNE(q.k) * scale), then (chunked P.V) the partial
// outputs [rows][n_kv][chunks][G][head_dim] f32. splits: blocks per (row, KV
// head) of the scores kernel. P.V runs one of two ways:
//   sliced: blocks per (row, KV head) = slices, each over head_dim / slices
//     dims (at least 16) and all keys -- few, short rows (no combine pass);
//   chunked: blocks per (row, KV head) = chunks of chunk_keys keys over all
//     dims (16-byte V loads), then a combine pass adds the chunks -- long or
//     many rows.
struct AttnLayout {
    uint64_t nck, splits, slices, scores, part, total;  // stats at byte 0
    uint64_t chunks, chunk_keys;                         // chunks == 0: sliced P.V
};

constexpr int kPvTile = 64;  // keys per tile of the chunked P.V
// The sliced P.V reads V in 4-byte pieces (a 16-dim slice of a key row is 32
// bytes): below this many keys per (row, KV head) pair, summed over the
// launch, it still wins by skipping the combine pass.
constexpr uint64_t kPvChunkedMinKeys = FH_PV_CHUNKED_MIN_KEYS;

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
    a.part = a.scores + round_up(rows * n_heads * max_len * 2);
    a.chunks = a.chunk_keys = 0;
    if (blocks * max_len >= kPvChunkedMinKeys) {
        const uint64_t tiles = (max_len + kPvTile - 1) / kPvTile;
        const uint64_t want_pv = blocks ? (kPvTargetBlocks + blocks - 1) / blocks : 1;
        uint64_t chunks = want_pv < tiles ? want_pv : tiles;
        if (chunks == 0) chunks = 1;
        a.chunk_keys = (tiles + chunks - 1) / chunks * kPvTile;
        a.chunks = (max_len + a.chunk_keys - 1) / a.chunk_keys;
    }
    a.total = a.part + (a.chunks > 1 ? round_up(rows * n_heads * a.chunks * head_dim * 4) : 0);
    return a;
}

// ROPE: q_src is the qkv rows, the block rotates its q heads and the row's
// key, and the block owning key `pos` writes the key and value to the cache.
// Otherwise q_src is the rotated q [rows, n_heads * HD] and the cache is
// complete. Rows whose position is >= pos_limit are skipped (the PV kernel
// writes their zero output).
//
// The dot products run on the matrix cores: v_mfma_f32_16x16x32_bf16 with
// the G query heads as A rows (rows >= G zero, fragments held for the whole
// block) and 16 keys as B columns; a lane loads 16 bytes of its key per
// instruction (16 key rows x 64 bytes per wavefront load). Each wavefront
// scores whole chunks of kAttnChunk keys on its own (chunks split +
// splits * (wave + 4 i)), so the loop has no block barrier. The results'
// live rows (G of the 16 heads) go through the wavefront's LDS slice to
// lane = key, one register per head: the rounding, exp and the chunk's max
// and sum then cost G operations per lane instead of 16, and each head's
// scores leave as one 256-byte store.
typedef __attribute__((ext_vector_type(8))) __bf16 attn_bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float attn_f32x4_t;

__device__ __forceinline__ attn_f32x4_t attn_mfma(const uint4 a, const uint4 b, const attn_f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(attn_bf16x8_t, a),
                                                   __builtin_bit_cast(attn_bf16x8_t, b), c, 0, 0, 0);
}

// The workspace keeps each score as the bf16 RNE(q.k); s = RNE(q.k) * scale
// is re-formed where it is used, as one rounded multiply (never contracted
// into a following subtraction), so it equals the value the scores kernels
// computed.
__device__ __forceinline__ float score_of(uint16_t qk, float scale) { return __fmul_rn(bf(qk), scale); }

// Key groups (16 keys) a scores wavefront keeps in flight.
#ifndef FH_ATTN_SCORES_DEPTH
#define FH_ATTN_SCORES_DEPTH 2
#endif
constexpr int kScoresDepth = FH_ATTN_SCORES_DEPTH;
static_assert(kScoresDepth == 2 || kScoresDepth == 4, "a chunk's 4 groups cycle through the buffers");

template <int HD, int G, bool ROPE>
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(
    const uint16_t *__restrict__ q_src, const uint16_t *__restrict__ cos_tab, const uint16_t *__restrict__ sin_tab,
    const uint32_t *__restrict__ positions, uint32_t pos_limit, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, uint64_t row_stride, uint32_t n_heads, uint32_t n_kv, uint32_t max_len,
    uint32_t nck, uint32_t splits, float scale, uint16_t *__restrict__ scores, float2 *__restrict__ stats) {
    constexpr int KS = HD / 32;       // MFMA k steps per key group
    constexpr uint32_t PPH = HD / 8;  // 8-dim pieces per head
    constexpr int NQ = (G + 3) / 4;   // 16-lane rows of the results holding live heads
    constexpr int HP = NQ * 4;        // head slots per key after the move
    static_assert(kAttnChunk == 64, "a chunk is 4 groups of 16 keys");
    static_assert(G <= 16, "query heads fit the MFMA rows");
    // rotated q heads (rows 0..G-1), the rotated new key (row G) and a row
    // the other threads write (G + 1)
    __shared__ __align__(16) uint16_t qb[ROPE ? G + 2 : 1][ROPE ? HD : 8];
    __shared__ __align__(16) uint4 vpark[ROPE ? kAttnThreads : 1];
    __shared__ __align__(16) float sc[kAttnWaves][kAttnChunk][HP];  // raw dot products, lane = key
    const uint32_t tid = threadIdx.x, r = blockIdx.y, kvh = blockIdx.x / splits, split = blockIdx.x % splits;
    const uint32_t pos = positions[r];
    if (pos >= pos_limit) return;
    const uint32_t ctx = pos < max_len ? pos + 1 : max_len;
    const uint32_t nact = (ctx + kAttnChunk - 1) / kAttnChunk;
    if (split >= nact) return;
    const uint32_t h0 = kvh * G;
    const uint32_t wave = tid >> 6, lane = tid & 63, col = lane & 15, quad = lane >> 4;
    const uint64_t cache = static_cast<uint64_t>(r) * row_stride + static_cast<uint64_t>(kvh) * max_len * HD;
    // keys below kmax come from the cache; with ROPE key pos is the new one (from LDS)
    const uint32_t kmax = ROPE ? pos : ctx;
    const uint32_t c_first = split + splits * wave, c_step = splits * kAttnWaves;
    // key groups (16 keys) of this wavefront; 0 for a wavefront without chunks
    const uint32_t total = c_first < nact ? (nact - c_first + c_step - 1) / c_step * 4 : 0;
    const uint16_t *kb = k_cache + cache + 8 * quad;
    // group f -> B fragments of its 16 keys (clamped past the context; past
    // the wavefront's last group, key 0's row, one line for the wavefront;
    // such values are masked or unused); each fragment is one 1 KB run of the
    // tiled K cache (k_tile)
    auto load_grp = [&](uint32_t f, uint4 (&b)[KS]) {
        const uint32_t fc = total ? (f < total ? f : total - 1) : 0;
        const uint32_t j = (c_first + (fc / 4) * c_step) * kAttnChunk + (fc % 4) * 16 + col;
        const uint32_t jc = j < kmax && f < total ? j : (kmax && f < total ? kmax - 1 : 0);
        const KTile t = k_tile(jc, max_len, HD);
#pragma unroll
        for (int st = 0; st < KS; ++st) b[st] = *reinterpret_cast<const uint4 *>(kb + t.base + st * t.stride);
    };
    // Loads go out in this order, unconditionally (clamped indices): the RoPE
    // inputs, the q fragments, then the first kScoresDepth key groups, so the
    // set-up waits for its own loads only.
    const bool hlive = col < static_cast<uint32_t>(G);
    const uint32_t hc = hlive ? col : 0;
    uint4 a[KS];
    uint4 x4, r4, c4, s4, v4;
    const uint32_t tr = tid < (G + 1) * PPH ? tid : 0;
    const uint32_t hh = tr / PPH, pp = tr % PPH;  // hh < G: query head h0 + hh; hh == G: the key
    const uint16_t *row = q_src + static_cast<uint64_t>(r) * (n_heads + 2 * n_kv) * HD;
    if constexpr (ROPE) {
        const uint16_t *head = row + static_cast<uint64_t>(hh < G ? h0 + hh : n_heads + kvh) * HD;
        const uint32_t partner = pp < PPH / 2 ? pp + PPH / 2 : pp - PPH / 2;
        x4 = *reinterpret_cast<const uint4 *>(head + pp * 8);
        r4 = *reinterpret_cast<const uint4 *>(head + partner * 8);
        c4 = *reinterpret_cast<const uint4 *>(cos_tab + static_cast<uint64_t>(pos) * HD + pp * 8);
        s4 = *reinterpret_cast<const uint4 *>(sin_tab + static_cast<uint64_t>(pos) * HD + pp * 8);
        const uint32_t tv = tid >= (G + 1) * PPH && tid < (G + 2) * PPH ? tid - (G + 1) * PPH : 0;
        v4 = *reinterpret_cast<const uint4 *>(row + static_cast<uint64_t>(n_heads + n_kv + kvh) * HD + tv * 8);
    } else {
#pragma unroll
        for (int st = 0; st < KS; ++st) {
            const uint4 v = *reinterpret_cast<const uint4 *>(q_src + (static_cast<uint64_t>(r) * n_heads + h0 + hc) * HD +
                                                             32 * st + 8 * quad);
            a[st] = hlive ? v : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    uint4 b[kScoresDepth][KS];  // key groups in flight
    // The key groups go out after the RoPE inputs and the new value, pinned
    // in that order: loads return in order, so the rotation waits for its own
    // loads only, not for the keys.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int grp = 0; grp < kScoresDepth; ++grp) load_grp(grp, b[grp]);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ROPE) {
        const bool owner = (pos / kAttnChunk) % splits == split;
        const uint4 ov = rope_apply(x4, r4, c4, s4, pp < PPH / 2);
        // Every thread writes its rotation and its value piece to LDS, uses
        // outside any branch: with only the branches below using them, the
        // loads would sink into those branches, behind the key loads, and
        // their waits would drain the keys.
        *reinterpret_cast<uint4 *>(&qb[tid < (G + 1) * PPH ? hh : G + 1][pp * 8]) = ov;
        vpark[tid] = v4;
        if (owner) {
            if (tid >= G * PPH && tid < (G + 1) * PPH)
                *reinterpret_cast<uint4 *>(k_cache + cache + k_offset(pos, pp * 8, max_len, HD)) = ov;
            else if (tid >= (G + 1) * PPH && tid < (G + 2) * PPH)
                *reinterpret_cast<uint4 *>(v_cache + cache + static_cast<uint64_t>(pos) * HD +
                                           (tid - (G + 1) * PPH) * 8) = v4;
        }
        __syncthreads();
        // A fragments: head `col` (zero for col >= G), dims 32 st + 8 quad.. of each step
#pragma unroll
        for (int st = 0; st < KS; ++st) {
            const uint4 v = *reinterpret_cast<const uint4 *>(&qb[hc][32 * st + 8 * quad]);
            a[st] = hlive ? v : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    if (total == 0) return;  // a wavefront without chunks (no barrier follows)
    const uint4 *kn = reinterpret_cast<const uint4 *>(&qb[ROPE ? G : 0][8 * quad]);
    for (uint32_t f0 = 0; f0 < total; f0 += 4) {
        const uint32_t c = c_first + (f0 / 4) * c_step;
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            uint4(&bg)[KS] = b[grp % kScoresDepth];
            if constexpr (ROPE) {
                if (c * kAttnChunk + grp * 16 + col == pos) {
#pragma unroll
                    for (int st = 0; st < KS; ++st) bg[st] = kn[4 * st];
                }
            }
            attn_f32x4_t d = attn_mfma(a[0], bg[0], attn_f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int st = 1; st < KS; ++st) d = attn_mfma(a[st], bg[st], d);
            // result lane (key col, row quad) holds heads 4 quad .. 4 quad + 3
            if (quad < static_cast<uint32_t>(NQ))
                *reinterpret_cast<float4 *>(&sc[wave][grp * 16 + col][4 * quad]) = make_float4(d[0], d[1], d[2], d[3]);
            load_grp(f0 + grp + kScoresDepth, bg);
        }
        __builtin_amdgcn_wave_barrier();  // this wavefront's writes before its reads
        float dv[HP];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const float4 v = *reinterpret_cast<const float4 *>(&sc[wave][lane][4 * q]);
            dv[4 * q] = v.x, dv[4 * q + 1] = v.y, dv[4 * q + 2] = v.z, dv[4 * q + 3] = v.w;
        }
        __builtin_amdgcn_wave_barrier();  // its reads before the next chunk's writes
        // lane = key c * 64 + lane: per head, the score and the chunk's
        // (max, sum of exp) over its 64 keys
        const uint32_t j = c * kAttnChunk + lane;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const uint16_t qk = rne(dv[h]);
            const float sv = j < ctx ? bf(qk) * scale : -INFINITY;
            const float m = wave_max(sv);
            const float l = wave_sum(expf(sv - m));
            const uint64_t hrow = static_cast<uint64_t>(r) * n_heads + h0 + h;
            if (j < ctx) scores[hrow * max_len + j] = qk;
            if (lane == 0) stats[hrow * nck + c] = make_float2(m, l);
        }
    }
}

// Prefill scores over query-row tiles: block (KV head, split, tile of
// QR = 16 / G query rows). The MFMA's A rows are (query row r / G, head
// r % G), all live when G divides 16, so each key fragment a wavefront loads
// serves QR rows of the tile instead of one (attn_scores_kernel serves one
// row per block and re-reads its keys for every row). Row qi attends keys
// 0 .. ctx_qi - 1 and a chunk is scored when any row of the tile reaches it.
// Scores and each (row, head)'s per-chunk (max, sum of exp) go to the
// workspace as attn_scores_kernel writes them; a chunk past a row's context
// writes nothing for that row (its P.V reads only its own chunks).
template <int HD, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_scores_tile_kernel(
    const uint16_t *__restrict__ q, const uint32_t *__restrict__ positions, uint32_t rows,
    const uint16_t *__restrict__ k_cache, uint32_t n_heads, uint32_t max_len, uint32_t nck, uint32_t splits,
    float scale, uint16_t *__restrict__ scores, float2 *__restrict__ stats) {
    constexpr int KS = HD / 32;             // MFMA k steps per key group
    constexpr uint32_t QR = 16 / G;         // query rows per tile
    constexpr uint32_t LIVE = QR * G;       // live A rows
    static_assert(G <= 16 && kAttnChunk == 64, "a chunk is 4 groups of 16 keys");
    const uint32_t tid = threadIdx.x, kvh = blockIdx.x / splits, split = blockIdx.x % splits;
    const uint32_t r0 = blockIdx.y * QR, h0 = kvh * G;
    const uint32_t wave = tid >> 6, lane = tid & 63, col = lane & 15, quad = lane >> 4;
    // contexts of the tile's rows (0 past the last row); the tile's longest
    uint32_t ctxq[QR];
    uint32_t cmax = 0;
#pragma unroll
    for (uint32_t qi = 0; qi < QR; ++qi) {
        const uint32_t r = r0 + qi;
        const uint32_t p = r < rows ? positions[r] : 0u;
        ctxq[qi] = r < rows ? (p < max_len ? p + 1 : max_len) : 0u;
        cmax = ctxq[qi] > cmax ? ctxq[qi] : cmax;
    }
    // the contexts of this lane's 4 result rows 4 quad + i (compile-time
    // selection: no dynamically indexed private array)
    uint32_t ctxr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t rr = quad * 4 + i;
        ctxr[i] = 0;
#pragma unroll
        for (uint32_t qi = 0; qi < QR; ++qi)
            if (rr < LIVE && rr / G == qi) ctxr[i] = ctxq[qi];
    }
    const uint32_t nact = (cmax + kAttnChunk - 1) / kAttnChunk;
    const uint32_t c_first = split + splits * wave, c_step = splits * kAttnWaves;
    const uint32_t total = c_first < nact ? (nact - c_first + c_step - 1) / c_step * 4 : 0;
    if (total == 0) return;  // a wavefront without chunks (no barrier in this kernel)
    const uint16_t *kb = k_cache + static_cast<uint64_t>(kvh) * max_len * HD + 8 * quad;
    auto load_grp = [&](uint32_t f, uint4 (&b)[KS]) {
        const uint32_t fc = f < total ? f : total - 1;
        const uint32_t j = (c_first + (fc / 4) * c_step) * kAttnChunk + (fc % 4) * 16 + col;
        const uint32_t jc = j < cmax ? j : cmax - 1;
        const KTile t = k_tile(jc, max_len, HD);
#pragma unroll
        for (int st = 0; st < KS; ++st) b[st] = *reinterpret_cast<const uint4 *>(kb + t.base + st * t.stride);
    };
    // A fragments: row col = (query row col / G, head col % G), dims 32 st + 8 quad
    const uint32_t qa = col / G, ha = col % G;
    const bool alive = col < LIVE && r0 + qa < rows;
    const uint16_t *qrow = q + (static_cast<uint64_t>(alive ? r0 + qa : 0) * n_heads + h0 + (alive ? ha : 0)) * HD + 8 * quad;
    uint4 a[KS];
#pragma unroll
    for (int st = 0; st < KS; ++st) {
        const uint4 v = *reinterpret_cast<const uint4 *>(qrow + 32 * st);
        a[st] = alive ? v : make_uint4(0u, 0u, 0u, 0u);
    }
    uint4 b0[KS], b1[KS];
    load_grp(0, b0);
    load_grp(1, b1);
    for (uint32_t f0 = 0; f0 < total; f0 += 4) {
        const uint32_t c = c_first + (f0 / 4) * c_step;
        float sv[4][4];      // [group][i]: result row quad * 4 + i, key c * 64 + group * 16 + col
        uint16_t qk[4][4];   // RNE(q.k) of the same entries, the stored form
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            uint4(&b)[KS] = grp % 2 ? b1 : b0;
            const uint32_t j = c * kAttnChunk + grp * 16 + col;
            attn_f32x4_t d = attn_mfma(a[0], b[0], attn_f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int st = 1; st < KS; ++st) d = attn_mfma(a[st], b[st], d);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qk[grp][i] = rne(d[i]);
                sv[grp][i] = j < ctxr[i] ? bf(qk[grp][i]) * scale : -INFINITY;
            }
            load_grp(f0 + grp + 2, b);
        }
        // per result row: (max, sum of exp) over the chunk's 64 keys
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float m = group_max<16>(fmaxf(fmaxf(sv[0][i], sv[1][i]), fmaxf(sv[2][i], sv[3][i])));
            const float l = group_sum<16>((expf(sv[0][i] - m) + expf(sv[1][i] - m)) + (expf(sv[2][i] - m) + expf(sv[3][i] - m)));
            const uint32_t rr = quad * 4 + i;
            if (rr < LIVE && c * kAttnChunk < ctxr[i]) {  // the row is live and reaches this chunk
                const uint64_t hrow = static_cast<uint64_t>(r0 + rr / G) * n_heads + h0 + rr % G;
                uint16_t *srow = scores + hrow * max_len + c * kAttnChunk + col;
#pragma unroll
                for (int grp = 0; grp < 4; ++grp)
                    if (c * kAttnChunk + grp * 16 + col < ctxr[i]) srow[grp * 16] = qk[grp][i];
                if (col == 0) stats[hrow * nck + c] = make_float2(m, l);
            }
        }
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
    uint32_t slices, float scale, const uint16_t *__restrict__ scores, const float2 *__restrict__ stats,
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
    const uint16_t *srow = scores + (static_cast<uint64_t>(r) * n_heads + h0) * max_len;
    // A tile: V of keys t0 + s + k * slots (this thread's dims) and the
    // scores s_j = RNE(q.k_j) * scale of entries i = tid + n * 256 of the
    // tile's [G][kTile] block.
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
            sr[n] = i < G * S::kTile && j < ctx ? score_of(srow[static_cast<uint64_t>(g) * max_len + j], scale) : 0.f;
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

// Chunked P.V: block (KV head, chunk, row) sums p_j v_j over the chunk's
// keys for every dim. A lane holds 8 dims of one key (16-byte loads; a
// wavefront load covers 64 / (HD/8) whole key rows). Each wavefront takes
// every 4th tile of 16 keys on its own: it computes the row's softmax
// statistics itself, stages its tile's probabilities in its own LDS slice
// (no block barrier in the loop) and keeps kPvDepth tiles of loads in flight. The
// lanes' and wavefronts' partials are added in a fixed order. With one chunk
// per row the result (RNE) goes to out, else the f32 partial goes to part
// for attn_combine_kernel.
#ifndef FH_PV_WAVE_TILE
#define FH_PV_WAVE_TILE 16
#endif
constexpr int kPvWaveTile = FH_PV_WAVE_TILE;  // keys per wavefront tile
// Tiles a chunked P.V wavefront keeps in flight.
#ifndef FH_PV_DEPTH
#define FH_PV_DEPTH 2
#endif
constexpr int kPvDepth = FH_PV_DEPTH;

template <int HD, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_pv_chunk_kernel(
    const uint16_t *__restrict__ v_cache, uint64_t row_stride, const uint32_t *__restrict__ positions,
    uint32_t pos_limit, uint32_t n_heads, uint32_t n_kv, uint32_t max_len, uint32_t nck, uint32_t chunks,
    uint32_t chunk_keys, float scale, const uint16_t *__restrict__ scores, const float2 *__restrict__ stats,
    uint16_t *__restrict__ out, float *__restrict__ part) {
    constexpr int LPK = HD / 8, KPI = 64 / LPK;  // lanes per key, keys per load
    constexpr int IT = kPvWaveTile / KPI;        // V loads per lane per tile
    constexpr int NSW = (G * kPvWaveTile + 63) / 64;  // score loads per lane per tile
    static_assert(IT >= 1, "a tile gives the wavefront whole loads");
    __shared__ float pw[kAttnWaves][G][kPvWaveTile];
    __shared__ float red[kAttnWaves][G][HD];
    const uint32_t tid = threadIdx.x, r = blockIdx.y, kvh = blockIdx.x / chunks, c = blockIdx.x % chunks;
    const uint32_t h0 = kvh * G;
    const uint32_t pos = positions[r];
    if (pos >= pos_limit) {  // a position the cache or the tables cannot hold: zero output (or the combine's)
        if (chunks == 1)
            for (uint32_t i = tid; i < G * HD; i += kAttnThreads) out[(static_cast<uint64_t>(r) * n_heads + h0) * HD + i] = 0;
        return;
    }
    const uint32_t ctx = pos < max_len ? pos + 1 : max_len;
    const uint32_t k0 = c * chunk_keys;
    if (k0 >= ctx) return;  // a chunk past the context (never chunk 0)
    const uint32_t k1 = min(k0 + chunk_keys, ctx);
    const uint32_t nact = (ctx + kAttnChunk - 1) / kAttnChunk;
    const uint32_t wave = tid >> 6, lane = tid & 63, kl = lane / LPK, dp = lane % LPK;
    const uint32_t nt = (k1 - k0 + kPvWaveTile - 1) / kPvWaveTile;           // tiles of the chunk
    const uint32_t wt = nt > wave ? (nt - wave + kAttnWaves - 1) / kAttnWaves : 0;  // this wavefront's
    const uint16_t *vb = v_cache + static_cast<uint64_t>(r) * row_stride + static_cast<uint64_t>(kvh) * max_len * HD +
                         dp * 8;
    const uint16_t *srow = scores + (static_cast<uint64_t>(r) * n_heads + h0) * max_len;
    // Tile i of this wavefront: its V rows for this lane, and the scores of
    // entries t = lane + 64 n of its [G][16] block. Keys past k1 and tiles past
    // the wavefront's last are clamped (loads stay unconditional; the values
    // are masked or unused).
    // Tiles past the wavefront's last read the chunk's first key (one line).
    auto load_tile = [&](uint32_t i, uint4 (&vr)[IT], float (&sr)[NSW]) {
        const bool live = i < wt;
        const uint32_t t0 = k0 + (wave + (live ? i : 0) * kAttnWaves) * kPvWaveTile;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const uint32_t j = t0 + it * KPI + kl;
            vr[it] = *reinterpret_cast<const uint4 *>(vb + static_cast<uint64_t>(live && j < k1 ? j : k0) * HD);
        }
#pragma unroll
        for (int n = 0; n < NSW; ++n) {
            const uint32_t t = lane + n * 64;
            const uint32_t g = t / kPvWaveTile < G ? t / kPvWaveTile : G - 1, j = t0 + t % kPvWaveTile;
            sr[n] = score_of(srow[static_cast<uint64_t>(live ? g : 0) * max_len + (live && j < k1 ? j : k0)], scale);
        }
    };
    constexpr int kDepth = kPvDepth;
    uint4 vt[kDepth][IT];
    float sct[kDepth][NSW];
    // The row's softmax statistics, per wavefront (M, S the same everywhere).
    // Up to 128 chunks they come from registers: every head's loads go out
    // first (unconditional, clamped), then the first tiles, pinned in that
    // order, so M and S wait for their own loads only (loads return in
    // order). Past the row's chunks the values are masked by arithmetic (a
    // select on a loaded value may become a branch around the load, whose
    // join would drain the tiles). Longer rows loop over the statistics.
    float mg[G], sg[G];
    const float2 *st0 = stats + (static_cast<uint64_t>(r) * n_heads + h0) * nck;
    const bool in_regs = nact <= 128;
    float2 sv[G][2];
    if (in_regs) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                const uint32_t cc = lane + 64 * n;
                sv[g][n] = st0[static_cast<uint64_t>(g) * nck + (cc < nact ? cc : nact - 1)];
            }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kDepth; ++q) load_tile(q, vt[q], sct[q]);
    __builtin_amdgcn_sched_barrier(0);
    if (in_regs) {
        float m_add[2], l_mul[2];  // 0 and 1 for the row's chunks, -inf and 0 past them
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const bool live = lane + 64 * n < nact;
            m_add[n] = live ? 0.f : -INFINITY;
            l_mul[n] = live ? 1.f : 0.f;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float m0 = sv[g][0].x + m_add[0], m1 = sv[g][1].x + m_add[1];
            mg[g] = wave_max(fmaxf(m0, m1));
            const float sum = sv[g][0].y * l_mul[0] * expf(m0 - mg[g]) + sv[g][1].y * l_mul[1] * expf(m1 - mg[g]);
            sg[g] = wave_sum(sum);
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float2 *st = st0 + static_cast<uint64_t>(g) * nck;
            float m = -INFINITY;
            for (uint32_t cc = lane; cc < nact; cc += 64) m = fmaxf(m, st[cc].x);
            mg[g] = wave_max(m);
            float sum = 0.f;
            for (uint32_t cc = lane; cc < nact; cc += 64) {
                const float2 v = st[cc];
                sum += v.y * expf(v.x - mg[g]);
            }
            sg[g] = wave_sum(sum);
        }
    }
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    // the statistics of the head each of this lane's probability entries
    // belongs to (fixed for the whole loop)
    float lm[NSW], ls[NSW];
#pragma unroll
    for (int n = 0; n < NSW; ++n) {
        const uint32_t g = (lane + n * 64) / kPvWaveTile;
        lm[n] = mg[0], ls[n] = sg[0];
#pragma unroll
        for (int gg = 1; gg < G; ++gg)
            if (gg == static_cast<int>(g)) lm[n] = mg[gg], ls[n] = sg[gg];
    }
    auto use_tile = [&](uint32_t i, const uint4 (&vr)[IT], const float (&sr)[NSW]) {
        const uint32_t t0 = k0 + (wave + i * kAttnWaves) * kPvWaveTile;
#pragma unroll
        for (int n = 0; n < NSW; ++n) {
            const uint32_t t = lane + n * 64, g = t / kPvWaveTile, jj = t % kPvWaveTile;
            const float pv = t0 + jj < k1 ? bf(rne(expf(sr[n] - lm[n]) / ls[n])) : 0.f;
            if (t < G * kPvWaveTile) pw[wave][g][jj] = pv;
        }
        __builtin_amdgcn_wave_barrier();  // this wavefront's writes before its reads
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const uint32_t jj = it * KPI + kl;
            float v[8];
            unpack8(vr[it], v);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float pj = pw[wave][g][jj];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[g][e] += pj * v[e];
            }
        }
        __builtin_amdgcn_wave_barrier();  // reads before the next tile's writes
    };
    for (uint32_t i = 0; i < wt; i += kDepth) {
#pragma unroll
        for (int q = 0; q < kDepth; ++q) {
            if (i + q < wt) use_tile(i + q, vt[q], sct[q]);
            load_tile(i + q + kDepth, vt[q], sct[q]);
        }
    }
    // keys of one dim piece sit LPK lanes apart: add them with shuffles, then
    // the wavefronts in order through LDS
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] += __shfl_xor(acc[g][e], off, 64);
    if (lane < static_cast<uint32_t>(LPK)) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) red[wave][g][dp * 8 + e] = acc[g][e];
    }
    __syncthreads();
    for (uint32_t i = tid; i < G * HD; i += kAttnThreads) {
        const uint32_t g = i / HD, d = i % HD;
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) o += red[w][g][d];
        if (chunks == 1)
            out[(static_cast<uint64_t>(r) * n_heads + h0) * HD + i] = rne(o);
        else
            part[((static_cast<uint64_t>(r) * n_kv + kvh) * chunks + c) * (G * HD) + i] = o;
    }
}

// Prefill P.V on the matrix cores: block (KV head, chunk, tile of R = 16 / G
// query rows), the MFMA's 16 A rows being (row r / G, head r % G) as in
// attn_scores_tile_kernel. A = the probabilities of 32 keys, formed from the
// workspace scores and the row's M and S by the rounding rule of the other
// P.V kernels; B = V of those keys for 16 dims. Wavefront w takes the
// chunk's 32-key steps w, w + 4, ...: it loads the keys' V coalesced (a lane
// holds 8 keys x 8 dims), transposes each 8 x 8 block of bf16 in registers
// and stores it as [dim][key] rows of its own LDS slice, so each B fragment
// (8 keys of one dim) is one 16-byte read. The wavefronts' sums are added in
// order through LDS: one chunk writes RNE(out), several write f32 partials
// for attn_combine_kernel. Rows with no key in the chunk write nothing.
constexpr int kPvtPitch = 40;  // bf16 per transposed V row in LDS: 32 keys + 8 of padding

template <int HD, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_pv_tile_kernel(
    const uint16_t *__restrict__ v_cache, const uint32_t *__restrict__ positions, uint32_t rows, uint32_t n_heads,
    uint32_t n_kv, uint32_t max_len, uint32_t nck, uint32_t chunks, uint32_t chunk_keys,
    float scale, const uint16_t *__restrict__ scores, const float2 *__restrict__ stats, uint16_t *__restrict__ out,
    float *__restrict__ part) {
    constexpr uint32_t R = 16 / G, LIVE = R * G;
    constexpr int DT = HD / 16;  // 16-dim tiles of the output
    static_assert(HD == 128, "a lane transposes 8 keys x 8 dims, 16 pieces per key row");
    static_assert(sizeof(uint16_t) * kAttnWaves * HD * kPvtPitch >= sizeof(float) * kAttnWaves * 16 * HD,
                  "the wavefronts' sums fit the transposed-V area");
    __shared__ __align__(16) uint16_t vt[kAttnWaves][HD][kPvtPitch];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, quad = lane >> 4;
    const uint32_t kvh = blockIdx.x / chunks, c = blockIdx.x % chunks;
    const uint32_t r0 = blockIdx.y * R, h0 = kvh * G;
    uint32_t ctxq[R];
    uint32_t cmax = 0;
#pragma unroll
    for (uint32_t qi = 0; qi < R; ++qi) {
        const uint32_t r = r0 + qi;
        const uint32_t p = r < rows ? positions[r] : 0u;
        ctxq[qi] = r < rows ? (p < max_len ? p + 1 : max_len) : 0u;
        cmax = ctxq[qi] > cmax ? ctxq[qi] : cmax;
    }
    const uint32_t k0 = c * chunk_keys;
    const uint32_t kend = k0 + chunk_keys < cmax ? k0 + chunk_keys : cmax;  // keys the tile reads in this chunk
    if (k0 >= kend) return;  // no row of the tile reaches this chunk (no barrier yet)
    // this lane's A row (query row qa, head ha) and its statistics
    const uint32_t qa = col / G, ha = col % G;
    const bool alive = col < LIVE && r0 + qa < rows;
    uint32_t ctx_a = 0;
#pragma unroll
    for (uint32_t qi = 0; qi < R; ++qi)
        if (alive && qa == qi) ctx_a = ctxq[qi];
    const uint64_t hrow = static_cast<uint64_t>(alive ? r0 + qa : 0) * n_heads + h0 + (alive ? ha : 0);
    const float2 *st = stats + hrow * nck;
    const uint32_t nact = (ctx_a + kAttnChunk - 1) / kAttnChunk;
    // M and S: the 4 quads of a row take chunks quad, quad + 4, ...; combined
    // over the quads in a fixed order, so all 4 hold the same values
    float mloc = -INFINITY;
    for (uint32_t cc = quad; cc < nact; cc += 4) mloc = fmaxf(mloc, st[cc].x);
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
    const float mrow = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    float sloc = 0.f;
    for (uint32_t cc = quad; cc < nact; cc += 4) {
        const float2 v = st[cc];
        sloc += v.y * expf(v.x - mrow);
    }
    sloc += __shfl_xor(sloc, 16, 64);
    const float srow_sum = sloc + __shfl_xor(sloc, 32, 64);
    const uint16_t *srow = scores + hrow * max_len;
    const uint32_t kend_a = alive ? (k0 + chunk_keys < ctx_a ? k0 + chunk_keys : ctx_a) : 0u;  // this row's keys end
    // V: lane (key octet j, piece pv) loads keys 8 j .. 8 j + 7 of a step, dims 8 pv .. 8 pv + 7
    const uint32_t vj = lane >> 4, pv = lane & 15;
    const uint16_t *vb = v_cache + static_cast<uint64_t>(kvh) * max_len * HD + pv * 8;
    const uint32_t nsteps = (kend - k0 + 31) / 32;
    auto load_v = [&](uint32_t s, uint4 (&v)[8]) {
        const uint32_t sc = s < nsteps ? s : nsteps - 1;
        const uint32_t kb = k0 + sc * 32 + 8 * vj;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t key = kb + t < kend ? kb + t : kend - 1;
            v[t] = *reinterpret_cast<const uint4 *>(vb + static_cast<uint64_t>(key) * HD);
        }
    };
    auto load_s = [&](uint32_t s, float (&sv)[8]) {
        const uint32_t sc = s < nsteps ? s : nsteps - 1;
        const uint32_t kb = k0 + sc * 32 + 8 * quad;
#pragma unroll
        for (int e = 0; e < 8; ++e) sv[e] = score_of(srow[kb + e < kend ? kb + e : k0], scale);
    };
    attn_f32x4_t acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = attn_f32x4_t{0.f, 0.f, 0.f, 0.f};
    uint16_t(*vw)[kPvtPitch] = vt[wave];
    uint4 va[8];
    float sa[8];
    uint32_t s = wave;
    if (s < nsteps) {
        load_v(s, va);
        load_s(s, sa);
    }
    for (; s < nsteps; s += kAttnWaves) {
        uint4 vn[8];
        float sn[8];
        const bool more = s + kAttnWaves < nsteps;
        if (more) {  // the next step's loads are in flight while this one is used
            load_v(s + kAttnWaves, vn);
            load_s(s + kAttnWaves, sn);
        }
        // transpose: dim 8 pv + d of keys 8 vj .. 8 vj + 7 as one 16-byte row piece
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 &a = va[2 * i], &b = va[2 * i + 1];
                const uint32_t aw = d / 2 == 0 ? a.x : d / 2 == 1 ? a.y : d / 2 == 2 ? a.z : a.w;
                const uint32_t bw = d / 2 == 0 ? b.x : d / 2 == 1 ? b.y : d / 2 == 2 ? b.z : b.w;
                w[i] = d % 2 ? (aw >> 16) | (bw & 0xFFFF0000u) : (aw & 0xFFFFu) | (bw << 16);
            }
            *reinterpret_cast<uint4 *>(&vw[8 * pv + d][8 * vj]) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        // A: the probabilities of keys 8 quad .. 8 quad + 7 of the step for this lane's row
        const uint32_t kb = k0 + s * 32 + 8 * quad;
        uint32_t pw2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p0 = kb + 2 * i < kend_a ? bf(rne(expf(sa[2 * i] - mrow) / srow_sum)) : 0.f;
            const float p1 = kb + 2 * i + 1 < kend_a ? bf(rne(expf(sa[2 * i + 1] - mrow) / srow_sum)) : 0.f;
            pw2[i] = (__float_as_uint(p0) >> 16) | (__float_as_uint(p1) & 0xFFFF0000u);
        }
        const uint4 a = make_uint4(pw2[0], pw2[1], pw2[2], pw2[3]);
        __builtin_amdgcn_wave_barrier();  // this wavefront's V rows before its reads
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const uint4 b = *reinterpret_cast<const uint4 *>(&vw[16 * t + col][8 * quad]);
            acc[t] = attn_mfma(a, b, acc[t]);
        }
        __builtin_amdgcn_wave_barrier();  // its reads before the next step's writes
        if (more) {
#pragma unroll
            for (int t = 0; t < 8; ++t) va[t] = vn[t];
#pragma unroll
            for (int e = 0; e < 8; ++e) sa[e] = sn[e];
        }
    }
    // the wavefronts' sums, added in wavefront order: result lane (dim col of
    // tile t, row quad) holds rows 4 quad + i
    __syncthreads();  // every wavefront is done with its V slice
    float(*red)[16][HD] = reinterpret_cast<float(*)[16][HD]>(&vt[0][0][0]);
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][quad * 4 + i][16 * t + col] = acc[t][i];
    __syncthreads();
    for (uint32_t o = tid; o < LIVE * HD; o += kAttnThreads) {
        const uint32_t rr = o / HD, d = o % HD, qi = rr / G, h = rr % G;
        uint32_t ctx_r = 0;
#pragma unroll
        for (uint32_t q = 0; q < R; ++q)
            if (q == qi) ctx_r = ctxq[q];
        if (k0 >= ctx_r) continue;  // past the row's context, or a row past the last
        const float v = ((red[0][rr][d] + red[1][rr][d]) + red[2][rr][d]) + red[3][rr][d];
        const uint32_t r = r0 + qi;
        if (chunks == 1)
            out[(static_cast<uint64_t>(r) * n_heads + h0 + h) * HD + d] = rne(v);
        else
            part[((static_cast<uint64_t>(r) * n_kv + kvh) * chunks + c) * (G * HD) + h * HD + d] = v;
    }
}

// Adds the chunked P.V partials of each (row, KV head): block (64 outputs,
// KV head, row); the 4 wavefronts each add a contiguous quarter of the row's
// active chunks in order (8 loads issued before their adds), then the
// quarters are added in order, so the sum is the same every run.
// With img (img_rows = the launch's rows, 2..8), the block also writes its 64
// outputs -- one quantisation group of the row, width % 64 == 0 -- into the
// o projection's staged-x image in mf_pack_kernel's layout (fragments by
// mf_slot, the group's X = sum of its values), and block (0, 0, 0) the zero
// slot and X = 0 for rows img_rows..7: the matrix-core GEMV then copies the
// image instead of staging x itself (q4_gemv_packed), with the same values.
constexpr int kCombineOuts = 64;

__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(
    const uint32_t *__restrict__ positions, uint32_t pos_limit, uint32_t n_heads, uint32_t n_kv, uint32_t width,
    uint32_t max_len, uint32_t chunks, uint32_t chunk_keys, const float *__restrict__ part,
    uint16_t *__restrict__ out, uint4 *__restrict__ img, uint32_t img_rows) {
    __shared__ float quarter_sum[kAttnWaves][kCombineOuts];
    __shared__ __align__(16) uint16_t ob[kCombineOuts];
    const uint32_t tid = threadIdx.x, e = tid % kCombineOuts, qw = tid / kCombineOuts;
    const uint32_t i = blockIdx.x * kCombineOuts + e, kvh = blockIdx.y, r = blockIdx.z;
    const uint32_t pos = positions[r];
    uint16_t *orow = out + (static_cast<uint64_t>(r) * n_kv + kvh) * width;  // heads kvh*G.. of row r
    // a position the cache or the tables cannot hold: zero output
    const bool live = pos < pos_limit;
    const uint32_t ctx = pos < max_len ? pos + 1 : max_len;
    const uint32_t nc = live ? (ctx + chunk_keys - 1) / chunk_keys : 0u;
    const uint32_t per = (nc + kAttnWaves - 1) / kAttnWaves;
    const uint32_t c0 = qw * per, c1 = min(c0 + per, nc);
    const float *pr = part + (static_cast<uint64_t>(r) * n_kv + kvh) * chunks * width + (i < width ? i : 0);
    float o = 0.f;
    for (uint32_t c = c0; c < c1; c += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = pr[static_cast<uint64_t>(c + u < c1 ? c + u : c0) * width];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (c + u < c1) o += v[u];
    }
    quarter_sum[qw][e] = o;
    __syncthreads();
    if (qw == 0) {
        float t = quarter_sum[0][e];
#pragma unroll
        for (int w = 1; w < kAttnWaves; ++w) t += quarter_sum[w][e];
        const uint16_t ov = live ? rne(t) : uint16_t{0};
        if (i < width) orow[i] = ov;
        ob[e] = ov;
    }
    if (img == nullptr) return;  // uniform over the launch
    __syncthreads();
    const uint32_t k = n_kv * width, ppr = k / 8;  // the o projection's x row
    float *xs = reinterpret_cast<float *>(img + static_cast<uint64_t>(img_rows) * ppr + 2);
    if (tid < 8) {  // pieces of the block's group: lanes 0..7, as the GEMV's own staging sums them
        const uint32_t g = (kvh * width + blockIdx.x * kCombineOuts) / kGroup;
        const uint4 p = gemv_permute(*reinterpret_cast<const uint4 *>(&ob[8 * tid]));
        img[mf_slot_rt(img_rows, r, g * 8 + tid)] = p;
        const float gsum = group_sum<8>(mf_piece_sum(p));
        if (tid == 0) xs[g * 8 + r] = gsum;
    }
    if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) {
        if (tid == 0) img[static_cast<uint64_t>(img_rows) * ppr] = make_uint4(0u, 0u, 0u, 0u);  // the zero slot
        const uint32_t G = k / kGroup;
        for (uint32_t j = tid; j < (8 - img_rows) * G; j += kAttnThreads) xs[(j % G) * 8 + img_rows + j / G] = 0.f;
    }
}

// Decode attention over a cache of at most kShortKeys positions in ONE
// launch: block (part, KV head, row) of 16 wavefronts, wavefront w owning
// chunk w (keys 64 w .. 64 w + 63).
//   1. Every block rotates the row's q and key (LDS); part 0 writes the new
//      key and value to the cache.
//   2. A wavefront scores its chunk on the matrix cores (the fragments of
//      attn_scores_kernel), then moves the live rows of the 16x16 results
//      (G of 16 heads) through LDS so that lane = key and one register per
//      head: the softmax arithmetic then runs on G values per lane, not 16.
//      s_j = RNE(q.k_j) * scale; the chunk's max per head goes to LDS.
//   3. M = max over the chunks; e_j = exp(s_j - M); the chunk's sum of e_j
//      per head goes to LDS.
//   4. S = sum of the chunk sums (a fixed 16-lane tree, the same in every
//      wavefront and block); p_j = RNE(e_j / S), the reference's rounding
//      point, into the wavefront's LDS slice.
//   5. The wavefront sums p_j v_j over its keys for the block's DB dims
//      (part * DB ..), lanes (dim pair, key slot); slots are added within
//      aligned lane groups, then the wavefronts' partials in wavefront order.
// Every output is a sum in a fixed order. The head_dim / DB parts of a KV
// head each read all of its keys (for the scores) and DB dims of its
// values; blocks of one KV head are n_kv apart in the grid, which the
// dispatcher deals round-robin to the XCDs, so with 8 KV heads a head's
// parts share an L2.
constexpr int kShortThreads = 1024;
constexpr int kShortWaves = kShortThreads / 64;
constexpr uint32_t kShortKeys = kShortWaves * kAttnChunk;

template <int HD, int G, int DB>
__global__ __launch_bounds__(kShortThreads) void attn_decode_short_kernel(
    const uint16_t *__restrict__ qkv, const uint16_t *__restrict__ cos_tab, const uint16_t *__restrict__ sin_tab,
    const uint32_t *__restrict__ positions, uint32_t pos_limit, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, uint64_t row_stride, uint32_t n_heads, uint32_t n_kv, uint32_t max_len,
    float scale, uint16_t *__restrict__ out) {
    constexpr int KS = HD / 32;           // MFMA k steps per key group
    constexpr uint32_t PPH = HD / 8;      // 8-dim pieces per head
    constexpr int NQ = (G + 3) / 4;       // 16-lane rows of the results holding live heads
    constexpr int HP = NQ * 4;            // head slots per key after the move
    constexpr int PAIRS = DB / 2;         // dim pairs of the block
    constexpr int SLOTS = 64 / PAIRS;     // key slots per wavefront (adjacent lanes)
    constexpr int KPS = kAttnChunk / SLOTS;  // keys per slot
    static_assert(HD == 64 || HD == 128, "a wavefront holds a chunk's key fragments in registers");
    static_assert(G <= kAttnMaxGroup && (G + 2) * PPH <= kShortThreads, "RoPE lanes fit the block");
    static_assert((DB == 4 || DB == 8 || DB == 16 || DB == 32) && HD % DB == 0, "32, 16, 8 or 4 key slots");
    __shared__ __align__(16) uint16_t qb[G][HD];
    __shared__ __align__(16) uint16_t knew[HD];
    __shared__ __align__(16) float sc[kShortWaves][kAttnChunk][HP];  // raw dot products, lane = key
    __shared__ __align__(16) float pw[kShortWaves][G][kAttnChunk];   // probabilities
    __shared__ float cmax[kShortWaves][G], csum[kShortWaves][G];
    __shared__ float red[kShortWaves][G][DB];
    const uint32_t tid = threadIdx.x, r = blockIdx.y, kvh = blockIdx.x % n_kv, part = blockIdx.x / n_kv;
    const uint32_t h0 = kvh * G, d0 = part * DB;
    const uint32_t wave = tid >> 6, lane = tid & 63, col = lane & 15, quad = lane >> 4;
    uint16_t *orow = out + (static_cast<uint64_t>(r) * n_heads + h0) * HD + d0;
    const uint32_t pos = positions[r];
    if (pos >= pos_limit) {  // a position the cache or the tables cannot hold: zero output, no cache write
        if (tid < G * DB) orow[(tid / DB) * HD + tid % DB] = 0;
        return;
    }
    const uint32_t ctx = pos + 1;  // pos < pos_limit <= max_len <= kShortKeys
    const uint32_t nact = (ctx + kAttnChunk - 1) / kAttnChunk;
    const bool active = wave < nact;
    const uint32_t c0 = wave * kAttnChunk;
    const uint64_t cache = static_cast<uint64_t>(r) * row_stride + static_cast<uint64_t>(kvh) * max_len * HD;
    const uint16_t *row = qkv + static_cast<uint64_t>(r) * (n_heads + 2 * n_kv) * HD;
    // RoPE inputs first (thread hh < G: query head h0 + hh, hh == G: the key;
    // then the value's pieces), so the set-up waits for its own loads only
    uint4 x4, r4, c4, s4, v4;
    const uint32_t tr = tid < (G + 1) * PPH ? tid : 0;
    const uint32_t hh = tr / PPH, pp = tr % PPH;
    const bool rope_wave = wave * 64 < (G + 2) * PPH;  // wavefronts holding RoPE or value lanes
    if (rope_wave) {
        const uint16_t *head = row + static_cast<uint64_t>(hh < G ? h0 + hh : n_heads + kvh) * HD;
        const uint32_t partner = pp < PPH / 2 ? pp + PPH / 2 : pp - PPH / 2;
        x4 = *reinterpret_cast<const uint4 *>(head + pp * 8);
        r4 = *reinterpret_cast<const uint4 *>(head + partner * 8);
        c4 = *reinterpret_cast<const uint4 *>(cos_tab + static_cast<uint64_t>(pos) * HD + pp * 8);
        s4 = *reinterpret_cast<const uint4 *>(sin_tab + static_cast<uint64_t>(pos) * HD + pp * 8);
        const uint32_t tv = tid >= (G + 1) * PPH && tid < (G + 2) * PPH ? tid - (G + 1) * PPH : 0;
        v4 = *reinterpret_cast<const uint4 *>(row + static_cast<uint64_t>(n_heads + n_kv + kvh) * HD + tv * 8);
    }
    // this wavefront's 4 key groups (keys below pos from the cache, clamped
    // otherwise: key pos comes from LDS, later ones are masked)
    uint4 b[4][KS];
    // V: lane (dim pair dp, slot vs) holds dims d0 + 2 dp, +1 of keys
    // c0 + KPS vs + t; keys past pos are zero, key pos is the new value
    const uint32_t dp = lane / SLOTS, vs = lane % SLOTS;
    uint32_t vr[KPS];
    const uint32_t vnew =
        *reinterpret_cast<const uint32_t *>(row + static_cast<uint64_t>(n_heads + n_kv + kvh) * HD + d0 + 2 * dp);
    if (active) {
        const uint16_t *kb = k_cache + cache + 8 * quad;
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            const uint32_t j = c0 + grp * 16 + col;
            const uint32_t jc = j < pos ? j : (pos ? pos - 1 : 0);
            const KTile t = k_tile(jc, max_len, HD);
#pragma unroll
            for (int st = 0; st < KS; ++st) b[grp][st] = *reinterpret_cast<const uint4 *>(kb + t.base + st * t.stride);
        }
        const uint16_t *vb = v_cache + cache + d0 + 2 * dp;
#pragma unroll
        for (int t = 0; t < KPS; ++t) {
            const uint32_t j = c0 + KPS * vs + t;
            const uint32_t jc = j < pos ? j : (pos ? pos - 1 : 0);
            vr[t] = *reinterpret_cast<const uint32_t *>(vb + static_cast<uint64_t>(jc) * HD);
        }
    }
    if (rope_wave) {
        const uint4 ov = rope_apply(x4, r4, c4, s4, pp < PPH / 2);
        if (tid < (G + 1) * PPH) {
            if (hh < G) {
                *reinterpret_cast<uint4 *>(&qb[hh][pp * 8]) = ov;
            } else {
                *reinterpret_cast<uint4 *>(knew + pp * 8) = ov;
                if (part == 0) *reinterpret_cast<uint4 *>(k_cache + cache + k_offset(pos, pp * 8, max_len, HD)) = ov;
            }
        } else if (part == 0 && tid < (G + 2) * PPH) {
            *reinterpret_cast<uint4 *>(v_cache + cache + static_cast<uint64_t>(pos) * HD + (tid - (G + 1) * PPH) * 8) = v4;
        }
    }
    __syncthreads();
    const uint32_t j = c0 + lane;  // this lane's key after the move
    float sv[G];
    if (active) {
        const bool hlive = col < static_cast<uint32_t>(G);
        const uint32_t hc = hlive ? col : 0;
        uint4 a[KS];
#pragma unroll
        for (int st = 0; st < KS; ++st) {
            const uint4 v = *reinterpret_cast<const uint4 *>(&qb[hc][32 * st + 8 * quad]);
            a[st] = hlive ? v : make_uint4(0u, 0u, 0u, 0u);
        }
        const uint4 *kn = reinterpret_cast<const uint4 *>(knew + 8 * quad);
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            if (c0 + grp * 16 + col == pos) {
#pragma unroll
                for (int st = 0; st < KS; ++st) b[grp][st] = kn[4 * st];
            }
            attn_f32x4_t d = attn_mfma(a[0], b[grp][0], attn_f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int st = 1; st < KS; ++st) d = attn_mfma(a[st], b[grp][st], d);
            // result lane (key col, row quad) holds heads 4 quad .. 4 quad + 3
            if (quad < static_cast<uint32_t>(NQ))
                *reinterpret_cast<float4 *>(&sc[wave][grp * 16 + col][4 * quad]) = make_float4(d[0], d[1], d[2], d[3]);
        }
        __builtin_amdgcn_wave_barrier();  // this wavefront's writes before its reads
        float dv[HP];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const float4 v = *reinterpret_cast<const float4 *>(&sc[wave][lane][4 * q]);
            dv[4 * q] = v.x, dv[4 * q + 1] = v.y, dv[4 * q + 2] = v.z, dv[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            sv[h] = j < ctx ? bf(rne(dv[h])) * scale : -INFINITY;
            const float m = wave_max(sv[h]);
            if (lane == 0) cmax[wave][h] = m;
        }
    }
    __syncthreads();
    // per-head totals over the chunks: row q of the wavefront reduces head
    // 4 n + q over chunk `col` (lanes past the active chunks hold the identity)
    auto row_reduce = [&](bool is_max, float (&res)[G]) {
#pragma unroll
        for (int n = 0; n < NQ; ++n) {
            const uint32_t h = 4 * n + quad;
            const bool live = col < nact && h < static_cast<uint32_t>(G);
            const uint32_t cc = live ? col : 0, hc = live ? h : 0;
            const float x = live ? (is_max ? cmax[cc][hc] : csum[cc][hc]) : (is_max ? -INFINITY : 0.f);
            const float t = is_max ? group_max<16>(x) : group_sum<16>(x);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (4 * n + q < G) res[4 * n + q] = lane_value(t, 16 * q);
        }
    };
    float e[G];
    if (active) {
        float mg[G];
        row_reduce(true, mg);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            e[h] = expf(sv[h] - mg[h]);
            const float l = wave_sum(e[h]);
            if (lane == 0) csum[wave][h] = l;
        }
    }
    __syncthreads();
    float acc[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;
    if (active) {
        float sg[G];
        row_reduce(false, sg);
#pragma unroll
        for (int h = 0; h < G; ++h) pw[wave][h][lane] = bf(rne(e[h] / sg[h]));
        __builtin_amdgcn_wave_barrier();  // this wavefront's probabilities before its reads
        if constexpr (KPS == 2) {
            float v0[2], v1[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t jk = c0 + KPS * vs + u;
                const uint32_t w = jk < pos ? vr[u] : (jk == pos ? vnew : 0u);
                v0[u] = bf(w & 0xFFFFu);
                v1[u] = bf(w >> 16);
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float2 p2 = *reinterpret_cast<const float2 *>(&pw[wave][g][KPS * vs]);
                acc[g][0] += p2.x * v0[0];
                acc[g][1] += p2.x * v1[0];
                acc[g][0] += p2.y * v0[1];
                acc[g][1] += p2.y * v1[1];
            }
        }
#pragma unroll
        for (int t4 = 0; t4 < KPS / 4; ++t4) {
            float v0[4], v1[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t t = 4 * t4 + u, jk = c0 + KPS * vs + t;
                const uint32_t w = jk < pos ? vr[t] : (jk == pos ? vnew : 0u);
                v0[u] = bf(w & 0xFFFFu);
                v1[u] = bf(w >> 16);
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float4 p4 = *reinterpret_cast<const float4 *>(&pw[wave][g][KPS * vs + 4 * t4]);
                acc[g][0] += p4.x * v0[0];
                acc[g][1] += p4.x * v1[0];
                acc[g][0] += p4.y * v0[1];
                acc[g][1] += p4.y * v1[1];
                acc[g][0] += p4.z * v0[2];
                acc[g][1] += p4.z * v1[2];
                acc[g][0] += p4.w * v0[3];
                acc[g][1] += p4.w * v1[3];
            }
        }
        // the slots of a dim pair are adjacent lanes: add them in their group
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if constexpr (SLOTS >= 8) {
                    acc[g][k] = group_sum<SLOTS>(acc[g][k]);
                } else {
                    acc[g][k] += dpp_mov<0xB1>(acc[g][k]);
                    acc[g][k] += dpp_mov<0x4E>(acc[g][k]);
                }
            }
        if (vs == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                red[wave][g][2 * dp] = acc[g][0];
                red[wave][g][2 * dp + 1] = acc[g][1];
            }
        }
    }
    __syncthreads();
    if (tid < G * DB) {
        const uint32_t g = tid / DB, dd = tid % DB;
        float o = red[0][g][dd];
        for (uint32_t w = 1; w < nact; ++w) o += red[w][g][dd];
        orow[g * HD + dd] = rne(o);
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
    uint4 *img = nullptr;   // decode: the o projection's x image (attn_combine_kernel), or null
    uint32_t img_rows = 0;  // its rows (the launch's rows)
};

template <int G, int P>
static void launch_pv(hipStream_t stream, uint32_t rows, const AttnLayout &a, const AttnArgs &x, uint32_t head_dim,
                      const uint16_t *scores, const float2 *stats) {
    const dim3 grid(static_cast<uint32_t>(x.n_kv * a.slices), rows);
    hipLaunchKernelGGL((attn_pv_kernel<G, P>), grid, dim3(kAttnThreads), 0, stream, x.v_cache, x.row_stride,
                       x.positions, x.pos_limit, x.n_heads, x.n_kv, head_dim, x.max_len,
                       static_cast<uint32_t>(a.nck), static_cast<uint32_t>(a.slices), x.scale, scores, stats, x.out);
}

template <int HD, int G, bool ROPE>
static void launch_attention(hipStream_t stream, uint32_t rows, const AttnLayout &a, const AttnArgs &x) {
    auto *stats = reinterpret_cast<float2 *>(x.ws);
    auto *scores = reinterpret_cast<uint16_t *>(x.ws + a.scores);
    if constexpr (ROPE) {
        const dim3 grid(static_cast<uint32_t>(x.n_kv * a.splits), rows);
        hipLaunchKernelGGL((attn_scores_kernel<HD, G, ROPE>), grid, dim3(kAttnThreads), 0, stream, x.q_src,
                           x.cos_tab, x.sin_tab, x.positions, x.pos_limit, x.k_cache, x.v_cache, x.row_stride,
                           x.n_heads, x.n_kv, x.max_len, static_cast<uint32_t>(a.nck),
                           static_cast<uint32_t>(a.splits), x.scale, scores, stats);
    } else {
        // query-row tiles (one shared cache); splits make about
        // kAttnTargetBlocks blocks in all, as for the per-row kernel
        constexpr uint32_t kQR = 16 / G;
        const uint64_t tiles = (rows + kQR - 1) / kQR;
        const uint64_t blocks = tiles * x.n_kv;
        const uint64_t want = (kAttnTargetBlocks + blocks - 1) / blocks;
        const uint32_t splits = static_cast<uint32_t>(want < a.nck ? want : a.nck);
        const dim3 grid(static_cast<uint32_t>(x.n_kv * splits), static_cast<uint32_t>(tiles));
        hipLaunchKernelGGL((attn_scores_tile_kernel<HD, G>), grid, dim3(kAttnThreads), 0, stream, x.q_src,
                           x.positions, rows, x.k_cache, x.n_heads, x.max_len, static_cast<uint32_t>(a.nck), splits,
                           x.scale, scores, stats);
    }
    if constexpr (!ROPE && HD == 128) {
        // prefill: P.V on the matrix cores over the same query-row tiles
        constexpr uint32_t kQR = 16 / G;
        const uint32_t tiles = (rows + kQR - 1) / kQR;
        const uint32_t chunks = a.chunks ? static_cast<uint32_t>(a.chunks) : 1u;
        const uint32_t ck = a.chunks ? static_cast<uint32_t>(a.chunk_keys) : x.max_len;
        float *part = reinterpret_cast<float *>(x.ws + a.part);
        hipLaunchKernelGGL((attn_pv_tile_kernel<HD, G>), dim3(x.n_kv * chunks, tiles), dim3(kAttnThreads), 0, stream,
                           x.v_cache, x.positions, rows, x.n_heads, x.n_kv, x.max_len, static_cast<uint32_t>(a.nck),
                           chunks, ck, x.scale, scores, stats, x.out, part);
        if (chunks > 1)
            hipLaunchKernelGGL(attn_combine_kernel, dim3((G * HD + kCombineOuts - 1) / kCombineOuts, x.n_kv, rows),
                               dim3(kAttnThreads), 0, stream, x.positions, x.pos_limit, x.n_heads, x.n_kv,
                               static_cast<uint32_t>(G * HD), x.max_len, chunks, ck, part, x.out, nullptr, 0u);
        return;
    }
    if (a.chunks) {
        const uint32_t chunks = static_cast<uint32_t>(a.chunks), ck = static_cast<uint32_t>(a.chunk_keys);
        float *part = reinterpret_cast<float *>(x.ws + a.part);
        hipLaunchKernelGGL((attn_pv_chunk_kernel<HD, G>), dim3(x.n_kv * chunks, rows), dim3(kAttnThreads), 0, stream,
                           x.v_cache, x.row_stride, x.positions, x.pos_limit, x.n_heads, x.n_kv, x.max_len,
                           static_cast<uint32_t>(a.nck), chunks, ck, x.scale, scores, stats, x.out, part);
        if (chunks > 1)
            hipLaunchKernelGGL(attn_combine_kernel, dim3((G * HD + kCombineOuts - 1) / kCombineOuts, x.n_kv, rows),
                               dim3(kAttnThreads), 0, stream, x.positions, x.pos_limit, x.n_heads, x.n_kv,
                               static_cast<uint32_t>(G * HD), x.max_len, chunks, ck, part, x.out,
                               ROPE ? x.img : nullptr, ROPE ? x.img_rows : 0u);
        return;
    }
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

// Caches of at most this many positions take attn_decode_short_kernel
// (head_dim 64 or 128).
#ifndef FH_DECODE_SHORT_MAX_LEN
#define FH_DECODE_SHORT_MAX_LEN 1024
#endif
constexpr uint32_t kDecodeShortMaxLen = FH_DECODE_SHORT_MAX_LEN;
static_assert(kDecodeShortMaxLen <= kShortKeys, "one chunk per wavefront");

#ifndef FH_DECODE_SHORT_DIMS
#define FH_DECODE_SHORT_DIMS 4
#endif
constexpr int kShortDims = FH_DECODE_SHORT_DIMS;  // V dims per block

template <int HD, int G>
static void launch_decode_short(hipStream_t stream, uint32_t rows, const AttnArgs &x) {
    // one wavefront per 64-key chunk the cache can hold (positions beyond
    // max_len take no chunk), and at least the RoPE and value lanes
    const uint32_t chunk_waves = (x.max_len + kAttnChunk - 1) / kAttnChunk;
    const uint32_t rope_waves = ((G + 2) * (HD / 8) + 63) / 64;
    // the output (and zero-output) writers are threads tid < G * kShortDims
    const uint32_t out_waves = (G * kShortDims + 63) / 64;
    uint32_t waves = chunk_waves > rope_waves ? chunk_waves : rope_waves;
    if (out_waves > waves) waves = out_waves;
    const dim3 grid(x.n_kv * (HD / kShortDims), rows);
    hipLaunchKernelGGL((attn_decode_short_kernel<HD, G, kShortDims>), grid, dim3(64 * waves), 0, stream, x.q_src, x.cos_tab,
                       x.sin_tab, x.positions, x.pos_limit, x.k_cache, x.v_cache, x.row_stride, x.n_heads, x.n_kv,
                       x.max_len, x.scale, x.out);
}

static bool launch_decode_short_shape(int64_t head_dim, int64_t g, hipStream_t stream, uint32_t rows,
                                      const AttnArgs &x) {
#define FH_SHORT_G(HD, GG)                                         \
    case GG:                                                       \
        launch_decode_short<HD, GG>(stream, rows, x);              \
        return true;
#define FH_SHORT_HD(HD)                                            \
    if (head_dim == HD) switch (g) {                               \
            FH_SHORT_G(HD, 1)                                      \
            FH_SHORT_G(HD, 2)                                      \
            FH_SHORT_G(HD, 3)                                      \
            FH_SHORT_G(HD, 4)                                      \
            FH_SHORT_G(HD, 5)                                      \
            FH_SHORT_G(HD, 6)                                      \
            FH_SHORT_G(HD, 7)                                      \
            FH_SHORT_G(HD, 8)                                      \
        }
    FH_SHORT_HD(64)
    FH_SHORT_HD(128)
#undef FH_SHORT_HD
#undef FH_SHORT_G
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

// The workspace holds fewer than rows * n_heads * (6 * max_len + 2 *
// head_dim) floats (scores, statistics, P.V partials); refuse sizes whose
// byte counts would not fit comfortably in 64 bits.
int check_attn_size(const char *fn, int64_t rows, int64_t n_heads, int64_t head_dim, int64_t max_len) {
    const long double floats = static_cast<long double>(rows) * n_heads * (6.0L * max_len + 2.0L * head_dim);
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
                    int64_t max_len, void *workspace, uint64_t workspace_bytes, AttnLayout *a,
                    bool workspace_is_allocation = true) {
    if (int rc = check_heads(fn, n_heads, n_kv, head_dim)) return rc;
    if (max_len == 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: empty KV cache", fn);
    if (int rc = check_attn_size(fn, rows, n_heads, head_dim, max_len)) return rc;
    *a = attn_layout(rows, n_heads, n_kv, head_dim, max_len);
    if (rows > 65535 || static_cast<uint64_t>(n_kv) * (a->splits + a->slices + a->chunks) > 0x7FFFFFFFu)
        return fail(FH_ERR_INDEX_TOO_LARGE, "%s: %lld rows x %llu splits exceed the grid", fn, (long long)rows,
                    (unsigned long long)(n_kv * a->splits));
    if (workspace_bytes < a->total)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: workspace of %llu bytes, %llu needed", fn,
                    (unsigned long long)workspace_bytes, (unsigned long long)a->total);
    if (reinterpret_cast<uintptr_t>(workspace) & 15u)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: workspace must be 16-byte aligned", fn);
    if (!workspace_is_allocation) return FH_OK;  // the device's static scratch, sized above
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
    // prompt-length calls that fill the device: the one-pass kernel
    // (attention_flash.hip), which leaves the workspace untouched
    return dispatch(dev, fn, [&] {
        if (!launch_attention_flash(dev->stream, dev->compute_units, q, positions, static_cast<uint32_t>(tokens),
                                    k_cache, v_cache, static_cast<uint32_t>(n_heads), static_cast<uint32_t>(n_kv),
                                    static_cast<uint32_t>(head_dim), static_cast<uint32_t>(max_len), scale, out, 1,
                                    0))
            launch_attention_shape<false>(head_dim, n_heads / n_kv, dev->stream, static_cast<uint32_t>(tokens), a, x);
    });
}

extern "C" int fh_decode_attention_workspace(int64_t batch, int64_t n_heads, int64_t n_kv, int64_t head_dim,
                                             int64_t max_len, uint64_t *bytes) {
    return workspace_bytes("fh_decode_attention_workspace", batch, n_heads, n_kv, head_dim, max_len, bytes);
}

// The no-allocation decode attention's workspace. A __device__ array exists
// once per GPU the library runs on (each holds its own copy from the first
// use until the process ends); host code reaches it only through the address
// hipGetSymbolAddress gives for that GPU, kept in fh_device::scratch.
constexpr uint64_t kScratchBytes = FH_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace fh {

// Called once per device at creation, with that device current.
int attention_scratch_setup(fh_device *dev) {
    void *ptr = nullptr;
    hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
        (void)hipGetLastError();  // clears the runtime's last-error slot
        return fail(FH_ERR_DEVICE_UNAVAILABLE, "fh_device_create: hipGetSymbolAddress(scratch) failed: %s",
                    hipGetErrorString(err));
    }
    dev->scratch = ptr;
    return FH_OK;
}

}  // namespace fh

namespace {

// fh_decode_attention with its workspace either a caller allocation (checked
// against the device's allocations) or the device's scratch array.
// img (the device's pack area, img_rows = batch): also leave the o
// projection's x image there when the chunked P.V's combine runs (*wrote).
int decode_attention(const char *fn, fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads,
                     int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab, const uint16_t *sin_tab,
                     int64_t table_len, const uint32_t *positions, uint16_t *k_cache, uint16_t *v_cache,
                     int64_t max_len, float scale, void *workspace, uint64_t workspace_bytes, bool scratch_ws,
                     uint16_t *out, uint4 *img = nullptr, bool *wrote = nullptr) {
    if (wrote) *wrote = false;
    if (int rc = check_usable(dev, fn)) return rc;
    if (int rc = fh_check_dims(fn, {batch, n_heads, n_kv, head_dim, table_len, max_len})) return rc;
    if (batch == 0) return FH_OK;
    AttnLayout a;
    if (scratch_ws) {
        if (int rc = check_heads(fn, n_heads, n_kv, head_dim)) return rc;
        if (max_len == 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: empty KV cache", fn);
        if (int rc = check_attn_size(fn, batch, n_heads, head_dim, max_len)) return rc;
        const uint64_t need = attn_layout(batch, n_heads, n_kv, head_dim, max_len).total;
        if (need > kScratchBytes)
            return fail(FH_ERR_UNSUPPORTED,
                        "%s: these sizes need a %llu-byte workspace; the static one holds %llu (use "
                        "fh_decode_attention with a caller workspace)",
                        fn, (unsigned long long)need, (unsigned long long)kScratchBytes);
        if (!dev->scratch) return fail(FH_ERR_DEVICE_UNAVAILABLE, "%s: the device has no scratch address", fn);
        workspace = dev->scratch;
        workspace_bytes = kScratchBytes;
    }
    if (int rc = check_attention(fn, dev, batch, n_heads, n_kv, head_dim, max_len, workspace, workspace_bytes, &a,
                                 !scratch_ws))
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
    AttnArgs x{qkv, cos_tab, sin_tab, positions, limit, k_cache, v_cache, row_stride,
               static_cast<uint32_t>(n_heads), static_cast<uint32_t>(n_kv), static_cast<uint32_t>(max_len),
               scale, static_cast<char *>(workspace), out};
    // the image holds 2..8 rows of a width the pack area takes, in whole groups
    const uint64_t img_k = static_cast<uint64_t>(n_heads) * head_dim;
    if (img && batch >= 2 && batch <= 8 && img_k % kGroup == 0 && img_k <= kMfPackMaxK) {
        x.img = img;
        x.img_rows = static_cast<uint32_t>(batch);
    }
    // short caches: one launch (no workspace use); otherwise scores, then P.V
    const bool short_cache = static_cast<uint64_t>(max_len) <= kDecodeShortMaxLen && head_dim != 256;
    dev->no_alloc = scratch_ws;
    bool combined = false;
    const int rc = dispatch(dev, fn, [&] {
        if (!short_cache ||
            !launch_decode_short_shape(head_dim, n_heads / n_kv, dev->stream, static_cast<uint32_t>(batch), x))
            combined = launch_attention_shape<true>(head_dim, n_heads / n_kv, dev->stream,
                                                    static_cast<uint32_t>(batch), a, x) &&
                       a.chunks > 1;
    });
    if (wrote) *wrote = rc == FH_OK && x.img != nullptr && combined;
    dev->no_alloc = false;
    return rc;
}

}  // namespace

namespace fh {

// fh_decode_attention for the batched decode step of fh_llama_forward: where
// the chunked P.V's combine runs (and 2..8 rows), it also leaves the o
// projection's x image in the device's pack area for q4_gemv_packed;
// *wrote tells whether it did.
int decode_attention_with_o_image(fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads, int64_t n_kv,
                                  int64_t head_dim, const uint16_t *cos_tab, const uint16_t *sin_tab,
                                  int64_t table_len, const uint32_t *positions, uint16_t *k_cache,
                                  uint16_t *v_cache, int64_t max_len, float scale, void *workspace,
                                  uint64_t workspace_bytes, uint16_t *out, bool *wrote) {
    return decode_attention("fh_llama_forward", dev, qkv, batch, n_heads, n_kv, head_dim, cos_tab, sin_tab,
                            table_len, positions, k_cache, v_cache, max_len, scale, workspace, workspace_bytes, false,
                            out, static_cast<uint4 *>(dev->pack_area), wrote);
}

}  // namespace fh

extern "C" int fh_decode_attention(fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads,
                                   int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab,
                                   const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
                                   uint16_t *k_cache, uint16_t *v_cache, int64_t max_len, float scale,
                                   void *workspace, uint64_t workspace_bytes, uint16_t *out) {
    return decode_attention("fh_decode_attention", dev, qkv, batch, n_heads, n_kv, head_dim, cos_tab, sin_tab,
                            table_len, positions, k_cache, v_cache, max_len, scale, workspace, workspace_bytes, false,
                            out);
}

extern "C" int fh_decode_attention_noalloc(fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads,
                                           int64_t n_kv, int64_t head_dim, const uint16_t *cos_tab,
                                           const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
                                           uint16_t *k_cache, uint16_t *v_cache, int64_t max_len, float scale,
                                           uint16_t *out) {
    return decode_attention("fh_decode_attention_noalloc", dev, qkv, batch, n_heads, n_kv, head_dim, cos_tab,
                            sin_tab, table_len, positions, k_cache, v_cache, max_len, scale, nullptr, 0, true, out);
}
