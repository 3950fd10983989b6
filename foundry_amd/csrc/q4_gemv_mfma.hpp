// q4 decode GEMV on the matrix cores, for 2..8 rows of x: the same product
// as q4_gemv_kernel (y[m, r] = sum_j x[m, j] * (s[r, j/64] * q[r, j] +
// b[r, j/64]), behind Linear::forward, src/nn/linear.rs:22-35), for the
// batched decode step (Decoder over batch rows, src/generate/mod.rs:150-204).
//
// With several rows the dot2 kernel spends 4 dot2 per row and weight word:
// at 8 rows the VALU, not HBM, sets its pace. Here v_mfma_f32_16x16x32_bf16
// does the multiply-adds:
// - Output tile: 16 weight rows (B columns). A lane holds B column l%16 and
//   K quarter q = l/16 and loads 16 bytes of its row per instruction: words
//   4q..4q+3 of a 16-word span, i.e. a pair of groups (q < 2: the even
//   group, q >= 2: the odd one). MFMA j takes word 4q + j from every quarter.
// - Groups stay apart in the sums: A row m (< 8) holds x row m on the even
//   quarters and zeros on the odd ones, A row 8 + m the reverse, so D rows
//   0..7 sum the even group and rows 8..15 the odd group (no wasted rows for
//   M <= 8). A lane's D rows then belong to its own quarter's group, so it
//   applies that group's scale and bias itself: y += s * d + (b - 128 s) * X
//   in fp32, d = sum x (128 + q) from the MFMAs, X = sum x staged in LDS.
// - The mask-and-or trick turns a word into bf16 (128 + q) pairs (nibbles e,
//   e+4) without conversions, exactly; x fragments are staged permuted to
//   match.
// - Scale and bias load 2*CH groups per instruction; weight loads run two
//   chunks (CH group pairs each) ahead of the MFMAs, across task boundaries,
//   with clamped (never guarded) addresses, so every wait counts exactly.
//   With kLaySb the scales and biases come interleaved per group pair (the
//   two scale halves, then the two bias halves: fh_q4_interleave's layout),
//   so one load brings a chunk's scales and biases together (CH <= 2). With
//   kLayTiled the words come from fh_q4_tile's copy, where the 16 rows of a
//   task's B tile hold each group pair's 64 bytes side by side: a wavefront
//   load then reads one contiguous KiB instead of 16 rows x 64 bytes.
// - Every block stages all of x in LDS. Plain x: the prologue loads it in
//   1 KB runs and permutes it into fragments. With RMSNorm (fh_q4_matmul_
//   rmsnorm, fh_q4_gate_up_silu) a separate pack kernel normalises x once
//   and writes the finished LDS image to the device's pack area, and the
//   prologue only copies it (global_load_lds_dwordx4, straight into LDS):
//   per-block normalisation of 8 rows was VALU-bound (about 8 us of every
//   launch).
// - Rows whose x does not fit LDS over the whole row (8 x 14336, the down
//   projection) run over K ranges: blockIdx.y picks the range, each block
//   stages that range of x, and the f32 partial tiles go to the device's
//   partial area for mf_combine_kernel (q4_matmul.hip) to add in order.
// - Work: blocks of 16 wavefronts, persistent; a task is one 16-column B
//   tile (16 weight rows, or 8 gate rows and their 8 up rows for the SiLU
//   epilogue) over a K slice; S wavefronts split K (S = 1..16) and add their
//   partial tiles in LDS in a fixed order, so the result is deterministic
//   and the same for every variant over one weight.
#pragma once

#include "decoder_common.hpp"
#include "q4_gemv.hpp"

namespace fh {

constexpr int kMfThreads = 1024;
constexpr int kMfWaves = kMfThreads / 64;
// LDS one block may use (gfx950 gives a workgroup up to 160 KB).
constexpr uint32_t kMfLdsLimit = 160 * 1024;

typedef __attribute__((ext_vector_type(8))) __bf16 mf_bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float mf_f32x4_t;

__device__ __forceinline__ mf_f32x4_t mf_mfma(const uint4 a, const uint4 b, const mf_f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mf_bf16x8_t, a),
                                                   __builtin_bit_cast(mf_bf16x8_t, b), c, 0, 0, 0);
}

// LDS bytes: staged x fragments, a zero slot and a dummy slot, group sums X
// [G][8], the partial tiles of the K split.
constexpr uint32_t kMfRedBytes = kMfWaves * 4 * 64 * 4;
__host__ __device__ constexpr uint32_t mf_lds_bytes(uint32_t m, uint32_t k) {
    return m * k * 2 + 32 + (k / kGroup) * 8 * 4 + kMfRedBytes;
}

// Areas for the K split's partial tiles: two when LDS has room (rounds
// alternate between them, so a round needs one block barrier instead of
// two), else one.
__host__ __device__ constexpr uint32_t mf_red_areas(uint32_t m, uint32_t k) {
    return mf_lds_bytes(m, k) + kMfRedBytes <= kMfLdsLimit ? 2u : 1u;
}

// 16-byte slots of the packed LDS image: fragments, the zero and dummy
// slots, X [G][8], rounded up to whole wavefronts (the tail lands in the
// K-split area, unused until the main loop).
__host__ __device__ constexpr uint32_t mf_image_slots(uint32_t m, uint32_t k) {
    return (m * k / 8 + 2 + (k / kGroup) * 2 + 63) / 64 * 64;
}

// Largest x row count (<= 8) whose staged copy fits the LDS budget.
inline uint32_t mf_rows_per_launch(uint32_t k) {
    uint32_t r = 8;
    while (r > 0 && mf_lds_bytes(r, k) > kMfLdsLimit) --r;
    return r;
}

// One chunk (CH group pairs) of operands as a lane holds them: 16 bytes of
// packed words per pair, and scale / bias of the chunk's groups (one dword
// per pair: even group low, odd group high).
template <int CH>
struct MfChunk {
    uint4 w[CH];
    uint32_t s[CH], b[CH];
};

// Decodes two packed words into bf16 pairs (128 + q_t, 128 + q_{t+4}); the
// shifts run on the 64-bit pair (bits crossing between the words land
// outside the mask).
__device__ __forceinline__ void mf_decode2(uint32_t w0, uint32_t w1, uint32_t magic, uint4 &b0, uint4 &b1) {
    constexpr uint32_t kM = 0x000F000Fu;
    const uint64_t ww = (static_cast<uint64_t>(w1) << 32) | w0;
    const uint64_t s1 = ww >> 4, s2 = ww >> 8, s3 = ww >> 12;
    b0 = make_uint4((w0 & kM) | magic, (static_cast<uint32_t>(s1) & kM) | magic,
                    (static_cast<uint32_t>(s2) & kM) | magic, (static_cast<uint32_t>(s3) & kM) | magic);
    b1 = make_uint4((w1 & kM) | magic, (static_cast<uint32_t>(s1 >> 32) & kM) | magic,
                    (static_cast<uint32_t>(s2 >> 32) & kM) | magic, (static_cast<uint32_t>(s3 >> 32) & kM) | magic);
}

// Sum of a staged (permuted) piece's 8 values.
__device__ __forceinline__ float mf_piece_sum(const uint4 p) {
    return ((bf16_to_f32(p.x & 0xFFFFu) + bf16_to_f32(p.y & 0xFFFFu)) +
            (bf16_to_f32(p.z & 0xFFFFu) + bf16_to_f32(p.w & 0xFFFFu))) +
           ((bf16_to_f32(p.x >> 16) + bf16_to_f32(p.y >> 16)) + (bf16_to_f32(p.z >> 16) + bf16_to_f32(p.w >> 16)));
}

// 16-byte pieces of plain x rows per thread the prologue stages in
// straight-line code (rounds of kMfThreads: 8 x 4096 values, 4 x 14336);
// beyond, it loops (and the first weight loads wait for it).
constexpr uint32_t kMfPlainRounds = 8;

// Swizzle of the fragment row for word w % 4 == j: XOR keeps the M rows of a
// fragment column on distinct slots, and spreads the 8 pieces of one group
// (j = 0..3, two word columns) over distinct LDS banks (M a power of two).
template <int M>
__host__ __device__ constexpr uint32_t mf_swz(uint32_t j) {
    return M == 8 ? 2 * j : M == 4 ? j : M == 2 ? (j >> 1) : 0u;
}

// LDS slot of column piece c (8 values) of x row m: word w = c % 16 of group
// pair p = c / 16 feeds MFMA j = w % 4 of quarter w / 4, so the slot is
// ((p * 4 + j) * 4 + w / 4) * M + (m ^ mf_swz(j)).
template <int M>
__device__ __forceinline__ uint32_t mf_slot(uint32_t m, uint32_t c) {
    const uint32_t p = c >> 4, w = c & 15, j = w & 3;
    return ((p * 4 + j) * 4 + (w >> 2)) * M + (m ^ mf_swz<M>(j));
}

// mf_slot for a row count known at run time (1..8), for writers of the
// image outside the GEMV's templates.
__device__ __forceinline__ uint32_t mf_slot_rt(uint32_t M, uint32_t m, uint32_t c) {
    const uint32_t p = c >> 4, w = c & 15, j = w & 3;
    const uint32_t swz = M == 8 ? 2 * j : M == 4 ? j : M == 2 ? (j >> 1) : 0u;
    return ((p * 4 + j) * 4 + (w >> 2)) * M + (m ^ swz);
}

// M: x rows (1..8). CH: group pairs per chunk (1, 2 or 4). ksplit:
// wavefronts per task (divides 16; k / 64 / ksplit is a multiple of 2 * CH).
// LAY: operand layouts, a set of the bits below.
// kLaySb: scale and bias are read from sbi (dword 2p of a row: the scales of
// groups 2p and 2p + 1, dword 2p + 1: their biases), not scales / biases.
// kLayTiled: the words are read from wt (fh_q4_tile: [task tile][group pair
// of the whole row][16 B-tile columns][16 words]), not wq.
constexpr int kLaySb = 1, kLayTiled = 2;

template <int M, int PRO, int EPI, int CH, int LAY>
__global__ __launch_bounds__(kMfThreads) void q4_gemv_mfma_kernel(
    const uint16_t *__restrict__ x, uint32_t x_ld, const uint32_t *__restrict__ wq,
    const uint16_t *__restrict__ scales, const uint16_t *__restrict__ biases, const uint32_t *__restrict__ sbi,
    const uint32_t *__restrict__ wt, uint32_t n, uint32_t k, void *__restrict__ y, uint32_t y_ld, int y_is_f32,
    uint32_t ksplit) {
    constexpr bool kPacked = PRO == kProRmsNorm;  // x: mf_pack_kernel's image of RMSNorm(x + res)
    constexpr bool SB = (LAY & kLaySb) != 0, TILED = (LAY & kLayTiled) != 0;
    static_assert(kMfWaves / 2 * M * 16 <= kMfThreads, "a K-split round stores one output per thread at most");
    static_assert(!SB || CH <= 2, "interleaved scale/bias: one load per chunk of at most 2 pairs");
    extern __shared__ uint4 lds[];
    const uint32_t G = k / kGroup;
    const uint32_t wpr = k / 8;  // packed words per row of the K range (x fragments)
    // K range blockIdx.y of gridDim.y: weight rows hold all of them; y takes
    // this range's f32 partial sums at [blockIdx.y][M][y_ld]. A row has
    // sb_ld scales, sb_ld biases, or sb_ld interleaved dwords.
    const uint32_t w_ld = wpr * gridDim.y, sb_ld = G * gridDim.y;
    // tiled words: group pairs per whole row, and this range's first pair
    const uint32_t wt_pairs = w_ld / 16, wt_p0 = blockIdx.y * (G / 2);
    if (gridDim.y > 1) {
        x += static_cast<uint64_t>(blockIdx.y) * k;
        wq += static_cast<uint64_t>(blockIdx.y) * wpr;
        scales += static_cast<uint64_t>(blockIdx.y) * G;
        biases += static_cast<uint64_t>(blockIdx.y) * G;
        sbi += static_cast<uint64_t>(blockIdx.y) * G;
        y = static_cast<float *>(y) + static_cast<uint64_t>(blockIdx.y) * M * y_ld;
    }
    // A task is one 16-column B tile: 16 weight rows, or with the SiLU
    // epilogue 8 gate rows and their 8 up rows (n / 2 rows on), so that every
    // variant over a weight has n / 16 tasks and spreads them alike.
    const uint32_t n_out = EPI == kEpiSiluMul ? n / 2 : n;
    const uint32_t tiles = n / 16;
    uint4 *xa = lds;                                         // [G/2][4 j][4 q][M] fragments
    const uint32_t zero = M * wpr;                           // a zero fragment (dead A lanes)
    const uint32_t dummy = zero + 1;                         // write-only slot for dead items
    float *xsum = reinterpret_cast<float *>(lds + dummy + 1);  // [G][8]
    float *red = xsum + G * 8;                               // [areas][16][4][64]
    const uint32_t red_areas = mf_red_areas(M, k);

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t col = lane & 15, quarter = lane >> 4, hi = quarter >> 1;
    const uint32_t slots = kMfWaves / ksplit;
    const uint32_t slot = wave / ksplit, ks = wave % ksplit;
    const uint32_t gs = G / ksplit;      // groups per task and wavefront
    const uint32_t cpt = gs / (2 * CH);  // chunks per task
    const uint32_t per_round = gridDim.x * slots;
    const uint32_t rounds = (tiles + per_round - 1) / per_round;
    const uint32_t total = rounds * cpt;  // chunks of this wavefront
    auto tile_of = [&](uint32_t r) { return (r * gridDim.x + blockIdx.x) * slots + slot; };

    // ---- weight operands ----
    auto wrow = [&](uint32_t tile) {
        return EPI == kEpiSiluMul ? (col < 8 ? 0u : n_out) + tile * 8 + (col & 7) : tile * 16 + col;
    };
    // chunk c (of this wavefront's sequence) -> operands; past the end, the
    // last chunk again (values unused)
    // Chunks past the end, and tiles past the last of a partial round, read
    // the first bytes of the operands instead (one line for the whole block,
    // at hand in L1): a reload of real operands would be waited for before
    // the last reduction. The choice is a select on uniform values, not a
    // branch, so every wait still counts exactly.
    auto load = [&](uint32_t c, MfChunk<CH> &cb) {
        const uint32_t cc = c < total ? c : total - 1;
        const uint32_t r = cc / cpt;
        const uint32_t p0 = (ks * gs) / 2 + (cc % cpt) * CH;  // first pair
        uint32_t tile = tile_of(r);
        const bool dead = c >= total || tile >= tiles;
        tile = tile < tiles ? tile : tiles - 1;
        const uint64_t row = wrow(tile);
        if constexpr (TILED) {
            // pair p of tile t: 1 KiB at ((t * pairs + p) * 16) * 16 words, column col at 16 col
            const uint4 *wp = reinterpret_cast<const uint4 *>(
                wt + ((static_cast<uint64_t>(tile) * wt_pairs + wt_p0 + p0) * 16 + col) * 16 + quarter * 4);
            if (dead) wp = reinterpret_cast<const uint4 *>(wt);
#pragma unroll
            for (int c2 = 0; c2 < CH; ++c2) cb.w[c2] = load_stream16(wp + c2 * 64);
        } else {
            const uint4 *wp = reinterpret_cast<const uint4 *>(wq + row * w_ld + p0 * 16 + quarter * 4);
            if (dead) wp = reinterpret_cast<const uint4 *>(wq);
#pragma unroll
            for (int c2 = 0; c2 < CH; ++c2) cb.w[c2] = load_stream16(wp + c2 * 4);
        }
        const uint16_t *sp = scales + row * sb_ld + p0 * 2, *bp = biases + row * sb_ld + p0 * 2;
        if (dead) sp = scales, bp = biases;
        const uint32_t *ip = dead ? sbi : sbi + row * sb_ld + p0 * 2;
        if constexpr (SB && CH == 2) {
            const uint4 v = *reinterpret_cast<const uint4 *>(ip);
            cb.s[0] = v.x, cb.b[0] = v.y, cb.s[1] = v.z, cb.b[1] = v.w;
        } else if constexpr (SB) {
            const uint2 v = *reinterpret_cast<const uint2 *>(ip);
            cb.s[0] = v.x, cb.b[0] = v.y;
        } else if constexpr (CH == 4) {
            const uint4 sv = *reinterpret_cast<const uint4 *>(sp), bv = *reinterpret_cast<const uint4 *>(bp);
            cb.s[0] = sv.x, cb.s[1] = sv.y, cb.s[2] = sv.z, cb.s[3] = sv.w;
            cb.b[0] = bv.x, cb.b[1] = bv.y, cb.b[2] = bv.z, cb.b[3] = bv.w;
        } else if constexpr (CH == 2) {
            const uint2 sv = *reinterpret_cast<const uint2 *>(sp), bv = *reinterpret_cast<const uint2 *>(bp);
            cb.s[0] = sv.x, cb.s[1] = sv.y;
            cb.b[0] = bv.x, cb.b[1] = bv.y;
        } else {
            cb.s[0] = *reinterpret_cast<const uint32_t *>(sp);
            cb.b[0] = *reinterpret_cast<const uint32_t *>(bp);
        }
    };
    MfChunk<CH> buf[2];
    // two chunks in flight, issued in buffer order (pinned) so the first
    // waits count the later loads instead of draining them
    auto prefetch = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        load(0, buf[0]);
        __builtin_amdgcn_sched_barrier(0);
        load(1, buf[1]);
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- prologue: stage x as fragments, and X ----
    if constexpr (kPacked) {
        // x is the LDS image mf_pack_kernel wrote (fragments, zero slot,
        // dummy slot, X, padded to whole wavefronts): loaded straight into
        // LDS, 1 KB per wavefront instruction, before the weights; the
        // barrier below waits for it
        const uint32_t total = mf_image_slots(M, k);
        for (uint32_t i0 = wave * 64; i0 < total; i0 += kMfThreads)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4 *>(x) + i0 + lane,
                                             (__attribute__((address_space(3))) void *)(lds + i0),
                                             16, 0, 0);
        prefetch();
    } else {
        // Piece Q (16 bytes, 8 values) is column piece Q % ppr of row Q / ppr.
        // Round i of thread t takes piece i * kMfThreads + t, so each load
        // instruction of a wavefront reads 1 KB of consecutive pieces, and a
        // group's 8 pieces sit in 8 neighbouring lanes (group sums by DPP).
        const uint32_t ppr = k / 8;  // pieces per row
        const uint32_t pieces = M * ppr;
        auto piece_load = [&](uint32_t q) {
            const uint32_t qc = q < pieces ? q : 0u;
            return *reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(qc / ppr) * x_ld + (qc % ppr) * 8);
        };
        // stores a piece (unpermuted values) as a fragment and its group's X
        auto piece_stage = [&](uint32_t q, const uint4 v) {
            const bool live = q < pieces;
            const uint32_t qc = live ? q : 0u;
            const uint32_t m = qc / ppr, c = qc % ppr;
            const uint4 p = gemv_permute(v);
            if (live) xa[mf_slot<M>(m, c)] = p;
            const float gsum = group_sum<8>(mf_piece_sum(p));
            if (live && (c & 7) == 0) xsum[(c >> 3) * 8 + m] = gsum;
        };
        constexpr uint32_t kRounds = kMfPlainRounds;
        if (pieces <= kRounds * kMfThreads) {
            uint4 v[kRounds];
#pragma unroll
            for (uint32_t rr = 0; rr < kRounds; ++rr) v[rr] = piece_load(threadIdx.x + rr * kMfThreads);
            prefetch();
#pragma unroll
            for (uint32_t rr = 0; rr < kRounds; ++rr) piece_stage(threadIdx.x + rr * kMfThreads, v[rr]);
        } else {
            for (uint32_t q0 = 0; q0 < pieces; q0 += kMfThreads)
                piece_stage(q0 + threadIdx.x, piece_load(q0 + threadIdx.x));
            prefetch();
        }
        // the zero fragment; X = 0 for rows M..7 (the pack image holds them)
        for (uint32_t t = threadIdx.x; t < (8 - M) * G; t += kMfThreads) xsum[(t % G) * 8 + M + t / G] = 0.f;
    }
    if (!kPacked && threadIdx.x == 0) xa[zero] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();

    // ---- main loop ----
    uint32_t magic = 0x43004300u;  // in a VGPR: v_and_or_b32 takes no literal on gfx9
    asm volatile("" : "+v"(magic));
    // A row of this lane: x row col % 8 on its own half's quarters, else the
    // zero fragment (stride 0: every fragment of a dead lane reads it)
    const uint32_t am = col & 7;
    const bool alive = (col >> 3) == hi && am < static_cast<uint32_t>(M);
    const uint4 *abase[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) abase[j] = alive ? xa + j * 4 * M + quarter * M + (am ^ mf_swz<M>(j)) : xa + zero;
    const uint32_t astride = alive ? 16 * M : 0;  // per pair

    mf_f32x4_t acc = mf_f32x4_t{0.f, 0.f, 0.f, 0.f};

    // the task of round r is complete: even + odd halves, the K slices,
    // epilogue, store. Output column c of a task: 16 of them, or with SiLU 8
    // (gate in B column c, up in column c + 8).
    constexpr uint32_t kOuts = EPI == kEpiSiluMul ? 8 : 16;
    auto finish = [&](uint32_t r) {
        auto store = [&](uint32_t m, uint32_t c, uint32_t tile, float v) {
            const uint32_t o = m * y_ld + tile * kOuts + c;  // < 2^31 (mf_eligible)
            if (y_is_f32)
                static_cast<float *>(y)[o] = v;
            else
                static_cast<uint16_t *>(y)[o] = static_cast<uint16_t>(f32_to_bf16_rne(v));
        };
        auto epilogue = [](float gsum, float usum) {
            if constexpr (EPI == kEpiSiluMul) {
                const float g = bf16_to_f32(f32_to_bf16_rne(gsum));
                const float u = bf16_to_f32(f32_to_bf16_rne(usum));
                return bf16_to_f32(f32_to_bf16_rne(g / (expf(-g) + 1.0f))) * u;
            } else {
                return gsum;
            }
        };
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = acc[i] + __shfl_xor(acc[i], 32, 64);  // lanes < 32: totals
        if (ksplit == 1) {
            const uint32_t tile = tile_of(r);
            float u[4];  // the up sums of the lane's gate column (SiLU)
#pragma unroll
            for (int i = 0; i < 4; ++i) u[i] = EPI == kEpiSiluMul ? __shfl_xor(v[i], 8, 64) : v[i];
            if (tile < tiles && quarter < 2 && col < kOuts) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m = quarter * 4 + i;
                    if (m < static_cast<uint32_t>(M)) store(m, col, tile, epilogue(v[i], u[i]));
                }
            }
        } else {
            // round r's area; with two, round r + 2 writes this one only after
            // every thread has passed round r + 1's barrier, i.e. after its reads
            float *rd = red + (red_areas == 2 ? (r & 1u) * (kMfRedBytes / 4) : 0u);
#pragma unroll
            for (int i = 0; i < 4; ++i) rd[(wave * 4 + i) * 64 + lane] = v[i];
            __syncthreads();
            // slots * M * 16 <= kMfThreads: one output per thread at most, and
            // no store loop (a store loop inside the main loop would make every
            // weight wait drain the whole pipeline)
            const uint32_t e = threadIdx.x;
            if (e < slots * M * 16) {
                const uint32_t sl = e / (M * 16), m = (e / 16) % M, c = e % 16;
                const uint32_t tile = (r * gridDim.x + blockIdx.x) * slots + sl;
                const uint32_t i = m & 3, ln = (m >> 2) * 16 + c;
                float sum = 0.f, usum = 0.f;
                for (uint32_t s = 0; s < ksplit; ++s) sum += rd[((sl * ksplit + s) * 4 + i) * 64 + ln];
                if constexpr (EPI == kEpiSiluMul)
                    for (uint32_t s = 0; s < ksplit; ++s) usum += rd[((sl * ksplit + s) * 4 + i) * 64 + ln + 8];
                if (tile < tiles && c < kOuts) store(m, c, tile, epilogue(sum, usum));
            }
            if (red_areas == 1) __syncthreads();
        }
    };

    uint32_t cr = 0, cc = 0;  // compute position: round, chunk in task
    // Chunks past `total` (to an even count) compute on reloaded operands and
    // are dropped: loads and MFMAs stay unconditional. total >= 1 for every
    // launch, so the loop runs its body before the first test (a loop that
    // might not run would let the prefetch sink below the prologue barrier).
    uint32_t c0 = 0;
    do {
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const uint32_t p0 = (ks * gs) / 2 + cc * CH;
#pragma unroll
            for (int c2 = 0; c2 < CH; ++c2) {
                const uint32_t p = p0 + c2;
                const float4 xv = *reinterpret_cast<const float4 *>(xsum + (2 * p + hi) * 8 + 4 * (quarter & 1));
                uint4 a[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) a[j] = abase[j][p * astride];
                const uint4 wv = buf[d].w[c2];
                uint4 b0, b1, b2, b3;
                mf_decode2(wv.x, wv.y, magic, b0, b1);
                mf_decode2(wv.z, wv.w, magic, b2, b3);
                mf_f32x4_t dv = mf_mfma(a[0], b0, mf_f32x4_t{0.f, 0.f, 0.f, 0.f});
                dv = mf_mfma(a[1], b1, dv);
                dv = mf_mfma(a[2], b2, dv);
                dv = mf_mfma(a[3], b3, dv);
                const uint32_t sb = hi ? buf[d].s[c2] >> 16 : buf[d].s[c2] & 0xFFFFu;
                const uint32_t bb = hi ? buf[d].b[c2] >> 16 : buf[d].b[c2] & 0xFFFFu;
                const float s = bf16_to_f32(sb);
                const float bc = fmaf(-128.f, s, bf16_to_f32(bb));
                acc[0] = fmaf(bc, xv.x, fmaf(s, dv[0], acc[0]));
                acc[1] = fmaf(bc, xv.y, fmaf(s, dv[1], acc[1]));
                acc[2] = fmaf(bc, xv.z, fmaf(s, dv[2], acc[2]));
                acc[3] = fmaf(bc, xv.w, fmaf(s, dv[3], acc[3]));
            }
            load(c0 + d + 2, buf[d]);
            if (cc == cpt - 1 && cr < rounds) {  // uniform across the block
                finish(cr);
                acc = mf_f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
            if (++cc == cpt) {
                cc = 0;
                ++cr;
            }
        }
        c0 += 2;
    } while (c0 < total);
}

// ---- the pack kernel: RMSNorm(x + res) once, as the GEMV's LDS image ----

constexpr uint32_t kMfPackMaxK = 16384;
constexpr int kMfPackThreads = 512;
constexpr int kMfPackPieces = kMfPackMaxK / 8 / kMfPackThreads;  // 16-byte pieces per thread
static_assert(mf_image_slots(8, kMfPackMaxK) * 16ull <= kPackAreaBytes, "the pack area holds the image of 8 rows");

// K ranges a split GEMV may use (the combine's loads are issued for all).
constexpr uint32_t kMfMaxRanges = 8;

// Block m (one per x row, k <= kMfPackMaxK): h = x (+ res) (to res_out when
// given), the row's scale = 1 / sqrt(mean(h^2) + eps) and x' = RNE(RNE(h *
// scale) * w), RmsNorm's rounding points (src/nn/norm.rs:32-50); x' goes to
// img as the GEMV's LDS image: fragments (mf_slot), the zero slot, a dummy
// slot, then X [G][8] = group sums of x' (block 0 writes the zero slot and the
// zeros of rows M..7). Sums run in a fixed order. P: 16-byte pieces per
// thread (k <= 8 * 512 * P).
// PARTS: x is not given; its row is formed here from the f32 partial sums of
// a GEMV split over `ranges` K ranges ([ranges][M][k]), added in range order
// and rounded to bf16 exactly as mf_combine_kernel would write it, so the
// combine's launch and its round trip through memory are saved.
template <int M, int P, bool PARTS>
__global__ __launch_bounds__(kMfPackThreads) void mf_pack_kernel(const uint16_t *__restrict__ x,
                                                                const float *__restrict__ part, uint32_t ranges,
                                                                GemvFusion fu, uint32_t k, uint4 *__restrict__ img) {
    __shared__ float red[kMfPackThreads / 64];
    const uint32_t m = blockIdx.x, ppr = k / 8, G = k / kGroup, t = threadIdx.x;
    const uint32_t lane = t & 63, wave = t >> 6;
    const bool has_res = fu.res != nullptr;
    const uint16_t *rr = (has_res ? fu.res : fu.w) + (has_res ? static_cast<uint64_t>(m) * k : 0u);  // used only with a residual
    uint4 h[P], r[P], w[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const uint32_t c = t + i * kMfPackThreads, cc = c < ppr ? c : 0u;
        if constexpr (PARTS) {
            float4 lo[kMfMaxRanges], hi[kMfMaxRanges];
#pragma unroll
            for (uint32_t q = 0; q < kMfMaxRanges; ++q) {
                const float *pp = part + (static_cast<uint64_t>(q < ranges ? q : 0u) * M + m) * k + cc * 8;
                lo[q] = *reinterpret_cast<const float4 *>(pp);
                hi[q] = *reinterpret_cast<const float4 *>(pp + 4);
            }
            float4 a = lo[0], b = hi[0];
#pragma unroll
            for (uint32_t q = 1; q < kMfMaxRanges; ++q)
                if (q < ranges) {
                    a = make_float4(a.x + lo[q].x, a.y + lo[q].y, a.z + lo[q].z, a.w + lo[q].w);
                    b = make_float4(b.x + hi[q].x, b.y + hi[q].y, b.z + hi[q].z, b.w + hi[q].w);
                }
            h[i] = make_uint4(f32x2_to_bf16x2_rne(a.x, a.y), f32x2_to_bf16x2_rne(a.z, a.w),
                              f32x2_to_bf16x2_rne(b.x, b.y), f32x2_to_bf16x2_rne(b.z, b.w));
        } else {
            h[i] = *reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(m) * k + cc * 8);
        }
        r[i] = *reinterpret_cast<const uint4 *>(rr + (has_res ? cc * 8 : 0u));
        w[i] = *reinterpret_cast<const uint4 *>(fu.w + cc * 8);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const uint32_t c = t + i * kMfPackThreads;
        const bool live = c < ppr;
        if (has_res) {
            h[i] = gemv_pairwise(h[i], r[i], [](float a, float b) { return a + b; });
            if (fu.res_out && live) *reinterpret_cast<uint4 *>(fu.res_out + static_cast<uint64_t>(m) * k + c * 8) = h[i];
        }
        const uint32_t w4[4] = {h[i].x, h[i].y, h[i].z, h[i].w};
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float lo = bf16_to_f32(w4[e] & 0xFFFFu), up = bf16_to_f32(w4[e] >> 16);
            sq += lo * lo;
            sq += up * up;
        }
        ss += live ? sq : 0.f;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kMfPackThreads / 64; ++i) tot += red[i];
    const float scale = 1.0f / sqrtf(tot * fu.dim_inv + fu.eps);
    float *xs = reinterpret_cast<float *>(img + static_cast<uint64_t>(M) * ppr + 2);
    if (m == 0 && t == 0) img[static_cast<uint64_t>(M) * ppr] = make_uint4(0u, 0u, 0u, 0u);  // the zero slot
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const uint32_t c = t + i * kMfPackThreads;
        const bool live = c < ppr;
        const uint4 p = gemv_permute(gemv_pairwise(h[i], w[i], [scale](float hh, float gg) {
            return bf16_to_f32(f32_to_bf16_rne(hh * scale)) * gg;
        }));
        if (live) img[mf_slot<M>(m, c)] = p;
        const float gsum = group_sum<8>(mf_piece_sum(p));
        if (live && (c & 7) == 0) xs[(c >> 3) * 8 + m] = gsum;
    }
    if (m == 0)
        for (uint32_t j = t; j < (8 - M) * G; j += kMfPackThreads) xs[(j % G) * 8 + M + j / G] = 0.f;
}

// Pieces per thread for rows of k values.
constexpr int mf_pack_pieces(uint32_t k) { return k <= 8u * kMfPackThreads ? 1 : k <= 16u * kMfPackThreads ? 2 : 4; }

template <int M, bool PARTS>
inline void launch_mf_pack_m(hipStream_t stream, const GemvArgs &a, void *area, const float *part,
                             uint32_t ranges) {
    switch (mf_pack_pieces(a.k)) {
        case 1:
            hipLaunchKernelGGL((mf_pack_kernel<M, 1, PARTS>), dim3(M), dim3(kMfPackThreads), 0, stream, a.x, part,
                               ranges, a.fu, a.k, static_cast<uint4 *>(area));
            break;
        case 2:
            hipLaunchKernelGGL((mf_pack_kernel<M, 2, PARTS>), dim3(M), dim3(kMfPackThreads), 0, stream, a.x, part,
                               ranges, a.fu, a.k, static_cast<uint4 *>(area));
            break;
        default:
            hipLaunchKernelGGL((mf_pack_kernel<M, 4, PARTS>), dim3(M), dim3(kMfPackThreads), 0, stream, a.x, part,
                               ranges, a.fu, a.k, static_cast<uint4 *>(area));
    }
}

// Picks the K split (wavefronts per task) from the weight's 16-row tiles, its
// groups and the CU count only (one block per CU), so that every variant over
// the same weight (SiLU pairs included) adds the same partial sums in the
// same order: the fewest rounds of tiles times groups per wavefront (the
// critical path), then the fewest rounds, then the smallest split (less
// reduction). A split leaves each wavefront a multiple of 2 groups; 0 if none
// does.
inline uint32_t pick_mf_split(uint32_t weight_tiles, uint32_t groups, uint32_t cus) {
    uint32_t best_s = 0;
    uint64_t best_cost = ~0ull, best_rounds = ~0ull;
    for (uint32_t s = 1; s <= static_cast<uint32_t>(kMfWaves); s *= 2) {
        if (groups % (s * 2) != 0) continue;
        const uint32_t slots = kMfWaves / s;
        const uint32_t need = (weight_tiles + slots - 1) / slots;
        const uint64_t blocks = need < cus ? need : cus;
        const uint64_t rounds = (weight_tiles + blocks * slots - 1) / (blocks * slots);
        const uint64_t cost = rounds * (groups / s);
        if (cost < best_cost || (cost == best_cost && rounds < best_rounds)) {
            best_s = s;
            best_cost = cost;
            best_rounds = rounds;
        }
    }
    return best_s;
}

template <int M, int PRO, int EPI, int CH, int LAY>
inline void launch_gemv_mfma_t(hipStream_t stream, uint32_t cus, const GemvArgs &a, uint32_t ksplit) {
    auto kernel = q4_gemv_mfma_kernel<M, PRO, EPI, CH, LAY>;
    const uint32_t lds = mf_lds_bytes(M, a.k) + (mf_red_areas(M, a.k) - 1) * kMfRedBytes;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kMfThreads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const uint32_t slots = kMfWaves / ksplit;
    const uint32_t need = (a.n / 16 + slots - 1) / slots;
    const uint32_t ranges = a.kranges > 1 ? a.kranges : 1;
    const uint32_t cap = (cus / ranges > 0 ? cus / ranges : 1) * static_cast<uint32_t>(per_cu);
    hipLaunchKernelGGL(kernel, dim3(need < cap ? need : cap, a.kranges > 1 ? a.kranges : 1), dim3(kMfThreads), lds,
                       stream, a.x, a.x_ld, a.wq, a.s, a.b, a.sb, a.wt, a.n, a.k, a.y, a.y_ld, a.y_is_f32, ksplit);
}

// Launches chunk width C with operand layouts `lay` (LAYS: the layouts other
// than the plain one are built for this prologue / epilogue pair). Four-pair
// chunks only run without the interleaved table (the dispatcher takes two
// pairs when it is given), so they read the plain layout.
template <int M, int P, int E, int C, bool LAYS>
inline void launch_gemv_mfma_lay(hipStream_t stream, uint32_t cus, const GemvArgs &a, uint32_t ksplit, int lay) {
    if constexpr (LAYS && C <= 2) {
        if (lay == (kLaySb | kLayTiled)) return launch_gemv_mfma_t<M, P, E, C, kLaySb | kLayTiled>(stream, cus, a, ksplit);
        if (lay == kLaySb) return launch_gemv_mfma_t<M, P, E, C, kLaySb>(stream, cus, a, ksplit);
    }
    launch_gemv_mfma_t<M, P, E, C, 0>(stream, cus, a, ksplit);
}

template <int M, int P, int E, bool LAYS>
inline void launch_gemv_mfma_ch(hipStream_t stream, uint32_t cus, const GemvArgs &a, uint32_t ksplit, int ch,
                                int lay) {
    if (ch == 4) launch_gemv_mfma_lay<M, P, E, 4, LAYS>(stream, cus, a, ksplit, lay);
    else if (ch == 2) launch_gemv_mfma_lay<M, P, E, 2, LAYS>(stream, cus, a, ksplit, lay);
    else launch_gemv_mfma_lay<M, P, E, 1, LAYS>(stream, cus, a, ksplit, lay);
}

// Whether the matrix-core GEMV takes this launch of 2..8 rows: k a multiple of
// 256 with a K split for it, n a multiple of 16 (whole B tiles; with SiLU
// [gate; up] rows, so 8 outputs per tile), 16-byte aligned operands,
// at least 2 x rows staged per launch (the caller splits larger m), and with
// RMSNorm rows the pack area can hold.
inline bool mf_eligible(uint32_t m, const GemvArgs &a) {
    if (m < 2 || m > 8 || a.k == 0 || a.k % (kGroup * 4) != 0 || a.n == 0 || a.n % 16 != 0 || a.x_ld % 8 != 0)
        return false;
    if ((reinterpret_cast<uintptr_t>(a.wq) | reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b) |
         reinterpret_cast<uintptr_t>(a.sb) | reinterpret_cast<uintptr_t>(a.wt)) & 15u)
        return false;
    if (a.pro == kProRmsNorm && a.k > kMfPackMaxK) return false;  // the pack area's row limit
    if (static_cast<uint64_t>(m) * a.y_ld >= (1ull << 31)) return false;  // 32-bit output offsets
    return mf_rows_per_launch(a.k) >= 2;
}

// Defined in q4_gemv_m<M>.hip.
template <int M>
void launch_gemv_mfma_m(hipStream_t stream, uint32_t cus, const GemvArgs &a);

// Chunk width: 4 group pairs when each wavefront's slice allows it (one
// 16-byte scale and one bias load per 8 groups), else 2, else 1, at most
// half the slice. With interleaved scales and biases (a.sb) the widest is 2
// pairs, read with one load per chunk: at 4 pairs the separate arrays take
// two loads, and two loads from the interleaved table measured slower (config-5
// decode 2,611 -> 2,596 tok/s), while 2 pairs from the table instead of 4
// from the arrays took the down projection 12.9 -> 11.5-12.0 us and the LM
// head 65.3 -> 63.7 us (same outputs). Tiled words (a.wt) come with the
// table, so they are read at 2 and 1 pairs per chunk.
template <int M>
inline void launch_gemv_mfma_dispatch(hipStream_t stream, uint32_t cus, const GemvArgs &a) {
    const uint32_t groups = a.k / kGroup;
    const uint32_t ranges = a.kranges > 1 ? a.kranges : 1;
    const uint32_t ksplit = pick_mf_split(a.n / 16, groups, cus / ranges > 0 ? cus / ranges : 1);
    const uint32_t gs = groups / ksplit;
    // Chunks go in pairs, so an odd chunk count per wavefront loads and
    // computes one chunk twice: take the widest chunk whose count (rounds of
    // tiles x chunks per task, rounds as launch_gemv_mfma_t sizes the grid at
    // one block per CU) is even or at least 5, else the narrowest.
    const uint32_t ranges_ = a.kranges > 1 ? a.kranges : 1;
    const uint32_t cap = cus / ranges_ > 0 ? cus / ranges_ : 1;
    const uint32_t slots = kMfWaves / ksplit;
    const uint32_t task_tiles = a.n / 16;
    const uint32_t need = (task_tiles + slots - 1) / slots;
    const uint32_t blocks = need < cap ? need : cap;
    const uint32_t rounds = (task_tiles + blocks * slots - 1) / (blocks * slots);
    int ch = 1;
    for (const int c : {a.sb != nullptr ? 2 : 4, 2, 1}) {
        if (gs % (2 * c) != 0) continue;
        const uint32_t total = rounds * (gs / (2 * c));
        if (total % 2 == 0 || total >= 5) {
            ch = c;
            break;
        }
    }
    // operand layouts given: the tiled words only with the interleaved
    // scales and biases (fh_llama_forward's weights carry both or neither);
    // no interleaved or tiled form of the SiLU epilogue without RMSNorm (the
    // decoder does not run it)
    const int lay = a.sb == nullptr ? 0 : a.wt == nullptr ? kLaySb : kLaySb | kLayTiled;
    if (a.epi == kEpiSiluMul) {
        if (a.pro == kProRmsNorm) launch_gemv_mfma_ch<M, kProRmsNorm, kEpiSiluMul, true>(stream, cus, a, ksplit, ch, lay);
        else launch_gemv_mfma_ch<M, kProNone, kEpiSiluMul, false>(stream, cus, a, ksplit, ch, 0);
    } else if (a.pro == kProRmsNorm) {
        launch_gemv_mfma_ch<M, kProRmsNorm, kEpiNone, true>(stream, cus, a, ksplit, ch, lay);
    } else {
        launch_gemv_mfma_ch<M, kProNone, kEpiNone, true>(stream, cus, a, ksplit, ch, lay);
    }
}

}  // namespace fh
