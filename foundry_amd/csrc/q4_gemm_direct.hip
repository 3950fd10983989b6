// q4 prefill GEMM with weights fed straight to the matrix cores:
// Y[m, r] = sum_j X[m, j] * RNE_bf16(s[r, j/64] * q[r, j] + b[r, j/64]).
// Replaces matmul_tiled (src/metal/kernels/matmul.metal:29-65) behind
// Linear::forward (src/nn/linear.rs:22-35) for prompt-length row counts whose
// 256 x 256 output tiles fill the chip.
//
// Design for CDNA4 (one 512-thread block per CU, 256 x 256 output tile, K
// step 64 = one quantisation group):
// - Eight wavefronts, two per SIMD, and both issue MFMAs all the time: on
//   gfx950 one wavefront issues a v_mfma_f32_32x32x16_bf16 at most every 32
//   clocks, and a second wavefront on the same SIMD doubles the rate
//   (measured: 2.2 PFLOP/s with one wavefront per SIMD, 4.4 with two).
//   Wavefront w owns X rows [128 (w / 4), +128) and output columns
//   [64 (w % 4), +64): a 128 x 64 tile, 4 x 2 accumulators (128 registers).
// - Weights skip LDS. Lane (col, h) of a 32-column B tile loads the 16 bytes
//   of its weight row that hold k = 32 h .. 32 h + 31 of the group (one
//   buffer_load_dwordx4) and dequantises them in registers; MFMA sub-step j
//   takes k = 32 h + 8 j .. + 7, and the X fragments are read in the same k
//   order, so every product is the plain GEMM's.
// - The dequantisation of the next sub-step (46 VALU instructions), the
//   next X fragments' LDS reads and the loads of later steps are interleaved
//   with each sub-step's eight MFMAs (sched_group_barrier), so they issue in
//   the MFMAs' shadow instead of in a phase of their own.
// - X goes through LDS in four stages per wavefront group of 128 rows,
//   brought by LDS DMA (buffer_load ... lds: no registers, no ds_write):
//   step s + 3's X is requested while step s computes and step s + 1's first
//   fragments are read at the end of step s, so one barrier per step
//   suffices. Rows are 128 bytes with their 16-byte pieces XOR-swizzled by
//   the row index, so 16-byte fragment reads are conflict-free without
//   padding (the DMA writes 64 consecutive 16-byte slots).
// - Dequantisation: exact nibble -> float (v_cvt_f32_ubyte of masked
//   bytes), fma(s, q, b), RNE to bf16: the fh_q4_dequant value whenever s*q
//   is finite.
// - The bf16 epilogue goes through LDS so that each lane stores 16
//   contiguous bytes of an output row (1 KiB per wavefront instruction)
//   instead of 2-byte values 8 KiB apart.
// - Tiles are dealt to XCDs in rectangles (blocks go round-robin over the 8
//   XCDs): the 32 blocks of one XCD share their X rows and weight rows in
//   that XCD's L2.
#include <type_traits>

#include "decoder_common.hpp"
#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

namespace {

constexpr int kDThreads = 512;
constexpr int kDBM = 256, kDBN = 256, kDBK = 64;
constexpr int kDPitch = kDBK;                     // bf16 per X row in LDS (swizzled pieces)
constexpr int kDRows = kDBM / 2;                  // X rows per wavefront group
constexpr int kDStage = kDRows * kDPitch;         // bf16 per group stage
constexpr int kDStages = 4;
constexpr uint32_t kDXLds = 2u * kDStages * kDStage * 2u;  // bytes, both groups
// Scales and biases go through LDS in chunks of 8 groups (8 K steps), two
// chunk buffers: [buffer][group][column][scale, bias], 4 bytes per (group,
// column), so the 32 columns a wavefront reads per step are consecutive
// dwords (no bank conflicts).
// (Loaded per step and per lane they cost 4 loads that each touch 32 cache
// lines for 256 useful bytes, and took 40% of the kernel.)
constexpr int kDSbGroups = 8;
constexpr uint32_t kDSbBuf = kDBN * kDSbGroups * 4;             // bytes per chunk buffer
constexpr uint32_t kDSbLds = 2 * kDSbBuf;
constexpr uint32_t kDLoopLds = kDXLds + kDSbLds;
// bf16 epilogue: each wavefront's 128 x 64 tile, row pitch 72
constexpr int kDOutPitch = 64 + 8;
constexpr uint32_t kDOutLds = 8u * 128u * kDOutPitch * 2u;
constexpr uint32_t kDLds = kDLoopLds > kDOutLds ? kDLoopLds : kDOutLds;
constexpr uint32_t kXcds = 8;
// Weight register sets: W(st) is requested kDWSets steps before its step
// (at the end of step st - kDWSets), into the set W(st - kDWSets) used. Four
// sets (three steps of lead, 244 VGPRs) measured no faster than two.
#ifndef FH_DIRECT_WSETS
#define FH_DIRECT_WSETS 2
#endif
constexpr int kDWSets = FH_DIRECT_WSETS;
static_assert(kDWSets == 2 || kDWSets == 4, "the 8-step chunk loop cycles through the sets");

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

// w & 0x0F0F0F0F as one v_and_b32 the compiler cannot fold into the byte
// conversions that follow (it would extract every nibble with its own
// v_bfe_u32, one more instruction per weight).
__device__ __forceinline__ uint32_t low_nibbles(uint32_t w) {
    uint32_t r;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(w));
    return r;
}

template <int I>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
    return static_cast<float>((v >> (8 * I)) & 0xFFu);
}

// 8 weights of one packed word (nibble e = weight e) -> bf16x8 in order.
__device__ __forceinline__ bf16x8_t dequant8(uint32_t w, float s, float b) {
    const uint32_t lo = low_nibbles(w);       // nibbles 0, 2, 4, 6 in bytes 0..3
    const uint32_t hi = low_nibbles(w >> 4);  // nibbles 1, 3, 5, 7
    uint4 o;
    o.x = f32x2_to_bf16x2_rne(fmaf(s, ubyte_f32<0>(lo), b), fmaf(s, ubyte_f32<0>(hi), b));
    o.y = f32x2_to_bf16x2_rne(fmaf(s, ubyte_f32<1>(lo), b), fmaf(s, ubyte_f32<1>(hi), b));
    o.z = f32x2_to_bf16x2_rne(fmaf(s, ubyte_f32<2>(lo), b), fmaf(s, ubyte_f32<2>(hi), b));
    o.w = f32x2_to_bf16x2_rne(fmaf(s, ubyte_f32<3>(lo), b), fmaf(s, ubyte_f32<3>(hi), b));
    return __builtin_bit_cast(bf16x8_t, o);
}

// One lane's packed weights of one step: for each of its two B tiles, the 4
// words of the group half it feeds.
struct WSet {
    uint4 w[2];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint64_t bytes) {
    // raw buffer (stride 0) over `bytes`; 0x00020000 is the gfx9 32-bit data
    // format word
    const uint32_t records = bytes < 0xFFFFFFFFull ? static_cast<uint32_t>(bytes) : 0xFFFFFFFFu;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), static_cast<short>(0), static_cast<int>(records),
                                             0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff),
                                                                           static_cast<int>(soff), 0));
}

// sched_group_barrier masks
constexpr int kSgMfma = 0x008, kSgValu = 0x002, kSgVmemRead = 0x020, kSgDsRead = 0x100;

}  // namespace

// Block L of the 1-D grid -> tile (tm, tn): L's XCD (L mod 8) takes a run of
// consecutive tiles in a grouped order (gm tile rows at a time, then every
// tile column), so each XCD works on a compact rectangle. A bijection for
// any tile count.
__device__ __forceinline__ void direct_tile(uint32_t L, uint32_t tiles_m, uint32_t tiles_n, uint32_t gm,
                                            uint32_t *tm, uint32_t *tn) {
    const uint32_t total = tiles_m * tiles_n;
    const uint32_t xcd = L % kXcds, slot = L / kXcds;
    const uint32_t base = total / kXcds, rem = total % kXcds;
    const uint32_t v = xcd * base + (xcd < rem ? xcd : rem) + slot;
    const uint32_t group = gm * tiles_n;
    const uint32_t g = v / group, r = v % group;
    const uint32_t rows_left = tiles_m - g * gm;
    const uint32_t gm_eff = rows_left < gm ? rows_left : gm;
    *tm = g * gm + r % gm_eff;
    *tn = r / gm_eff;
}

// y_mode: 0 bf16 through the LDS epilogue (n % 8 == 0, y 16-byte aligned),
// 1 bf16 stored per value, 2 f32 stored per value, 3 the MLP activation:
// the weight rows are [gate (f) | up (f)] (n = 2 f, f % 128 == 0), tile
// column tn covers gate rows [128 tn, +128) and the matching up rows, and y
// is act [m][f] = silu_mul1(RNE(gate), RNE(up)) (y 16-byte aligned). With
// gridDim.y = S > 1 the block takes K range blockIdx.y (k_len of the k
// columns, k = S k_len) and writes its f32 partial tile to y[blockIdx.y][m][n]
// (y_mode 2).
__global__ __launch_bounds__(kDThreads) void q4_gemm_direct_kernel(
    const uint16_t *__restrict__ x, uint32_t x_ld, const uint32_t *__restrict__ wq,
    const uint16_t *__restrict__ scales, const uint16_t *__restrict__ biases, uint32_t m, uint32_t n, uint32_t k,
    void *__restrict__ y, int y_mode, uint32_t tiles_m, uint32_t tiles_n, uint32_t gm, uint32_t k_len) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t grp = wave >> 2, wc = wave & 3;
    uint32_t tm, tn;
    direct_tile(blockIdx.x, tiles_m, tiles_n, gm, &tm, &tn);
    const uint32_t m0 = tm * kDBM, n0 = tn * kDBN;
    // weight row of the tile's column lc (mode 3: gate rows, then their up rows)
    const uint32_t f = n / 2;
    auto weight_row = [&](uint32_t lc) {
        return y_mode == 3 ? (lc < kDBN / 2 ? tn * (kDBN / 2) + lc : f + tn * (kDBN / 2) + lc - kDBN / 2) : n0 + lc;
    };
    const uint32_t kw = k / 8, kg = k / kGroup;  // row strides (words, groups)
    const uint32_t steps = k_len / kDBK;
    {
        const uint32_t k0 = blockIdx.y * k_len;
        x += k0;
        wq += k0 / 8;
        scales += k0 / kGroup;
        biases += k0 / kGroup;
        y = static_cast<float *>(y) + static_cast<uint64_t>(blockIdx.y) * m * n;  // y_mode 2 when blockIdx.y > 0
    }
    const uint32_t h = lane >> 5;

    uint16_t *const xs_base = smem + grp * kDStages * kDStage;  // this group's stages

    // X staging by LDS DMA: wavefront (g, c) brings rows [32 c, 32 c + 32)
    // of its group's 128-row step tile, as 4 chunks of 8 rows (1 KiB each,
    // lane i -> row 8 q + i / 8, slot i % 8). Slot s of row r holds piece
    // s ^ ((r / 2) % 8): a 128-byte row covers half the 64 banks, so the 16
    // rows of one 16-lane fragment read (one piece each) start at 16
    // distinct 4-bank offsets, (r % 2) * 32 + 4 * slot, and hit all 64
    // banks once. (With s ^ (r % 8), rows r and r + 8 of a read collided.)
    uint32_t xoff[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t row = m0 + grp * kDRows + wc * 32 + q * 8 + (lane >> 3);
        row = row < m ? row : m - 1;
        const uint32_t piece = (lane & 7) ^ ((4 * q + (lane >> 4)) & 7);
        xoff[q] = (row * x_ld + piece * 8) * 2;
    }
    // weights: B tile jj's column for this lane; rows past n read row 0
    uint32_t woff[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        uint32_t col = weight_row(wc * 64 + jj * 32 + (lane & 31));
        col = col < n ? col : 0;
        woff[jj] = (col * kw + 4 * h) * 4;
    }
    // scale/bias chunks: thread t loads the 8 scales (group 0) or biases
    // (group 1) of tile column t % 256 for one chunk: 16 bytes per 8 steps
    uint32_t sbcol = weight_row(tid & 255);
    sbcol = sbcol < n ? sbcol : 0;
    const uint32_t sbgoff = sbcol * kg * 2;
    const uint32_t chunks = k_len / kGroup / kDSbGroups;
    char *const sb_lds = reinterpret_cast<char *>(smem) + kDXLds;
    // this lane's dword of B tile jj in a chunk buffer, group 0
    uint32_t sbread[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) sbread[jj] = (wc * 64 + jj * 32 + (lane & 31)) * 4;

    // Loads are buffer loads: a per-lane 32-bit byte offset plus the step's
    // offset as a scalar (readfirstlane keeps it scalar), so no lane keeps a
    // 64-bit address of its own.
    const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(x, static_cast<uint64_t>(m) * x_ld * 2);
    const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wq, static_cast<uint64_t>(n) * k / 2);
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scales, static_cast<uint64_t>(n) * kg * 2);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(biases, static_cast<uint64_t>(n) * kg * 2);
    const uint32_t last = steps - 1;
    auto dma_x = [&](uint32_t st) {
        const uint32_t so = __builtin_amdgcn_readfirstlane((st < last ? st : last) * kDBK * 2);
        uint16_t *xs = xs_base + (st % kDStages) * kDStage + wc * 32 * kDPitch;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void *)(xs + q * 8 * kDPitch), 16,
                                                 static_cast<int>(xoff[q]), static_cast<int>(so), 0, 0);
    };
    auto load_w = [&](WSet &ws, uint32_t st) {
        st = st < last ? st : last;
        const uint32_t wso = __builtin_amdgcn_readfirstlane(st * 32);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) ws.w[jj] = buf_load16(rw, woff[jj], wso);
    };
    // chunk c's 16 bytes for this thread (chunks past the last re-read it)
    auto load_sb = [&](uint32_t c) {
        c = c < chunks ? c : chunks - 1;
        return buf_load16(grp ? rb : rs, sbgoff, __builtin_amdgcn_readfirstlane(c * kDSbGroups * 2));
    };
    // ... stored as [group][column][scale, bias] into chunk c's buffer
    auto store_sb = [&](const uint4 &v, uint32_t c) {
        uint16_t *dst = reinterpret_cast<uint16_t *>(sb_lds + (c & 1) * kDSbBuf + (tid & 255) * 4) + grp;
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int g = 0; g < kDSbGroups; ++g) dst[g * kDBN * 2] = static_cast<uint16_t>(d[g / 2] >> (16 * (g % 2)));
    };
    // step st's (scale | bias << 16) for this lane's two B tiles
    auto read_sb = [&](uint32_t st, uint32_t (&sb)[2]) {
        const char *base = sb_lds + ((st / kDSbGroups) & 1) * kDSbBuf + (st % kDSbGroups) * kDBN * 4;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) sb[jj] = *reinterpret_cast<const uint32_t *>(base + sbread[jj]);
    };
    // sub-step j's B fragments of both tiles from a step's weights
    auto dequant = [&](const WSet &ws, const uint32_t (&sb)[2], int j, bf16x8_t (&b)[2]) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const float s = __uint_as_float(sb[jj] << 16);
            const float bb = __uint_as_float(sb[jj] & 0xFFFF0000u);
            const uint32_t w = j == 0 ? ws.w[jj].x : j == 1 ? ws.w[jj].y : j == 2 ? ws.w[jj].z : ws.w[jj].w;
            b[jj] = dequant8(w, s, bb);
        }
    };
    // A fragment of lane l for sub-step j of tile i: row 32 i + l % 32,
    // k = 32 h + 8 j .. + 7, i.e. piece 4 h + j in slot (4 h + j) ^ (l / 2 % 8)
    const uint32_t frag = (lane & 31) * kDPitch + (((4 * h) ^ ((lane >> 1) & 7)) * 8);
    auto read_a = [&](uint32_t st, int j, bf16x8_t (&a)[4]) {
        const uint16_t *xs = xs_base + (st % kDStages) * kDStage + (frag ^ (8 * j));
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const bf16x8_t *>(xs + i * 32 * kDPitch);
    };

    f32x16_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0.f;

    // Prologue: X(0..2) staged, the weights of steps 0 .. kDWSets - 1
    // loaded; sub-step (0, 0)'s B fragments and sub-steps (0, 0), (0, 1)'s A
    // fragments ready.
    WSet ws[kDWSets];
    uint4 sbr = load_sb(0);
    dma_x(0);
    dma_x(1);
    dma_x(2);
    __builtin_amdgcn_sched_barrier(0);
    load_w(ws[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    store_sb(sbr, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 1; i < kDWSets; ++i) load_w(ws[i], i);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);  // every DMA of X(0..2) has landed
    bf16x8_t b[2][2], a[2][4];
    uint32_t sb0[2], sb1[2];
    __syncthreads();
    read_sb(0, sb0);
    dequant(ws[0], sb0, 0, b[0]);
    read_a(0, 0, a[0]);
    read_a(0, 1, a[1]);

    // Step st, sub-step j: the eight MFMAs of (st, j), interleaved with
    // - the dequantisation of the next sub-step ((st, j + 1), or (st + 1, 0)),
    // - the A reads of the sub-step after next ((st, j + 2), or (st + 1, j - 2)),
    // - at j = 0: the DMA of X(st + 3) into the stage step st - 1 read; at
    //   j = 3: the load of W(st + kDWSets) into the set that W(st) used (its
    //   last sub-step was dequantised at j = 2);
    // - at j = 1: the LDS read of step st + 1's scales and biases; in the
    //   first step of a chunk (st % 8 == 0) the load of chunk st / 8 + 1, and
    //   in its fifth step the store of that chunk into the other buffer
    //   (read from step st + 4 on; its previous contents, chunk st / 8 - 1,
    //   were last read in step st - 5).
    // One barrier per step, after sub-step 3: it publishes X(st + 2) and
    // retires every read of the stage the next step's DMA reuses.
    // q = st % 8 is a compile-time constant: the chunk loop below runs its
    // eight steps unrolled, so no load sits under a branch (a branch's join
    // would wait for every load in flight).
    auto step = [&](uint32_t st, auto qc, WSet &cur, WSet &nxt, const uint32_t (&sbc)[2], uint32_t (&sbn)[2]) {
        constexpr uint32_t q = decltype(qc)::value;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bf16x8_t (&ac)[4] = a[j % 2];
            bf16x8_t (&bc)[2] = b[j % 2];
            bf16x8_t (&bn)[2] = b[(j + 1) % 2];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 2; ++jj)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ac[i], bc[jj], acc[i][jj], 0, 0, 0);
            if (j == 0) dma_x(st + 3);
            if (j == 1) {
                read_sb(st + 1, sbn);
                if (q == 0) sbr = load_sb(st / kDSbGroups + 1);
                if (q == 4) store_sb(sbr, st / kDSbGroups + 1);
            }
            if (j < 3)
                dequant(cur, sbc, j + 1, bn);
            else
                dequant(nxt, sbn, 0, bn);
            if (j < 2)
                read_a(st, j + 2, ac);
            else
                read_a(st + 1, j - 2, ac);
            if (j == 3) load_w(cur, st + kDWSets);
            // 8 MFMAs, each followed by its share of the sub-step's other work
            if (j == 0) {
                __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
                __builtin_amdgcn_sched_group_barrier(kSgVmemRead, 4, 0);  // the X DMA
            } else if (j == 3) {
                __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
                __builtin_amdgcn_sched_group_barrier(kSgVmemRead, 6, 0);
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if ((j == 0 && q >= 2) || (j == 3 && q >= 1) || (j == 1 || j == 2))
                    __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
                __builtin_amdgcn_sched_group_barrier(kSgValu, 6, 0);
                if (q % 2 == 1) __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
            }
            // each sub-step is its own scheduling region, so that loads keep
            // their sub-step (and the X loads their place before the weight
            // loads, which the next step's wait counts rely on)
            __builtin_amdgcn_sched_barrier(0);
            if (j == 3) {
                // X(st + 2)'s DMA (issued in step st - 1) has landed: only
                // W(st - 1 + kDWSets), X(st + 3), W(st + kDWSets) and, in the
                // first step of a chunk, one scale/bias chunk were issued
                // after it (vmcnt(8), or 9); this wavefront's LDS
                // writes and reads are done (lgkmcnt(0)). The barrier is a
                // bare s_barrier: a workgroup fence would also wait for the
                // DMA of X(st + 3).
                __builtin_amdgcn_s_waitcnt(q == 0 ? 0x0079 : 0x0078);
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    for (uint32_t st = 0; st < steps; st += kDSbGroups) {
        step(st, std::integral_constant<uint32_t, 0>{}, ws[0 % kDWSets], ws[1 % kDWSets], sb0, sb1);
        step(st + 1, std::integral_constant<uint32_t, 1>{}, ws[1 % kDWSets], ws[2 % kDWSets], sb1, sb0);
        step(st + 2, std::integral_constant<uint32_t, 2>{}, ws[2 % kDWSets], ws[3 % kDWSets], sb0, sb1);
        step(st + 3, std::integral_constant<uint32_t, 3>{}, ws[3 % kDWSets], ws[4 % kDWSets], sb1, sb0);
        step(st + 4, std::integral_constant<uint32_t, 4>{}, ws[4 % kDWSets], ws[5 % kDWSets], sb0, sb1);
        step(st + 5, std::integral_constant<uint32_t, 5>{}, ws[5 % kDWSets], ws[6 % kDWSets], sb1, sb0);
        step(st + 6, std::integral_constant<uint32_t, 6>{}, ws[6 % kDWSets], ws[7 % kDWSets], sb0, sb1);
        step(st + 7, std::integral_constant<uint32_t, 7>{}, ws[7 % kDWSets], ws[8 % kDWSets], sb1, sb0);
    }

    // the DMAs of the last steps (re-reads of the last X tile) land before
    // any wavefront reuses the LDS
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __builtin_amdgcn_s_barrier();
    const uint32_t row_base = m0 + grp * kDRows + 4 * h;
    if (y_mode == 3) {
        // every wavefront's 128 x 64 tile to LDS as bf16 (pitch 72); then
        // the group's 256 threads form its 128 x 128 activations, gate
        // column c from wavefront c / 64 and up column c from wavefront
        // 2 + c / 64, 16 output bytes per piece
        uint16_t *const os = smem + wave * 128 * kDOutPitch;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t row = i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
                    os[row * kDOutPitch + jj * 32 + (lane & 31)] = static_cast<uint16_t>(f32_to_bf16_rne(acc[i][jj][r]));
                }
        __syncthreads();
        const uint16_t *const gs = smem + grp * 4 * 128 * kDOutPitch;
        uint16_t *const yb = static_cast<uint16_t *>(y);
        const uint32_t gt = tid & 255;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const uint32_t piece = p * 256 + gt, r = piece / 16, c = (piece % 16) * 8;
            const uint16_t *g = gs + (c / 64) * 128 * kDOutPitch + r * kDOutPitch + c % 64;
            const uint4 gv = *reinterpret_cast<const uint4 *>(g);
            const uint4 uv = *reinterpret_cast<const uint4 *>(g + 2 * 128 * kDOutPitch);
            const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
            uint32_t ow[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ow[e] = silu_mul1(gw[e] & 0xFFFFu, uw[e] & 0xFFFFu) |
                        (static_cast<uint32_t>(silu_mul1(gw[e] >> 16, uw[e] >> 16)) << 16);
            const uint32_t row = m0 + grp * kDRows + r;
            if (row < m)
                *reinterpret_cast<uint4 *>(yb + static_cast<uint64_t>(row) * f + tn * (kDBN / 2) + c) =
                    make_uint4(ow[0], ow[1], ow[2], ow[3]);
        }
        return;
    }
    if (y_mode == 0) {
        // bf16 via LDS: the wavefront's 128 x 64 tile, row-major (pitch 72),
        // then 16-byte row pieces: 8 lanes per 128-byte row, 8 rows per store
        uint16_t *const os = smem + wave * 128 * kDOutPitch;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t row = i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
                    os[row * kDOutPitch + jj * 32 + (lane & 31)] = static_cast<uint16_t>(f32_to_bf16_rne(acc[i][jj][r]));
                }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's own LDS writes
        __builtin_amdgcn_wave_barrier();
        const uint32_t col = n0 + wc * 64 + (lane & 7) * 8;
        uint16_t *const yb = static_cast<uint16_t *>(y);
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            const uint32_t r = p * 8 + (lane >> 3);
            const uint32_t row = m0 + grp * kDRows + r;
            const uint4 v = *reinterpret_cast<const uint4 *>(os + r * kDOutPitch + (lane & 7) * 8);
            if (row < m && col < n) *reinterpret_cast<uint4 *>(yb + static_cast<uint64_t>(row) * n + col) = v;
        }
        return;
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const uint32_t col = n0 + wc * 64 + jj * 32 + (lane & 31);
        if (col >= n) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = row_base + i * 32 + 8 * (r / 4) + (r % 4);
                if (row >= m) continue;
                const uint64_t o = static_cast<uint64_t>(row) * n + col;
                if (y_mode == 2)
                    static_cast<float *>(y)[o] = acc[i][jj][r];
                else
                    static_cast<uint16_t *>(y)[o] = static_cast<uint16_t>(f32_to_bf16_rne(acc[i][jj][r]));
            }
    }
}

// Rows of tiles per XCD rectangle: the count that minimises the X and
// weight bytes one XCD brings in (gm tile rows of X, per_xcd / gm tile
// columns of weights; a tile reads k_len columns of 256 rows of each).
static uint32_t xcd_rect_rows(uint64_t tiles, uint32_t tiles_m, uint32_t tiles_n, uint32_t k_len) {
    const uint64_t per_xcd = (tiles + kXcds - 1) / kXcds;
    const double x_tile = 256.0 * k_len * 2, w_tile = 256.0 * (k_len / 2 + 4 * (k_len / 64));
    uint32_t gm = 1;
    double best = 1e300;
    for (uint32_t g = 1; g <= tiles_m && g <= per_xcd; ++g) {
        const double cols = static_cast<double>((per_xcd + g - 1) / g);
        const double bytes = g * x_tile + (cols < tiles_n ? cols : tiles_n) * w_tile;
        if (bytes < best) best = bytes, gm = g;
    }
    return gm;
}

// The kernel's dynamic LDS above the default limit, requested once.
static void direct_lds_opt_in() {
    static bool done = false;
    if (!done) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(q4_gemm_direct_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kDLds);
        done = true;
    }
}

// Launches the direct-weight GEMM when it applies: 256 x 256 tiles that fill
// the chip (the 2048 x 8192 x 3072 gate/up shape has exactly 256), or fill
// at least 3/4 of it over two K ranges (the 2048 x 3072 x 8192 down shape:
// 96 tiles, 192 blocks), k a multiple of 512 per range (whole scale/bias
// chunks) and every per-lane byte offset within 32 bits. Returns 0 when it
// does not apply, 1 when y was written, 2 when the two ranges' f32 partials
// were left in `area` ([2][m][n], for the caller to add in order).
uint32_t launch_q4_gemm_direct(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld,
                               const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n,
                               uint32_t k, void *y, int y_is_f32, void *area) {
    const uint32_t tiles_m = (m + kDBM - 1) / kDBM, tiles_n = (n + kDBN - 1) / kDBN;
    const uint64_t tiles = static_cast<uint64_t>(tiles_m) * tiles_n;
    uint32_t splits = 1;
    if (tiles < cus) {
        if (area == nullptr || 8 * tiles < 3ull * cus || k % (2 * kDSbGroups * kDBK) != 0 ||
            2ull * m * n * 4 > kPartialAreaBytes)
            return 0;
        splits = 2;
    }
    // k % 512: whole scale/bias chunks of 8 groups (and whole pairs of steps)
    if (tiles > 0x7FFFFFFFull || k % (kDSbGroups * kDBK) != 0 || k == 0 || m == 0) return 0;
    if (static_cast<uint64_t>(m) * x_ld * 2 >= (1ull << 32) || static_cast<uint64_t>(n) * k / 2 >= (1ull << 32))
        return 0;
    direct_lds_opt_in();
    const uint32_t gm = xcd_rect_rows(tiles, tiles_m, tiles_n, k / splits);
    if (splits > 1) {
        hipLaunchKernelGGL(q4_gemm_direct_kernel, dim3(static_cast<uint32_t>(tiles), splits), dim3(kDThreads), kDLds,
                           stream, x, x_ld, wq, s, b, m, n, k, area, 2, tiles_m, tiles_n, gm, k / splits);
        return splits;
    }
    const int y_mode = y_is_f32 ? 2 : (n % 8 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) ? 0 : 1;
    hipLaunchKernelGGL(q4_gemm_direct_kernel, dim3(static_cast<uint32_t>(tiles)), dim3(kDThreads), kDLds, stream, x,
                       x_ld, wq, s, b, m, n, k, y, y_mode, tiles_m, tiles_n, gm, k);
    return 1;
}

// act [m][f] = silu_mul1 of the [gate; up] GEMM (n = 2 f weight rows) in one
// launch (y_mode 3), when its 256-row x 128-pair tiles fill the chip with no
// K split, f % 128 == 0, k % 512 == 0, act 16-byte aligned and every byte
// offset within 32 bits. Returns false when it does not apply.
bool launch_q4_gemm_direct_silu(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld,
                                const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t f,
                                uint32_t k, uint16_t *act) {
    const uint32_t n = 2 * f;
    const uint32_t tiles_m = (m + kDBM - 1) / kDBM, tiles_n = f / (kDBN / 2);
    const uint64_t tiles = static_cast<uint64_t>(tiles_m) * tiles_n;
    if (f == 0 || f % (kDBN / 2) != 0 || m == 0 || tiles < cus || tiles > 0x7FFFFFFFull || k == 0 ||
        k % (kDSbGroups * kDBK) != 0 || (reinterpret_cast<uintptr_t>(act) & 15) != 0)
        return false;
    if (static_cast<uint64_t>(m) * x_ld * 2 >= (1ull << 32) || static_cast<uint64_t>(n) * k / 2 >= (1ull << 32))
        return false;
    direct_lds_opt_in();
    const uint32_t gm = xcd_rect_rows(tiles, tiles_m, tiles_n, k);  // a tile reads 256 weight rows either way
    hipLaunchKernelGGL(q4_gemm_direct_kernel, dim3(static_cast<uint32_t>(tiles)), dim3(kDThreads), kDLds, stream, x,
                       x_ld, wq, s, b, m, n, k, act, 3, tiles_m, tiles_n, gm, k);
    return true;
}

}  // namespace fh
