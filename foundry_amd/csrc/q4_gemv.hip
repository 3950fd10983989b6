// Shape selection and dispatch of the q4 decode GEMV (kernel in q4_gemv.hpp;
// one translation unit per row count, q4_gemv_m<M>.hip, so they build in
// parallel).
#include "q4_gemv_mfma.hpp"

namespace fh {

// Largest count of x rows whose staged copy fits the LDS budget at this k
// (norm: the RMSNorm prologue also stages the k-wide norm weight).
uint32_t gemv_rows_per_launch(uint32_t k, bool norm) {
    const uint32_t per_row = gemv_lds_bytes(1, k);
    const uint32_t fixed = norm ? k * 2 : 0;
    if (per_row == 0) return 8;
    if (fixed >= kGemvLdsLimit) return 0;
    uint32_t r = (kGemvLdsLimit - fixed) / per_row;
    return r > 8 ? 8 : r;
}

struct GemvShape {
    uint32_t lanes, cpl;
};
#define FH_GEMV_SHAPE_ENTRY(LL, CC) {LL, CC},
constexpr GemvShape kGemvShapes[] = {FH_GEMV_SHAPES(FH_GEMV_SHAPE_ENTRY)};
#undef FH_GEMV_SHAPE_ENTRY

// Picks the shape for k and n. Preferred: one segment covers K exactly (no
// guards, one pass). Among those, the fewest lanes per row that still gives
// at least 16 wavefronts per CU (less reduction work per output); for small n,
// the most lanes per row (more, shorter wavefronts: a shorter compute tail).
// Otherwise 64 lanes x 8 chunks, walking K in segments.
// max_lanes: the SiLU epilogue pairs rows inside a wavefront (at most 32
// lanes per row).
static GemvShape pick_gemv_shape(uint32_t n, uint32_t k, uint32_t cus, uint32_t max_lanes) {
    const uint32_t chunks = k / 32;
    const GemvShape *best = nullptr;
    for (const GemvShape &sh : kGemvShapes) {
        if (chunks == 0 || chunks != sh.lanes * sh.cpl || sh.lanes > max_lanes) continue;
        const uint64_t waves = (static_cast<uint64_t>(n) * sh.lanes + 63) / 64;
        if (best == nullptr) {
            best = &sh;
            continue;
        }
        const uint64_t best_waves = (static_cast<uint64_t>(n) * best->lanes + 63) / 64;
        const bool enough = waves >= 16ull * cus, best_enough = best_waves >= 16ull * cus;
        if (enough && (!best_enough || sh.lanes < best->lanes)) best = &sh;
        else if (!enough && !best_enough && sh.lanes > best->lanes) best = &sh;
    }
    if (best) return *best;
    if (chunks <= 32) return {16, 2};
    return max_lanes >= 64 ? GemvShape{64, 8} : GemvShape{32, 8};
}

// Launches the GEMV for m in [1, 8] rows of x whose staged copy fits LDS;
// the caller splits larger m (see gemv_rows_per_launch).
void launch_q4_gemv(hipStream_t stream, uint32_t cus, int m, const GemvArgs &a) {
    const GemvShape sh = pick_gemv_shape(a.n, a.k, cus, a.epi == kEpiSiluMul ? 32 : 64);
    switch (m) {
        case 1: launch_gemv_m<1>(sh.lanes, sh.cpl, stream, cus, a); break;
        case 2: launch_gemv_m<2>(sh.lanes, sh.cpl, stream, cus, a); break;
        case 3: launch_gemv_m<3>(sh.lanes, sh.cpl, stream, cus, a); break;
        case 4: launch_gemv_m<4>(sh.lanes, sh.cpl, stream, cus, a); break;
        case 5: launch_gemv_m<5>(sh.lanes, sh.cpl, stream, cus, a); break;
        case 6: launch_gemv_m<6>(sh.lanes, sh.cpl, stream, cus, a); break;
        case 7: launch_gemv_m<7>(sh.lanes, sh.cpl, stream, cus, a); break;
        default: launch_gemv_m<8>(sh.lanes, sh.cpl, stream, cus, a);
    }
}

// Launches the matrix-core GEMV for m (2..8) rows whose staged x fits its
// LDS budget (the caller checks mf_eligible and splits rows).
void launch_q4_gemv_mfma(hipStream_t stream, uint32_t cus, int m, const GemvArgs &a) {
    switch (m) {
        case 2: launch_gemv_mfma_m<2>(stream, cus, a); break;
        case 3: launch_gemv_mfma_m<3>(stream, cus, a); break;
        case 4: launch_gemv_mfma_m<4>(stream, cus, a); break;
        case 5: launch_gemv_mfma_m<5>(stream, cus, a); break;
        case 6: launch_gemv_mfma_m<6>(stream, cus, a); break;
        case 7: launch_gemv_mfma_m<7>(stream, cus, a); break;
        default: launch_gemv_mfma_m<8>(stream, cus, a);
    }
}

// Launches the pack kernel for m (2..8) RMSNorm rows of a (k <= kMfPackMaxK)
// into the device's pack area; with part, the rows are the ranges' f32 sums
// [ranges][m][k] instead of a.x.
void launch_mf_pack(hipStream_t stream, int m, const GemvArgs &a, void *area, const float *part,
                    uint32_t ranges) {
#define FH_PACK_CASE(MM)                                                          \
    case MM:                                                                      \
        if (part)                                                                 \
            launch_mf_pack_m<MM, true>(stream, a, area, part, ranges);            \
        else                                                                      \
            launch_mf_pack_m<MM, false>(stream, a, area, nullptr, 0);             \
        break;
    switch (m) {
        FH_PACK_CASE(2)
        FH_PACK_CASE(3)
        FH_PACK_CASE(4)
        FH_PACK_CASE(5)
        FH_PACK_CASE(6)
        FH_PACK_CASE(7)
        default: FH_PACK_CASE(8)
    }
#undef FH_PACK_CASE
}

}  // namespace fh
