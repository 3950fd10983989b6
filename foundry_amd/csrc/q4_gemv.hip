// Shape selection and dispatch of the q4 decode GEMV (kernel in q4_gemv.hpp;
// one translation unit per row count, q4_gemv_m<M>.hip, so they build in
// parallel).
#include "q4_gemv.hpp"

namespace fh {

// Largest count of x rows whose staged copy fits the LDS budget at this k.
uint32_t gemv_rows_per_launch(uint32_t k) {
    const uint32_t per_row = gemv_lds_bytes(1, k);
    if (per_row == 0) return 8;
    uint32_t r = kGemvLdsLimit / per_row;
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
static GemvShape pick_gemv_shape(uint32_t n, uint32_t k, uint32_t cus) {
    const uint32_t chunks = k / 32;
    const GemvShape *best = nullptr;
    for (const GemvShape &sh : kGemvShapes) {
        if (chunks == 0 || chunks != sh.lanes * sh.cpl) continue;
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
    return {64, 8};
}

// Launches the GEMV for m in [1, 8] rows of x whose staged copy fits LDS;
// the caller splits larger m (see gemv_rows_per_launch).
void launch_q4_gemv(hipStream_t stream, uint32_t cus, int m, const uint16_t *x, uint32_t x_ld,
                    const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t n,
                    uint32_t k, void *y, uint32_t y_ld, int y_is_f32) {
    const GemvShape sh = pick_gemv_shape(n, k, cus);
#define FH_GEMV_M(MM)                                                                             \
    case MM:                                                                                      \
        launch_gemv_m<MM>(sh.lanes, sh.cpl, stream, cus, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); \
        break;
    switch (m) {
        FH_GEMV_M(1)
        FH_GEMV_M(2)
        FH_GEMV_M(3)
        FH_GEMV_M(4)
        FH_GEMV_M(5)
        FH_GEMV_M(6)
        FH_GEMV_M(7)
        default: launch_gemv_m<8>(sh.lanes, sh.cpl, stream, cus, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32);
    }
#undef FH_GEMV_M
}

}  // namespace fh
