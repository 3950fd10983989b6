// q4 decode GEMV instances for 7 rows of x.
#include "q4_gemv.hpp"

namespace fh {

template <>
void launch_gemv_m<7>(uint32_t lanes, uint32_t cpl, hipStream_t stream, uint32_t cus,
                      const uint16_t *x, uint32_t x_ld, const uint32_t *wq, const uint16_t *s,
                      const uint16_t *b, uint32_t n, uint32_t k, void *y, uint32_t y_ld,
                      int y_is_f32) {
#define FH_GEMV_SHAPE(LL, CC)                                                                  \
    if (lanes == LL && cpl == CC) {                                                             \
        launch_gemv_mlc<7, LL, CC>(stream, cus, x, x_ld, wq, s, b, n, k, y, y_ld, y_is_f32); \
        return;                                                                                \
    }
    FH_GEMV_SHAPES(FH_GEMV_SHAPE)
#undef FH_GEMV_SHAPE
}

}  // namespace fh
