// q4 decode GEMV instances (dot2 and matrix-core kernels) for 4 rows of x.
#include "q4_gemv_mfma.hpp"

namespace fh {

template <>
void launch_gemv_m<4>(uint32_t lanes, uint32_t cpl, hipStream_t stream, uint32_t cus, const GemvArgs &a) {
#define FH_GEMV_SHAPE(LL, CC)                                   \
    if (lanes == LL && cpl == CC) {                              \
        launch_gemv_mlc<4, LL, CC>(stream, cus, a);             \
        return;                                                 \
    }
    FH_GEMV_SHAPES(FH_GEMV_SHAPE)
#undef FH_GEMV_SHAPE
}

template <>
void launch_gemv_mfma_m<4>(hipStream_t stream, uint32_t cus, const GemvArgs &a) {
    launch_gemv_mfma_dispatch<4>(stream, cus, a);
}

}  // namespace fh
