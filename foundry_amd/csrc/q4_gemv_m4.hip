// q4 decode GEMV instances for 4 rows of x.
#include "q4_gemv.hpp"

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

}  // namespace fh
