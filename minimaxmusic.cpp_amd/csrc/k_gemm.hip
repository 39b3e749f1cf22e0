// k_gemm.hip - MFMA GEMM for quantized weights at token counts (M > 8).
#include "mmhip_device.h"
#include "mmhip_internal.h"

namespace mmhip {

int gemm_q(int wtype, const void * W, int64_t N, int64_t K, int64_t row_stride, const float * x, int64_t ldx, int64_t M,
           float * y, int64_t ldy, hipStream_t stream) {
    (void) W; (void) N; (void) K; (void) row_stride; (void) x; (void) ldx; (void) y; (void) ldy; (void) stream;
    return set_error(MMHIP_ERR_UNSUPPORTED, "mul_mat: GEMM path (type %d, M=%lld) not built yet", wtype, (long long) M);
}

}  // namespace mmhip
