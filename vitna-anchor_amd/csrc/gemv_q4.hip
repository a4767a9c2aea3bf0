/**
 * gemv_q4.hip - Instantiations of the dense-projection GEMV (gemv_impl.h) for
 * some dtype combinations of the q/k/v, o and head matrices.
 */

#include "gemv_impl.h"

hipError_t gemv_combo_q4(const gemv_args& a, int d0, int d1, int d2, hipStream_t s, bool* served) {
    constexpr int Q8 = VITNA_DTYPE_Q8_0, Q4 = VITNA_DTYPE_Q4_K, Q6 = VITNA_DTYPE_Q6_K, F = VITNA_DTYPE_F32;
    (void)Q8; (void)Q4; (void)Q6; (void)F;
    GEMV_CASE(Q4, Q4, Q6)
    GEMV_CASE(Q4, Q4, Q4)
    GEMV_CASE(Q4, Q6, Q6)
    *served = false;
    return hipErrorInvalidValue;
}
