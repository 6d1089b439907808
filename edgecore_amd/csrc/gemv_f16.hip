// f16-weight instantiations of the fused GEMV (gemv_impl.h).
#include "gemv_impl.h"

namespace ec {

hipError_t gemv_f16_fused(const GemvArgs &a, int epi, int pro, hipStream_t s) {
#define EC_CASE(E, P) \
  if (epi == E && pro == P) return gemv_launch_shape<WT_F16, E, P>(a, s);
  EC_CASE(EPI_STORE, PRO_F32)
  EC_CASE(EPI_STORE, PRO_RMS)
  EC_CASE(EPI_STORE, PRO_LN)
  EC_CASE(EPI_BIAS, PRO_LN)
  EC_CASE(EPI_RESID, PRO_F32)
  EC_CASE(EPI_BIAS_RESID, PRO_F32)
  EC_CASE(EPI_SWIGLU, PRO_RMS)
  EC_CASE(EPI_BIAS_GELU, PRO_LN)
#undef EC_CASE
  return hipErrorInvalidValue;
}

}  // namespace ec
