// int8-weight instantiations of the fused GEMV (gemv_impl.h).
#include "gemv_impl.h"

namespace ec {

hipError_t gemv_i8_fused(const GemvArgs &a, int epi, int pro, hipStream_t s) {
#define EC_CASE(E, P) \
  if (epi == E && pro == P) return gemv_launch_shape<WT_I8, E, P>(a, s);
  EC_CASE(EPI_STORE, PRO_I8)
  EC_CASE(EPI_STORE, PRO_RMS)
  EC_CASE(EPI_STORE, PRO_LN)
  EC_CASE(EPI_RESID, PRO_QUANT)
  EC_CASE(EPI_SWIGLU, PRO_RMS)
  EC_CASE(EPI_GELU, PRO_LN)
#undef EC_CASE
  return hipErrorInvalidValue;
}

}  // namespace ec
