// int8-weight instantiations of the fused GEMV (gemv_impl.h).
#include "gemv_impl.h"

namespace ec {

int gemv_pick_lpr(int wt, int epi, int K, int N);

template <int LPR>
static hipError_t i8_case(const GemvArgs &a, int epi, int pro, int mt, hipStream_t s) {
#define EC_CASE(E, P) \
  if (epi == E && pro == P) return gemv_launch_mt<WT_I8, LPR, E, P>(a, mt, s);
  EC_CASE(EPI_STORE, PRO_I8)
  EC_CASE(EPI_STORE, PRO_RMS)
  EC_CASE(EPI_STORE, PRO_LN)
  EC_CASE(EPI_RESID, PRO_QUANT)
  EC_CASE(EPI_SWIGLU, PRO_RMS)
  EC_CASE(EPI_GELU, PRO_LN)
#undef EC_CASE
  return hipErrorInvalidValue;
}

int gemv_pick_mt(int M);

hipError_t gemv_i8_fused(const GemvArgs &a, int epi, int pro, hipStream_t s) {
  const int mt = gemv_pick_mt(a.M);
  return gemv_pick_lpr(WT_I8, epi, a.K, a.N) == 64 ? i8_case<64>(a, epi, pro, mt, s)
                                                   : i8_case<16>(a, epi, pro, mt, s);
}

}  // namespace ec
