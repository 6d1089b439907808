// f16-weight instantiations of the fused GEMV (gemv_impl.h).
#include "gemv_impl.h"

namespace ec {

int gemv_pick_lpr(int wt, int epi, int K, int N);
int gemv_pick_mt(int M);

template <int LPR>
static hipError_t w16_case(const GemvArgs &a, int epi, int pro, int mt, hipStream_t s) {
#define EC_CASE(E, P) \
  if (epi == E && pro == P) return gemv_launch_mt<WT_F16, LPR, E, P>(a, mt, s);
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

hipError_t gemv_f16_fused(const GemvArgs &a, int epi, int pro, hipStream_t s) {
  const int mt = gemv_pick_mt(a.M);
  return gemv_pick_lpr(WT_F16, epi, a.K, a.N) == 64 ? w16_case<64>(a, epi, pro, mt, s)
                                                   : w16_case<32>(a, epi, pro, mt, s);
}

}  // namespace ec
