// Instantiations of the multi-pass row GEMV (gemv_rows_lm.h).
#include "gemv_rows_lm.h"

namespace spectra {

gemv_rows_lm_fn gemv_rows_lm_pick(int g, int spr, bool bf, int pro) {
#define SPECTRA_LM_CASE(G_, S_, R_, X_)                                                                 \
  if (g == G_ && spr == S_) {                                                                        \
    if (pro == kProRms) return bf ? nullptr : gemv_rows_lm_kernel<G_, S_, R_, X_, false, kProRms>;       \
    if (pro == kProNone) return bf ? gemv_rows_lm_kernel<G_, S_, R_, X_, true, kProNone>                  \
                                   : gemv_rows_lm_kernel<G_, S_, R_, X_, false, kProNone>;                \
    return nullptr;                                                                                  \
  }
  SPECTRA_LM_CASE(32, 3, 2, 1)
  SPECTRA_LM_CASE(64, 1, 2, 1)
  SPECTRA_LM_CASE(64, 2, 2, 1)
#undef SPECTRA_LM_CASE
  return nullptr;
}

}  // namespace spectra
