// GEMV kernel instantiations for fp16 activations.
#include "gemv_kernel.h"

namespace spectra {

gemv_fn gemv_pick_f16(int fmt, int mt, int rpw, bool wide) {
  return fmt == SPECTRA_FMT_NF4 ? pick_kernel<SPECTRA_FMT_NF4, false>(mt, rpw, wide)
                                : pick_kernel<SPECTRA_FMT_ASYM_G32, false>(mt, rpw, wide);
}

gemv_fn gemv_pick_f16_pro(int pro, int rpw, bool wide) {
  if (wide)
    return pro == kProRms ? pick_wide<SPECTRA_FMT_NF4, false, kProRms>(rpw)
                          : pick_wide<SPECTRA_FMT_NF4, false, kProSiluMul>(rpw);
  return pro == kProRms ? pick_pro_rpw<kProRms>(rpw) : pick_pro_rpw<kProSiluMul>(rpw);
}

}  // namespace spectra
