// GEMV kernel instantiations for bf16 activations.
#include "gemv_kernel.h"

namespace spectra {

gemv_fn gemv_pick_bf16(int fmt, int mt, int rpw, bool wide) {
  return fmt == SPECTRA_FMT_NF4 ? pick_kernel<SPECTRA_FMT_NF4, true>(mt, rpw, wide)
                                : pick_kernel<SPECTRA_FMT_ASYM_G32, true>(mt, rpw, wide);
}

}  // namespace spectra
