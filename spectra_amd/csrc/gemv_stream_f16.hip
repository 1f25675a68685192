// Stream GEMV kernel instantiations for fp16 activations (plain, RMSNorm and SiLU-mul prologues).
#include "gemv_stream.h"

namespace spectra {

gemv_stream_fn gemv_stream_pick_f16(int ns, int pro) {
  if (pro == kProRms) return stream_pick_ns<false, kProRms>(ns);
  if (pro == kProSiluMul) return stream_pick_ns<false, kProSiluMul>(ns);
  return stream_pick_ns<false, kProNone>(ns);
}

}  // namespace spectra
