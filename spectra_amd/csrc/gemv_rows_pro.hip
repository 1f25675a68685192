// Row-owning GEMV instantiations with the fused RMSNorm and SiLU-mul prologues (fp16).
#include "gemv_rows_inst.h"

namespace spectra {

gemv_rows_fn gemv_rows_pick_pro(int g, int spr, int rpg, int xc, bool split, int pro) {
  if (pro == kProRms) return rows_pick_combo<false, kProRms>(g, spr, rpg, xc, split);
  if (pro == kProSiluMul) return rows_pick_combo<false, kProSiluMul>(g, spr, rpg, xc, split);
  return nullptr;
}

}  // namespace spectra
