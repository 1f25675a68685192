// Row-owning GEMV instantiations without a prologue (fp16 and bf16 activations).
#include "gemv_rows_inst.h"

namespace spectra {

gemv_rows_fn gemv_rows_pick_plain(int g, int spr, int rpg, int xc, bool split, bool bf) {
  return bf ? rows_pick_combo<true, kProNone>(g, spr, rpg, xc, split)
            : rows_pick_combo<false, kProNone>(g, spr, rpg, xc, split);
}

}  // namespace spectra
