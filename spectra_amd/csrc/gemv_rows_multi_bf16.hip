// Row-owning GEMV instantiations for 2 .. 4 bf16 activation rows.
#include "gemv_rows_multi.h"

namespace spectra {

gemv_rows_fn gemv_rows_pick_multi_bf16(int g, int spr, int rpg, int xc, bool split, int mr) {
  return rows_pick_multi_combo<true>(g, spr, rpg, xc, split, mr);
}

}  // namespace spectra
