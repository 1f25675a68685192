// Row-owning GEMV instantiations for 2 .. 4 activation rows (no prologue), K = 3072, 4096
// and 8192: the every-wave-produces combinations, the only ones the several-row plan picks
// (it tries them first, and whenever none fits no split plan fits either: both need the
// row waves within 16 waves).  Each is built for the row counts whose accumulators,
// residual values, decoded slots and activation runs stay in registers (rows per group x
// rows <= 12: no scratch).
#pragma once

#include "gemv_rows_inst.h"

namespace spectra {

//  (group size, slots per row, rows per group, chunks per producer wave, split)
#define SPECTRA_ROWS_MULTI_COMBOS(X)                                                  \
  X(32, 3, 1, 1, false) X(32, 3, 2, 1, false)                      /* K = 3072 */     \
  X(64, 2, 1, 1, false) X(64, 2, 2, 1, false) X(64, 2, 4, 1, false) /* K = 4096 */    \
  X(64, 4, 1, 1, false) X(64, 4, 2, 1, false)                      /* K = 8192 */

template <bool BF>
gemv_rows_fn rows_pick_multi_combo(int g, int spr, int rpg, int xc, bool split, int mr) {
#define SPECTRA_ROWS_MULTI_CASE(G_, S_, R_, X_, P_)                                     \
  if (g == G_ && spr == S_ && rpg == R_ && xc == X_ && split == P_) {                  \
    if (R_ * mr > 12) return nullptr;                                                   \
    if (mr == 2) return gemv_rows_kernel<G_, S_, R_, X_, BF, kProNone, P_, 2>;         \
    if (mr == 3) return gemv_rows_kernel<G_, S_, R_, X_, BF, kProNone, P_, 3>;         \
    if (mr == 4) return gemv_rows_kernel<G_, S_, R_, X_, BF, kProNone, P_, (R_ <= 3 ? 4 : 2)>; \
    return nullptr;                                                                     \
  }
  SPECTRA_ROWS_MULTI_COMBOS(SPECTRA_ROWS_MULTI_CASE)
#undef SPECTRA_ROWS_MULTI_CASE
  return nullptr;
}

}  // namespace spectra
