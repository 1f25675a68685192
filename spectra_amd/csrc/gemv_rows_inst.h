// Row-owning GEMV instantiations: the (group size, slots per row, rows per group, chunks
// per producer wave, split) combinations the planner can pick, K = 1024 .. 14336.
#pragma once

#include "gemv_rows.h"

namespace spectra {

#define SPECTRA_ROWS_COMBOS(X)                                                                          \
  X(32, 1, 1, 1, true) X(32, 1, 2, 1, true) X(32, 1, 4, 1, true)                     /* K = 1024 */  \
  X(64, 1, 1, 1, true) X(64, 1, 2, 1, true) X(64, 1, 4, 1, true)                     /* K = 2048 */  \
  X(32, 3, 1, 1, true) X(32, 3, 2, 1, true) X(32, 3, 2, 1, false)                      /* K = 3072 */ \
  X(64, 2, 1, 1, true) X(64, 2, 2, 1, true) X(64, 2, 4, 1, true) X(64, 2, 4, 1, false) /* K = 4096 */ \
  X(64, 4, 1, 2, true) X(64, 4, 1, 4, true) X(64, 4, 2, 2, true) X(64, 4, 2, 4, true)               \
  X(64, 4, 2, 1, false)                                                              /* K = 8192 */  \
  X(64, 7, 1, 2, true) X(64, 7, 1, 4, true)                                          /* K = 14336 */

template <bool BF, int PRO>
gemv_rows_fn rows_pick_combo(int g, int spr, int rpg, int xc, bool split) {
#define SPECTRA_ROWS_CASE(G_, S_, R_, X_, P_) \
  if (g == G_ && spr == S_ && rpg == R_ && xc == X_ && split == P_) return gemv_rows_kernel<G_, S_, R_, X_, BF, PRO, P_>;
  SPECTRA_ROWS_COMBOS(SPECTRA_ROWS_CASE)
#undef SPECTRA_ROWS_CASE
  return nullptr;
}

gemv_rows_fn gemv_rows_pick_plain(int g, int spr, int rpg, int xc, bool split, bool bf);
gemv_rows_fn gemv_rows_pick_pro(int g, int spr, int rpg, int xc, bool split, int pro);
// 2 .. 4 activation rows, no prologue (nullptr where the combination is not built for mr rows)
gemv_rows_fn gemv_rows_pick_multi_f16(int g, int spr, int rpg, int xc, bool split, int mr);
gemv_rows_fn gemv_rows_pick_multi_bf16(int g, int spr, int rpg, int xc, bool split, int mr);

}  // namespace spectra
