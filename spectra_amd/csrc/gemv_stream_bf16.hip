// Stream GEMV kernel instantiations for bf16 activations.
#include "gemv_stream.h"

namespace spectra {

gemv_stream_fn gemv_stream_pick_bf16(int ns) { return stream_pick_ns<true, kProNone>(ns); }

}  // namespace spectra
