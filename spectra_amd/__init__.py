"""spectra_amd -- MI355X (gfx950) W4A16 quantized-linear path of SPECTRA.

Host-side mirror of the reference's operator surface for this path:
  spectra_amd.kernels     fused_w4a16_gemv_hdsq, batched_w4a16_gemm (kernels.py)
  spectra_amd.engine      SpectraFusedLinear (engine.py:35-124)
  spectra_amd.compressor  Format A / Format B quantizers (compressor.py:22-156)
All compute runs in the hand-written HIP library libspectra_hip.so (C ABI in
include/spectra_hip.h), built by ``python -m spectra_amd._build``.
"""
from . import _lib  # noqa: F401

__version__ = "0.1.0"


def library_version() -> str:
    return _lib.load().spectra_version().decode()
