"""CPU oracle for SPECTRA's W4A16 quantized-linear path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``spectra_amd``) may import,
call, link or execute anything under ``oracle/``.  The only permitted callers
are ``tests/``, ``__graft_entry__.smoke()`` (as the checker) and the
``cpu_baseline`` leg of ``bench.py`` (as the timed CPU restatement).

Everything here is a from-scratch numpy restatement of the reference's
arithmetic (``/root/reference/spectra/{compressor,engine,kernels}.py`` and
``/root/reference/tests/test_kernels.py``).  Each function cites the file:line
it follows and states which check pins it (see ``tests/test_oracle.py``).

Pinning status per function:
  quantize_group32      pinned: the reference's 3 known-answer tests
                        (tests/test_quantizer.py:19-55) + reconstruction bound
                        + bit-equality with torch's evaluation of the same
                        fp32 op sequence.
  pack/unpack layouts   pinned: engine.py:189-198 unpack semantics restated
                        independently + round trip on all 256 byte values.
  dequant_group32       pinned: closed form + torch evaluation.
  fwht                  pinned: dense Sylvester matrix (scipy.linalg.hadamard)
                        in fp64, involution H.H = I, exact integer inputs.
  nf4_quantize          pinned: brute-force nearest code in fp64, exact
                        reconstruction of every code point, monotonicity.
  nf4_dequant           pinned: closed form + torch evaluation.
  linear_ref            pinned: fp64 matmul (numpy) vs float32 torch matmul.
  select_outlier_columns pinned: golden vectors written by the reference's own
                        _isolate_hdsq_outliers (tests/golden/make_outlier_golden.py)
                        + closed-form invariants (Gaussian kurtosis, dominant column).
"""
from .spectra_oracle import *  # noqa: F401,F403
