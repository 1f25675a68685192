"""``SpectraFusedLinear``: the reference's quantized linear module (engine.py:35-124)
on the MI355X library.

Same constructor, ``set_weights`` and ``forward`` contract; the weight
descriptor is built once per ``set_weights`` so a forward call is one C-ABI
call (plus the output allocation) on the current stream -- capturable in a
HIP graph.  Format B operands arrive through keyword-only arguments.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .kernels import GEMV_MAX_M, QWeightOperands, w4a16_linear

__all__ = ["SpectraFusedLinear"]


class SpectraFusedLinear(nn.Module):
    """Drop-in quantized linear: packed 4-bit weights, scales, zeros and outliers
    (engine.py:35-88); rows <= GEMV_MAX_M go to the GEMV family, larger batches to
    the MFMA GEMM (engine.py:94-124)."""

    def __init__(self, in_features: int, out_features: int, group_size: int = 32, has_bias: bool = False,
                 enable_hdsq: bool = True, marlin_layout: bool = False, *, codebook: str = "asym",
                 hadamard_block: int = 0):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        self.enable_hdsq = enable_hdsq
        self.marlin_layout = marlin_layout
        self.codebook = codebook
        self.hadamard_block = hadamard_block
        self.register_buffer("packed_weight", None)
        self.register_buffer("scales", None)
        self.register_buffer("zeros", None)
        self.register_buffer("outlier_idx", None)
        self.register_buffer("outlier_weight", None)
        self.register_buffer("outlier_rowptr", None)
        if has_bias:  # engine.py:64-65
            self.register_parameter("bias", nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16)))
        else:
            self.register_parameter("bias", None)
        self._ops: Optional[QWeightOperands] = None

    def set_weights(self, packed_w: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor],
                    bias: Optional[torch.Tensor] = None, outlier_idx: Optional[torch.Tensor] = None,
                    outlier_weight: Optional[torch.Tensor] = None, marlin_layout: bool = False, *,
                    outlier_rowptr: Optional[torch.Tensor] = None, codebook: Optional[str] = None,
                    hadamard_block: Optional[int] = None):
        """engine.py:69-88, plus Format B: codebook="nf4" with ``zeros=None``, CSR outliers
        given as ``outlier_rowptr`` + ``outlier_idx`` (col) + ``outlier_weight`` (val)."""
        self.packed_weight = packed_w
        self.scales = scales
        self.zeros = zeros
        self.marlin_layout = marlin_layout
        if codebook is not None:
            self.codebook = codebook
        if hadamard_block is not None:
            self.hadamard_block = hadamard_block
        if bias is not None:
            self.bias = nn.Parameter(bias, requires_grad=False)
        if outlier_idx is not None and outlier_weight is not None:
            self.enable_hdsq = True
            self.outlier_idx = outlier_idx
            self.outlier_weight = outlier_weight
            self.outlier_rowptr = outlier_rowptr
        self._ops = None

    def _operands(self) -> QWeightOperands:
        if self._ops is None:
            use_o = self.enable_hdsq and self.outlier_idx is not None and self.outlier_weight is not None
            gs = self.group_size if self.codebook == "asym" else (self.group_size if self.group_size != 32 else 64)
            self._ops = QWeightOperands(
                self.packed_weight, self.scales, self.zeros, self.in_features, codebook=self.codebook,
                group_size=gs, hadamard_block=self.hadamard_block, marlin_layout=self.marlin_layout,
                outlier_idx=self.outlier_idx if use_o else None, outlier_w=self.outlier_weight if use_o else None,
                outlier_rowptr=self.outlier_rowptr if use_o else None, bias=self.bias)
        return self._ops

    def _apply(self, fn, *args, **kwargs):  # device/dtype moves invalidate the descriptor
        self._ops = None
        return super()._apply(fn, *args, **kwargs)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        total_tokens = x.numel() // self.in_features
        if total_tokens == 0:
            return x.new_empty(x.shape[:-1] + (self.out_features,))
        y = w4a16_linear(self._operands(), x.reshape(total_tokens, self.in_features))
        return y.reshape(x.shape[:-1] + (self.out_features,)).to(x.dtype)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, codebook={self.codebook}, "
                f"group_size={self.group_size}, hadamard_block={self.hadamard_block}, "
                f"marlin_layout={self.marlin_layout}, gemv_rows<={GEMV_MAX_M}")
