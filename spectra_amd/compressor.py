"""Weight quantizers running on the GPU (libspectra_hip.so).

Format A restates ``SpectraCompressor._quantize_chunk_group32`` /
``_compute_group32_quant`` (compressor.py:71-156) bit for bit; Format B is the
NF4 + Hadamard + CSR format (built on compressor.py:22-42).  The operand
decode the reference's loader performs on device (engine.py:1007-1021: zero
point nibble unpack, idx widening) is provided as torch ops on the same device.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib as L
from .kernels import _DT, _dtype_code, _rows, _stream

__all__ = ["SpectraCompressor", "quantize_group32", "compute_group32_quant", "unpack_zeros", "NF4Weight",
           "quantize_nf4", "csr_from_mask", "select_outlier_columns"]


class SpectraCompressor:
    """Config surface of the reference compressor (compressor.py:44-61) for this path."""

    def __init__(self, group_size: int = 32, base_outlier_ratio: float = 0.01, adaptive_kurtosis: bool = True,
                 hadamard_incoherence: bool = False, trust_remote_code: bool = False):
        if group_size != 32:  # compressor.py:53-54
            raise ValueError(f"SPECTRA currently requires group_size=32 (Group-32 microscales). "
                             f"Received group_size={group_size}.")
        if hadamard_incoherence:  # compressor.py:55-56 (Format A keeps the reference's rule)
            raise NotImplementedError("hadamard_incoherence is disabled pending paired online activation "
                                      "transformation support.")
        self.group_size = group_size
        self.base_outlier_ratio = base_outlier_ratio
        self.adaptive_kurtosis = adaptive_kurtosis
        self.hadamard_incoherence = hadamard_incoherence
        self.trust_remote_code = trust_remote_code

    @staticmethod
    def _quantize_chunk_group32(w_chunk: torch.Tensor, group_size: int = 32):
        return quantize_group32(w_chunk, group_size=group_size)

    @staticmethod
    def _compute_group32_quant(w: torch.Tensor, group_size: int = 32, outlier_idx: Optional[torch.Tensor] = None):
        return compute_group32_quant(w, group_size=group_size, outlier_idx=outlier_idx)

    def _isolate_hdsq_outliers(self, w: torch.Tensor, norm_vector: Optional[torch.Tensor] = None):
        """compressor.py:158-215: returns (w with the outlier columns zeroed when N <= 4096, else
        None; outlier column indices int32 on the CPU, ascending; the outlier columns in w's
        dtype; ratio; kurtosis).  The selection runs on the GPU (spectra_outlier_columns)."""
        idx, ratio, kurtosis = select_outlier_columns(w, norm_vector, self.base_outlier_ratio,
                                                      self.adaptive_kurtosis)
        idx_cpu = idx.cpu().contiguous()
        outlier_w = w[:, idx_cpu.long().to(w.device)].contiguous()
        w_dense = None
        if w.shape[0] <= 4096:  # compressor.py:208-210
            w_dense = w.clone()
            w_dense[:, idx_cpu.long().to(w.device)] = 0.0
        return w_dense, idx_cpu, outlier_w, ratio, kurtosis


def _weights(w: torch.Tensor, device: Optional[torch.device]) -> Tuple[torch.Tensor, int]:
    if device is None:
        device = w.device if w.is_cuda else torch.device("cuda")
    w = w.to(device)
    if w.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        w = w.float()
    return _rows(w, "w")


def quantize_group32(w: torch.Tensor, group_size: int = 32, outlier_idx: Optional[torch.Tensor] = None,
                     device: Optional[torch.device] = None):
    """Format A quantizer: returns (packed uint8 [N,K/2] marlin layout, scales fp16 [N,K/32],
    packed zero points uint8 [N, ceil(K/64)]) on the GPU (compressor.py:71-112)."""
    if w.dim() != 2:
        raise ValueError("w must be 2-D")
    n, k = w.shape
    if k % 32:
        raise ValueError(f"K ({k}) must be divisible by group_size (32)")
    w2, ldw = _weights(w, device)
    dev = w2.device
    packed = torch.empty((n, k // 2), dtype=torch.uint8, device=dev)
    scales = torch.empty((n, k // 32), dtype=torch.float16, device=dev)
    pz = torch.empty((n, (k // 32 + 1) // 2), dtype=torch.uint8, device=dev)
    idx = None
    if outlier_idx is not None:
        idx = torch.sort(outlier_idx.to(device=dev, dtype=torch.int64).reshape(-1)).values.contiguous()
    lib = L.load()
    L.check("spectra_quantize_group32", lib.spectra_quantize_group32(
        w2.data_ptr(), ldw, _dtype_code(w2, _DT.keys(), "w"), n, k, int(group_size),
        idx.data_ptr() if idx is not None else None, idx.numel() if idx is not None else 0,
        packed.data_ptr(), scales.data_ptr(), pz.data_ptr(), _stream(dev)))
    return packed, scales, pz


def compute_group32_quant(w: torch.Tensor, group_size: int = 32, outlier_idx: Optional[torch.Tensor] = None,
                          device: Optional[torch.device] = None):
    """``_compute_group32_quant`` (compressor.py:114-156): outlier columns zeroed, then quantized."""
    return quantize_group32(w, group_size=group_size, outlier_idx=outlier_idx, device=device)


def unpack_zeros(packed_zeros: torch.Tensor, k: int, group_size: int = 32) -> torch.Tensor:
    """Loader operand decode (engine.py:1007-1012): two zero points per byte -> uint8 [N, K/32]
    (returned as the same non-contiguous slice the reference binds)."""
    pz = packed_zeros
    z = torch.empty((pz.shape[0], pz.shape[1] * 2), dtype=torch.uint8, device=pz.device)
    z[:, 0::2] = pz & 0x0F
    z[:, 1::2] = (pz >> 4) & 0x0F
    return z[:, : k // group_size]


@dataclass
class NF4Weight:
    """Format B operands of one linear: NF4 nibbles, fp16 absmax, CSR outliers."""
    packed: torch.Tensor          # uint8 [N, K/2]
    absmax: torch.Tensor          # fp16 [N, K/blocksize]
    rowptr: torch.Tensor          # int32 [N+1]
    col: torch.Tensor             # int32 [nnz]
    val: torch.Tensor             # fp16 [nnz]
    k: int
    blocksize: int = 64
    hadamard_block: int = 0
    marlin_layout: bool = True

    @property
    def n(self) -> int:
        return self.packed.shape[0]

    def kernel_kwargs(self) -> dict:
        """Arguments for fused_w4a16_gemv_hdsq / batched_w4a16_gemm."""
        kw = dict(codebook="nf4", group_size=self.blocksize, hadamard_block=self.hadamard_block)
        if self.col.numel():
            kw.update(outlier_rowptr=self.rowptr)
        return kw

    def outliers(self):
        return (self.col, self.val) if self.col.numel() else (None, None)

    def nbytes(self) -> int:
        """Stored bytes of all operands (the algorithmic weight bytes of one pass)."""
        return sum(t.numel() * t.element_size() for t in (self.packed, self.absmax, self.rowptr, self.col, self.val))


def csr_from_mask(mask: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Row-major CSR positions (rowptr int32 [N+1], col int32 [nnz]) of a boolean mask, on its device."""
    n = mask.shape[0]
    rows, cols = torch.nonzero(mask, as_tuple=True)
    counts = torch.bincount(rows, minlength=n)
    rowptr = torch.zeros(n + 1, dtype=torch.int64, device=mask.device)
    rowptr[1:] = torch.cumsum(counts, 0)
    return rowptr.to(torch.int32), cols.to(torch.int32)


def quantize_nf4(w: torch.Tensor, blocksize: int = 64, hadamard_block: int = 0,
                 outlier_mask: Optional[torch.Tensor] = None, marlin_layout: bool = True,
                 device: Optional[torch.device] = None) -> NF4Weight:
    """Format B quantizer on the GPU: optional blockwise FWHT of the rows, CSR outliers
    (positions from ``outlier_mask`` in the stored basis) kept in fp16 and zeroed, fp16
    absmax per block, nearest NF4 code (fp32 distances, lowest index on ties)."""
    if w.dim() != 2:
        raise ValueError("w must be 2-D")
    n, k = w.shape
    w2, ldw = _weights(w, device)
    dev = w2.device
    packed = torch.empty((n, k // 2), dtype=torch.uint8, device=dev)
    absmax = torch.empty((n, k // blocksize), dtype=torch.float16, device=dev)
    if outlier_mask is not None:
        rowptr, col = csr_from_mask(outlier_mask.to(dev))
    else:
        rowptr, col = torch.zeros(n + 1, dtype=torch.int32, device=dev), torch.zeros(0, dtype=torch.int32, device=dev)
    val = torch.empty(col.numel(), dtype=torch.float16, device=dev)
    has = col.numel() > 0
    lib = L.load()
    L.check("spectra_quantize_nf4", lib.spectra_quantize_nf4(
        w2.data_ptr(), ldw, _dtype_code(w2, _DT.keys(), "w"), n, k, int(blocksize), int(hadamard_block),
        int(bool(marlin_layout)), rowptr.data_ptr() if has else None, col.data_ptr() if has else None,
        val.data_ptr() if has else None, packed.data_ptr(), absmax.data_ptr(), _stream(dev)))
    return NF4Weight(packed, absmax, rowptr, col, val, k, blocksize, hadamard_block, bool(marlin_layout))


def select_outlier_columns(w: torch.Tensor, norm_vector: Optional[torch.Tensor] = None, base_ratio: float = 0.01,
                           adaptive: bool = True, device: Optional[torch.device] = None):
    """Outlier-column selection on the GPU (compressor.py:158-206): returns (idx int32 [n_out]
    ascending, on the GPU; ratio; kurtosis)."""
    if w.dim() != 2:
        raise ValueError("w must be 2-D")
    n, k = w.shape
    w2, ldw = _weights(w, device)
    dev = w2.device
    norm = None
    if norm_vector is not None and norm_vector.numel() == k:  # compressor.py:183-184
        norm = norm_vector.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    lib = L.load()
    ws = torch.empty(max(int(lib.spectra_outlier_columns_workspace(k)), 4), dtype=torch.uint8, device=dev)
    idx = torch.empty(k, dtype=torch.int32, device=dev)
    cnt = torch.empty(1, dtype=torch.int32, device=dev)
    stats = torch.empty(2, dtype=torch.float32, device=dev)
    L.check("spectra_outlier_columns", lib.spectra_outlier_columns(
        w2.data_ptr(), ldw, _dtype_code(w2, _DT.keys(), "w"), n, k, norm.data_ptr() if norm is not None else None,
        float(base_ratio), int(bool(adaptive)), idx.data_ptr(), cnt.data_ptr(), stats.data_ptr(), ws.data_ptr(),
        ws.numel(), _stream(dev)))
    n_out = int(cnt.item())
    st = stats.cpu()
    return idx[:n_out], float(st[0]), float(st[1])
