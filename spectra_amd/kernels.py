"""Drop-in replacements for the reference's ``spectra/kernels.py`` entry points.

``fused_w4a16_gemv_hdsq`` and ``batched_w4a16_gemm`` keep the reference's
positional signatures (kernels.py:132-142, :333-341) and argument meaning; the
Format B (NF4 + Hadamard + CSR) operands are reached through keyword-only
arguments whose defaults leave Format A calls unchanged:

    codebook="asym" | "nf4"     Format A (q - z) * s   |  Format B NF4 * absmax
    group_size=None             32 for Format A, NF4 block size (default 64)
    hadamard_block=0            blockwise FWHT of the activations (0 = none)
    outlier_rowptr=None         when given, outlier_idx / outlier_w are the CSR
                                col (int32 [nnz]) / val (fp16 [nnz]) arrays
    bias=None                   (batched only) fused bias, as engine.py:122-123

All work runs in libspectra_hip.so on the current HIP stream; nothing here
computes on the host and there is no fallback path.
"""
from __future__ import annotations

import ctypes
import weakref
from collections import OrderedDict
from typing import List, Optional, Tuple

import torch

from . import _lib as L

__all__ = ["fused_w4a16_gemv_hdsq", "batched_w4a16_gemm", "w4a16_linear", "w4_dequant", "fwht_rows",
           "QWeightOperands", "GEMV_MAX_M", "w4_embedding", "rmsnorm", "rope_append", "attend_decode",
           "attend_workspace_bytes", "silu_mul", "greedy_next", "argmax_slots", "greedy_finish",
           "w4a16_gemv_fused", "kv4_quantize",
           "kv4_dequantize", "attend_decode_q4", "validate_outliers"]

GEMV_MAX_M = 4  # rows served by the GEMV family; larger batches go to the MFMA GEMM
# rows from which the GEMM entry runs the prefill library path (W_eff dequantized in the
# activations' dtype, one hipBLASLt GEMM) when the workspace holds it: kPrefillMinM in
# csrc/prefill.hip
PREFILL_LIBRARY_MIN_M = 512


def prefill_rotates_weights(m: int, n: int, k: int, hadamard_block: int) -> bool:
    """Whether the prefill library path puts the Hadamard rotation on the weights (W_eff H / sqrt(b)
    from the row dequant, the activations read as given) rather than on the activations: its rule
    in csrc/prefill.hip for 16-byte aligned activations with a row stride a multiple of 8 (as this
    module passes them): m >= PREFILL_LIBRARY_MIN_M, 4 m >= n, K a multiple of 512, blocks of
    2 .. 512."""
    return (m >= PREFILL_LIBRARY_MIN_M and 4 * m >= n and k % 512 == 0 and 2 <= hadamard_block <= 512
            and hadamard_block & (hadamard_block - 1) == 0)

_DT = {torch.float16: L.F16, torch.bfloat16: L.BF16, torch.float32: L.F32}
_TORCH_DT = {v: k for k, v in _DT.items()}


def _dtype_code(t: torch.Tensor, allowed, what: str) -> int:
    if t.dtype not in allowed:
        raise ValueError(f"{what} must be one of {[str(a) for a in allowed]}, got {t.dtype}")
    return _DT[t.dtype]


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _rows(t: torch.Tensor, name: str, align: int = 1) -> Tuple[torch.Tensor, int]:
    """2-D operand with unit inner stride (and optional base/row alignment in bytes)."""
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        t = t.contiguous()
    es = t.element_size()
    if align > 1 and (t.data_ptr() % align or (t.stride(0) * es) % align):
        t = t.contiguous().clone() if t.is_contiguous() else t.contiguous()
        if t.data_ptr() % align or (t.stride(0) * es) % align:
            raise ValueError(f"{name}: cannot satisfy {align}-byte row alignment for shape {tuple(t.shape)}")
    return t, t.stride(0)


def validate_outliers(n: int, k: int, *, rowptr: Optional[torch.Tensor] = None, col: Optional[torch.Tensor] = None,
                      val: Optional[torch.Tensor] = None, idx: Optional[torch.Tensor] = None,
                      ow: Optional[torch.Tensor] = None) -> None:
    """Raise ValueError unless the outlier side tensors index inside W[N, K]: CSR ``rowptr``
    [N+1] starting at 0, never decreasing and ending at nnz, ``col`` in [0, K) and ``val`` of
    nnz entries; dense ``idx`` in [0, K) with ``ow`` [N, n_out].  The kernels use these
    values as addresses, so a corrupt side tensor would read out of bounds.  Works on any
    device; one host read of the result."""
    if rowptr is not None:
        nnz = 0 if col is None else col.numel()
        if rowptr.dim() != 1 or rowptr.numel() != n + 1:
            raise ValueError(f"CSR rowptr must have N+1={n + 1} entries, got {tuple(rowptr.shape)}")
        if val is None or val.numel() != nnz:
            raise ValueError(f"CSR col and val must both have nnz entries ({nnz} vs {None if val is None else val.numel()})")
        rp = rowptr.to(torch.int64)
        ok = (rp[0] == 0) & (rp[-1] == nnz) & torch.all(rp[1:] >= rp[:-1])
        if nnz:
            c = col.to(torch.int64)
            ok = ok & torch.all((c >= 0) & (c < k))
        if not bool(ok):
            raise ValueError("corrupt CSR outliers: rowptr must start at 0, never decrease and end at nnz, "
                             f"and every column must lie in [0, K={k})")
    if idx is not None:
        if ow is not None and (ow.dim() != 2 or ow.shape[0] != n or ow.shape[1] != idx.numel()):
            raise ValueError(f"outlier_w must be [N, n_out] = [{n}, {idx.numel()}], got {tuple(ow.shape)}")
        if idx.numel() and not bool(torch.all((idx >= 0) & (idx < k))):
            raise ValueError(f"outlier column indices must lie in [0, K={k})")


def layout_word(codebook: str, group_size: int, hadamard_block: int, marlin_layout: bool) -> int:
    """The weight-layout argument of torch.ops.spectra_hip.w4a16_linear: bit 0 the codebook
    (1 = NF4, 0 = Format A), bit 1 the Marlin nibble order, bits 2-13 the group / block size,
    bits 14-25 the Hadamard block (0 = none)."""
    if codebook not in ("asym", "nf4"):
        raise ValueError(f"codebook must be 'asym' or 'nf4', got {codebook!r}")
    if not (0 < group_size < 4096 and 0 <= hadamard_block < 4096):
        raise ValueError(f"group_size {group_size} / hadamard_block {hadamard_block} out of range")
    return (codebook == "nf4") | (bool(marlin_layout) << 1) | (group_size << 2) | (hadamard_block << 14)


class QWeightOperands:
    """Validated device operands of one quantized weight + its C descriptor.

    Keeps every tensor it hands to the library alive for as long as the
    descriptor is used.
    """

    def __init__(self, packed: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor], k: int, *,
                 codebook: str = "asym", group_size: Optional[int] = None, hadamard_block: int = 0,
                 marlin_layout: bool = False, outlier_idx: Optional[torch.Tensor] = None,
                 outlier_w: Optional[torch.Tensor] = None, outlier_rowptr: Optional[torch.Tensor] = None,
                 bias: Optional[torch.Tensor] = None, packed_align: int = 16, hold_inputs: bool = True):
        # hold_inputs=False: keep only the tensors made here (conversions, copies); the caller's
        # own tensors must then outlive every use of the descriptor (the functional API's
        # cache drops an entry as soon as one of them is freed)
        inputs = {id(t) for t in (packed, scales, zeros, outlier_idx, outlier_w, outlier_rowptr, bias) if t is not None}
        if not packed.is_cuda:
            raise ValueError("packed weights must be on the GPU")
        dev = packed.device
        if packed.dtype != torch.uint8:
            raise ValueError(f"packed weights must be uint8, got {packed.dtype}")
        n = packed.shape[0]
        if codebook not in ("asym", "nf4"):
            raise ValueError(f"codebook must be 'asym' or 'nf4', got {codebook!r}")
        fmt = L.FMT_ASYM_G32 if codebook == "asym" else L.FMT_NF4
        gs = group_size if group_size is not None else (32 if fmt == L.FMT_ASYM_G32 else 64)
        if k <= 0 or k % 2 or packed.shape[1] != k // 2:
            raise ValueError(f"packed weights {tuple(packed.shape)} do not match K={k} (need [N, K/2])")
        if k % gs:
            raise ValueError(f"K={k} is not a multiple of group_size {gs}")
        keep: List[torch.Tensor] = []
        packed, ldp = _rows(packed, "packed_w", packed_align)
        keep.append(packed)
        for t, what in ((scales, "scales"), (zeros, "zeros"), (bias, "bias")):
            if t is not None and t.device != dev:
                raise ValueError(f"{what} is on {t.device}, the packed weights on {dev}")
        if scales.dtype != torch.float16:
            raise ValueError(f"scales must be float16, got {scales.dtype}")
        if scales.shape[0] != n or scales.shape[1] < k // gs:
            raise ValueError(f"scales {tuple(scales.shape)} do not match [N={n}, K/group={k // gs}]")
        scales, lds = _rows(scales, "scales")
        keep.append(scales)
        w = L.QWeight()
        w.n, w.k, w.format, w.group_size = n, k, fmt, gs
        w.hadamard_block, w.marlin_layout = int(hadamard_block), int(bool(marlin_layout))
        w.packed, w.packed_stride = packed.data_ptr(), ldp
        w.scales, w.scales_stride = scales.data_ptr(), lds
        if fmt == L.FMT_ASYM_G32:
            if zeros is None:
                raise ValueError("Format A needs zero points")
            if zeros.dtype != torch.uint8 or zeros.shape[0] != n or zeros.shape[1] < k // 32:
                raise ValueError(f"zeros must be uint8 [N, K/32] (unpacked), got {zeros.dtype} {tuple(zeros.shape)}")
            zeros, ldz = _rows(zeros, "zeros")
            keep.append(zeros)
            w.zeros, w.zeros_stride = zeros.data_ptr(), ldz
        w.outlier_kind = L.OUTLIERS_NONE
        if outlier_rowptr is not None:
            if outlier_idx is None or outlier_w is None:
                raise ValueError("CSR outliers need outlier_rowptr, outlier_idx (col) and outlier_w (val)")
            rp = outlier_rowptr.to(device=dev, dtype=torch.int32).contiguous()
            col = outlier_idx.to(device=dev, dtype=torch.int32).contiguous()
            if outlier_w.dtype != torch.float16:
                raise ValueError(f"CSR outlier values must be float16, got {outlier_w.dtype}")
            val = outlier_w.to(device=dev).contiguous()
            if rp.numel() != n + 1 or col.numel() != val.numel():
                raise ValueError("CSR shapes: rowptr [N+1], col and val [nnz]")
            validate_outliers(n, k, rowptr=rp, col=col, val=val)
            keep += [rp, col, val]
            w.outlier_kind = L.OUTLIERS_CSR
            w.csr_rowptr, w.csr_col, w.csr_val, w.csr_nnz = rp.data_ptr(), col.data_ptr(), val.data_ptr(), col.numel()
        elif outlier_idx is not None and outlier_w is not None:
            idx = outlier_idx.to(device=dev, dtype=torch.int64).contiguous()
            ow = outlier_w.to(device=dev)
            validate_outliers(n, k, idx=idx, ow=ow)
            odt = _dtype_code(ow, (torch.float16, torch.bfloat16), "outlier_w")
            ow, ldow = _rows(ow, "outlier_w")
            keep += [idx, ow]
            w.outlier_kind = L.OUTLIERS_COLUMNS
            w.num_outliers = idx.numel()
            w.outlier_idx, w.outlier_w, w.outlier_w_stride, w.outlier_w_dtype = idx.data_ptr(), ow.data_ptr(), ldow, odt
        if bias is not None:
            if bias.numel() != n:
                raise ValueError(f"bias must have N={n} elements")
            b = bias.detach().reshape(n).contiguous()
            w.bias, w.bias_dtype = b.data_ptr(), _dtype_code(b, _DT.keys(), "bias")
            keep.append(b)
        self.desc = w
        self.keep = keep if hold_inputs else [t for t in keep if id(t) not in inputs]
        # the same operands as the arguments after x of torch.ops.spectra_hip.w4a16_linear
        # (validated above; the operator trusts them); only when the caller's tensors are held
        self.op_args = None
        if hold_inputs:
            csr = w.outlier_kind == L.OUTLIERS_CSR
            cols = w.outlier_kind == L.OUTLIERS_COLUMNS
            self.op_args = (packed, scales, zeros if fmt == L.FMT_ASYM_G32 else None,
                            col if csr else idx if cols else None, val if csr else ow if cols else None,
                            rp if csr else None, b if bias is not None else None,
                            layout_word(codebook, gs, int(hadamard_block), bool(marlin_layout)))
        self.n, self.k, self.device = n, k, dev

    def ptr(self):
        return ctypes.byref(self.desc)


class _OperandCache:
    """Descriptors of the functional API, keyed by the identity, address, shape, strides, dtype
    and version (in-place writes bump it) of every operand tensor: a weight passed again is
    neither rebuilt nor re-validated.  An entry holds no reference to the caller's tensors and
    is dropped when any of them is freed (weak references); at most ``cap`` entries (LRU)."""

    def __init__(self, cap: int = 256):
        self.cap = cap
        self.d: "OrderedDict" = OrderedDict()

    def get(self, tensors, scalars, build) -> QWeightOperands:
        key = (scalars, tuple(None if t is None else (id(t), t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype,
                                                       t.device, t._version) for t in tensors))
        hit = self.d.get(key)
        if hit is not None and all((r is None) == (t is None) and (r is None or r() is t)
                                   for r, t in zip(hit[0], tensors)):
            self.d.move_to_end(key)
            return hit[1]
        ops = build()
        d = self.d
        refs = tuple(None if t is None else weakref.ref(t, lambda _r, k=key: d.pop(k, None)) for t in tensors)
        d[key] = (refs, ops)
        while len(d) > self.cap:
            d.popitem(last=False)
        return ops


_OPS = _OperandCache()


def _cached_operands(packed, scales, zeros, k, *, codebook, group_size, hadamard_block, marlin_layout, outlier_idx,
                     outlier_w, outlier_rowptr, bias=None, packed_align=16) -> QWeightOperands:
    tensors = (packed, scales, zeros, outlier_idx, outlier_w, outlier_rowptr, bias)
    scalars = (k, codebook, group_size, hadamard_block, bool(marlin_layout), packed_align)
    return _OPS.get(tensors, scalars, lambda: QWeightOperands(
        packed, scales, zeros, k, codebook=codebook, group_size=group_size, hadamard_block=hadamard_block,
        marlin_layout=marlin_layout, outlier_idx=outlier_idx, outlier_w=outlier_w, outlier_rowptr=outlier_rowptr,
        bias=bias, packed_align=packed_align, hold_inputs=False))


def _run_linear(ops: QWeightOperands, x2: torch.Tensor, out2: torch.Tensor, family: str) -> None:
    lib = L.load()
    m, k = x2.shape
    adt = _DT[x2.dtype]
    stream = _stream(x2.device)
    if family == "linear" and m == 1:
        family = "gemv"  # one row: the GEMV family, no workspace
    if family == "gemv":
        st = lib.spectra_w4a16_gemv(ops.ptr(), x2.data_ptr(), x2.stride(0), m, adt, out2.data_ptr(),
                                    out2.stride(0), stream)
        if st != L.ERR_UNSUPPORTED:  # operand combinations the GEMV family does not serve run on the GEMM
            L.check("spectra_w4a16_gemv", st)
            return
        family = "gemm"
    ws_bytes = lib.spectra_w4a16_gemm_workspace(ops.ptr(), m, adt)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=x2.device)
    fn = lib.spectra_w4a16_gemm if family == "gemm" else lib.spectra_w4a16_linear
    L.check(fn.__name__, fn(ops.ptr(), x2.data_ptr(), x2.stride(0), m, adt, out2.data_ptr(), out2.stride(0),
                            ws.data_ptr(), ws.numel(), stream))


def _activations(x: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.dtype]:
    """[M, K] fp16/bf16 view with a 16-byte aligned base and row stride; fp32 inputs are
    computed in fp16 like the reference's compute dtype (kernels.py:347-348)."""
    if not x.is_cuda:
        raise ValueError("activations must be on the GPU")
    if x.shape[-1] != k:
        raise ValueError(f"activation inner dim {x.shape[-1]} != K={k}")
    in_dtype = x.dtype
    x2 = x.reshape(-1, k)
    if x2.dtype not in (torch.float16, torch.bfloat16):
        x2 = x2.to(torch.float16)
    x2, _ = _rows(x2, "x", 16)
    return x2, in_dtype


def fused_w4a16_gemv_hdsq(x: torch.Tensor, packed_w: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor],
                          bias: Optional[torch.Tensor] = None, outlier_idx: Optional[torch.Tensor] = None,
                          outlier_w: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                          marlin_layout: bool = False, *, codebook: str = "asym", group_size: Optional[int] = None,
                          hadamard_block: int = 0, outlier_rowptr: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode GEMV (kernels.py:132-184): ``out[b] = x[b] . W_eff^T + bias``.

    x is [K] or [B, K].  Rows up to GEMV_MAX_M run on the GEMV family; the reference
    kernel reads only row 0 (kernels.py:42-98), here every row is computed (larger B
    goes to the MFMA GEMM family).
    """
    orig_1d = x.dim() == 1
    if orig_1d:
        x = x.unsqueeze(0)
    if x.dim() != 2:
        raise ValueError(f"x must be [K] or [B, K], got {tuple(x.shape)}")
    B, K = x.shape
    ops = _cached_operands(packed_w, scales, zeros, K, codebook=codebook, group_size=group_size,
                           hadamard_block=hadamard_block, marlin_layout=marlin_layout, outlier_idx=outlier_idx,
                           outlier_w=outlier_w, outlier_rowptr=outlier_rowptr, bias=bias)
    x2, in_dtype = _activations(x, K)
    N = ops.n
    if out is None:
        out = torch.empty((B, N), device=x.device, dtype=in_dtype)
    if out.shape != (B, N):
        raise ValueError(f"out must be [B={B}, N={N}], got {tuple(out.shape)}")
    target = out if (out.dtype == x2.dtype and out.stride(1) == 1) else torch.empty((B, N), device=x.device,
                                                                                      dtype=x2.dtype)
    _run_linear(ops, x2, target, "linear" if B <= GEMV_MAX_M else "gemm")
    if target is not out:
        out.copy_(target)
    return out.squeeze(0) if orig_1d else out


def batched_w4a16_gemm(a: torch.Tensor, packed_b: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor],
                       outlier_idx: Optional[torch.Tensor] = None, outlier_w: Optional[torch.Tensor] = None,
                       marlin_layout: bool = False, *, codebook: str = "asym", group_size: Optional[int] = None,
                       hadamard_block: int = 0, outlier_rowptr: Optional[torch.Tensor] = None,
                       bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Batched / prefill GEMM (kernels.py:333-389): ``c = a . W_eff^T`` over all leading dims,
    returned in ``a.dtype`` with shape ``a.shape[:-1] + (N,)``."""
    K = a.shape[-1]
    ops = _cached_operands(packed_b, scales, zeros, K, codebook=codebook, group_size=group_size,
                           hadamard_block=hadamard_block, marlin_layout=marlin_layout, outlier_idx=outlier_idx,
                           outlier_w=outlier_w, outlier_rowptr=outlier_rowptr, bias=bias)
    x2, in_dtype = _activations(a, K)
    c = torch.empty((x2.shape[0], ops.n), device=a.device, dtype=x2.dtype)
    _run_linear(ops, x2, c, "gemm")
    return c.reshape(a.shape[:-1] + (ops.n,)).to(in_dtype)


def w4a16_linear(ops: QWeightOperands, x: torch.Tensor) -> torch.Tensor:
    """Module dispatch through the C ABI (engine.py:90-124): GEMV family for up to
    GEMV_MAX_M rows, MFMA GEMM otherwise.  Returns ``x.shape[:-1] + (N,)`` in x.dtype."""
    x2, in_dtype = _activations(x, ops.k)
    out = torch.empty((x2.shape[0], ops.n), device=x.device, dtype=x2.dtype)
    _run_linear(ops, x2, out, "linear")
    return out.reshape(x.shape[:-1] + (ops.n,)).to(in_dtype)


def w4_dequant(packed: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor], *, k: Optional[int] = None,
               out_dtype: torch.dtype = torch.float16, codebook: str = "asym", group_size: Optional[int] = None,
               marlin_layout: bool = False, outlier_idx: Optional[torch.Tensor] = None,
               outlier_w: Optional[torch.Tensor] = None, outlier_rowptr: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Materialise W_eff [N, K] bit-exactly (tests/test_kernels.py:31-39, engine.py:185-210)."""
    k = k if k is not None else packed.shape[1] * 2
    ops = _cached_operands(packed, scales, zeros, k, codebook=codebook, group_size=group_size, hadamard_block=0,
                           marlin_layout=marlin_layout, outlier_idx=outlier_idx, outlier_w=outlier_w,
                           outlier_rowptr=outlier_rowptr, packed_align=1)
    out = torch.empty((ops.n, k), device=packed.device, dtype=out_dtype)
    lib = L.load()
    L.check("spectra_w4_dequant", lib.spectra_w4_dequant(ops.ptr(), out.data_ptr(), out.stride(0),
                                                          _dtype_code(out, _DT.keys(), "out_dtype"),
                                                          _stream(out.device)))
    return out


def w4_embedding(ops: QWeightOperands, ids: torch.Tensor, out_dtype: torch.dtype = torch.float16,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Gather-dequantize rows ``ids`` of a quantized weight (engine.py:167-212), bit-identical
    to the same rows of ``w4_dequant``.  Returns ``ids.shape + (K,)``."""
    if not ids.is_cuda:
        raise ValueError("ids must be on the GPU")
    flat = ids.reshape(-1)
    if flat.dtype != torch.int64:
        flat = flat.to(torch.int64)
    flat = flat.contiguous()
    if out is None:
        out = torch.empty((flat.numel(), ops.k), device=ids.device, dtype=out_dtype)
    lib = L.load()
    L.check("spectra_w4_embedding", lib.spectra_w4_embedding(ops.ptr(), flat.data_ptr(), flat.numel(), out.data_ptr(),
                                                              out.stride(0), _dtype_code(out, _DT.keys(), "out"),
                                                              _stream(ids.device)))
    return out.reshape(tuple(ids.shape) + (ops.k,))


def fwht_rows(x: torch.Tensor, block: int, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Blockwise normalised FWHT of the last dim (compressor.py:29-42), fp32 arithmetic."""
    if not x.is_cuda:
        raise ValueError("x must be on the GPU")
    k = x.shape[-1]
    x2, ldx = _rows(x.reshape(-1, k), "x")
    out = torch.empty(x2.shape, device=x.device, dtype=out_dtype or x.dtype)
    lib = L.load()
    L.check("spectra_fwht_rows", lib.spectra_fwht_rows(x2.data_ptr(), ldx, _dtype_code(x2, _DT.keys(), "x"),
                                                        x2.shape[0], k, int(block), out.data_ptr(), out.stride(0),
                                                        _dtype_code(out, _DT.keys(), "out"), _stream(x.device)))
    return out.reshape(x.shape)


# ---------------------------------------------------------------------------
# decode-layer kernels between the linears (engine.py:1240-1250 fuses the same
# submodules with Inductor; engine.py:1387-1415 keeps the static KV cache)
# ---------------------------------------------------------------------------
def _need_f16(t: torch.Tensor, name: str, contiguous: bool = True) -> None:
    if not t.is_cuda or t.dtype != torch.float16:
        raise ValueError(f"{name} must be an fp16 GPU tensor")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def rmsnorm(h: torch.Tensor, weight: torch.Tensor, eps: float, residual: Optional[torch.Tensor] = None,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``h`` += ``residual`` in place (fp16 rounding) when given, then returns
    fp16(h * rsqrt(mean(h^2) + eps) * weight) over the last dimension."""
    _need_f16(h, "h")
    hidden = h.shape[-1]
    if residual is not None:
        _need_f16(residual, "residual")
        if residual.shape != h.shape:
            raise ValueError("residual must have h's shape")
    if weight.dtype != torch.float32 or not weight.is_contiguous() or weight.numel() != hidden:
        raise ValueError("weight must be contiguous fp32 [hidden]")
    if out is None:
        out = torch.empty_like(h)
    _need_f16(out, "out")
    lib = L.load()
    L.check("spectra_rmsnorm", lib.spectra_rmsnorm(h.data_ptr(), residual.data_ptr() if residual is not None else None,
                                                    weight.data_ptr(), float(eps), h.numel() // hidden, hidden,
                                                    out.data_ptr(), _stream(h.device)))
    return out


def rope_append(qkv: torch.Tensor, pos: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int,
                kv_heads: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rotates the q/k heads of fused-QKV rows ``qkv`` [T, (heads + 2 kv_heads) * d] at
    positions ``pos`` (int64 [T]), appends k and v to ``k_cache`` / ``v_cache`` [kv, L, d];
    returns the rotated q [T, heads, d]."""
    _need_f16(qkv, "qkv", contiguous=False)
    _need_f16(k_cache, "k_cache")
    _need_f16(v_cache, "v_cache")
    kv, lmax, hd = k_cache.shape
    if v_cache.shape != k_cache.shape or kv != kv_heads:
        raise ValueError("k_cache and v_cache must be [kv_heads, L, d]")
    qkv2, ld = _rows(qkv.reshape(-1, qkv.shape[-1]), "qkv")
    T = qkv2.shape[0]
    if pos.dtype != torch.int64 or not pos.is_contiguous() or pos.numel() != T:
        raise ValueError("pos must be contiguous int64 [T]")
    for t, name in ((cos, "cos"), (sin, "sin")):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.shape != (lmax, hd // 2):
            raise ValueError(f"{name} must be contiguous fp32 [L, d/2]")
    if q_out is None:
        q_out = torch.empty((T, heads, hd), device=qkv.device, dtype=torch.float16)
    _need_f16(q_out, "q_out")
    lib = L.load()
    L.check("spectra_rope_append", lib.spectra_rope_append(qkv2.data_ptr(), ld, T, pos.data_ptr(), cos.data_ptr(),
                                                            sin.data_ptr(), heads, kv_heads, hd, lmax,
                                                            q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                                            _stream(qkv.device)))
    return q_out


def attend_workspace_bytes(heads: int, head_dim: int, max_seq: int) -> int:
    return int(L.load().spectra_attend_workspace(heads, head_dim, max_seq))


def attend_decode(qkv: torch.Tensor, pos: torch.Tensor, cos: Optional[torch.Tensor], sin: Optional[torch.Tensor],
                  heads: int, kv_heads: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  workspace: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode attention of the fused-QKV row ``qkv`` [(heads + 2 kv_heads) * d] of the token at
    position ``pos`` (int64 [1] on the device): rotates q and k (``cos``/``sin`` fp32 [L, d/2],
    None = no rotation), appends k and v to the caches [kv, L, d], attends over [0, pos];
    returns fp16 [heads, d].  ``workspace`` (uint8, ``attend_workspace_bytes`` or more): the
    merge's per-KV-head arrival counters at its start, then the span partials.  It must be
    zero before its first use; every complete call leaves the counters at zero, so one
    workspace serves later calls of any shape that fits it, but overlapping calls on one
    workspace race.  Default: a fresh zeroed buffer."""
    _need_f16(qkv, "qkv")
    _need_f16(k_cache, "k_cache")
    _need_f16(v_cache, "v_cache")
    kv, lmax, hd = k_cache.shape
    if v_cache.shape != k_cache.shape or kv != kv_heads or qkv.numel() != (heads + 2 * kv_heads) * hd:
        raise ValueError("qkv must hold (heads + 2 kv_heads) * d values and the caches be [kv_heads, L, d]")
    if pos.dtype != torch.int64 or pos.numel() != 1:
        raise ValueError("pos must be int64 [1]")
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin must both be given or both be None")
    for t, name in ((cos, "cos"), (sin, "sin")):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous() or t.shape != (lmax, hd // 2)):
            raise ValueError(f"{name} must be contiguous fp32 [L, d/2]")
    need = attend_workspace_bytes(heads, hd, lmax)
    if workspace is None:  # (zeroed: the merge's arrival counters; every call leaves them at zero)
        workspace = torch.zeros(need, device=qkv.device, dtype=torch.uint8)
    if out is None:
        out = torch.empty((heads, hd), device=qkv.device, dtype=torch.float16)
    _need_f16(out, "out")
    lib = L.load()
    L.check("spectra_attend_decode", lib.spectra_attend_decode(
        qkv.data_ptr(), pos.data_ptr(), cos.data_ptr() if cos is not None else None,
        sin.data_ptr() if sin is not None else None, heads, kv, hd, lmax, k_cache.data_ptr(), v_cache.data_ptr(),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(), _stream(qkv.device)))
    return out


def silu_mul(gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp16(silu(g) * u) of fused gate_up rows [T, 2 I] -> [T, I]."""
    _need_f16(gate_up, "gate_up", contiguous=False)
    g2, ld = _rows(gate_up.reshape(-1, gate_up.shape[-1]), "gate_up")
    inter = g2.shape[1] // 2
    if out is None:
        out = torch.empty((g2.shape[0], inter), device=gate_up.device, dtype=torch.float16)
    _need_f16(out, "out")
    lib = L.load()
    L.check("spectra_silu_mul", lib.spectra_silu_mul(g2.data_ptr(), ld, g2.shape[0], inter, out.data_ptr(),
                                                      _stream(gate_up.device)))
    return out


def greedy_next(logits: torch.Tensor, token: torch.Tensor, history: Optional[torch.Tensor] = None,
                pos: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Temperature-0 sampling (engine.py:1690-1697): ``token`` (int64 [1]) = argmax of the fp16
    ``logits`` (lowest index on ties, as torch.argmax); with ``pos`` (int64 [1]) also
    ``history[pos + 1] = token`` and ``pos += 1``, all on the device."""
    _need_f16(logits, "logits")
    for t, name in ((token, "token"), (history, "history"), (pos, "pos")):
        if t is not None and (t.dtype != torch.int64 or not t.is_cuda or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous int64 GPU tensor")
    lib = L.load()
    L.check("spectra_greedy_next", lib.spectra_greedy_next(logits.data_ptr(), logits.numel(), token.data_ptr(),
                                                            history.data_ptr() if history is not None else None,
                                                            history.numel() if history is not None else 0,
                                                            pos.data_ptr() if pos is not None else None,
                                                            _stream(logits.device)))
    return token


def argmax_slots(device: Optional[torch.device] = None) -> torch.Tensor:
    """Zeroed slots for a GEMV's fused greedy pick (``w4a16_gemv_fused(argmax_key=...)``)."""
    return torch.zeros(L.ARGMAX_SLOTS * L.ARGMAX_STRIDE, dtype=torch.int64, device=device or torch.device("cuda"))


def greedy_finish(argmax_key: torch.Tensor, token: torch.Tensor, history: Optional[torch.Tensor] = None,
                  pos: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``greedy_next`` for outputs whose pick a fused GEMV gathered into ``argmax_key``: same
    token, history and position update; leaves the slots at 0 for the next pick."""
    if argmax_key.dtype != torch.int64 or argmax_key.numel() != L.ARGMAX_SLOTS * L.ARGMAX_STRIDE or \
            not argmax_key.is_cuda or not argmax_key.is_contiguous():
        raise ValueError("argmax_key must come from argmax_slots()")
    for t, name in ((token, "token"), (history, "history"), (pos, "pos")):
        if t is not None and (t.dtype != torch.int64 or not t.is_cuda or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous int64 GPU tensor")
    lib = L.load()
    L.check("spectra_greedy_finish", lib.spectra_greedy_finish(argmax_key.data_ptr(), token.data_ptr(),
                                                                history.data_ptr() if history is not None else None,
                                                                history.numel() if history is not None else 0,
                                                                pos.data_ptr() if pos is not None else None,
                                                                _stream(argmax_key.device)))
    return token


def w4a16_gemv_fused(ops: QWeightOperands, x: torch.Tensor, *, prologue: str = "none",
                     norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-5,
                     residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                     argmax_key: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One-row GEMV with a decoder layer's neighbouring work fused in:

    * ``prologue="rmsnorm"``: x is the residual stream h; computes linear(rmsnorm(h)) with
      ``norm_weight`` (fp16 [K]) and ``eps``;
    * ``prologue="silu_mul"``: x is a fused gate_up row [2K]; computes linear(silu(g) * u);
    * ``residual`` [1, N]: returns residual + linear(...) (fp16 roundings of both, as the
      separate add); ``out`` may be ``residual`` itself (in-place update);
    * ``argmax_key`` (``argmax_slots()``): the greedy pick of the stored outputs gathered
      in the epilogue, for ``greedy_finish``.
    """
    codes = {"none": L.PROLOGUE_NONE, "rmsnorm": L.PROLOGUE_RMSNORM, "silu_mul": L.PROLOGUE_SILU_MUL}
    if prologue not in codes:
        raise ValueError(f"prologue must be one of {list(codes)}")
    _need_f16(x, "x", contiguous=False)
    kin = 2 * ops.k if prologue == "silu_mul" else ops.k
    if x.shape[-1] != kin:
        raise ValueError(f"x must have {kin} values per row")
    x2, ldx = _rows(x.reshape(-1, kin), "x", 16)
    fu = L.GemvFusion()
    fu.prologue = codes[prologue]
    fu.eps = float(eps)
    if prologue == "rmsnorm":
        if norm_weight is None or norm_weight.dtype != torch.float16 or norm_weight.numel() != ops.k:
            raise ValueError("rmsnorm needs an fp16 norm_weight of K values")
        nw = norm_weight.contiguous()
        fu.norm_weight = nw.data_ptr()
    if out is None:
        out = torch.empty((x2.shape[0], ops.n), device=x.device, dtype=torch.float16)
    _need_f16(out, "out", contiguous=False)
    out2 = out.reshape(-1, ops.n)
    if residual is not None:
        _need_f16(residual, "residual", contiguous=False)
        r2 = residual.reshape(-1, ops.n)
        if r2.stride(1) != 1:
            raise ValueError("residual rows must be contiguous")
        fu.residual, fu.residual_stride = r2.data_ptr(), r2.stride(0)
    if argmax_key is not None:
        if argmax_key.dtype != torch.int64 or argmax_key.numel() != L.ARGMAX_SLOTS * L.ARGMAX_STRIDE or \
                not argmax_key.is_cuda or not argmax_key.is_contiguous():
            raise ValueError("argmax_key must come from argmax_slots()")
        fu.argmax_key = argmax_key.data_ptr()
    lib = L.load()
    L.check("spectra_w4a16_gemv_fused", lib.spectra_w4a16_gemv_fused(ops.ptr(), x2.data_ptr(), ldx, x2.shape[0],
                                                                      L.F16, ctypes.byref(fu), out2.data_ptr(),
                                                                      out2.stride(0), _stream(x.device)))
    return out


# ---------------------------------------------------------------------------
# the 4-bit KV cache (engine.py:614-700)
# ---------------------------------------------------------------------------
def kv4_quantize(x: torch.Tensor, out: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None,
                 out_rows: Optional[int] = None):
    """Quantize fp16 rows ``x`` [..., rows, d] (leading dims = heads) like the reference's
    ``_quantize``: returns (codes uint8 [..., out_rows, d/2], scales fp16 [..., out_rows, d/32],
    zeros uint8 [..., out_rows, d/32]); with ``out`` the rows go to the first ``rows`` of
    each head's ``out_rows`` (e.g. a cache of max_seq positions)."""
    _need_f16(x, "x", contiguous=False)
    d = x.shape[-1]
    rows = x.shape[-2]
    x3 = x.reshape(-1, rows, d) if x.dim() != 2 else x.reshape(1, rows, d)
    if x3.stride(-1) != 1:
        raise ValueError("x rows must be contiguous")
    heads = x3.shape[0]
    orows = out_rows or rows
    if out is None:
        lead = tuple(x.shape[:-2])
        out = (torch.empty(lead + (orows, d // 2), device=x.device, dtype=torch.uint8),
               torch.empty(lead + (orows, d // 32), device=x.device, dtype=torch.float16),
               torch.empty(lead + (orows, d // 32), device=x.device, dtype=torch.uint8))
    codes, scales, zeros = out
    lib = L.load()
    L.check("spectra_kv4_quantize", lib.spectra_kv4_quantize(x3.data_ptr(), x3.stride(1), rows, heads, x3.stride(0), d,
                                                              codes.data_ptr(), scales.data_ptr(), zeros.data_ptr(),
                                                              orows, _stream(x.device)))
    return out


def kv4_dequantize(codes: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor) -> torch.Tensor:
    """The reference's ``_dequantize``: (q - z) * s as bf16 [rows, d]."""
    d = codes.shape[-1] * 2
    rows = codes.numel() // (d // 2)
    out = torch.empty(codes.shape[:-1] + (d,), device=codes.device, dtype=torch.bfloat16)
    # contiguous operands bound to names: a temporary copy must outlive the launch that reads it
    codes_c, scales_c, zeros_c = codes.contiguous(), scales.contiguous(), zeros.contiguous()
    lib = L.load()
    L.check("spectra_kv4_dequantize", lib.spectra_kv4_dequantize(codes_c.data_ptr(), scales_c.data_ptr(),
                                                                  zeros_c.data_ptr(), rows, d,
                                                                  out.data_ptr(), _stream(codes.device)))
    return out


def attend_decode_q4(qkv: torch.Tensor, pos: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int,
                     kv_heads: int, k_window: torch.Tensor, v_window: torch.Tensor, k4, v4,
                     workspace: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``attend_decode`` over a 4-bit cache: ``k4`` / ``v4`` = (codes [kv, L, d/2], scales
    [kv, L, d/32], zeros [kv, L, d/32]) hold every position; ``k_window`` / ``v_window``
    [kv, W, d] fp16 rings hold the last W positions (slot = position % W).  ``workspace``:
    as for ``attend_decode`` (zero before its first use, counters first, no overlapping calls)."""
    _need_f16(qkv, "qkv")
    _need_f16(k_window, "k_window")
    _need_f16(v_window, "v_window")
    kv, w, hd = k_window.shape
    lmax = k4[0].shape[1]
    if v_window.shape != k_window.shape or kv != kv_heads or k4[0].shape != (kv, lmax, hd // 2):
        raise ValueError("windows [kv_heads, W, d] and codes [kv_heads, L, d/2] expected")
    if qkv.numel() != (heads + 2 * kv_heads) * hd:
        raise ValueError("qkv must hold (heads + 2 kv_heads) * d values")
    if pos.dtype != torch.int64 or pos.numel() != 1:
        raise ValueError("pos must be int64 [1]")
    for t, name in ((cos, "cos"), (sin, "sin")):  # the kernel reads row pos of each
        if t.dtype != torch.float32 or not t.is_contiguous() or t.shape != (lmax, hd // 2):
            raise ValueError(f"{name} must be contiguous fp32 [L, d/2]")
    for cache, name in ((k4, "k4"), (v4, "v4")):  # codes, fp16 scales, uint8 zero points
        codes, sc, zp = cache
        if codes.shape != (kv, lmax, hd // 2) or codes.dtype != torch.uint8 or \
                sc.shape != (kv, lmax, hd // 32) or sc.dtype != torch.float16 or \
                zp.shape != (kv, lmax, hd // 32) or zp.dtype != torch.uint8 or \
                not all(t.is_contiguous() and t.device == qkv.device for t in cache):
            raise ValueError(f"{name} must be contiguous (codes uint8 [kv, L, d/2], scales fp16 and "
                             f"zero points uint8 [kv, L, d/32]) on the qkv's device")
    need = attend_workspace_bytes(heads, hd, lmax)
    if workspace is None:  # (zeroed: the merge's arrival counters; every call leaves them at zero)
        workspace = torch.zeros(need, device=qkv.device, dtype=torch.uint8)
    if out is None:
        out = torch.empty((heads, hd), device=qkv.device, dtype=torch.float16)
    ptrs = [t.data_ptr() for t in (k_window, v_window, k4[0], v4[0], k4[1], v4[1], k4[2], v4[2])]
    lib = L.load()
    L.check("spectra_attend_decode_q4", lib.spectra_attend_decode_q4(
        qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), heads, kv, hd, lmax, w, *ptrs,
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(), _stream(qkv.device)))
    return out
