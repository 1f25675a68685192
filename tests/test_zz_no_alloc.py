"""The no-allocation entry point spectra_w4a16_linear_noalloc, called through the C ABI,
against spectra_w4a16_linear with a caller workspace (the same kernels: bit-identical
outputs): two calls in a row on the GPU's shared scratch, the second with a smaller input,
then a single row, a Format A weight, and a call whose workspace exceeds the scratch
(rejected before any launch, the output left untouched)."""
import numpy as np
import pytest
import torch

import oracle as O
from spectra_amd import _lib as L
from spectra_amd import compressor as C
from spectra_amd import kernels as K

pytestmark = pytest.mark.gpu


def case(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _nf4_operands(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    mask = torch.rand(n, k, generator=g) < 0.005
    w[mask] = (torch.randn(int(mask.sum()), generator=g) * 0.2).half()
    q = C.quantize_nf4(w.cuda(), 64, 0, mask.cuda(), True)
    col, val = q.outliers()
    return K.QWeightOperands(q.packed, q.absmax, None, k, codebook="nf4", group_size=64, hadamard_block=128,
                             marlin_layout=True, outlier_idx=col, outlier_w=val, outlier_rowptr=q.rowptr)


def _format_a_operands(n, k, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    idx = np.sort(rng.permutation(k)[:9]).astype(np.int64)
    packed, scales, pz = O.compute_group32_quant(w.astype(np.float32), idx)
    zeros = C.unpack_zeros(torch.from_numpy(pz), k).contiguous().cuda()
    return K.QWeightOperands(torch.from_numpy(packed).cuda(), torch.from_numpy(scales).cuda(), zeros, k,
                             marlin_layout=True, outlier_idx=torch.from_numpy(idx).cuda(),
                             outlier_w=torch.from_numpy(w[:, idx].copy()).cuda())


def _with_workspace(lib, ops, x, out):
    m = x.shape[0]
    ws_bytes = lib.spectra_w4a16_gemm_workspace(ops.ptr(), m, L.F16)
    ws = torch.empty(max(int(ws_bytes), 256), dtype=torch.uint8, device="cuda")
    st = lib.spectra_w4a16_linear(ops.ptr(), x.data_ptr(), x.stride(0), m, L.F16, out.data_ptr(), out.stride(0),
                                  ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    L.check("spectra_w4a16_linear", st)


def _noalloc(lib, ops, x, out):
    return lib.spectra_w4a16_linear_noalloc(ops.ptr(), x.data_ptr(), x.stride(0), x.shape[0], L.F16, out.data_ptr(),
                                            out.stride(0), torch.cuda.current_stream().cuda_stream)


def test_noalloc_matches_workspace_entry(hip):
    lib = hip
    n, k = 5120, 3072
    ops = _nf4_operands(n, k, 11)
    g = torch.Generator().manual_seed(12)
    # two calls in a row on the shared scratch, the second smaller; then one row
    for m in (8, 3, 1):
        case(n=n, k=k, m=m, fmt="nf4")
        x = torch.randn(m, k, generator=g).half().cuda()
        ref = torch.empty(m, n, dtype=torch.float16, device="cuda")
        got = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda")
        _with_workspace(lib, ops, x, ref)
        L.check("spectra_w4a16_linear_noalloc", _noalloc(lib, ops, x, got))
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"m={m}: no-allocation output differs from the workspace entry"


def test_noalloc_format_a(hip):
    lib = hip
    n, k = 700, 2048
    ops = _format_a_operands(n, k, 13)
    g = torch.Generator().manual_seed(14)
    for m in (16, 5):
        case(n=n, k=k, m=m, fmt="asym_g32")
        x = torch.randn(m, k, generator=g).half().cuda()
        ref = torch.empty(m, n, dtype=torch.float16, device="cuda")
        got = torch.empty(m, n, dtype=torch.float16, device="cuda")
        _with_workspace(lib, ops, x, ref)
        L.check("spectra_w4a16_linear_noalloc", _noalloc(lib, ops, x, got))
        torch.cuda.synchronize()
        assert torch.equal(got, ref)


def test_noalloc_prompt_rows_on_the_mfma_family(hip):
    """From 512 rows the full workspace query includes the library GEMM path's dequantized
    weight (here 16 MiB, beyond the scratch); the no-allocation entry counts only the MFMA
    family's buffers (about 1.3 MiB here), so the call runs from the scratch on that family:
    against the workspace entry (the library path, the same fp16 operands) within 1e-2."""
    lib = hip
    n, k, m = 16384, 512, 1024
    case(n=n, k=k, m=m, fmt="nf4")
    ops = _nf4_operands(n, k, 16)
    assert lib.spectra_w4a16_gemm_workspace(ops.ptr(), m, L.F16) > 8 << 20
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(17)).half().cuda()
    ref = torch.empty(m, n, dtype=torch.float16, device="cuda")
    got = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda")
    _with_workspace(lib, ops, x, ref)
    L.check("spectra_w4a16_linear_noalloc", _noalloc(lib, ops, x, got))
    torch.cuda.synchronize()
    err = (got.float() - ref.float()).abs().max().item()
    assert err <= 1e-2, f"max-abs {err}"


def test_noalloc_rejects_workspace_beyond_scratch(hip):
    lib = hip
    n, k, m = 1024, 4096, 2048  # the prefill GEMM needs > 8 MiB of workspace at this m
    case(n=n, k=k, m=m, fmt="nf4")
    ops = _nf4_operands(n, k, 15)
    need = lib.spectra_w4a16_gemm_workspace(ops.ptr(), m, L.F16)
    assert need > 8 << 20
    x = torch.zeros(m, k, dtype=torch.float16, device="cuda")
    out = torch.full((m, n), 7.0, dtype=torch.float16, device="cuda")
    st = _noalloc(lib, ops, x, out)
    torch.cuda.synchronize()
    assert st == L.ERR_WORKSPACE
    assert "scratch" in lib.spectra_last_error().decode()
    assert torch.all(out == 7.0), "a rejected call must not launch anything"
