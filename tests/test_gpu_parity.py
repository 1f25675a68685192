"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Bars:
  * quantizers, FWHT and W_eff dequant: bit-exact;
  * GEMV / GEMM outputs, fp16: max-abs <= 1e-2 and L2-relative <= 1e-3 against
    y_ref = fp32(FWHT(x)) @ fp32(W_eff)^T accumulated in float64.  Where |y_ref|
    >= 16 one fp16 output ulp exceeds 1e-2, so the per-element bar is
    max(1e-2, 1 ulp); the L2-relative bar applies to outputs of >= 64 elements
    (on a single element it only measures that element's cancellation);
  * bf16 outputs: bf16 rounding alone is ~2^-9 relative, so the bar is max error
    <= 1 bf16 ulp of |y_ref| (+1e-2 absolute) and L2-relative <= 5e-3.  For bf16
    the reference is the float32 dequant (W_eff in float32), the arithmetic of the
    reference GEMV itself (kernels.py:73-74): W_eff rounded to bf16 would add a
    2^-9 weight error that the kernels do not make (they keep >= fp16 precision).
Every case prints its parameters first so a failure names it.
"""
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O
from spectra_amd import _lib as L
from spectra_amd import compressor as C
from spectra_amd import kernels as K
from spectra_amd.engine import SpectraFusedEmbedding, SpectraFusedLinear

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
TDT = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


def case(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def cuda(a, dtype=None):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16 and dtype == torch.bfloat16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda()
    t = torch.from_numpy(a).cuda()
    return t if dtype is None else t.to(dtype)


def host(t, dtype="float16"):
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def check_y(y, y_ref, dtype):
    yv = y.detach().float().cpu().double().numpy().reshape(y_ref.shape)
    err = np.abs(yv - y_ref)
    rel = np.linalg.norm(yv - y_ref) / max(np.linalg.norm(y_ref), 1e-30)
    big = y_ref.size >= 64
    if dtype == torch.float16:
        ulp = np.spacing(np.abs(y_ref).astype(np.float16)).astype(np.float64)
        assert np.all(err <= np.maximum(1e-2, ulp)), f"max-abs {err.max()} (excess over bar {np.max(err - np.maximum(1e-2, ulp))})"
        assert not big or rel <= 1e-3, f"rel-L2 {rel}"
    else:
        ulp = np.abs(O.bf16_bits_to_f32(O.f32_to_bf16_bits(y_ref.astype(np.float32)))).astype(np.float64) * 2.0 ** -7
        assert np.all(err <= ulp + 1e-2), f"max excess {np.max(err - ulp)}"
        assert not big or rel <= 5e-3, f"rel-L2 {rel}"
    return err.max(), rel


def rand_np(rng, shape, scale=1.0, dtype=np.float16):
    return (rng.standard_normal(shape) * scale).astype(dtype)


# ---------------------------------------------------------------------------
# quantizers / FWHT / dequant: bit-exact
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("wdt", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("n,k,n_out", [(128, 256, 0), (64, 1024, 9), (3, 96, 2)])
def test_quantize_group32_bitexact(hip, wdt, n, k, n_out):
    case(wdt=wdt, n=n, k=k, n_out=n_out)
    rng = np.random.default_rng(n * k + n_out)
    w32 = rand_np(rng, (n, k), 0.05, np.float32)
    w32[0, :32] = 2.5       # KAT groups (tests/test_quantizer.py:19-55)
    w32[1, :32] = -4.25
    w32[2, :32] = 0.0
    wt = cuda(w32, TDT[wdt])
    w_exact = wt.float().cpu().numpy()  # the values the GPU sees
    idx = np.sort(rng.permutation(k)[:n_out]).astype(np.int64) if n_out else None
    packed, scales, pz = C.compute_group32_quant(wt, outlier_idx=cuda(idx) if idx is not None else None)
    rp, rs, rz = O.compute_group32_quant(w_exact, idx)
    assert np.array_equal(host(packed), rp)
    assert np.array_equal(host(scales), rs)
    assert np.array_equal(host(pz), rz)


@pytest.mark.parametrize("had", [0, 128, 64])
@pytest.mark.parametrize("marlin", [True, False])
@pytest.mark.parametrize("outliers", [False, True])
def test_quantize_nf4_bitexact(hip, had, marlin, outliers):
    case(had=had, marlin=marlin, outliers=outliers)
    rng = np.random.default_rng(100 + had + marlin * 7 + outliers)
    n, k = 48, 1024
    w = rand_np(rng, (n, k), 0.02)
    w[3, 64:128] = 0  # zero block
    mask = rng.random((n, k)) < 0.005 if outliers else None
    q = C.quantize_nf4(cuda(w), blocksize=64, hadamard_block=had, outlier_mask=cuda(mask) if outliers else None,
                       marlin_layout=marlin)
    r = O.nf4_quantize(w, "float16", blocksize=64, hadamard_block=had, outlier_mask=mask, marlin=marlin)
    assert np.array_equal(host(q.packed), r["packed"])
    assert np.array_equal(host(q.absmax), r["absmax"])
    assert np.array_equal(host(q.rowptr), r["rowptr"])
    assert np.array_equal(host(q.col), r["col"])
    assert np.array_equal(host(q.val), r["val"])


def test_golden_format_b_quantizer(hip):
    g = np.load(os.path.join(HERE, "golden", "format_b_small.npz"))
    q = C.quantize_nf4(cuda(g["w"]), 64, 0, cuda(g["mask"]), True)
    assert np.array_equal(host(q.packed), g["packed"]) and np.array_equal(host(q.absmax), g["absmax"])
    assert np.array_equal(host(q.val), g["val"])
    qr = C.quantize_nf4(cuda(g["w_plain"]), 64, int(g["had"]), None, False)
    assert np.array_equal(host(qr.packed), g["packed_rot"]) and np.array_equal(host(qr.absmax), g["absmax_rot"])


@pytest.mark.parametrize("block", [2, 8, 128, 512, 1024])
@pytest.mark.parametrize("in_dt", ["float32", "float16", "bfloat16"])
def test_fwht_bitexact(hip, block, in_dt):
    case(block=block, in_dt=in_dt)
    rng = np.random.default_rng(block)
    x = rand_np(rng, (7, 2048), 1.0, np.float32)
    xt = cuda(x, TDT[in_dt])
    y = K.fwht_rows(xt, block, out_dtype=torch.float32)
    ref = O.rotate_blocks(xt.float().cpu().numpy(), block)
    assert np.array_equal(host(y), ref)


@pytest.mark.parametrize("out_dt", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("marlin", [True, False])
def test_dequant_format_a_bitexact(hip, out_dt, marlin):
    case(out_dt=out_dt, marlin=marlin)
    g = np.load(os.path.join(HERE, "golden", "format_a_small.npz"))
    z = cuda(g["zeros"])
    w = K.w4_dequant(cuda(g["packed"]), cuda(g["scales"]), z, out_dtype=TDT[out_dt], codebook="asym",
                     marlin_layout=marlin, outlier_idx=cuda(g["idx"]), outlier_w=cuda(g["ow"]))
    ref = O.apply_outlier_columns(O.dequant_group32(g["packed"], g["scales"], g["zeros"], marlin, out_dt),
                                  g["idx"], g["ow"], out_dt)
    assert np.array_equal(host(w), ref)
    if out_dt == "float16" and marlin:
        assert np.array_equal(host(w), g["w_deq"])  # golden fixture


@pytest.mark.parametrize("out_dt", ["float16", "bfloat16", "float32"])
def test_dequant_format_b_bitexact(hip, out_dt):
    case(out_dt=out_dt)
    g = np.load(os.path.join(HERE, "golden", "format_b_small.npz"))
    w = K.w4_dequant(cuda(g["packed"]), cuda(g["absmax"]), None, out_dtype=TDT[out_dt], codebook="nf4",
                     group_size=64, marlin_layout=True, outlier_idx=cuda(g["col"]), outlier_w=cuda(g["val"]),
                     outlier_rowptr=cuda(g["rowptr"]))
    ref = O.nf4_dequant(g["packed"], g["absmax"], True, out_dt, g["rowptr"], g["col"], g["val"])
    assert np.array_equal(host(w), ref)
    if out_dt == "float16":
        assert np.array_equal(host(w), g["w_eff16"])
    if out_dt == "bfloat16":
        assert np.array_equal(host(w), g["w_effbf"])


@pytest.mark.parametrize("out_dt", ["float16", "bfloat16", "float32"])
def test_dequant_every_code_and_scale(hip, out_dt):
    """Every NF4 code under every finite fp16 absmax (63488 blocks of 64, each holding the 16
    codes four times), dequantized by the row kernel: bit-exact against the oracle's fp32
    product and its rounding to the output dtype (one rounding to fp32, then one to 16 bits)."""
    case(out_dt=out_dt)
    bits = np.arange(65536, dtype=np.uint32)
    finite = bits[((bits >> 10) & 0x1F) != 0x1F].astype(np.uint16)  # 63488 patterns
    n, k = 248, 16384
    absmax = finite.view(np.float16).reshape(n, k // 64)
    codes = (np.arange(k) % 16).astype(np.uint8)
    packed = np.tile((codes[0::2] | (codes[1::2] << 4)).astype(np.uint8), (n, 1))  # natural nibble order
    ref = O.nf4_dequant(packed, absmax, False, out_dt)
    ops = K.QWeightOperands(cuda(packed), cuda(absmax), None, k, codebook="nf4", group_size=64, marlin_layout=False)
    out = torch.empty((n, k), dtype=TDT[out_dt], device="cuda")
    L.check("spectra_w4_dequant", lib_dequant(ops, out, k, out_dt))
    got = host(out)
    if out_dt == "float32":
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    else:
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def lib_dequant(ops, out, ldo, out_dt):
    return L.load().spectra_w4_dequant(ops.ptr(), out.data_ptr(), ldo, K._DT[TDT[out_dt]], K._stream(out.device))


@pytest.mark.parametrize("fmt,marlin,out_dt,n_out", [
    ("nf4", False, "float16", 0), ("nf4", True, "bfloat16", 0), ("nf4", False, "float32", 0),
    ("asym", True, "bfloat16", 16), ("asym", False, "float32", 150), ("asym", True, "float16", 150),
])
def test_dequant_row_and_general_kernels(hip, fmt, marlin, out_dt, n_out):
    """spectra_w4_dequant runs the row kernel (a 16-byte chunk of packed bytes per lane, the
    row's outliers stored over it afterwards) when rows and output are 16-byte aligned, and
    the general kernel otherwise (here an output row stride of K + 1): both bit-exact against
    the oracle, CSR and column outliers included.  K = 8192 spans several of the row kernel's
    segments, each storing its own outliers; 3% CSR outliers (about 245 a row) and 150 outlier
    columns exceed the 128 entries a lane group preloads, so the remainder loop runs too."""
    case(fmt=fmt, marlin=marlin, out_dt=out_dt, n_out=n_out)
    n, k = 120, 8192
    if fmt == "nf4":
        q, _ = _format_b(11, n, k, 0, ratio=0.03, marlin=marlin)
        ref = O.nf4_dequant(q["packed"], q["absmax"], marlin, out_dt, q["rowptr"], q["col"], q["val"])
        ops = K.QWeightOperands(cuda(q["packed"]), cuda(q["absmax"]), None, k, codebook="nf4", group_size=64,
                                marlin_layout=marlin, outlier_idx=cuda(q["col"]), outlier_w=cuda(q["val"]),
                                outlier_rowptr=cuda(q["rowptr"]))
    else:
        packed, scales, z, idx, ow, _ = _format_a(12, n, k, n_out)
        ref = O.apply_outlier_columns(O.dequant_group32(packed, scales, z, marlin, out_dt), idx, ow, out_dt)
        ops = K.QWeightOperands(cuda(packed), cuda(scales), cuda(z), k, codebook="asym", marlin_layout=marlin,
                                outlier_idx=cuda(idx), outlier_w=cuda(ow))
    lib = L.load()
    for ldo in (k, k + 1):
        out = torch.full((n, ldo), float("nan"), dtype=TDT[out_dt], device="cuda")
        L.check("spectra_w4_dequant", lib.spectra_w4_dequant(ops.ptr(), out.data_ptr(), ldo, K._DT[TDT[out_dt]],
                                                             K._stream(out.device)))
        assert np.array_equal(host(out[:, :k].contiguous()), ref), f"ldo={ldo}"


# ---------------------------------------------------------------------------
# Format A GEMV / GEMM (the reference's own test cases, tests/test_kernels.py:43-70)
# ---------------------------------------------------------------------------
def _format_a(seed, n, k, n_out, act="float16", ref_dtype=None):
    rng = np.random.default_rng(seed)
    w = rand_np(rng, (n, k), 1.0)
    idx = np.sort(rng.permutation(k)[:n_out]).astype(np.int64) if n_out else None
    packed, scales, pz = O.compute_group32_quant(w.astype(np.float32), idx)
    z = O.unpack_zeros(pz, k // 32)
    rd = ref_dtype or act
    w_deq = O.dequant_group32(packed, scales, z, True, rd)
    ow = None
    if n_out:
        ow = w[:, idx] if act == "float16" else O.round_to(w[:, idx].astype(np.float32), act)
        w_deq = O.apply_outlier_columns(w_deq, idx, ow, rd)
    return packed, scales, z, idx, ow, w_deq


@pytest.mark.parametrize("act", ["float16", "bfloat16"])
@pytest.mark.parametrize("m", [1, 2, 4, 8])
@pytest.mark.parametrize("n_out", [0, 16])
def test_format_a_reference_cases(hip, act, m, n_out):
    case(act=act, m=m, n_out=n_out)
    packed, scales, z, idx, ow, w_deq = _format_a(42, 128, 256, n_out, act)
    w_ref = w_deq if act == "float16" else _format_a(42, 128, 256, n_out, act, ref_dtype="float32")[-1]
    rng = np.random.default_rng(m)
    x = rand_np(rng, (m, 256), 1.0, np.float32)
    x = O.round_to(x, act)
    xt = cuda(x, TDT[act])
    y_ref = O.format_a_linear_ref(x, act, w_ref, w_dtype="float16" if act == "float16" else "float32")
    kw = dict(outlier_idx=cuda(idx) if n_out else None, outlier_w=cuda(ow, TDT[act]) if n_out else None,
              marlin_layout=True)
    if m == 1:
        y = K.fused_w4a16_gemv_hdsq(xt, cuda(packed), cuda(scales), cuda(z), **kw)
    else:
        y = K.batched_w4a16_gemm(xt, cuda(packed), cuda(scales), cuda(z), **kw)
    assert y.dtype == TDT[act] and y.shape == (m, 128)
    # the reference's own bar (tests/test_kernels.py:48-49; it tests fp16 only) ...
    if act == "float16":
        assert np.abs(y.float().cpu().double().numpy() - y_ref).max() <= 0.05
    # ... and this build's
    check_y(y, y_ref, TDT[act])


@pytest.mark.parametrize("m", [1, 3, 4, 5, 16, 33])
@pytest.mark.parametrize("marlin", [True, False])
def test_format_a_gemv_gemm_with_bias(hip, m, marlin):
    case(m=m, marlin=marlin)
    rng = np.random.default_rng(m + 10 * marlin)
    n, k = 200, 1536
    w = rand_np(rng, (n, k), 0.05)
    idx = np.sort(rng.permutation(k)[:20]).astype(np.int64)
    packed, scales, pz = O.compute_group32_quant(w.astype(np.float32), idx)
    if not marlin:  # same codes, even-odd nibble order
        packed = O.pack_nibbles(O.unpack_nibbles(packed, True), False)
    z = O.unpack_zeros(pz, k // 32)
    ow = w[:, idx]
    w_deq = O.apply_outlier_columns(O.dequant_group32(packed, scales, z, marlin, "float16"), idx, ow, "float16")
    b = rand_np(rng, (n,), 0.5)
    x = rand_np(rng, (m, k), 1.0)
    y_ref = O.format_a_linear_ref(x, "float16", w_deq, bias=b)
    lin = SpectraFusedLinear(k, n, 32, has_bias=True, marlin_layout=marlin).cuda()
    lin.set_weights(cuda(packed), cuda(scales), cuda(z), bias=cuda(b), outlier_idx=cuda(idx), outlier_weight=cuda(ow),
                    marlin_layout=marlin)
    y = lin(cuda(x))
    check_y(y, y_ref, torch.float16)


# ---------------------------------------------------------------------------
# Format B (NF4 + Hadamard + CSR)
# ---------------------------------------------------------------------------
def _format_b(seed, n, k, had, ratio=0.005, marlin=True, scale=0.02):
    rng = np.random.default_rng(seed)
    w = rand_np(rng, (n, k), scale)
    mask = rng.random((n, k)) < ratio
    w[mask] = (np.abs(rng.standard_normal(mask.sum())) * 0.2 * np.sign(rng.standard_normal(mask.sum()))).astype(
        np.float16)
    q = O.nf4_quantize(w, "float16", 64, 0, mask if ratio > 0 else None, marlin)
    return q, rng


@pytest.mark.parametrize("act", ["float16", "bfloat16"])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("had", [0, 128])
@pytest.mark.parametrize("marlin", [True, False])
def test_format_b_gemv(hip, act, m, had, marlin):
    case(act=act, m=m, had=had, marlin=marlin)
    q, rng = _format_b(m * 3 + had + marlin, 257, 3072, had, marlin=marlin)
    rd = act if act == "float16" else "float32"
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], marlin, rd, q["rowptr"], q["col"], q["val"])
    x = O.round_to(rand_np(rng, (m, 3072), 1.0, np.float32), act)
    b = rand_np(rng, (257,), 0.1)
    y_ref = O.linear_ref(x, act, w_eff, rd, hadamard_block=had, bias=b)
    y = K.fused_w4a16_gemv_hdsq(cuda(x, TDT[act]), cuda(q["packed"]), cuda(q["absmax"]), None, bias=cuda(b),
                                outlier_idx=cuda(q["col"]), outlier_w=cuda(q["val"]), marlin_layout=marlin,
                                codebook="nf4", group_size=64, hadamard_block=had, outlier_rowptr=cuda(q["rowptr"]))
    check_y(y, y_ref, TDT[act])


def test_golden_format_b_gemv(hip):
    g = np.load(os.path.join(HERE, "golden", "format_b_small.npz"))
    y = K.fused_w4a16_gemv_hdsq(cuda(g["x"]), cuda(g["packed"]), cuda(g["absmax"]), None, outlier_idx=cuda(g["col"]),
                                outlier_w=cuda(g["val"]), marlin_layout=True, codebook="nf4", group_size=64,
                                hadamard_block=int(g["had"]), outlier_rowptr=cuda(g["rowptr"]))
    check_y(y, g["y_ref"], torch.float16)


@pytest.mark.parametrize("n,k", [(1, 1024), (33, 256), (100, 1536), (513, 4096), (64, 8192), (40, 14336)])
def test_format_b_gemv_shapes(hip, n, k):
    case(n=n, k=k)
    q, rng = _format_b(n + k, n, k, 128)
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], True, "float16", q["rowptr"], q["col"], q["val"])
    x = rand_np(rng, (1, k), 1.0)
    y_ref = O.linear_ref(x, "float16", w_eff, "float16", hadamard_block=128)
    y = K.fused_w4a16_gemv_hdsq(cuda(x[0]), cuda(q["packed"]), cuda(q["absmax"]), None, outlier_idx=cuda(q["col"]),
                                outlier_w=cuda(q["val"]), marlin_layout=True, codebook="nf4", hadamard_block=128,
                                outlier_rowptr=cuda(q["rowptr"]))
    assert y.shape == (n,)
    check_y(y.unsqueeze(0), y_ref, torch.float16)


def _stream_operands(seed, n, k, had, marlin):
    """Format B operands with 0.5% outliers plus one row holding an outlier in every fourth
    column (far more entries than a lane group has lanes)."""
    rng = np.random.default_rng(seed)
    w = rand_np(rng, (n, k), 0.02)
    mask = rng.random((n, k)) < 0.005
    mask[5, ::4] = True
    w[mask] = (rng.standard_normal(mask.sum()) * 0.2).astype(np.float16)
    q = O.nf4_quantize(w, "float16", 64, 0, mask, marlin)
    return q, rng


@pytest.mark.parametrize("k,had,marlin,act,bias", [
    (5120, 128, True, "float16", True),    # K / 1024 = 5: no row-owning plan
    (6144, 128, False, "bfloat16", False),
    (5120, 0, False, "float16", False),
    (1024, 16, True, "float16", True),     # Hadamard blocks the row-owning kernel does not take
    (1024, 32, False, "bfloat16", True),
    (1024, 64, True, "bfloat16", False),
    (1024, 256, False, "float16", False),
    (1024, 512, True, "float16", True),
])
def test_stream_gemv_shapes(hip, k, had, marlin, act, bias):
    """One-row shapes served by the streaming GEMV kernel (the M=1 NF4 shapes the row-owning
    kernel's plan does not cover): fp16 / bf16 activations, both nibble orders, Hadamard
    blocks 16-512, bias, and a row with more CSR entries than lanes, against the oracle."""
    case(k=k, had=had, marlin=marlin, act=act, bias=bias)
    n = 700
    q, rng = _stream_operands(k + had + marlin, n, k, had, marlin)
    rd = act if act == "float16" else "float32"
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], marlin, rd, q["rowptr"], q["col"], q["val"])
    x = O.round_to(rand_np(rng, (1, k), 1.0, np.float32), act)
    b = rand_np(rng, (n,), 0.1) if bias else None
    y_ref = O.linear_ref(x, act, w_eff, rd, hadamard_block=had, bias=b)
    y = K.fused_w4a16_gemv_hdsq(cuda(x, TDT[act]), cuda(q["packed"]), cuda(q["absmax"]), None,
                                bias=cuda(b) if bias else None, outlier_idx=cuda(q["col"]), outlier_w=cuda(q["val"]),
                                marlin_layout=marlin, codebook="nf4", group_size=64, hadamard_block=had,
                                outlier_rowptr=cuda(q["rowptr"]))
    check_y(y, y_ref, TDT[act])


@pytest.mark.parametrize("n,k,had,marlin,act,prologue", [
    (40000, 3072, 128, True, "float16", None),      # lane groups of 32, passes of 32 rows
    (45000, 4096, 0, False, "bfloat16", None),      # lane groups of 64, passes of 16 rows
    (41000, 2048, 128, True, "float16", "rmsnorm"),
])
def test_multipass_gemv_shapes(hip, n, k, had, marlin, act, prologue):
    """One-row shapes with more rows per CU (150-180) than the row-owning plan holds, served
    by the multi-pass row kernel (the lm_head's): passes with the next pass's loads in flight,
    partial last passes, the last workgroup's shorter row range, a row with more CSR entries
    than lanes, and its greedy pick.  The operands come from the GPU quantizer; its codes and
    the GPU dequant are pinned bit for bit to the oracle on sampled rows (pass and workgroup
    boundaries, the dense-outlier row), then y is checked against the oracle product on that
    W_eff."""
    case(n=n, k=k, had=had, marlin=marlin, act=act, prologue=prologue)
    g = torch.Generator().manual_seed(n + k)
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    mask = torch.rand(n, k, generator=g) < 0.005
    mask[5, ::4] = True
    w[mask] = (torch.randn(int(mask.sum()), generator=g) * 0.2).half()
    q = C.quantize_nf4(w.cuda(), 64, 0, mask.cuda(), marlin)
    rd = act if act == "float16" else "float32"
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    R = -(-n // ncu)
    pr = 32 if (k // 1024) % 2 else 16  # rows per pass: 8 waves x 2 rows x (64 / lanes per group)
    rows = sorted({0, 5, pr - 1, pr, R - 1, R, R + pr, (n // R) * R - 1, (n // R) * R, n - 1})
    rows = np.array([r for r in rows if r < n])
    sub = O.nf4_quantize(w.numpy()[rows], "float16", 64, 0, mask.numpy()[rows], marlin)
    assert np.array_equal(host(q.packed)[rows], sub["packed"]) and np.array_equal(host(q.absmax)[rows], sub["absmax"])
    w_eff_t = K.w4_dequant(q.packed, q.absmax, None, out_dtype=TDT[rd], codebook="nf4", marlin_layout=marlin,
                           outlier_idx=q.col, outlier_w=q.val, outlier_rowptr=q.rowptr)
    w_eff = host(w_eff_t)
    del w_eff_t
    ref_rows = O.nf4_dequant(sub["packed"], sub["absmax"], marlin, rd, sub["rowptr"], sub["col"], sub["val"])
    assert np.array_equal(w_eff[rows], ref_rows)
    ops = K.QWeightOperands(q.packed, q.absmax, None, k, codebook="nf4", group_size=64, hadamard_block=had,
                            marlin_layout=marlin, outlier_idx=q.col, outlier_w=q.val, outlier_rowptr=q.rowptr)
    slots = K.argmax_slots()
    token = torch.zeros(1, dtype=torch.int64, device="cuda")
    rng = np.random.default_rng(n)
    if prologue == "rmsnorm":
        h = (rng.standard_normal((1, k)) * 3).astype(np.float16)
        nw = (rng.random(k) + 0.5).astype(np.float16)
        y = K.w4a16_gemv_fused(ops, cuda(h), prologue="rmsnorm", norm_weight=cuda(nw), eps=1e-5, argmax_key=slots)
        hf = h.astype(np.float64)
        x, xdt = (hf / np.sqrt((hf * hf).mean() + 1e-5) * nw.astype(np.float64)).astype(np.float32), "float32"
    else:
        x, xdt = O.round_to(rand_np(rng, (1, k), 1.0, np.float32), act), act
        if act == "float16":
            y = K.w4a16_gemv_fused(ops, cuda(x, TDT[act]), argmax_key=slots)
        else:  # (the fused entry's pick takes fp16 activations)
            y = K.w4a16_linear(ops, cuda(x, TDT[act]))
    check_y(y, O.linear_ref(x, xdt, w_eff, rd, hadamard_block=had), TDT[act])
    if act == "float16":
        K.greedy_finish(slots, token)
        assert int(token) == int(torch.argmax(y.float().reshape(-1)))


@pytest.mark.parametrize("k,had,marlin,prologue", [(6144, 128, True, "rmsnorm"), (5120, 128, False, "rmsnorm"),
                                                   (5120, 128, True, "silu_mul"), (1024, 64, False, "silu_mul")])
def test_stream_gemv_prologues(hip, k, had, marlin, prologue):
    """The streaming GEMV kernel's fused prologues (RMSNorm of the residual stream, SiLU-mul of
    a fused gate_up row) and residual epilogue against the oracle: RMSNorm in fp64, the SiLU-mul
    activations taken from the separate kernel (the prologue is bit-identical to it); the
    residual add bit-identical to the separate fp16 add."""
    case(k=k, had=had, marlin=marlin, prologue=prologue)
    n = 900
    q, rng = _stream_operands(k + had, n, k, had, marlin)
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], marlin, "float16", q["rowptr"], q["col"], q["val"])
    ops = K.QWeightOperands(cuda(q["packed"]), cuda(q["absmax"]), None, k, codebook="nf4", group_size=64,
                            hadamard_block=had, marlin_layout=marlin, outlier_idx=cuda(q["col"]),
                            outlier_w=cuda(q["val"]), outlier_rowptr=cuda(q["rowptr"]))
    if prologue == "rmsnorm":
        h = (rng.standard_normal((1, k)) * 3).astype(np.float16)
        nw = (rng.random(k) + 0.5).astype(np.float16)
        y = K.w4a16_gemv_fused(ops, cuda(h), prologue="rmsnorm", norm_weight=cuda(nw), eps=1e-5)
        hf = h.astype(np.float64)
        x_eff = (hf / np.sqrt((hf * hf).mean() + 1e-5) * nw.astype(np.float64)).astype(np.float32)
        check_y(y, O.linear_ref(x_eff, "float32", w_eff, "float16", hadamard_block=had), torch.float16)
        return
    gu = cuda((rng.standard_normal((1, 2 * k)) * 2).astype(np.float16))
    act = K.silu_mul(gu)
    y = K.w4a16_gemv_fused(ops, gu, prologue="silu_mul")
    check_y(y, O.linear_ref(host(act), "float16", w_eff, "float16", hadamard_block=had), torch.float16)
    res = cuda((rng.standard_normal((1, n)) * 4).astype(np.float16))
    expect = res + y
    out = K.w4a16_gemv_fused(ops, gu, prologue="silu_mul", residual=res, out=res)
    assert out.data_ptr() == res.data_ptr() and torch.equal(res, expect)


@pytest.mark.parametrize("act", ["float16", "bfloat16"])
@pytest.mark.parametrize("m", [5, 16, 64, 130])
def test_format_b_gemm(hip, act, m):
    case(act=act, m=m)
    n, k = 320, 2048
    q, rng = _format_b(m, n, k, 128, ratio=0.01)
    rd = act if act == "float16" else "float32"
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], True, rd, q["rowptr"], q["col"], q["val"])
    x = O.round_to(rand_np(rng, (m, k), 1.0, np.float32), act)
    y_ref = O.linear_ref(x, act, w_eff, rd, hadamard_block=128)
    y = K.batched_w4a16_gemm(cuda(x, TDT[act]), cuda(q["packed"]), cuda(q["absmax"]), None,
                             outlier_idx=cuda(q["col"]), outlier_w=cuda(q["val"]), marlin_layout=True, codebook="nf4",
                             hadamard_block=128, outlier_rowptr=cuda(q["rowptr"]))
    check_y(y, y_ref, TDT[act])


@pytest.mark.parametrize("act,bias_dt,ldo_pad,ratio", [
    ("float16", "float16", 0, 0.01),    # the library GEMM, bias in its epilogue
    ("float16", "float32", 0, 0.01),
    ("bfloat16", "bfloat16", 0, 0.01),
    ("bfloat16", "float32", 0, 0.01),
    ("float16", "float16", 0, 0.08),    # ~160 outliers a row: more than a lane group preloads
    ("float16", "float16", 3, 0.01),    # row stride not a multiple of 8: served by the MFMA family
])
def test_prefill_library_path(hip, act, bias_dt, ldo_pad, ratio):
    """From PREFILL_LIBRARY_MIN_M rows the dequantized weights run on the library GEMM in the
    activations' dtype (the reference kernel's operand type, kernels.py:238-242), fp32
    accumulation, the output in that dtype.  The Hadamard rotation goes onto the weights there
    (x_rot . W_eff^T = x . (W_eff H / sqrt(b))^T, H symmetric): the oracle's reference takes
    the activations as given and the oracle's fp32 W_eff rotated blockwise and rounded to the
    activations' dtype.  With bias, one row 300 times larger than the others (on the library
    path; the strided output runs on the MFMA family, against rotated activations rounded
    to its fp16 operands, its rows unit-scale)."""
    case(act=act, bias_dt=bias_dt, ldo_pad=ldo_pad, ratio=ratio)
    m, n, k = 1100, 520, 2048
    q, rng = _format_b(7 + ldo_pad, n, k, 128, ratio=ratio)
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], True, act, q["rowptr"], q["col"], q["val"])
    x = rand_np(rng, (m, k), 1.0, np.float32)
    if ldo_pad == 0:
        x[7] *= 300.0
    x = O.round_to(x, act)
    b = O.round_to((rng.standard_normal(n) * 0.5).astype(np.float32), bias_dt)
    if ldo_pad == 0:  # the library path, here with the rotation on the weights
        assert K.prefill_rotates_weights(m, n, k, 128)
        w_rot = O.round_to(O.rotate_blocks(O.nf4_dequant(q["packed"], q["absmax"], True, "float32", q["rowptr"],
                                                         q["col"], q["val"]), 128), act)
        y_ref = O.linear_ref(x, act, w_rot, act, bias=b, bias_dtype=bias_dt)
    else:
        y_ref = O.linear_ref(x, act, w_eff, act, hadamard_block=128, bias=b, bias_dtype=bias_dt, round_x_to=act)
    ops = K.QWeightOperands(cuda(q["packed"]), cuda(q["absmax"]), None, k, codebook="nf4", group_size=64,
                            hadamard_block=128, marlin_layout=True, outlier_idx=cuda(q["col"]),
                            outlier_w=cuda(q["val"]), outlier_rowptr=cuda(q["rowptr"]), bias=cuda(b, TDT[bias_dt]))
    y = torch.full((m, n + ldo_pad), float("nan"), dtype=TDT[act], device="cuda")[:, :n]
    K._run_linear(ops, cuda(x, TDT[act]), y, "gemm")
    check_y(y, y_ref, TDT[act])


def test_prefill_library_path_format_a(hip):
    """The library path on a Format A weight (groups of 32, dense outlier columns)."""
    case(m=1024, n=384, k=1536)
    packed, scales, z, idx, ow, w_deq = _format_a(31, 384, 1536, 16)
    rng = np.random.default_rng(32)
    x = O.round_to(rand_np(rng, (1024, 1536), 1.0, np.float32), "float16")
    y_ref = O.linear_ref(x, "float16", w_deq, "float16")
    y = K.batched_w4a16_gemm(cuda(x), cuda(packed), cuda(scales), cuda(z), outlier_idx=cuda(idx), outlier_w=cuda(ow),
                             marlin_layout=True)
    check_y(y, y_ref, torch.float16)


@pytest.mark.parametrize("act", ["float16", "bfloat16"])
@pytest.mark.parametrize("m", [2, 3, 5, 8, 13, 16])
@pytest.mark.parametrize("n,k,had,marlin", [
    (257, 3072, 128, True),     # one 16-row tile per workgroup, 3 chunks per wave
    (4112, 1024, 0, False),     # two tiles per workgroup, plain nibble order, no rotation
    (8200, 1024, 128, True),    # four tiles per workgroup, ragged last workgroup
    (48, 14336, 128, True),     # two rounds of 7 chunks per wave
    (40, 640, 64, True),        # five waves of one chunk
])
def test_format_b_small_batch(hip, act, m, n, k, had, marlin):
    """The MFMA small-batch family (2 <= M <= 16) through batched_w4a16_gemm, with bias."""
    case(act=act, m=m, n=n, k=k, had=had, marlin=marlin)
    q, rng = _format_b(m * 7 + n + k, n, k, had, marlin=marlin)
    rd = act if act == "float16" else "float32"
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], marlin, rd, q["rowptr"], q["col"], q["val"])
    x = O.round_to(rand_np(rng, (m, k), 1.0, np.float32), act)
    b = rand_np(rng, (n,), 0.1)
    y_ref = O.linear_ref(x, act, w_eff, rd, hadamard_block=had, bias=b)
    lin = SpectraFusedLinear(k, n, 64, has_bias=True, codebook="nf4", hadamard_block=had, marlin_layout=marlin).cuda()
    lin.set_weights(cuda(q["packed"]), cuda(q["absmax"]), None, bias=cuda(b), outlier_idx=cuda(q["col"]),
                    outlier_weight=cuda(q["val"]), marlin_layout=marlin, outlier_rowptr=cuda(q["rowptr"]))
    y = K.batched_w4a16_gemm(cuda(x, TDT[act]), cuda(q["packed"]), cuda(q["absmax"]), None,
                             outlier_idx=cuda(q["col"]), outlier_w=cuda(q["val"]), marlin_layout=marlin,
                             codebook="nf4", hadamard_block=had, outlier_rowptr=cuda(q["rowptr"]))
    y = y + cuda(b, TDT[act])  # batched_w4a16_gemm has no bias (kernels.py:333-341): engine.py:122-123 adds it
    check_y(y, y_ref, TDT[act])
    if m > 4:  # the module dispatch sends m > 4 to the same family, bias in the kernel epilogue
        check_y(lin(cuda(x, TDT[act])), y_ref, TDT[act])


@pytest.mark.parametrize("m", [1, 3, 5, 16])
def test_nf4_block32_module_and_embedding(hip, m):
    """NF4 with 32-element blocks (absmax [N, K/32]) through the modules built with group_size=32:
    the GPU quantizer bit-exact against the oracle, the linear (one row: the GEMV; more: the
    small-batch / GEMM families) against the oracle's product, the embedding rows bit-exact."""
    case(m=m, block=32)
    n, k, had = 384, 3072, 128
    rng = np.random.default_rng(320 + m)
    w = rand_np(rng, (n, k), 0.02)
    mask = rng.random((n, k)) < 0.005
    w[mask] = (rng.standard_normal(mask.sum()) * 0.2).astype(np.float16)
    ref = O.nf4_quantize(w, "float16", 32, 0, mask, True)
    q = C.quantize_nf4(cuda(w), 32, 0, cuda(mask), True)
    assert q.absmax.shape == (n, k // 32)
    assert np.array_equal(host(q.packed), ref["packed"]) and np.array_equal(host(q.absmax), ref["absmax"])
    w_eff = O.nf4_dequant(ref["packed"], ref["absmax"], True, "float16", ref["rowptr"], ref["col"], ref["val"],
                          blocksize=32)
    lin = SpectraFusedLinear(k, n, 32, codebook="nf4", hadamard_block=had, marlin_layout=True).cuda()
    lin.set_weights(q.packed, q.absmax, None, outlier_idx=q.col, outlier_weight=q.val, marlin_layout=True,
                    outlier_rowptr=q.rowptr)
    x = rand_np(rng, (m, k), 1.0)
    check_y(lin(cuda(x)), O.linear_ref(x, "float16", w_eff, "float16", hadamard_block=had), torch.float16)
    emb = SpectraFusedEmbedding(n, k, 32, True, codebook="nf4").cuda()
    emb.set_weights(q.packed, q.absmax, None, q.col, q.val, True, outlier_rowptr=q.rowptr)
    ids = torch.tensor([0, n - 1, 17, 200], device="cuda")
    assert np.array_equal(host(emb(ids)), w_eff[ids.cpu().numpy()])


@pytest.mark.parametrize("nnz", [1, 3, 5])
def test_tiny_csr(hip, nnz):
    """CSR arrays shorter than one 4-entry load group (read per entry, never as a group)."""
    n, k = 64, 256
    q, rng = _format_b(nnz, n, k, 0, ratio=0.0)
    mask = np.zeros((n, k), bool)
    mask.reshape(-1)[rng.permutation(n * k)[:nnz]] = True
    w = rand_np(rng, (n, k), 0.02)
    qq = O.nf4_quantize(w, "float16", 64, 0, mask, True)
    w_eff = O.nf4_dequant(qq["packed"], qq["absmax"], True, "float16", qq["rowptr"], qq["col"], qq["val"])
    for m in (1, 8):
        case(nnz=nnz, m=m)
        x = rand_np(rng, (m, k), 1.0)
        y_ref = O.linear_ref(x, "float16", w_eff, "float16")
        fn = K.fused_w4a16_gemv_hdsq if m <= 4 else K.batched_w4a16_gemm
        # exactly-sized side tensors: no slack after the last entry
        col = torch.from_numpy(qq["col"].copy()).cuda()
        val = torch.from_numpy(qq["val"].copy()).cuda()
        y = fn(cuda(x), cuda(qq["packed"]), cuda(qq["absmax"]), None, outlier_idx=col, outlier_w=val,
               marlin_layout=True, codebook="nf4", outlier_rowptr=cuda(qq["rowptr"]))
        check_y(y, y_ref, torch.float16)


def test_dense_outlier_rows(hip):
    """A row with many outliers in one 64-wide tile exercises the GEMM's slow path and
    the GEMV's beyond-register entries."""
    n, k = 130, 1024
    q, rng = _format_b(5, n, k, 0, ratio=0.0)
    mask = np.zeros((n, k), bool)
    mask[7, 64:128] = True          # 64 outliers in one tile
    mask[100, :] = True             # a fully dense row
    mask[129, ::3] = True
    w = rand_np(rng, (n, k), 0.02)
    qq = O.nf4_quantize(w, "float16", 64, 0, mask, True)
    w_eff = O.nf4_dequant(qq["packed"], qq["absmax"], True, "float16", qq["rowptr"], qq["col"], qq["val"])
    for m in (1, 4, 20):
        case(m=m)
        x = rand_np(rng, (m, k), 1.0)
        y_ref = O.linear_ref(x, "float16", w_eff, "float16")
        fn = K.fused_w4a16_gemv_hdsq if m <= 4 else K.batched_w4a16_gemm
        y = fn(cuda(x), cuda(qq["packed"]), cuda(qq["absmax"]), None, outlier_idx=cuda(qq["col"]),
               outlier_w=cuda(qq["val"]), marlin_layout=True, codebook="nf4", outlier_rowptr=cuda(qq["rowptr"]))
        check_y(y, y_ref, torch.float16)


@pytest.mark.parametrize("m", [40, 300])
def test_gemm_split_k_outliers_across_splits(hip, m):
    """Few output tiles -> the GEMM splits K (8 splits of 512 here); outlier runs that cross
    split boundaries, a fully dense row and a bias must land in exactly one split each."""
    case(m=m)
    n, k = 256, 4096
    rng = np.random.default_rng(m)
    w = rand_np(rng, (n, k), 0.02)
    mask = rng.random((n, k)) < 0.005
    mask[3, 480:560] = True          # crosses the boundary at k = 512
    mask[200, 1000:1100] = True      # crosses k = 1024
    mask[77, :] = True               # every column
    qq = O.nf4_quantize(w, "float16", 64, 0, mask, True)
    w_eff = O.nf4_dequant(qq["packed"], qq["absmax"], True, "float16", qq["rowptr"], qq["col"], qq["val"])
    x = rand_np(rng, (m, k), 1.0)
    b = rand_np(rng, (n,), 0.5)
    y_ref = O.linear_ref(x, "float16", w_eff, "float16", hadamard_block=128, bias=b)
    lin = SpectraFusedLinear(k, n, 64, has_bias=True, codebook="nf4", hadamard_block=128).cuda()
    lin.set_weights(cuda(qq["packed"]), cuda(qq["absmax"]), None, bias=cuda(b), outlier_idx=cuda(qq["col"]),
                    outlier_weight=cuda(qq["val"]), marlin_layout=True, outlier_rowptr=cuda(qq["rowptr"]))
    y = lin(cuda(x))
    check_y(y, y_ref, torch.float16)
    assert torch.equal(lin(cuda(x)), y)  # the split partials are summed in a fixed order


# ---------------------------------------------------------------------------
# BASELINE shapes (configs 1-3) at full size, M=1..16, against the oracle
# ---------------------------------------------------------------------------
def _sampled_rows_bitexact(q, w, mask, out_dtype):
    """Rows 0, 1, N/2 and N-1 of a full-size quantization: packed codes, absmax, CSR and
    W_eff (dequantized by the HIP kernel in ``out_dtype``) bit-identical to the oracle's
    quantizer and dequant run on the same source rows."""
    n = w.shape[0]
    rows = np.array([0, 1, n // 2, n - 1])
    wn = w.numpy()[rows]
    mk = mask.numpy()[rows] if mask is not None else None
    sub = O.nf4_quantize(wn, "float16", 64, 0, mk, True)
    assert np.array_equal(host(q.packed)[rows], sub["packed"]) and np.array_equal(host(q.absmax)[rows], sub["absmax"])
    rp = host(q.rowptr).astype(np.int64)
    for i, r in enumerate(rows):
        assert np.array_equal(host(q.col)[rp[r]:rp[r + 1]], sub["col"][sub["rowptr"][i]:sub["rowptr"][i + 1]])
        assert np.array_equal(host(q.val)[rp[r]:rp[r + 1]].view(np.uint16),
                              sub["val"][sub["rowptr"][i]:sub["rowptr"][i + 1]].view(np.uint16))
    w_eff = K.w4_dequant(q.packed, q.absmax, None, out_dtype=TDT[out_dtype], codebook="nf4", marlin_layout=True,
                         outlier_idx=q.col if q.col.numel() else None, outlier_w=q.val if q.col.numel() else None,
                         outlier_rowptr=q.rowptr if q.col.numel() else None)
    ref = O.nf4_dequant(sub["packed"], sub["absmax"], True, out_dtype, sub["rowptr"], sub["col"], sub["val"])
    assert np.array_equal(host(w_eff)[rows], ref)  # bf16 compares as bit patterns on both sides
    return w_eff


@pytest.mark.parametrize("name,n,k,had,ratio,ms", [
    ("cfg1", 4096, 4096, 0, 0.0, (1,)),
    ("cfg2_qkv", 5120, 3072, 128, 0.005, (1,)),
    ("cfg2_down", 3072, 8192, 128, 0.005, (1, 4, 8, 16)),
    ("cfg3_gate_up", 16384, 3072, 128, 0.005, (2, 4, 8, 16)),
])
def test_baseline_shapes(hip, name, n, k, had, ratio, ms):
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    mask = None
    if ratio:
        nnz = int(round(ratio * n * k))
        pos = torch.randperm(n * k, generator=g)[:nnz]
        vals = (torch.randn(nnz, generator=g).abs() * 0.2 * torch.sign(torch.randn(nnz, generator=g))).half()
        w.view(-1)[pos] = vals
        mask = torch.zeros(n * k, dtype=torch.bool)
        mask[pos] = True
        mask = mask.view(n, k)
    q = C.quantize_nf4(w.cuda(), 64, 0, mask.cuda() if mask is not None else None, True)
    # the full-size quantizer and dequant agree bit for bit with the oracle on sampled rows
    _sampled_rows_bitexact(q, w, mask, "float16")
    w_eff_t = K.w4_dequant(q.packed, q.absmax, None, codebook="nf4", marlin_layout=True,
                           outlier_idx=q.col if q.col.numel() else None, outlier_w=q.val if q.col.numel() else None,
                           outlier_rowptr=q.rowptr if q.col.numel() else None)
    w_eff = O.nf4_dequant(host(q.packed), host(q.absmax), True, "float16", host(q.rowptr), host(q.col), host(q.val))
    assert np.array_equal(host(w_eff_t), w_eff)
    for m in ms:
        case(name=name, m=m)
        x = (torch.randn(m, k, generator=g)).half()
        y_ref = O.linear_ref(x.numpy(), "float16", w_eff, "float16", hadamard_block=had)
        q.hadamard_block = had  # the synthetic matrix is the stored (rotated-basis) weight
        kw = q.kernel_kwargs()
        col, val = q.outliers()
        fn = K.fused_w4a16_gemv_hdsq if m <= 4 else K.batched_w4a16_gemm
        y = fn(x.cuda(), q.packed, q.absmax, None, outlier_idx=col, outlier_w=val, marlin_layout=True, **kw)
        err, rel = check_y(y, y_ref, torch.float16)
        print(f"{name} m={m}: max-abs {err:.3e} rel-L2 {rel:.3e}", flush=True)
        if 2 <= m <= 4:  # the GEMV entry itself (the module dispatch sends wide shapes to the small-batch family)
            ops = K.QWeightOperands(q.packed, q.absmax, None, k, marlin_layout=True, outlier_idx=col, outlier_w=val,
                                    **kw)
            yg = torch.empty(m, n, dtype=torch.float16, device="cuda")
            K._run_linear(ops, x.cuda(), yg, "gemv")
            err, rel = check_y(yg, y_ref, torch.float16)
            print(f"{name} m={m} GEMV entry: max-abs {err:.3e} rel-L2 {rel:.3e}", flush=True)


@pytest.mark.parametrize("m,k,n", [
    (448, 4096, 14336),   # hand-written GEMM: 256-wide tiles, K split in two
    (2048, 4096, 14336),  # cfg4's first GEMM at full size (library path)
    (2048, 14336, 4096),  # cfg4's second GEMM at full size (library path)
    (384, 8192, 3072),    # hand-written GEMM: 128-wide tiles, K split in five
    (512, 8192, 3072),    # the library path's first row count
])
def test_prefill_gemm_against_torch_fp32(hip, m, k, n):
    """cfg4 shape class: fp32 torch reference on the GPU built from the bit-exact dequant
    and FWHT kernels (0.5% CSR outliers, bf16 activations).  Below PREFILL_LIBRARY_MIN_M rows the
    hand-written MFMA GEMM (fp16 operands, per-row scale) is held to the fp32 operands; from
    there the library GEMM computes on bf16 operands like the reference's kernel
    (kernels.py:238-242).  With the rotation on the weights (prefill_rotates_weights) the
    reference product takes the activations as given and the fp32 W_eff rotated blockwise (the
    HIP FWHT, pinned to the oracle) and rounded to bf16; otherwise W_eff and the rotated
    activations rounded to bf16."""
    case(m=m, k=k, n=n)
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    nnz = int(round(0.005 * n * k))
    pos = torch.randperm(n * k, generator=g)[:nnz]
    mask = torch.zeros(n * k, dtype=torch.bool)
    mask[pos] = True
    w.view(-1)[pos] = (torch.randn(nnz, generator=g) * 0.2).half()
    q = C.quantize_nf4(w.cuda(), 64, 0, mask.view(n, k).cuda(), True)
    x = torch.randn(m, k, generator=g).bfloat16().cuda()
    y = K.batched_w4a16_gemm(x, q.packed, q.absmax, None, outlier_idx=q.col, outlier_w=q.val, marlin_layout=True,
                             **q.kernel_kwargs() | dict(hadamard_block=128))
    # the reference's operands are the oracle's on sampled rows: quantized codes, CSR and W_eff
    # (float32 and bf16) bit for bit, and the rotated activations
    w_eff = _sampled_rows_bitexact(q, w, mask.view(n, k), "float32")
    w_bf = _sampled_rows_bitexact(q, w, mask.view(n, k), "bfloat16")
    x_rot = K.fwht_rows(x, 128, out_dtype=torch.float32)
    xr = np.array([0, m // 2, m - 1])
    assert np.array_equal(host(x_rot)[xr], O.rotate_blocks(O.to_f32(host(x)[xr], "bfloat16"), 128))
    if K.prefill_rotates_weights(m, n, k, 128):
        w_eff = K.fwht_rows(w_eff.float(), 128, out_dtype=torch.float32).bfloat16()
        x_rot = x.float()
    elif m >= K.PREFILL_LIBRARY_MIN_M:
        w_eff, x_rot = w_bf.float(), x_rot.bfloat16().float()
    y_t = (x_rot @ w_eff.float().T).double().cpu().numpy()
    check_y(y, y_t, torch.bfloat16)


@pytest.mark.parametrize("act", ["float16", "bfloat16"])
@pytest.mark.parametrize("n,k,m,had,marlin,bias", [
    (3072, 8192, 2, 128, True, False),    # cfg3 down_proj, one row per lane group
    (3072, 8192, 4, 128, True, True),
    (8448, 3072, 3, 128, True, False),    # K = 3072 past 32 rows per workgroup (cfg3 gate_up's
    (8448, 3072, 4, 0, False, True),      # plan): two rows per 32-lane group
    (4096, 4096, 3, 128, False, True),    # K = 4096
    (301, 8192, 4, 128, True, False),     # ragged: two rows per workgroup, the last one short
])
def test_rows_gemv_several_rows(hip, act, n, k, m, had, marlin, bias):
    """The row-owning GEMV with 2-4 activation rows (one weight read, each slot decoded once
    for the rows): bit-identical to one single-row call per row (the same per-row arithmetic)
    and within the dtype's bar of the oracle's float64 product, x rows ldx apart and output
    rows ldo apart (both padded)."""
    case(act=act, n=n, k=k, m=m, had=had, marlin=marlin, bias=bias)
    q, rng = _format_b(n * 7 + k + m + had, n, k, had, marlin=marlin)
    rd = act if act == "float16" else "float32"
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], marlin, rd, q["rowptr"], q["col"], q["val"])
    x = O.round_to(rand_np(rng, (m, k), 1.0, np.float32), act)
    b = rand_np(rng, (n,), 0.1) if bias else None
    y_ref = O.linear_ref(x, act, w_eff, rd, hadamard_block=had, bias=b)
    ops = K.QWeightOperands(cuda(q["packed"]), cuda(q["absmax"]), None, k, codebook="nf4", group_size=64,
                            hadamard_block=had, marlin_layout=marlin, bias=cuda(b) if bias else None,
                            outlier_idx=cuda(q["col"]), outlier_w=cuda(q["val"]), outlier_rowptr=cuda(q["rowptr"]))
    lib = L.load()
    dt, code = TDT[act], (L.F16 if act == "float16" else L.BF16)
    xp = torch.zeros(m, k + 64, dtype=dt, device="cuda")
    xp[:, :k] = cuda(x, dt)
    stream = torch.cuda.current_stream().cuda_stream
    y = torch.full((m, n + 5), float("nan"), dtype=dt, device="cuda")
    L.check("spectra_w4a16_gemv", lib.spectra_w4a16_gemv(ops.ptr(), xp.data_ptr(), xp.stride(0), m, code,
                                                          y.data_ptr(), y.stride(0), stream))
    ys = torch.full((m, n), float("nan"), dtype=dt, device="cuda")
    for i in range(m):
        L.check("spectra_w4a16_gemv", lib.spectra_w4a16_gemv(ops.ptr(), xp[i].data_ptr(), xp.stride(0), 1, code,
                                                              ys[i].data_ptr(), n, stream))
    torch.cuda.synchronize()
    assert torch.isnan(y[:, n:]).all(), "a store past the row"
    assert torch.equal(y[:, :n], ys), "several-row output differs from single-row calls"
    check_y(y[:, :n], y_ref, dt)


@pytest.mark.parametrize("m", [2, 4])
def test_linear_dispatch_with_and_without_workspace(hip, m):
    """spectra_w4a16_linear on a wide layer the row-owning GEMV does not plan (N=16384,
    K=5120: K / 1024 odd and not 3; the older multi-row GEMV plan needs more than one
    workgroup per CU): with the workspace the rows go to the small-batch family, with none
    (or one too small) they stay on the GEMV; both against the fp32 reference."""
    import ctypes
    from spectra_amd import _lib as L
    case(m=m)
    n, k = 16384, 5120
    g = torch.Generator().manual_seed(m)
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    nnz = int(round(0.005 * n * k))
    pos = torch.randperm(n * k, generator=g)[:nnz]
    mask = torch.zeros(n * k, dtype=torch.bool)
    mask[pos] = True
    w.view(-1)[pos] = (torch.randn(nnz, generator=g) * 0.2).half()
    q = C.quantize_nf4(w.cuda(), 64, 0, mask.view(n, k).cuda(), True)
    q.hadamard_block = 128
    col, val = q.outliers()
    ops = K.QWeightOperands(q.packed, q.absmax, None, k, marlin_layout=True, outlier_idx=col, outlier_w=val,
                            **q.kernel_kwargs())
    x = torch.randn(m, k, generator=g).half().cuda()
    w_eff = K.w4_dequant(q.packed, q.absmax, None, out_dtype=torch.float32, codebook="nf4", marlin_layout=True,
                         outlier_idx=q.col, outlier_w=q.val, outlier_rowptr=q.rowptr)
    y_t = (K.fwht_rows(x, 128, out_dtype=torch.float32) @ w_eff.T).double().cpu().numpy()
    lib = L.load()
    stream = torch.cuda.current_stream().cuda_stream
    need = int(lib.spectra_w4a16_gemm_workspace(ctypes.byref(ops.desc), m, L.F16))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    outs = []
    for wptr, wbytes in ((ws.data_ptr(), need), (None, 0), (ws.data_ptr(), need - 256)):
        y = torch.full((m, n), float("nan"), dtype=torch.float16, device="cuda")
        st = lib.spectra_w4a16_linear(ctypes.byref(ops.desc), x.data_ptr(), k, m, L.F16, y.data_ptr(), n, wptr,
                                      wbytes, stream)
        assert st == L.OK, lib.spectra_last_error()
        check_y(y, y_t, torch.float16)
        outs.append(y)
    assert torch.equal(outs[1], outs[2])  # both stayed on the GEMV


# ---------------------------------------------------------------------------
# engineering properties
# ---------------------------------------------------------------------------
def test_determinism_and_graph_replay(hip):
    q, rng = _format_b(3, 1024, 4096, 128)
    args = (cuda(q["packed"]), cuda(q["absmax"]), None)
    kw = dict(outlier_idx=cuda(q["col"]), outlier_w=cuda(q["val"]), marlin_layout=True, codebook="nf4",
              hadamard_block=128, outlier_rowptr=cuda(q["rowptr"]))
    lin = SpectraFusedLinear(4096, 1024, 64, codebook="nf4", hadamard_block=128).cuda()
    lin.set_weights(*args, outlier_idx=kw["outlier_idx"], outlier_weight=kw["outlier_w"], marlin_layout=True,
                    outlier_rowptr=kw["outlier_rowptr"])
    x1 = cuda(rand_np(rng, (1, 4096), 1.0))
    x3 = cuda(rand_np(rng, (3, 4096), 1.0))  # the row-owning GEMV with three activation rows
    x8 = cuda(rand_np(rng, (8, 4096), 1.0))
    e1, e3, e8 = lin(x1), lin(x3), lin(x8)
    assert torch.equal(lin(x1), e1) and torch.equal(lin(x3), e3) and torch.equal(lin(x8), e8)  # bitwise deterministic
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            lin(x1), lin(x3), lin(x8)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g1 = lin(x1)
        g3 = lin(x3)
        g8 = lin(x8)
    for _ in range(3):
        g1.zero_()
        g3.zero_()
        g8.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g1, e1) and torch.equal(g3, e3) and torch.equal(g8, e8)
        _ = lin(x1)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("k,n", [(4096, 14336), (14336, 4096)])
def test_prefill_library_path_graph_replay(hip, k, n):
    """cfg4's two shapes through the module at M=2048, bf16: the prefill library path (a
    Stream-K algorithm on the first shape, the rotated weights on the second).  Two eager calls
    (the first times the candidates) agree bit for bit; then the call is captured in a graph
    and replayed three times with eager work between the replays, each replay equal to the
    eager output bit for bit."""
    case(k=k, n=n)
    g = torch.Generator().manual_seed(k)
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    mask = torch.rand(n, k, generator=g) < 0.005
    q = C.quantize_nf4(w.cuda(), 64, 128, mask.cuda(), True)
    lin = SpectraFusedLinear(k, n, 64, codebook="nf4", hadamard_block=128).cuda()
    lin.set_weights(q.packed, q.absmax, None, outlier_idx=q.col, outlier_weight=q.val, marlin_layout=True,
                    outlier_rowptr=q.rowptr)
    x = torch.randn(K.PREFILL_LIBRARY_MIN_M * 4, k, generator=g).bfloat16().cuda()
    e = lin(x)
    assert torch.equal(lin(x), e)  # bitwise deterministic
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            lin(x)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gy = lin(x)
    for _ in range(3):
        gy.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gy, e)
        _ = lin(x)  # eager work between replays
        torch.cuda.synchronize()


def test_functional_api_reuses_and_validates_descriptors(hip):
    """fused_w4a16_gemv_hdsq builds (and validates) a weight's descriptor once: a second call
    with the same tensors reuses it, an in-place write to an operand rebuilds and re-validates
    it (a column past K raises before any launch), and freeing the operands drops the entry."""
    import gc
    q, rng = _format_b(77, 64, 1024, 128)
    t = {k: cuda(q[k]) for k in ("packed", "absmax", "rowptr", "col", "val")}
    x = cuda(rand_np(rng, (1, 1024), 1.0))

    def call():
        return K.fused_w4a16_gemv_hdsq(x, t["packed"], t["absmax"], None, outlier_idx=t["col"], outlier_w=t["val"],
                                       marlin_layout=True, codebook="nf4", hadamard_block=128,
                                       outlier_rowptr=t["rowptr"])
    gc.collect()
    n0 = len(K._OPS.d)
    y1 = call()
    assert len(K._OPS.d) == n0 + 1
    y2 = call()
    assert len(K._OPS.d) == n0 + 1 and torch.equal(y1, y2)
    t["col"][0] = 1024  # past K: the next call re-validates and refuses
    with pytest.raises(ValueError):
        call()
    del t, y1, y2
    gc.collect()
    assert len(K._OPS.d) == n0


def test_module_edge_cases(hip):
    q, rng = _format_b(9, 64, 256, 0, ratio=0.0)
    lin = SpectraFusedLinear(256, 64, 64, codebook="nf4").cuda()
    lin.set_weights(cuda(q["packed"]), cuda(q["absmax"]), None, marlin_layout=True)
    assert lin(torch.empty(0, 256, dtype=torch.float16, device="cuda")).shape == (0, 64)
    x = cuda(rand_np(rng, (2, 3, 256), 1.0))
    y = lin(x)
    assert y.shape == (2, 3, 64)
    w_eff = O.nf4_dequant(q["packed"], q["absmax"], True, "float16")
    check_y(y.reshape(6, 64), O.linear_ref(host(x).reshape(6, 256), "float16", w_eff, "float16"), torch.float16)
    with pytest.raises(ValueError):
        K.fused_w4a16_gemv_hdsq(x.reshape(6, 256)[:, :128], cuda(q["packed"]), cuda(q["absmax"]), None,
                                codebook="nf4")
    with pytest.raises(ValueError):
        C.SpectraCompressor(group_size=64)
    with pytest.raises(NotImplementedError):
        C.SpectraCompressor(hadamard_incoherence=True)


# ---------------------------------------------------------------------------
# outlier-column selection (compressor.py:158-215)
# ---------------------------------------------------------------------------
def test_outlier_selection_reference_vectors(hip):
    """The GPU selection against the reference's own _isolate_hdsq_outliers outputs."""
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_outlier_golden import cases, make_inputs
    g = np.load(os.path.join(HERE, "golden", "outlier_select.npz"))
    comp = C.SpectraCompressor()
    for i, (name, n, k, dt, heavy, with_norm) in enumerate(cases()):
        case(name=name, n=n, k=k)
        w, norm = make_inputs(i, n, k, dt, heavy, with_norm)
        w_dense, idx, ow, ratio, kurt = comp._isolate_hdsq_outliers(w.cuda(), norm)
        assert idx.dtype == torch.int32 and idx.device.type == "cpu"
        assert np.array_equal(idx.numpy(), g[f"{name}/idx"]), name
        assert abs(ratio - float(g[f"{name}/ratio"])) <= 1e-6 * ratio
        assert abs(kurt - float(g[f"{name}/kurtosis"])) <= 1e-4 * kurt
        assert torch.equal(ow.cpu(), w[:, idx.long()])
        if n <= 4096:
            assert torch.equal(w_dense[:, idx.long().cuda()].cpu(), torch.zeros(n, idx.numel(), dtype=w.dtype))
        else:
            assert w_dense is None


@pytest.mark.parametrize("adaptive", [True, False])
def test_outlier_selection_against_oracle(hip, adaptive):
    rng = np.random.default_rng(11 + adaptive)
    n, k = 3072, 8192
    w = rand_np(rng, (n, k), 0.02)
    cols = rng.permutation(k)[:60]
    w[:, cols] *= (1 + 10 * rng.random(60)).astype(np.float16)
    norm = (rng.random(k) + 0.5).astype(np.float32)
    case(n=n, k=k, adaptive=adaptive)
    idx, ratio, kurt = C.select_outlier_columns(cuda(w), torch.from_numpy(norm), 0.01, adaptive)
    o_idx, o_ratio, o_kurt = O.select_outlier_columns(w, "float16", norm, 0.01, adaptive)
    assert np.array_equal(host(idx), o_idx)
    assert abs(ratio - o_ratio) <= 1e-6 * o_ratio and abs(kurt - o_kurt) <= 1e-4 * o_kurt
