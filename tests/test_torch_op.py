"""The registered operator torch.ops.spectra_hip.w4a16_linear (spectra_amd/csrc/torch_ops.cpp).

CPU: the operator library loads, registers its schema and gives output shapes through its
Meta kernel (no launch).  GPU: it returns exactly what the C ABI returns through ctypes
(the same entry point on the same operands, so bit-equal), for one row, small batches and
prefill, Format A and Format B, fp16 / bf16 / fp32 activations and strided or misaligned
rows; the module routes through it; a HIP graph replays it; torch.compile traces it
without a graph break.
"""
import numpy as np
import pytest
import torch

import oracle as O
from spectra_amd import _lib as L
from spectra_amd import kernels as K
from spectra_amd.engine import SpectraFusedLinear


def _ops():
    return L.load_torch_ops()


def test_operator_schema_and_meta_shapes():
    op = _ops().w4a16_linear
    schema = str(op.default._schema)
    for arg in ("Tensor x", "Tensor packed_w", "Tensor scales", "Tensor? zeros", "Tensor? outlier_idx",
                "Tensor? outlier_w", "Tensor? outlier_rowptr", "Tensor? bias", "int layout"):
        assert arg in schema, schema
    lw = K.layout_word("nf4", 64, 128, True)
    p = torch.empty(96, 128, dtype=torch.uint8, device="meta")
    s = torch.empty(96, 4, dtype=torch.float16, device="meta")
    for shape, dt in (((1, 256), torch.float16), ((2, 3, 256), torch.bfloat16), ((256,), torch.float32),
                      ((0, 256), torch.float16)):
        y = op(torch.empty(shape, dtype=dt, device="meta"), p, s, None, None, None, None, None, lw)
        assert y.shape == shape[:-1] + (96,) and y.dtype == dt
    with pytest.raises(RuntimeError):  # bits above the layout fields
        op(torch.empty(1, 256, dtype=torch.float16, device="meta"), p, s, None, None, None, None, None, 1 << 26)


def test_layout_word_fields():
    """The bit fields the operator decodes (torch_ops.cpp decode_layout)."""
    assert K.layout_word("asym", 32, 0, False) == 32 << 2
    assert K.layout_word("nf4", 64, 0, False) == 1 | 64 << 2
    assert K.layout_word("nf4", 64, 128, True) == 1 | 2 | 64 << 2 | 128 << 14
    assert K.layout_word("asym", 32, 1024, True) == 2 | 32 << 2 | 1024 << 14
    with pytest.raises(ValueError):
        K.layout_word("int8", 32, 0, False)
    with pytest.raises(ValueError):
        K.layout_word("nf4", 4096, 0, False)


def test_operator_rejects_host_tensors():
    p = torch.zeros(64, 128, dtype=torch.uint8)
    s = torch.ones(64, 4, dtype=torch.float16)
    with pytest.raises((RuntimeError, NotImplementedError)):
        _ops().w4a16_linear(torch.zeros(1, 256, dtype=torch.float16), p, s, None, None, None, None, None,
                            K.layout_word("nf4", 64, 0, True))


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
def _nf4(seed, n, k, had):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    mask = rng.random((n, k)) < 0.005
    w[mask] = (rng.standard_normal(int(mask.sum())) * 0.2).astype(np.float16)
    q = O.nf4_quantize(w, "float16", 64, 0, mask, True)
    t = {k_: torch.from_numpy(np.ascontiguousarray(q[k_])).cuda() for k_ in ("packed", "absmax", "rowptr", "col", "val")}
    b = torch.from_numpy((rng.standard_normal(n) * 0.1).astype(np.float16)).cuda()
    ops = K.QWeightOperands(t["packed"], t["absmax"], None, k, codebook="nf4", group_size=64, hadamard_block=had,
                            marlin_layout=True, outlier_idx=t["col"], outlier_w=t["val"], outlier_rowptr=t["rowptr"],
                            bias=b)
    return ops, rng


def _format_a(seed, n, k):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    idx = np.sort(rng.permutation(k)[:12]).astype(np.int64)
    packed, scales, pz = O.compute_group32_quant(w, idx)
    z = O.unpack_zeros(pz, k // 32)
    ow = w[:, idx].astype(np.float16)
    b = (rng.standard_normal(n) * 0.5).astype(np.float16)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    ops = K.QWeightOperands(cu(packed), cu(scales), cu(z), k, codebook="asym", group_size=32, marlin_layout=True,
                            outlier_idx=cu(idx), outlier_w=cu(ow), bias=cu(b))
    return ops, rng


def _both(ops, x):
    y_op = _ops().w4a16_linear(x, *ops.op_args)
    y_abi = K.w4a16_linear(ops, x)
    torch.cuda.synchronize()
    assert y_op.shape == y_abi.shape and y_op.dtype == x.dtype == y_abi.dtype
    assert torch.equal(y_op, y_abi)
    return y_op


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 80])
@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_operator_matches_c_abi_nf4(hip, m, act):
    print(f"case: nf4 had=128 CSR bias m={m} act={act}", flush=True)
    ops, rng = _nf4(m, 1040, 3072, 128)
    x = torch.from_numpy(rng.standard_normal((m, 3072)).astype(np.float32)).to(act).cuda()
    _both(ops, x)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 3, 40])
def test_operator_matches_c_abi_format_a(hip, m):
    print(f"case: format A columns bias m={m}", flush=True)
    ops, rng = _format_a(100 + m, 200, 1536)
    x = torch.from_numpy(rng.standard_normal((m, 1536)).astype(np.float16)).cuda()
    _both(ops, x)


@pytest.mark.gpu
def test_operator_activation_layouts(hip):
    print("case: fp32, 3-D, strided, misaligned and empty activations", flush=True)
    ops, rng = _nf4(5, 512, 1024, 128)
    base = torch.from_numpy(rng.standard_normal((6, 2048)).astype(np.float32)).cuda()
    _both(ops, base[:, :1024].contiguous())                      # float32 in, float32 out
    _both(ops, base[:, :1024].half().reshape(2, 3, 1024))         # leading dims kept
    _both(ops, base.half()[:, 1024:])                             # row stride 2048
    flat = base.half().reshape(-1)
    _both(ops, flat[1:1 + 4 * 1024].reshape(4, 1024))             # base 2 bytes past alignment
    _both(ops, flat[8:8 + 1024])                                   # one row, 1-D
    assert _ops().w4a16_linear(base[:0, :1024].half(), *ops.op_args).shape == (0, 512)
    with pytest.raises(RuntimeError):
        _ops().w4a16_linear(base[:, :1000].half(), *ops.op_args)  # K mismatch


@pytest.mark.gpu
def test_module_runs_the_operator_in_a_graph(hip):
    """The module's call is the operator; captured in a HIP graph it replays to the eager
    result, with eager work between replays."""
    ops, rng = _nf4(11, 1024, 4096, 128)
    packed, absmax, _, col, val, rp, b, _ = ops.op_args
    lin = SpectraFusedLinear(4096, 1024, 64, has_bias=True, codebook="nf4", hadamard_block=128).cuda()
    lin.set_weights(packed, absmax, None, bias=b, outlier_idx=col, outlier_weight=val, marlin_layout=True,
                    outlier_rowptr=rp)
    x1 = torch.from_numpy(rng.standard_normal((1, 4096)).astype(np.float16)).cuda()
    x8 = torch.from_numpy(rng.standard_normal((8, 4096)).astype(np.float16)).cuda()
    e1, e8 = lin(x1), lin(x8)
    assert lin._op_args is not None
    assert torch.equal(e1, _both(ops, x1)) and torch.equal(e8, _both(ops, x8))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lin(x1), lin(x8)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g1 = lin(x1)
        g8 = lin(x8)
    for _ in range(3):
        g1.zero_()
        g8.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g1, e1) and torch.equal(g8, e8)
        _ = lin(x8)
        torch.cuda.synchronize()


@pytest.mark.gpu
def test_module_compiles_without_graph_break(hip):
    """torch.compile(fullgraph=True) traces the module's call through the operator's schema
    and Meta kernel (a graph break would raise); the compiled call returns the eager result."""
    ops, rng = _nf4(12, 256, 1024, 128)
    packed, absmax, _, col, val, rp, b, _ = ops.op_args
    lin = SpectraFusedLinear(1024, 256, 64, has_bias=True, codebook="nf4", hadamard_block=128).cuda()
    lin.set_weights(packed, absmax, None, bias=b, outlier_idx=col, outlier_weight=val, marlin_layout=True,
                    outlier_rowptr=rp)
    x = torch.from_numpy(rng.standard_normal((3, 1024)).astype(np.float16)).cuda()
    eager = lin(x)  # binds the operands outside the trace
    f = torch.compile(lambda t: lin(t) * 2, fullgraph=True, backend="aot_eager")
    torch.testing.assert_close(f(x), eager * 2, rtol=0, atol=0)
