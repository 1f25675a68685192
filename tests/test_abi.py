"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, the ctypes descriptor matches the C struct layout, and argument
validation rejects bad descriptors before any device work."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from spectra_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "spectra_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(spectra_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = L.load()
    declared = _declared_functions()
    assert declared, "no functions parsed from the header"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/spectra_hip.h but not exported"
    assert set(declared) == set(L.SIGNATURES), "ctypes signature table out of sync with the header"
    assert lib.spectra_version().decode().startswith("spectra_hip")


def test_qweight_layout_matches_c():
    fields = [f[0] for f in L.QWeight._fields_]
    src = "#include <stdio.h>\n#include <stddef.h>\n#include \"spectra_hip.h\"\nint main(void){\n"
    src += 'printf("%zu\\n", sizeof(spectra_qweight_t));\n'
    for f in fields:
        src += f'printf("%zu\\n", offsetof(spectra_qweight_t, {f}));\n'
    src += "return 0;}\n"
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        vals = [int(v) for v in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(L.QWeight)
    for f, off in zip(fields, vals[1:]):
        assert getattr(L.QWeight, f).offset == off, f


def _desc(**kw):
    w = L.QWeight()
    w.n, w.k, w.format, w.group_size = 128, 256, L.FMT_NF4, 64
    w.packed, w.packed_stride = 0x1000, 128
    w.scales, w.scales_stride = 0x2000, 4
    for k, v in kw.items():
        setattr(w, k, v)
    return w


@pytest.mark.parametrize("bad, msg", [
    (dict(n=0), "positive"),
    (dict(k=100), "multiple of 32"),
    (dict(format=7), "unknown format"),
    (dict(format=L.FMT_ASYM_G32, group_size=64), "group_size 32"),
    (dict(group_size=48), "power of two"),
    (dict(hadamard_block=96), "hadamard_block"),
    (dict(packed_stride=64), "packed row stride"),
    (dict(outlier_kind=L.OUTLIERS_CSR), "rowptr"),
    (dict(outlier_kind=L.OUTLIERS_COLUMNS, num_outliers=3), "idx and w"),
])
def test_descriptor_validation(bad, msg):
    lib = L.load()
    w = _desc(**bad)
    st = lib.spectra_w4_dequant(ctypes.byref(w), ctypes.c_void_p(0x3000), 256, L.F16, None)
    assert st == L.ERR_INVALID
    assert msg in lib.spectra_last_error().decode()


def test_entry_points_reject_bad_arguments():
    lib = L.load()
    w = _desc()
    assert lib.spectra_w4a16_gemv(None, None, 0, 1, L.F16, None, 0, None) == L.ERR_INVALID
    assert lib.spectra_w4a16_gemv(ctypes.byref(w), 0x4000, 256, 5, L.F16, 0x5000, 128, None) == L.ERR_INVALID
    assert "1 <= m <= 4" in lib.spectra_last_error().decode()
    assert lib.spectra_w4a16_gemv(ctypes.byref(w), 0x4000, 256, 1, L.F32, 0x5000, 128, None) == L.ERR_INVALID
    # GEMM: workspace is mandatory and sized by the query
    need = lib.spectra_w4a16_gemm_workspace(ctypes.byref(w), 100, L.F16)
    assert need >= 100 * 256 * 2
    assert lib.spectra_w4a16_gemm(ctypes.byref(w), 0x4000, 256, 100, L.F16, 0x5000, 128, None, 0,
                                  None) == L.ERR_WORKSPACE
    # Format A quantizer keeps the reference's group-32 rule (compressor.py:53-54)
    assert lib.spectra_quantize_group32(0x1000, 64, L.F16, 2, 64, 64, None, 0, 0x2000, 0x3000, 0x4000,
                                        None) == L.ERR_INVALID
    assert "group_size=32" in lib.spectra_last_error().decode()
    assert lib.spectra_fwht_rows(0x1000, 96, L.F32, 2, 96, 96, 0x2000, 96, L.F32, None) == L.ERR_INVALID
    # measurement kernels: geometry, alignment and size checks before any launch
    assert lib.spectra_measure_empty(0, 64, None) == L.ERR_INVALID
    assert lib.spectra_measure_read(0x1008, 1024, 4, 64, 0x2000, None) == L.ERR_INVALID  # unaligned source
    assert lib.spectra_measure_read(0x1000, 1000, 4, 64, 0x2000, None) == L.ERR_INVALID  # not a multiple of 16
    assert lib.spectra_measure_read(0x1000, 1024, 4, 100, 0x2000, None) == L.ERR_INVALID  # block not of whole waves
    assert lib.spectra_measure_read(0x1000, 1 << 30, 1, 64, 0x2000, None) == L.ERR_UNSUPPORTED  # > 16 loads/thread


def test_decode_kernels_reject_bad_arguments():
    lib = L.load()
    p = ctypes.c_void_p(0x1000)
    assert lib.spectra_rmsnorm(None, None, p, 1e-5, 1, 64, p, None) == L.ERR_INVALID
    assert lib.spectra_rmsnorm(p, None, p, 1e-5, 0, 64, p, None) == L.ERR_INVALID
    # heads must be a multiple of kv_heads; qkv rows must hold heads + 2 kv_heads heads
    assert lib.spectra_rope_append(p, 1024, 1, p, p, p, 6, 4, 64, 128, p, p, p, None) == L.ERR_INVALID
    assert lib.spectra_rope_append(p, 100, 1, p, p, p, 4, 2, 64, 128, p, p, p, None) == L.ERR_INVALID
    assert "stride" in lib.spectra_last_error().decode()
    # 64 spans of 64 positions for max_seq 4096; the partials are fp32 [heads][spans][d + 2]
    assert lib.spectra_attend_spans(4096) == 64 and lib.spectra_attend_spans(4097) == 65
    # partials rounded up to 256 bytes, then one 256-byte arrival counter per head
    assert lib.spectra_attend_workspace(24, 128, 1000) == (24 * 16 * 130 * 4 + 255) // 256 * 256 + 24 * 256
    args = (p, p, p, p)
    assert lib.spectra_attend_decode(*args, 24, 8, 128, 1024, p, p, None, 0, p, None) == L.ERR_WORKSPACE
    assert lib.spectra_attend_decode(*args, 24, 8, 48, 1024, p, p, p, 1 << 20, p, None) == L.ERR_INVALID
    # the 4-bit cache quantizes groups of 32 dims: head_dim 16 is refused before any launch
    assert lib.spectra_attend_decode_q4(*args, 4, 2, 16, 64, 16, p, p, p, p, p, p, p, p, p, 1 << 20, p,
                                        None) == L.ERR_INVALID
    assert "head_dim" in lib.spectra_last_error().decode()
    # 10 query heads per KV head: past both kernels (the MFMA kernel serves up to 8 at head_dim
    # >= 64, the other 1, 2, 3, 4, 6 or 8)
    assert lib.spectra_attend_decode(*args, 80, 8, 128, 1024, p, p, p, 1 << 24, p, None) == L.ERR_UNSUPPORTED
    assert lib.spectra_attend_decode(*args, 20, 4, 32, 1024, p, p, p, 1 << 24, p, None) == L.ERR_UNSUPPORTED
    assert lib.spectra_attend_decode(*args, 24, 8, 96, 1024, p, p, p, 1 << 24, p, None) == L.ERR_INVALID
    assert lib.spectra_attend_decode(p, p, p, None, 24, 8, 128, 1024, p, p, p, 1 << 24, p, None) == L.ERR_INVALID
    assert lib.spectra_silu_mul(p, 100, 1, 64, p, None) == L.ERR_INVALID
    assert lib.spectra_greedy_next(p, 0, p, None, 0, None, None) == L.ERR_INVALID
    assert lib.spectra_greedy_next(p, 10, p, p, 10, None, None) == L.ERR_INVALID  # history needs pos
