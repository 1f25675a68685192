"""Writes golden vectors for the 4-bit KV-cache quantizer (reference spectra/engine.py:614-680
``SpectraGroup32QuantizedLayer._quantize`` / ``_dequantize``: per row of the head
dimension, groups of 32, asymmetric min-max codes 0..15, fp16 scales, uint8 zero points,
two codes per byte).

Nothing in the reference's tests pins these functions, and the module that holds them
imports GPU-only packages, so the two methods alone are compiled from the module's syntax
tree (in this build container, on the CPU) and run on seeded inputs.  The fixture
``kv4_quant.npz`` holds inputs and outputs only.

    python tests/golden/make_kv4_golden.py /path/to/reference
"""
from __future__ import annotations

import ast
import os
import sys

sys.dont_write_bytecode = True  # loading the reference by path must leave no __pycache__ in its tree

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "kv4_quant.npz")


def load_reference_quantizer(root: str):
    path = os.path.join(root, "spectra", "engine.py")
    tree = ast.parse(open(path).read(), filename=path)
    cls = next(n for n in tree.body if isinstance(n, ast.ClassDef) and n.name == "SpectraGroup32QuantizedLayer")
    fns = [n for n in cls.body if isinstance(n, ast.FunctionDef) and n.name in ("_quantize", "_dequantize")]
    holder = ast.ClassDef(name="RefKV4", bases=[], keywords=[], body=fns, decorator_list=[])
    mod = ast.Module(body=[holder], type_ignores=[])
    ast.fix_missing_locations(mod)
    ns = {"torch": torch}
    exec(compile(mod, path, "exec"), ns)
    q = ns["RefKV4"]()
    q.group_size = 32
    return q


def cases():
    """(name, dtype, rows, D, seed, special) -- special groups: constant / zero / one-signed."""
    return [("bf16_128", torch.bfloat16, 37, 128, 1, True),
            ("fp16_128", torch.float16, 37, 128, 2, True),
            ("fp16_64", torch.float16, 20, 64, 3, False),
            ("bf16_96", torch.bfloat16, 9, 96, 4, False)]   # 96 = 3 groups


def make_input(dtype, rows, d, seed, special):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(rows, d, generator=g) * torch.exp(torch.randn(rows, 1, generator=g))
    if special:
        t[0, :32] = 0.0            # all-zero group
        t[1, 32:64] = 1.5          # constant positive
        t[2, 64:96] = -0.25        # constant negative
        t[3, :32] = t[3, :32].abs() + 0.5   # one-signed positive (zero point 0 after clamp)
        t[4, 32:64] = -t[4, 32:64].abs() - 2.0
    return t.to(dtype)


def main(root: str) -> None:
    q = load_reference_quantizer(root)
    out = {}
    for name, dt, rows, d, seed, special in cases():
        t = make_input(dt, rows, d, seed, special)
        packed, scales, zeros, shape, pad = q._quantize(t)
        deq = q._dequantize((packed, scales, zeros, shape, pad))
        out[name + "_x"] = t.view(torch.int16).numpy() if dt == torch.bfloat16 else t.numpy()
        out[name + "_packed"] = packed.numpy()
        out[name + "_scales"] = scales.numpy()
        out[name + "_zeros"] = zeros.numpy()
        out[name + "_deq"] = deq.view(torch.int16).numpy()  # bf16 bits
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
