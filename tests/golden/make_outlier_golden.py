"""Writes golden vectors for the outlier-column selection (reference
spectra/compressor.py:158-215 ``_isolate_hdsq_outliers``): column saliency, kurtosis,
adaptive ratio, topk and sort.

Nothing else pins this function -- its column choice depends on torch's reduction order
and topk tie-breaking -- so its input/output vectors are taken from the reference module
itself, loaded by path in this (build) container on the CPU.  The fixture holds data only
(inputs and outputs); the reference never travels with the repository.

    python tests/golden/make_outlier_golden.py /path/to/reference
"""
from __future__ import annotations

import hashlib
import importlib.util
import os
import sys

sys.dont_write_bytecode = True  # loading the reference by path must leave no __pycache__ in its tree

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference_compressor(root: str):
    path = os.path.join(root, "spectra", "compressor.py")
    spec = importlib.util.spec_from_file_location("reference_compressor", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def make_inputs(i, n, k, dt, heavy, with_norm):
    """Seeded CPU inputs of case i (the test regenerates them and checks their hash)."""
    g = torch.Generator().manual_seed(1000 + i)
    w = torch.randn(n, k, generator=g) * 0.02
    if heavy:
        cols = torch.randperm(k, generator=g)[:heavy]
        w[:, cols] *= 1.0 + 20.0 * torch.rand(heavy, generator=g)
    w = w.to(dt)
    norm = (torch.rand(k, generator=g) * 2.0 + 0.1) if with_norm else None
    return w, norm


def digest(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def cases():
    """(name, N, K, dtype, heavy-tail columns, with norm vector)."""
    return [
        ("gauss_fp16_norm", 96, 768, torch.float16, 0, True),
        ("heavy_fp16", 256, 1024, torch.float16, 12, False),
        ("heavy_bf16_norm", 128, 2048, torch.bfloat16, 40, True),
        ("tall_fp32", 4200, 256, torch.float32, 6, True),   # N > 4096: the chunked column norms
    ]


def main(root: str) -> None:
    ref = load_reference_compressor(root)
    comp = ref.SpectraCompressor()  # group 32, base ratio 0.01, adaptive kurtosis
    out = {}
    for i, (name, n, k, dt, heavy, with_norm) in enumerate(cases()):
        w, norm = make_inputs(i, n, k, dt, heavy, with_norm)
        w_dense, idx, ow, ratio, kurt = comp._isolate_hdsq_outliers(w, norm)
        assert torch.equal(ow, w[:, idx.long()])
        store = {"idx": idx.numpy().astype(np.int32), "ratio": np.float64(ratio), "kurtosis": np.float64(kurt),
                 "w_sha256": np.array(digest(w)), "norm_sha256": np.array(digest(norm) if norm is not None else "")}
        for key, val in store.items():
            out[f"{name}/{key}"] = val
        out[f"{name}/meta"] = np.array([i, n, k, {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}[dt], heavy,
                                        int(with_norm)], np.int64)
        print(f"{name}: N={n} K={k} ratio={ratio:.6f} kurtosis={kurt:.4f} n_out={idx.numel()}")
    np.savez_compressed(os.path.join(HERE, "outlier_select.npz"), **out)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
