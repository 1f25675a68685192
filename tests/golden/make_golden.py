"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

Inputs are drawn from numpy's seeded PCG64 so they are identical on any machine;
expected outputs come from oracle/ (pinned by tests/test_oracle.py).  The
fixtures are data only: inputs, packed operands, W_eff and float64 y_ref.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402


def format_a(seed=42, n=128, k=256, n_out=16, m=4):
    """The reference test's shape (tests/test_kernels.py:12-41): N=128, K=256, 16 outlier columns."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float16)
    idx = np.sort(rng.permutation(k)[:n_out]).astype(np.int64)
    ow = w[:, idx].copy()
    packed, scales, pz = O.compute_group32_quant(w.astype(np.float32), idx)
    z = O.unpack_zeros(pz, k // 32)
    w_deq = O.apply_outlier_columns(O.dequant_group32(packed, scales, z, marlin=True, out_dtype="float16"),
                                    idx, ow, "float16")
    x = rng.standard_normal((m, k)).astype(np.float16)
    y = O.format_a_linear_ref(x, "float16", w_deq)
    return dict(w=w, idx=idx, ow=ow, packed=packed, scales=scales, packed_zeros=pz, zeros=z, w_deq=w_deq, x=x,
                y_ref=y)


def format_b(seed=7, n=96, k=512, had=128, m=3, ratio=0.005):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    nnz = int(round(ratio * n * k))
    flat = rng.choice(n * k, size=nnz, replace=False)
    mask = np.zeros(n * k, bool)
    mask[flat] = True
    mask = mask.reshape(n, k)
    vals = (np.abs(rng.standard_normal(nnz)) * 0.2 * np.where(rng.random(nnz) < 0.5, -1, 1)).astype(np.float16)
    w_planted = w.copy()
    w_planted[mask] = vals[np.argsort(flat)]
    q = O.nf4_quantize(w_planted, "float16", blocksize=64, hadamard_block=0, outlier_mask=mask, marlin=True)
    w_eff16 = O.nf4_dequant(q["packed"], q["absmax"], True, "float16", q["rowptr"], q["col"], q["val"])
    w_effbf = O.nf4_dequant(q["packed"], q["absmax"], True, "bfloat16", q["rowptr"], q["col"], q["val"])
    x = rng.standard_normal((m, k)).astype(np.float16)
    y = O.linear_ref(x, "float16", w_eff16, "float16", hadamard_block=had)
    # the same weights quantized after a row rotation (the compressor's Hadamard option)
    qr = O.nf4_quantize(w, "float16", blocksize=64, hadamard_block=had, outlier_mask=None, marlin=False)
    return dict(w=w_planted, mask=mask, packed=q["packed"], absmax=q["absmax"], rowptr=q["rowptr"], col=q["col"],
                val=q["val"], w_eff16=w_eff16, w_effbf=w_effbf, x=x, y_ref=y, had=np.int64(had),
                w_plain=w, packed_rot=qr["packed"], absmax_rot=qr["absmax"])


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "format_a_small.npz"), **format_a())
    np.savez_compressed(os.path.join(HERE, "format_b_small.npz"), **format_b())
    print("wrote", os.listdir(HERE))
