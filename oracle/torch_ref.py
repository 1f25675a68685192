"""torch restatement of SPECTRA's W4A16 path and of the Llama-shaped decode it serves
(test infrastructure only, like the rest of ``oracle/``).

The same arithmetic as ``spectra_oracle`` (numpy), written with torch ops so that it runs
on the host cores with torch's thread pool (the CPU baseline of ``bench.py``) or on any
other device.  It never touches the product (``spectra_amd``): operands come in as plain
tensors.

Pinning (``tests/test_oracle.py``): ``nf4_dequant`` and ``fwht`` are bit-identical to the
numpy oracle (whose own pins are listed in ``oracle/__init__.py``); ``linear_a`` /
``linear_b`` agree with ``spectra_oracle.linear_ref`` to float32 rounding; the decoder
pieces satisfy closed forms (RoPE preserves norms and rotates by the position's angles,
attention over one position returns its value row, RMSNorm of a constant row is the norm
weight); ``Decoder`` and ``rope_inv_freq`` reproduce Hugging Face's ``LlamaForCausalLM``
(the reference engine's model class, engine.py:919-939) on a tiny grouped-query Llama, for
the unscaled and the llama3-scaled RoPE table: logits of a 96-token prefill and 4 decode
steps, greedy tokens and the inverse-frequency tables (fixture
``tests/golden/llama_hf_decode.npz``, written by ``tests/golden/make_llama_golden.py``).
``Decoder`` is then the checker of the GPU decoder in ``tests/test_decoder.py``.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence

import torch

from .spectra_oracle import NF4_CODEBOOK

__all__ = ["nf4_dequant", "fwht_blocks", "linear_a", "linear_b", "rms_norm", "rope", "rope_inv_freq", "attention",
           "Decoder"]

_CODES = torch.from_numpy(NF4_CODEBOOK.copy())  # compressor.py:22-27, float32


def _unpack(packed: torch.Tensor, marlin: bool) -> torch.Tensor:
    """uint8 [N, K/2] -> code indices int64 [N, K] (compressor.py:99-102 marlin interleave:
    byte j of a 32-run holds q[j] (low) and q[j+16] (high); plain: q[2j], q[2j+1])."""
    lo = (packed & 0x0F).to(torch.int64)
    hi = (packed >> 4).to(torch.int64)
    n = packed.shape[0]
    if marlin:
        lo = lo.reshape(n, -1, 16)
        hi = hi.reshape(n, -1, 16)
        return torch.cat([lo, hi], dim=-1).reshape(n, -1)
    return torch.stack([lo, hi], dim=-1).reshape(n, -1)


def nf4_dequant(packed: torch.Tensor, absmax: torch.Tensor, rowptr: Optional[torch.Tensor] = None,
                col: Optional[torch.Tensor] = None, val: Optional[torch.Tensor] = None, *, marlin: bool = True,
                blocksize: int = 64, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """W_eff = round_out(float32(NF4[q]) * float32(absmax)), then CSR positions := round_out(val)
    (the Format B dequant of ``spectra_oracle.nf4_dequant``; engine.py:204-210 for the
    reference's own Format A analogue)."""
    q = _unpack(packed, marlin)
    n, k = q.shape
    codes = _CODES.to(packed.device)[q].reshape(n, k // blocksize, blocksize)
    w = (codes * absmax.to(torch.float32)[..., None]).reshape(n, k).to(out_dtype)
    if rowptr is not None and col is not None and col.numel():
        rows = torch.repeat_interleave(torch.arange(n, device=packed.device), torch.diff(rowptr.to(torch.int64)))
        w[rows, col.to(torch.int64)] = val.to(torch.float32).to(out_dtype)
    return w


def fwht_blocks(x: torch.Tensor, block: int) -> torch.Tensor:
    """Normalised Walsh-Hadamard transform of every ``block``-wide block of the last axis, in
    float32, in the reference's stage order h = 1, 2, 4, ... and normalisation (compressor.py:29-42)."""
    x = x.to(torch.float32)
    if block == 0:
        return x.clone()
    shape = x.shape
    r = x.reshape(-1, block).clone()
    h = 1
    while h < block:
        v = r.reshape(-1, block // (2 * h), 2, h)
        a, b = v[:, :, 0, :].clone(), v[:, :, 1, :].clone()
        v[:, :, 0, :] = a + b
        v[:, :, 1, :] = a - b
        h *= 2
    return (r / torch.tensor(math.sqrt(block), dtype=torch.float32)).reshape(shape)


def linear_a(x: torch.Tensor, packed: torch.Tensor, absmax: torch.Tensor, rowptr, col, val, *, hadamard_block: int,
             blocksize: int = 64, marlin: bool = True) -> torch.Tensor:
    """Variant A, the per-call reference path a torch fallback of SpectraFusedLinear would
    take (tests/test_kernels.py:31-46, engine.py:186-210): dequantize W_eff, rotate x, float32
    product, output in x's dtype."""
    w = nf4_dequant(packed, absmax, rowptr, col, val, marlin=marlin, blocksize=blocksize)
    return (fwht_blocks(x, hadamard_block) @ w.T).to(x.dtype)


def linear_b(x: torch.Tensor, w_eff: torch.Tensor, *, hadamard_block: int) -> torch.Tensor:
    """Variant B: the float32 product alone on a pre-dequantized float32 W_eff (the CPU lower bound)."""
    return (fwht_blocks(x, hadamard_block) @ w_eff.T).to(x.dtype)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Llama RMSNorm in float32: x * rsqrt(mean(x^2) + eps) * w."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rope_inv_freq(head_dim: int, theta: float, scaling: Optional[dict] = None) -> torch.Tensor:
    """Inverse RoPE frequencies theta^(-2i/d), i < d/2, as float32.  ``scaling`` with
    ``rope_type: llama3`` applies Llama 3.1's published frequency scaling, element by element
    in float64: wavelength w = 2 pi / f; w below original_context / high_freq_factor keeps f,
    w above original_context / low_freq_factor takes f / factor, between them
    f ((1 - s) / factor + s) with s = (original_context / w - low) / (high - low)."""
    base = (torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim)
    inv = 1.0 / (theta ** base)
    kind = (scaling or {}).get("rope_type", (scaling or {}).get("type", "default"))
    if kind == "default":
        return inv
    if kind != "llama3":
        raise ValueError(f"rope_type {kind!r} is not restated here")
    factor = float(scaling["factor"])
    lo, hi = float(scaling["low_freq_factor"]), float(scaling["high_freq_factor"])
    ctx = float(scaling["original_max_position_embeddings"])
    out = []
    for f in inv.tolist():
        w = 2.0 * math.pi / f
        if w < ctx / hi:
            out.append(f)
        elif w > ctx / lo:
            out.append(f / factor)
        else:
            s = (ctx / w - lo) / (hi - lo)
            out.append((1.0 - s) * f / factor + s * f)
    return torch.tensor(out, dtype=torch.float64).to(torch.float32)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotary embedding, half-split (Llama's rotate_half): x [T, H, d], cos/sin [T, d/2]."""
    h2 = x.shape[-1] // 2
    c, s = cos[:, None, :], sin[:, None, :]
    a, b = x[..., :h2], x[..., h2:]
    return torch.cat([a * c - b * s, b * c + a * s], dim=-1)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """Causal grouped-query attention in float32: q [T, H, d] at positions ``pos`` over k, v
    [L, Hkv, d] (positions 0..L-1); returns [T, H * d]."""
    T, H, d = q.shape
    g = H // k.shape[1]
    kk = k.repeat_interleave(g, dim=1).permute(1, 2, 0).contiguous()  # [H, d, L]
    vv = v.repeat_interleave(g, dim=1).permute(1, 0, 2).contiguous()  # [H, L, d]
    s = torch.matmul(q.permute(1, 0, 2).contiguous(), kk) / math.sqrt(d)
    L = k.shape[0]
    s = s.masked_fill((torch.arange(L, device=q.device)[None, :] > pos[:, None])[None], float("-inf"))
    a = torch.matmul(torch.softmax(s, -1), vv)  # [H, T, d]
    return a.permute(1, 0, 2).reshape(T, H * d)


class Decoder:
    """float32 Llama-shaped decoder on pre-dequantized weights (the workload of BASELINE
    configs[4], engine.py:1801-1860): per layer the fused QKV and gate_up projections
    (layers[i] = (W_qkv, W_o, W_gate_up, W_down), each float32 [N, K] in the rotated basis
    with its Hadamard block ``had[i]``), RMSNorm, RoPE, grouped-query attention over a
    growing KV cache, SiLU-mul; ``norms`` holds 2 per layer then the final one; the logits
    come from ``head`` (float32 [vocab, hidden]).  ``rope_scaling``: the config's RoPE
    parameters (``rope_inv_freq``); None for the unscaled table."""

    def __init__(self, layers: Sequence[Sequence[torch.Tensor]], had: Sequence[Sequence[int]], norms: List[torch.Tensor],
                 emb: torch.Tensor, head: torch.Tensor, *, heads: int, kv_heads: int, rope_theta: float,
                 rms_eps: float, max_seq: int, rope_scaling: Optional[dict] = None):
        self.layers, self.had, self.norms, self.emb, self.head = layers, had, norms, emb, head
        self.heads, self.kv_heads, self.eps = heads, kv_heads, rms_eps
        self.hidden = emb.shape[1]
        self.hd = self.hidden // heads
        self.inter = layers[0][2].shape[0] // 2
        dev = emb.device
        inv = rope_inv_freq(self.hd, rope_theta, rope_scaling).to(dev)
        ang = torch.arange(max_seq, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos, self.sin = torch.cos(ang), torch.sin(ang)
        self.k: List[torch.Tensor] = []
        self.v: List[torch.Tensor] = []

    def lin(self, x: torch.Tensor, w: torch.Tensor, had: int) -> torch.Tensor:
        return fwht_blocks(x, had) @ w.T

    def forward(self, ids: torch.Tensor, pos0: int) -> torch.Tensor:
        """Logits of the last of the tokens ``ids`` at positions pos0.. (the cache grows)."""
        hd, H, Hkv = self.hd, self.heads, self.kv_heads
        T = ids.numel()
        pos = torch.arange(pos0, pos0 + T, device=ids.device)
        h = self.emb[ids]
        for li, (wqkv, wo, wgu, wd) in enumerate(self.layers):
            hq, ho, hg, hdn = self.had[li]
            qkv = self.lin(rms_norm(h, self.norms[2 * li], self.eps), wqkv, hq)
            q = qkv[:, : H * hd].reshape(T, H, hd)
            k = qkv[:, H * hd: (H + Hkv) * hd].reshape(T, Hkv, hd)
            v = qkv[:, (H + Hkv) * hd:].reshape(T, Hkv, hd)
            q, k = rope(q, self.cos[pos], self.sin[pos]), rope(k, self.cos[pos], self.sin[pos])
            if li == len(self.k):
                self.k.append(k)
                self.v.append(v)
            else:
                self.k[li] = torch.cat([self.k[li], k])
                self.v[li] = torch.cat([self.v[li], v])
            h = h + self.lin(attention(q, self.k[li], self.v[li], pos), wo, ho)
            gu = self.lin(rms_norm(h, self.norms[2 * li + 1], self.eps), wgu, hg)
            h = h + self.lin(torch.nn.functional.silu(gu[:, : self.inter]) * gu[:, self.inter:], wd, hdn)
        return rms_norm(h[-1:], self.norms[-1], self.eps) @ self.head.T
