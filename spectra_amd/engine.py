"""``SpectraFusedLinear``: the reference's quantized linear module (engine.py:35-124)
on the MI355X library.

Same constructor, ``set_weights`` and ``forward`` contract; the weight
descriptor is built once per ``set_weights`` so a forward call is one C-ABI
call (plus the output allocation) on the current stream -- capturable in a
HIP graph.  Format B operands arrive through keyword-only arguments.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn

from .kernels import GEMV_MAX_M, QWeightOperands, w4_embedding, w4a16_linear

__all__ = ["SpectraFusedLinear", "SpectraFusedEmbedding", "DecoderConfig", "SpectraDecoder"]


class SpectraFusedLinear(nn.Module):
    """Drop-in quantized linear: packed 4-bit weights, scales, zeros and outliers
    (engine.py:35-88); rows <= GEMV_MAX_M go to the GEMV family, larger batches to
    the MFMA GEMM (engine.py:94-124)."""

    def __init__(self, in_features: int, out_features: int, group_size: int = 32, has_bias: bool = False,
                 enable_hdsq: bool = True, marlin_layout: bool = False, *, codebook: str = "asym",
                 hadamard_block: int = 0):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        self.enable_hdsq = enable_hdsq
        self.marlin_layout = marlin_layout
        self.codebook = codebook
        self.hadamard_block = hadamard_block
        self.register_buffer("packed_weight", None)
        self.register_buffer("scales", None)
        self.register_buffer("zeros", None)
        self.register_buffer("outlier_idx", None)
        self.register_buffer("outlier_weight", None)
        self.register_buffer("outlier_rowptr", None)
        if has_bias:  # engine.py:64-65
            self.register_parameter("bias", nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16)))
        else:
            self.register_parameter("bias", None)
        self._ops: Optional[QWeightOperands] = None

    def set_weights(self, packed_w: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor],
                    bias: Optional[torch.Tensor] = None, outlier_idx: Optional[torch.Tensor] = None,
                    outlier_weight: Optional[torch.Tensor] = None, marlin_layout: bool = False, *,
                    outlier_rowptr: Optional[torch.Tensor] = None, codebook: Optional[str] = None,
                    hadamard_block: Optional[int] = None):
        """engine.py:69-88, plus Format B: codebook="nf4" with ``zeros=None``, CSR outliers
        given as ``outlier_rowptr`` + ``outlier_idx`` (col) + ``outlier_weight`` (val)."""
        self.packed_weight = packed_w
        self.scales = scales
        self.zeros = zeros
        self.marlin_layout = marlin_layout
        if codebook is not None:
            self.codebook = codebook
        if hadamard_block is not None:
            self.hadamard_block = hadamard_block
        if bias is not None:
            self.bias = nn.Parameter(bias, requires_grad=False)
        if outlier_idx is not None and outlier_weight is not None:
            self.enable_hdsq = True
            self.outlier_idx = outlier_idx
            self.outlier_weight = outlier_weight
            self.outlier_rowptr = outlier_rowptr
        self._ops = None

    def _operands(self) -> QWeightOperands:
        if self._ops is None:
            use_o = self.enable_hdsq and self.outlier_idx is not None and self.outlier_weight is not None
            gs = self.group_size if self.codebook == "asym" else (self.group_size if self.group_size != 32 else 64)
            self._ops = QWeightOperands(
                self.packed_weight, self.scales, self.zeros, self.in_features, codebook=self.codebook,
                group_size=gs, hadamard_block=self.hadamard_block, marlin_layout=self.marlin_layout,
                outlier_idx=self.outlier_idx if use_o else None, outlier_w=self.outlier_weight if use_o else None,
                outlier_rowptr=self.outlier_rowptr if use_o else None, bias=self.bias)
        return self._ops

    def _apply(self, fn, *args, **kwargs):  # device/dtype moves invalidate the descriptor
        self._ops = None
        return super()._apply(fn, *args, **kwargs)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        total_tokens = x.numel() // self.in_features
        if total_tokens == 0:
            return x.new_empty(x.shape[:-1] + (self.out_features,))
        y = w4a16_linear(self._operands(), x.reshape(total_tokens, self.in_features))
        return y.reshape(x.shape[:-1] + (self.out_features,)).to(x.dtype)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, codebook={self.codebook}, "
                f"group_size={self.group_size}, hadamard_block={self.hadamard_block}, "
                f"marlin_layout={self.marlin_layout}, gemv_rows<={GEMV_MAX_M}")


# ---------------------------------------------------------------------------
# Embedding (engine.py:125-212)
# ---------------------------------------------------------------------------
class SpectraFusedEmbedding(nn.Module):
    """Quantized embedding (engine.py:125-212): keeps the packed weight and gathers /
    dequantizes only the requested rows, in one kernel (``spectra_w4_embedding``).  Same
    constructor, ``set_weights`` and forward contract as the reference; Format B operands
    through keyword-only arguments.  Zero points may be given packed (two per byte,
    engine.py:177-183) or unpacked."""

    def __init__(self, num_embeddings: int, embedding_dim: int, group_size: int = 32, marlin_layout: bool = False,
                 *, codebook: str = "asym"):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.group_size = group_size
        self.marlin_layout = marlin_layout
        self.codebook = codebook
        self.register_buffer("packed_weight", None)
        self.register_buffer("scales", None)
        self.register_buffer("zeros", None)
        self.register_buffer("outlier_idx", None)
        self.register_buffer("outlier_weight", None)
        self.register_buffer("outlier_rowptr", None)
        self.target_dtype: Optional[torch.dtype] = None
        self._ops: Optional[QWeightOperands] = None

    def set_weights(self, packed_w: torch.Tensor, scales: torch.Tensor, zeros: Optional[torch.Tensor],
                    outlier_idx: Optional[torch.Tensor] = None, outlier_weight: Optional[torch.Tensor] = None,
                    marlin_layout: bool = False, *, outlier_rowptr: Optional[torch.Tensor] = None,
                    codebook: Optional[str] = None):
        self.packed_weight, self.scales, self.zeros = packed_w, scales, zeros
        self.outlier_idx, self.outlier_weight, self.outlier_rowptr = outlier_idx, outlier_weight, outlier_rowptr
        self.marlin_layout = marlin_layout
        if codebook is not None:
            self.codebook = codebook
        self._ops = None

    def operands(self) -> QWeightOperands:
        if self._ops is None:
            zeros = self.zeros
            gs = self.group_size if self.codebook == "asym" else (self.group_size if self.group_size != 32 else 64)
            if self.codebook == "asym" and zeros is not None and zeros.shape[1] < self.scales.shape[1]:
                from .compressor import unpack_zeros  # engine.py:177-183: two zero points per byte
                zeros = unpack_zeros(zeros, self.embedding_dim)
            self._ops = QWeightOperands(self.packed_weight, self.scales, zeros, self.embedding_dim,
                                        codebook=self.codebook, group_size=gs, marlin_layout=self.marlin_layout,
                                        outlier_idx=self.outlier_idx, outlier_w=self.outlier_weight,
                                        outlier_rowptr=self.outlier_rowptr, packed_align=1)
        return self._ops

    def _apply(self, fn, *args, **kwargs):
        self._ops = None
        return super()._apply(fn, *args, **kwargs)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        # engine.py:204: the outlier dtype, else the scale dtype (fp16)
        dt = self.target_dtype or (self.outlier_weight.dtype if self.outlier_weight is not None else self.scales.dtype)
        return w4_embedding(self.operands(), input_ids, out_dtype=dt)


# ---------------------------------------------------------------------------
# Llama-shaped decoder on the quantized linears (the cfg5 workload)
# ---------------------------------------------------------------------------
@dataclass
class DecoderConfig:
    """Llama-3.2-3B shape by default."""
    layers: int = 28
    hidden: int = 3072
    heads: int = 24
    kv_heads: int = 8
    inter: int = 8192
    vocab: int = 128256
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5
    max_seq: int = 1024
    hadamard_block: int = 128
    outlier_ratio: float = 0.005
    seed: int = 0

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


def _synthetic_nf4(n: int, k: int, gen: torch.Generator, had: int, ratio: float, dev) -> "NF4Weight":
    """Random-init weight N(0, 0.02), ``ratio`` of it replaced by fp16 outliers |N(0, 0.2)| with a
    random sign, quantized to NF4 (block 64) with CSR outliers; taken as stored in the rotated basis."""
    from .compressor import quantize_nf4
    w = torch.randn(n, k, generator=gen, device=dev, dtype=torch.float32).mul_(0.02).half()
    mask = None
    if ratio > 0:
        mask = torch.rand(n, k, generator=gen, device=dev) < ratio
        mag = torch.randn(n, k, generator=gen, device=dev).abs_().mul_(0.2).half()
        sign = torch.rand(n, k, generator=gen, device=dev) < 0.5
        w = torch.where(mask, torch.where(sign, -mag, mag), w)
        del mag, sign
    q = quantize_nf4(w, 64, 0, mask, True)
    q.hadamard_block = had
    return q


class SpectraDecoder(nn.Module):
    """Batch-1 Llama-shaped decoder whose every linear is a Format B ``SpectraFusedLinear``
    (fused QKV and gate_up per layer, engine.py:409-437), with a tied quantized embedding /
    lm_head (engine.py:1124-1168) and an fp16 KV cache.  Norms, RoPE, attention and the
    sampling are torch ops.  A decode step is fully device-side (token, position and cache
    index live in device tensors), so it is captured once as a HIP graph and replayed per
    token (engine.py:1801-1860)."""

    def __init__(self, cfg: DecoderConfig = DecoderConfig(), device: Optional[torch.device] = None):
        super().__init__()
        dev = device or torch.device("cuda")
        self.cfg = cfg
        c = cfg
        hd, kvd = c.head_dim, c.kv_heads * c.head_dim
        gen = torch.Generator(device=dev).manual_seed(c.seed)
        self.layers_q = []

        def linear(n, k):
            q = _synthetic_nf4(n, k, gen, c.hadamard_block, c.outlier_ratio, dev)
            lin = SpectraFusedLinear(k, n, 64, codebook="nf4", hadamard_block=c.hadamard_block).to(dev)
            col, val = q.outliers()
            lin.set_weights(q.packed, q.absmax, None, outlier_idx=col, outlier_weight=val, marlin_layout=True,
                            outlier_rowptr=q.rowptr if col is not None else None)
            return lin, q

        self.blocks = []
        for _ in range(c.layers):
            qkv, q1 = linear(c.hidden + 2 * kvd, c.hidden)
            o, q2 = linear(c.hidden, c.hidden)
            gu, q3 = linear(2 * c.inter, c.hidden)
            down, q4 = linear(c.hidden, c.inter)
            self.blocks.append(dict(qkv=qkv, o=o, gate_up=gu, down=down))
            self.layers_q.append((q1, q2, q3, q4))
        # tied embedding / lm_head: NF4 without rotation (the gather returns the stored rows)
        qe = _synthetic_nf4(c.vocab, c.hidden, gen, 0, c.outlier_ratio, dev)
        self.embed_q = qe
        col, val = qe.outliers()
        self.embed = SpectraFusedEmbedding(c.vocab, c.hidden, 64, True, codebook="nf4")
        self.embed.set_weights(qe.packed, qe.absmax, None, col, val, True,
                               outlier_rowptr=qe.rowptr if col is not None else None)
        self.lm_head = SpectraFusedLinear(c.hidden, c.vocab, 64, codebook="nf4").to(dev)
        self.lm_head.set_weights(qe.packed, qe.absmax, None, outlier_idx=col, outlier_weight=val, marlin_layout=True,
                                 outlier_rowptr=qe.rowptr if col is not None else None)
        self.norm_w = [torch.ones(c.hidden, device=dev, dtype=torch.float32) for _ in range(2 * c.layers + 1)]
        # KV cache: K stored transposed [kv, head_dim, max_seq] so the score product needs no copy
        self.k_cache = torch.zeros(c.layers, c.kv_heads, hd, c.max_seq, device=dev, dtype=torch.float16)
        self.v_cache = torch.zeros(c.layers, c.kv_heads, c.max_seq, hd, device=dev, dtype=torch.float16)
        inv = 1.0 / (c.rope_theta ** (torch.arange(0, hd, 2, device=dev, dtype=torch.float32) / hd))
        ang = torch.arange(c.max_seq, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos, self.sin = torch.cos(ang), torch.sin(ang)  # [max_seq, hd/2]
        self.arange = torch.arange(c.max_seq, device=dev)
        # device-side decode state
        self.cur_id = torch.zeros(1, dtype=torch.int64, device=dev)
        self.cur_pos = torch.zeros(1, dtype=torch.int64, device=dev)
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.graph_logits: Optional[torch.Tensor] = None
        self.device = dev

    # -- building blocks ---------------------------------------------------------------------
    def _rms(self, x: torch.Tensor, i: int) -> torch.Tensor:
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.cfg.rms_eps) * self.norm_w[i]).half()

    def _rope(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        # x [T, h, hd]; rotate pairs (i, i + hd/2) (Llama rotate_half convention), fp32
        h2 = x.shape[-1] // 2
        xf = x.float()
        a, b = xf[..., :h2], xf[..., h2:]
        c, s = cos[:, None, :], sin[:, None, :]
        return torch.cat([a * c - b * s, b * c + a * s], dim=-1).half()

    def _layer(self, li: int, h: torch.Tensor, pos: torch.Tensor, causal_len: Optional[int]) -> torch.Tensor:
        """One decoder layer for T tokens at positions ``pos`` (device int64 [T]).  Prefill:
        causal_len = T (positions 0..T-1); decode: None (one token, masked over the cache)."""
        c, blk = self.cfg, self.blocks[li]
        hd, T = c.head_dim, h.shape[0]
        g = c.heads // c.kv_heads
        x = self._rms(h, 2 * li)
        qkv = blk["qkv"](x)
        q = qkv[:, : c.hidden].reshape(T, c.heads, hd)
        k = qkv[:, c.hidden: c.hidden + c.kv_heads * hd].reshape(T, c.kv_heads, hd)
        v = qkv[:, c.hidden + c.kv_heads * hd:].reshape(T, c.kv_heads, hd)
        cos, sin = self.cos.index_select(0, pos), self.sin.index_select(0, pos)
        q, k = self._rope(q, cos, sin), self._rope(k, cos, sin)
        self.k_cache[li].index_copy_(2, pos, k.permute(1, 2, 0).contiguous())
        self.v_cache[li].index_copy_(1, pos, v.permute(1, 0, 2).contiguous())
        qg = q.permute(1, 0, 2).reshape(c.kv_heads, g * T, hd).contiguous()  # head = kv * g + j
        if causal_len is not None:
            L = causal_len
            kt, vv = self.k_cache[li][:, :, :L].contiguous(), self.v_cache[li][:, :L, :].contiguous()
        else:
            kt, vv = self.k_cache[li], self.v_cache[li]
        s = torch.matmul(qg, kt).float() * (1.0 / math.sqrt(hd))  # [kv, g*T, L]
        if causal_len is not None:
            qpos = pos.repeat(g)  # row r = j * T + t -> position pos[t]
            mask = self.arange[:L][None, :] > qpos[:, None]
        else:
            mask = (self.arange > pos[0])[None, :]
        s = s.masked_fill(mask[None], float("-inf"))
        p = torch.softmax(s, dim=-1).half()
        a = torch.matmul(p, vv)  # [kv, g*T, hd]
        a = a.reshape(c.heads, T, hd).permute(1, 0, 2).reshape(T, c.hidden)
        h = h + blk["o"](a)
        x = self._rms(h, 2 * li + 1)
        gu = blk["gate_up"](x)
        act = (torch.nn.functional.silu(gu[:, : c.inter].float()) * gu[:, c.inter:].float()).half()
        return h + blk["down"](act)

    def forward_tokens(self, ids: torch.Tensor, pos: torch.Tensor, causal_len: Optional[int]) -> torch.Tensor:
        h = self.embed(ids)
        for li in range(self.cfg.layers):
            h = self._layer(li, h, pos, causal_len)
        return self.lm_head(self._rms(h[-1:], 2 * self.cfg.layers))  # logits of the last token [1, vocab]

    # -- generation --------------------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        T = prompt.numel()
        pos = self.arange[:T]
        logits = self.forward_tokens(prompt.reshape(-1).to(self.device), pos, T)
        self.cur_id.copy_(torch.argmax(logits[0]).reshape(1))
        self.cur_pos.fill_(T)
        return logits

    def _decode_step(self) -> torch.Tensor:
        logits = self.forward_tokens(self.cur_id, self.cur_pos, None)
        self.cur_id.copy_(torch.argmax(logits[0]).reshape(1))
        self.cur_pos.add_(1)
        return logits

    @torch.no_grad()
    def capture_decode(self) -> None:
        """Capture one decode step (all linears, attention and the argmax) as a HIP graph."""
        saved = (self.cur_id.clone(), self.cur_pos.clone(), self.k_cache.clone(), self.v_cache.clone())
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._decode_step()  # warm-up (allocations outside the capture)
        torch.cuda.current_stream().wait_stream(s)
        self.cur_id.copy_(saved[0])
        self.cur_pos.copy_(saved[1])
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.graph_logits = self._decode_step()
        # the capture does not execute: restore the state the warm-up changed
        self.cur_id.copy_(saved[0])
        self.cur_pos.copy_(saved[1])
        self.k_cache.copy_(saved[2])
        self.v_cache.copy_(saved[3])

    @torch.no_grad()
    def decode(self, steps: int, use_graph: bool = True) -> torch.Tensor:
        """``steps`` greedy tokens after a prefill; returns them (device int64 [steps])."""
        out = torch.empty(steps, dtype=torch.int64, device=self.device)
        if use_graph and self.graph is None:
            self.capture_decode()
        for i in range(steps):
            out[i : i + 1].copy_(self.cur_id)
            if use_graph:
                self.graph.replay()
            else:
                self._decode_step()
        return out
