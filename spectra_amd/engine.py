"""``SpectraFusedLinear``: the reference's quantized linear module (engine.py:35-124)
on the MI355X library.

Same constructor, ``set_weights`` and ``forward`` contract; the weight
descriptor is built once per ``set_weights`` so a forward call is one C-ABI
call (plus the output allocation) on the current stream -- capturable in a
HIP graph.  Format B operands arrive through keyword-only arguments.
"""
from __future__ import annotations

import math
import warnings
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn

from . import _lib as L
from .kernels import (GEMV_MAX_M, QWeightOperands, argmax_slots, attend_decode, attend_decode_q4,
                      attend_workspace_bytes, greedy_finish, greedy_next, kv4_quantize, rmsnorm, rope_append, silu_mul,
                      w4_embedding, w4a16_gemv_fused, w4a16_linear)

__all__ = ["SpectraFusedLinear", "SpectraFusedEmbedding", "DecoderConfig", "SpectraDecoder", "rope_inv_freq"]


def _block(group_size: Optional[int], codebook: str) -> int:
    """The quantization block: as given, else the codebook's own (32 for Format A, 64 for NF4)."""
    if group_size is not None:
        return int(group_size)
    return 32 if codebook == "asym" else 64


class SpectraFusedLinear(nn.Module):
    """Drop-in quantized linear: packed 4-bit weights, scales, zeros and outliers
    (engine.py:35-88); rows <= GEMV_MAX_M go to the GEMV family, larger batches to
    the MFMA GEMM (engine.py:94-124)."""

    def __init__(self, in_features: int, out_features: int, group_size: Optional[int] = None,
                 has_bias: bool = False, enable_hdsq: bool = True, marlin_layout: bool = False, *,
                 codebook: str = "asym", hadamard_block: int = 0):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        # None: the codebook's own block (32 for Format A as engine.py:42, 64 for NF4); an
        # explicit value is used as given
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
        self._op_args: Optional[tuple] = None

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
        self._op_args = None

    def _operands(self) -> QWeightOperands:
        if self._ops is None:
            use_o = self.enable_hdsq and self.outlier_idx is not None and self.outlier_weight is not None
            self._ops = QWeightOperands(
                self.packed_weight, self.scales, self.zeros, self.in_features, codebook=self.codebook,
                group_size=_block(self.group_size, self.codebook), hadamard_block=self.hadamard_block,
                marlin_layout=self.marlin_layout,
                outlier_idx=self.outlier_idx if use_o else None, outlier_w=self.outlier_weight if use_o else None,
                outlier_rowptr=self.outlier_rowptr if use_o else None, bias=self.bias)
        return self._ops

    def _apply(self, fn, *args, **kwargs):  # device/dtype moves invalidate the descriptor
        self._ops = None
        self._op_args = None
        return super()._apply(fn, *args, **kwargs)

    # validation and conversion of the operands (host reads of the outlier tensors) happen
    # once, eagerly, outside any torch.compile trace
    @torch.compiler.disable
    def _bind(self) -> tuple:
        L.load_torch_ops()
        args = self._operands().op_args
        if args is None:
            raise RuntimeError("operands built without holding their tensors cannot feed the operator")
        self._op_args = args
        return args

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """One call of the registered operator torch.ops.spectra_hip.w4a16_linear: GEMV
        family for one row, small-batch / GEMM families for more (engine.py:90-124).  The
        operator has a schema and a shape function, so torch.compile traces through it where
        the reference marks forward @torch.compiler.disable (engine.py:90)."""
        args = self._op_args
        if args is None:
            args = self._bind()
        return torch.ops.spectra_hip.w4a16_linear.default(x, *args)

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

    def __init__(self, num_embeddings: int, embedding_dim: int, group_size: Optional[int] = None,
                 marlin_layout: bool = False, *, codebook: str = "asym"):
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
            gs = _block(self.group_size, self.codebook)
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
    kv_bits: int = 16        # 16: fp16 cache; 4: the reference's 4-bit cache (engine.py:614-700)
    kv_window: int = 128     # kv_bits 4: recent positions also kept in fp16 (engine.py:685 residual_length)
    hadamard_block: int = 128
    outlier_ratio: float = 0.005
    seed: int = 0
    rope_scaling: Optional[dict] = None  # the RoPE parameters ``rope_inv_freq`` applies; None: unscaled

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


def rope_inv_freq(head_dim: int, theta: float, scaling: Optional[dict] = None) -> torch.Tensor:
    """float32 inverse RoPE frequencies theta^(-2i/d) for i < d/2 (transformers' default table,
    which the reference's loader installs in every rotary module: engine.py:1172-1179).
    ``scaling`` with ``rope_type`` ``llama3`` applies the Llama 3.1 frequency scaling: with
    wavelength w = 2 pi / f, frequencies whose w is shorter than original_context /
    high_freq_factor stay, those longer than original_context / low_freq_factor are divided
    by ``factor``, and between them s = (original_context / w - low) / (high - low) blends
    f / factor and f.  Any other ``rope_type`` raises ``ValueError``."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    kind = (scaling or {}).get("rope_type", (scaling or {}).get("type", "default"))
    if kind == "default":
        return inv
    if kind != "llama3":
        raise ValueError(f"rope_type {kind!r} is not supported (default and llama3 are)")
    try:
        factor, lo, hi = float(scaling["factor"]), float(scaling["low_freq_factor"]), float(scaling["high_freq_factor"])
        ctx = float(scaling["original_max_position_embeddings"])
    except KeyError as e:
        raise ValueError(f"llama3 rope parameters lack {e.args[0]!r}") from None
    wavelen = (2.0 * math.pi) / inv
    blend = ((ctx / wavelen - lo) / (hi - lo)).clamp(0.0, 1.0)
    scaled = inv / factor
    return torch.where(wavelen < ctx / hi, inv,
                       torch.where(wavelen > ctx / lo, scaled, (1.0 - blend) * scaled + blend * inv))


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
    """Batch-1 Llama-shaped decoder whose every linear is a ``SpectraFusedLinear`` -- Format
    B (fused QKV and gate_up per layer, engine.py:409-437) or Format A (the container's
    separate projections, engine.py:1004-1025) -- with a tied quantized embedding /
    lm_head (engine.py:1124-1168) and an fp16 KV cache.  Between the linears a layer runs
    the library's fused kernels (residual add + RMSNorm, RoPE + cache append, split-sequence
    decode attention, SiLU-mul) where the reference relies on Inductor fusion
    (engine.py:1240-1250); prefill attention over the prompt is a torch product.  A decode
    step is fully device-side (token, position and cache index live in device tensors), so
    it is captured once as a HIP graph and replayed per token (engine.py:1801-1860)."""

    def __init__(self, cfg: DecoderConfig = DecoderConfig(), device: Optional[torch.device] = None,
                 weights: Optional[dict] = None):
        """``weights`` (default: random init from ``cfg.seed``): ``layers`` = per layer
        (qkv, o, gate_up, down) ``NF4Weight``s or ``FormatAWeight``s -- qkv and gate_up may
        also be lists of the parts (q, k, v / gate, up) -- ``embed`` (the gather's rows, no
        rotation), ``lm_head`` (None = tied to ``embed``), ``norms`` = the 2 * layers + 1
        RMSNorm weights."""
        super().__init__()
        dev = device or torch.device("cuda")
        self.cfg = cfg
        c = cfg
        hd = c.head_dim
        if weights is None:
            weights = self._random_weights(c, dev)
        if len(weights["layers"]) != c.layers or len(weights["norms"]) != 2 * c.layers + 1:
            raise ValueError("weights do not match the config's layer count")

        from .container import FormatAWeight

        def linear(q):
            if isinstance(q, FormatAWeight):  # engine.py:1004-1025: group 32, no rotation
                lin = SpectraFusedLinear(q.k, q.n, 32, marlin_layout=q.marlin_layout).to(dev)
                lin.set_weights(q.packed, q.scales, q.zeros, outlier_idx=q.outlier_idx, outlier_weight=q.outlier_w,
                                marlin_layout=q.marlin_layout)
                return lin
            lin = SpectraFusedLinear(q.k, q.n, q.blocksize, codebook="nf4", hadamard_block=q.hadamard_block).to(dev)
            col, val = q.outliers()
            lin.set_weights(q.packed, q.absmax, None, outlier_idx=col, outlier_weight=val, marlin_layout=q.marlin_layout,
                            outlier_rowptr=q.rowptr if col is not None else None)
            return lin

        def parts(q):  # a weight, or the parts of one concatenated along N
            return list(q) if isinstance(q, (list, tuple)) else [q]

        self.layers_q = [tuple(weights["layers"][i]) for i in range(c.layers)]
        # qkv / gate_up: the parts' linears, each writing its columns of the fused output
        self.blocks = [dict(qkv=[linear(p) for p in parts(a)], o=linear(b), gate_up=[linear(p) for p in parts(g)],
                            down=linear(d)) for a, b, g, d in self.layers_q]
        qe = weights["embed"]
        self.embed_q = qe
        if isinstance(qe, FormatAWeight):
            self.embed = SpectraFusedEmbedding(c.vocab, c.hidden, 32, qe.marlin_layout)
            self.embed.set_weights(qe.packed, qe.scales, qe.zeros, qe.outlier_idx, qe.outlier_w, qe.marlin_layout)
        else:
            col, val = qe.outliers()
            self.embed = SpectraFusedEmbedding(c.vocab, c.hidden, qe.blocksize, qe.marlin_layout, codebook="nf4")
            self.embed.set_weights(qe.packed, qe.absmax, None, col, val, qe.marlin_layout,
                                   outlier_rowptr=qe.rowptr if col is not None else None)
        self.lm_q = weights.get("lm_head") or qe
        self.lm_head = linear(self.lm_q)
        # the fused decode step (RMSNorm / SiLU-mul prologues, one GEMV per fused projection)
        # needs NF4 linears throughout; otherwise the step runs the norms and SiLU-mul as
        # their own kernels and one GEMV per part
        self.fused = all(len(b["qkv"]) == 1 and len(b["gate_up"]) == 1 for b in self.blocks) and all(
            lin.codebook == "nf4" for b in self.blocks for lin in b["qkv"] + b["gate_up"] + [b["o"], b["down"]]) and \
            self.lm_head.codebook == "nf4"
        self.norm_w = [w.to(device=dev, dtype=torch.float32).contiguous() for w in weights["norms"]]
        self.norm_w16 = [w.half() for w in self.norm_w]  # the fused GEMV prologues read fp16 weights
        # KV cache [layer, kv, max_seq, head_dim]: a position's head is one 16-byte-aligned run
        if c.kv_bits not in (16, 4):
            raise ValueError("kv_bits must be 16 or 4")
        if c.kv_bits == 16:
            self.k_cache = torch.zeros(c.layers, c.kv_heads, c.max_seq, hd, device=dev, dtype=torch.float16)
            self.v_cache = torch.zeros(c.layers, c.kv_heads, c.max_seq, hd, device=dev, dtype=torch.float16)
        else:  # every position in 4 bits + fp16 rings of the last kv_window positions
            w = min(c.kv_window, c.max_seq)
            self.k_cache = torch.zeros(c.layers, c.kv_heads, w, hd, device=dev, dtype=torch.float16)
            self.v_cache = torch.zeros(c.layers, c.kv_heads, w, hd, device=dev, dtype=torch.float16)

            def q4():
                return (torch.zeros(c.layers, c.kv_heads, c.max_seq, hd // 2, device=dev, dtype=torch.uint8),
                        torch.zeros(c.layers, c.kv_heads, c.max_seq, hd // 32, device=dev, dtype=torch.float16),
                        torch.zeros(c.layers, c.kv_heads, c.max_seq, hd // 32, device=dev, dtype=torch.uint8))
            self.k4, self.v4 = q4(), q4()
        inv = rope_inv_freq(hd, c.rope_theta, c.rope_scaling).to(dev)
        ang = torch.arange(c.max_seq, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos, self.sin = torch.cos(ang), torch.sin(ang)  # [max_seq, hd/2]
        self.arange = torch.arange(c.max_seq, device=dev)
        # attention partials and the merge's arrival counters (zero before the first call)
        self.attn_ws = torch.zeros(attend_workspace_bytes(c.heads, hd, c.max_seq), device=dev, dtype=torch.uint8)
        # device-side decode state
        self.cur_id = torch.zeros(1, dtype=torch.int64, device=dev)
        self.cur_pos = torch.zeros(1, dtype=torch.int64, device=dev)
        self.history = torch.zeros(c.max_seq + 1, dtype=torch.int64, device=dev)  # token at each position
        self.pick = argmax_slots(dev)  # the lm_head GEMV's fused greedy pick (left at 0 by greedy_finish)
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.graph_logits: Optional[torch.Tensor] = None
        self.device = dev

    @staticmethod
    def _random_weights(c: DecoderConfig, dev) -> dict:
        gen = torch.Generator(device=dev).manual_seed(c.seed)
        kvd = c.kv_heads * c.head_dim

        def nf4(n, k, had):
            return _synthetic_nf4(n, k, gen, had, c.outlier_ratio, dev)

        layers = []
        for _ in range(c.layers):
            layers.append((nf4(c.hidden + 2 * kvd, c.hidden, c.hadamard_block), nf4(c.hidden, c.hidden, c.hadamard_block),
                           nf4(2 * c.inter, c.hidden, c.hadamard_block), nf4(c.hidden, c.inter, c.hadamard_block)))
        # tied embedding / lm_head: NF4 without rotation (the gather returns the stored rows)
        embed = nf4(c.vocab, c.hidden, 0)
        norms = [torch.ones(c.hidden, device=dev, dtype=torch.float32) for _ in range(2 * c.layers + 1)]
        return dict(layers=layers, embed=embed, lm_head=None, norms=norms)

    @classmethod
    def from_trdc(cls, path, device: Optional[torch.device] = None, max_seq: int = 1024,
                  rope: str = "reference") -> "SpectraDecoder":
        """A decoder on the quantized tensors of a TRDC container (engine.py:798-1080 binds a
        container's tensors to the model's modules by name): HF Llama names, norms from the
        lossless tensors, lm_head tied to the embedding when the container has none.
        Format B (``nf4_*``) q/k/v and gate/up are concatenated along N at load (exact: every
        Format B operand is row-local); Format A (``q4_g32_hdsq``) parts stay separate
        linears, since their dense outlier columns are per tensor.

        ``rope``: ``"reference"`` decodes with the unscaled table of the config's
        ``rope_theta`` whatever ``rope_type`` the config names, as the reference's loader
        does (engine.py:1170-1179 replaces every rotary module's table by
        ``compute_default_rope_parameters``), and warns when the config names a scaling;
        ``"config"`` applies the config's scaling (``rope_inv_freq``: llama3; other types
        raise ``ValueError``)."""
        from .compressor import NF4Weight
        from .container import FORMAT_A, TrdcReader, nf4_concat
        if rope not in ("reference", "config"):
            raise ValueError("rope must be 'reference' or 'config'")
        dev = device or torch.device("cuda")
        with TrdcReader(path) as rd:
            cf = rd.config
            rp = cf.get("rope_parameters") or cf.get("rope_scaling") or {}
            theta = cf.get("rope_theta") or rp.get("rope_theta") or 10000.0
            kind = rp.get("rope_type", rp.get("type", "default"))
            scaling = None
            if kind != "default":
                if rope == "config":
                    scaling = dict(rp)
                    rope_inv_freq(2, 1.0, scaling)  # unsupported types and missing keys raise here
                else:
                    warnings.warn(f"container config names rope_type {kind!r}; decoding with the unscaled "
                                  "table as the reference's loader does (from_trdc(..., rope='config') "
                                  "applies the scaling)", stacklevel=2)
            c = DecoderConfig(layers=cf["num_hidden_layers"], hidden=cf["hidden_size"],
                              heads=cf["num_attention_heads"],
                              kv_heads=cf.get("num_key_value_heads") or cf["num_attention_heads"],
                              inter=cf["intermediate_size"], vocab=cf["vocab_size"],
                              rope_theta=float(theta), rope_scaling=scaling,
                              rms_eps=float(cf.get("rms_norm_eps") or 1e-6), max_seq=max_seq)
            if cf.get("head_dim") not in (None, c.head_dim):
                raise ValueError(f"head_dim {cf.get('head_dim')} != hidden / heads ({c.head_dim})")

            def q4(name):
                if name not in rd.tensors:
                    raise ValueError(f"container has no tensor {name!r}")
                t = rd.tensors[name]["type"]
                if not (t.startswith("nf4_") or t in (FORMAT_A, "q4_g32")):
                    raise ValueError(f"{name!r} is {t!r}: the decoder runs 4-bit quantized tensors")
                return rd.load(name, dev)

            def fuse(names):
                ws = [q4(n) for n in names]
                return nf4_concat(ws) if all(isinstance(w, NF4Weight) for w in ws) else ws

            def vec(name):
                return rd.load(name, dev).float()

            layers, norms = [], []
            for i in range(c.layers):
                p = f"model.layers.{i}."
                a = p + "self_attn."
                m = p + "mlp."
                layers.append((fuse([a + "q_proj.weight", a + "k_proj.weight", a + "v_proj.weight"]),
                               q4(a + "o_proj.weight"),
                               fuse([m + "gate_proj.weight", m + "up_proj.weight"]),
                               q4(m + "down_proj.weight")))
                norms += [vec(p + "input_layernorm.weight"), vec(p + "post_attention_layernorm.weight")]
            norms.append(vec("model.norm.weight"))
            embed = q4("model.embed_tokens.weight")
            head = q4("lm_head.weight") if "lm_head.weight" in rd.tensors else None
        return cls(c, dev, dict(layers=layers, embed=embed, lm_head=head, norms=norms))

    # -- building blocks ---------------------------------------------------------------------
    def _layer(self, li: int, h: torch.Tensor, delta: Optional[torch.Tensor], pos: torch.Tensor,
               causal_len: Optional[int]) -> torch.Tensor:
        """One prefill layer for T tokens at positions 0..T-1 (``pos``, device int64 [T];
        causal_len = T).  ``h`` is the residual stream, updated in place with the previous
        layer's output ``delta``; returns this layer's MLP output (added by the next norm)."""
        c, blk = self.cfg, self.blocks[li]
        hd, T = c.head_dim, h.shape[0]
        g = c.heads // c.kv_heads
        x = rmsnorm(h, self.norm_w[2 * li], c.rms_eps, residual=delta)
        qkv = self._project(blk["qkv"], x)
        L = causal_len
        if c.kv_bits == 16:
            kc, vc = self.k_cache[li], self.v_cache[li]
        else:  # the prompt attends in full precision; the cache keeps it in 4 bits (+ the window)
            kc = torch.empty(c.kv_heads, L, hd, device=h.device, dtype=torch.float16)
            vc = torch.empty_like(kc)
        q = rope_append(qkv, pos, self.cos[:kc.shape[1]].contiguous(), self.sin[:kc.shape[1]].contiguous(), c.heads,
                        c.kv_heads, kc, vc)
        if c.kv_bits == 4:
            k4 = tuple(t[li] for t in self.k4)
            v4 = tuple(t[li] for t in self.v4)
            kv4_quantize(kc, out=k4, out_rows=c.max_seq)
            kv4_quantize(vc, out=v4, out_rows=c.max_seq)
            w = self.k_cache.shape[2]
            last = self.arange[max(0, L - w):L]  # the window's positions -> ring slots position % window
            self.k_cache[li].index_copy_(1, last % w, kc[:, last])
            self.v_cache[li].index_copy_(1, last % w, vc[:, last])
        qg = q.permute(1, 0, 2).reshape(c.kv_heads, g * T, hd).contiguous()  # head = kv * g + j
        kt = kc[:, :L, :].transpose(1, 2).contiguous()  # [kv, hd, L]
        vv = vc[:, :L, :].contiguous()
        s = torch.matmul(qg, kt).float() * (1.0 / math.sqrt(hd))  # [kv, g*T, L]
        qpos = pos.repeat(g)  # row r = j * T + t -> position pos[t]
        s = s.masked_fill((self.arange[:L][None, :] > qpos[:, None])[None], float("-inf"))
        a = torch.matmul(torch.softmax(s, dim=-1).half(), vv)  # [kv, g*T, hd]
        a = a.reshape(c.heads, T, hd).permute(1, 0, 2).reshape(T, c.hidden)
        o = blk["o"](a)
        x = rmsnorm(h, self.norm_w[2 * li + 1], c.rms_eps, residual=o)
        return blk["down"](silu_mul(self._project(blk["gate_up"], x)))

    @staticmethod
    def _project(parts, x: torch.Tensor) -> torch.Tensor:
        """The fused projection of ``x`` through the parts' linears (columns in part order)."""
        if len(parts) == 1:
            return parts[0](x)
        return torch.cat([p(x) for p in parts], dim=-1)

    @staticmethod
    def _gemv_parts(parts, x: torch.Tensor) -> torch.Tensor:
        """One-row ``_project``: each part's GEMV writes its columns of one output row."""
        out = torch.empty((1, sum(p.out_features for p in parts)), device=x.device, dtype=torch.float16)
        off = 0
        for p in parts:
            w4a16_gemv_fused(p._operands(), x, out=out[:, off: off + p.out_features])
            off += p.out_features
        return out

    def _layer_decode(self, li: int, h: torch.Tensor, pos: torch.Tensor) -> None:
        """One decoder layer for the token at device position ``pos``, five kernels: the
        span merge rides in the attention kernel, the RMSNorms ride in the QKV / gate_up GEMV prologues, SiLU-mul in the down_proj prologue,
        the residual adds in the o_proj / down_proj epilogues (``h`` updated in place).
        Without NF4 linears throughout (``fused`` False) the norms and SiLU-mul are kernels
        of their own and each part of QKV / gate_up its own GEMV."""
        c, blk = self.cfg, self.blocks[li]
        if self.fused:
            qkv = w4a16_gemv_fused(blk["qkv"][0]._operands(), h, prologue="rmsnorm",
                                   norm_weight=self.norm_w16[2 * li], eps=c.rms_eps)
        else:
            qkv = self._gemv_parts(blk["qkv"], rmsnorm(h, self.norm_w[2 * li], c.rms_eps))
        if c.kv_bits == 16:
            a = attend_decode(qkv, pos, self.cos, self.sin, c.heads, c.kv_heads, self.k_cache[li], self.v_cache[li],
                              self.attn_ws)
        else:
            a = attend_decode_q4(qkv, pos, self.cos, self.sin, c.heads, c.kv_heads, self.k_cache[li],
                                 self.v_cache[li], tuple(t[li] for t in self.k4), tuple(t[li] for t in self.v4),
                                 self.attn_ws)
        w4a16_gemv_fused(blk["o"]._operands(), a.reshape(1, c.hidden), residual=h, out=h)
        if self.fused:
            gu = w4a16_gemv_fused(blk["gate_up"][0]._operands(), h, prologue="rmsnorm",
                                  norm_weight=self.norm_w16[2 * li + 1], eps=c.rms_eps)
            w4a16_gemv_fused(blk["down"]._operands(), gu, prologue="silu_mul", residual=h, out=h)
        else:
            gu = self._gemv_parts(blk["gate_up"], rmsnorm(h, self.norm_w[2 * li + 1], c.rms_eps))
            w4a16_gemv_fused(blk["down"]._operands(), silu_mul(gu), residual=h, out=h)

    def forward_tokens(self, ids: torch.Tensor, pos: torch.Tensor, causal_len: Optional[int],
                       pick: bool = False) -> torch.Tensor:
        """Logits of the last token.  ``pick`` (decode only): the lm_head GEMV also gathers the
        greedy pick into ``self.pick``, which ``greedy_finish`` must then consume."""
        h = self.embed(ids)
        c = self.cfg
        if causal_len is None:  # decode: one token, fused GEMVs
            for li in range(c.layers):
                self._layer_decode(li, h, pos)
            key = self.pick if pick else None
            if not self.fused:
                return w4a16_gemv_fused(self.lm_head._operands(), rmsnorm(h, self.norm_w[-1], c.rms_eps),
                                        argmax_key=key)
            return w4a16_gemv_fused(self.lm_head._operands(), h, prologue="rmsnorm", norm_weight=self.norm_w16[-1],
                                    eps=c.rms_eps, argmax_key=key)
        delta = None
        for li in range(c.layers):
            delta = self._layer(li, h, delta, pos, causal_len)
        x = rmsnorm(h[-1:], self.norm_w[2 * c.layers], c.rms_eps, residual=delta[-1:])
        return self.lm_head(x)  # logits of the last token [1, vocab]

    # -- generation --------------------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        T = prompt.numel()
        if T >= self.cfg.max_seq:
            raise ValueError(f"prompt of {T} tokens does not fit max_seq={self.cfg.max_seq}")
        ids = prompt.reshape(-1).to(self.device)
        self.history[:T].copy_(ids)
        self.cur_pos.fill_(T - 1)
        logits = self.forward_tokens(ids, self.arange[:T], T)
        greedy_next(logits[0], self.cur_id, self.history, self.cur_pos)  # history[T], cur_pos = T
        return logits

    def _decode_step(self) -> torch.Tensor:
        logits = self.forward_tokens(self.cur_id, self.cur_pos, None, pick=True)  # the pick rides on the lm_head
        greedy_finish(self.pick, self.cur_id, self.history, self.cur_pos)
        return logits

    def cache_tensors(self):
        """Every tensor of the KV cache (fp16 cache, or 4-bit codes / scales / zeros + rings)."""
        extra = list(self.k4) + list(self.v4) if self.cfg.kv_bits == 4 else []
        return [self.k_cache, self.v_cache] + extra

    @torch.no_grad()
    def capture_decode(self) -> None:
        """Capture one decode step (all linears, attention and the sampling) as a HIP graph."""
        saved = (self.cur_id.clone(), self.cur_pos.clone(), self.history.clone(),
                 [t.clone() for t in self.cache_tensors()])
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
        self.history.copy_(saved[2])
        for t, b in zip(self.cache_tensors(), saved[3]):
            t.copy_(b)

    @torch.no_grad()
    def decode(self, steps: int, use_graph: bool = True) -> torch.Tensor:
        """``steps`` greedy decode steps after a prefill; returns the tokens they consumed (the
        first is the prefill's prediction), a device int64 [steps] view of the history."""
        p0 = int(self.cur_pos)  # one host read before the loop; the steps themselves never sync
        if p0 + steps > self.cfg.max_seq:
            raise ValueError(f"{steps} steps from position {p0} exceed max_seq={self.cfg.max_seq}")
        if use_graph and self.graph is None:
            self.capture_decode()
        for _ in range(steps):
            if use_graph:
                self.graph.replay()
            else:
                self._decode_step()
        return self.history[p0: p0 + steps]
