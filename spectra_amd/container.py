"""The TRDC model container: the reference's checkpoint format, read and written here
(reference spectra/compressor.py:20 magic, :393-635 ``compress``; spectra/engine.py:798-1080
the loader), with one more tensor type for Format B.

Layout (little-endian): ``b"TRDC4B01"`` | ``<QQ`` manifest offset, manifest length | the
tensors' bytes, one after the other | the JSON manifest.  Per tensor the manifest holds
``type``, ``shape``, ``offset`` and the lengths of its parts, which follow each other from
``offset``:

* ``q4_g32_hdsq`` (Format A, the reference's type, written byte-identically): packed uint8
  [N, K/2] (marlin nibble order), scales fp16 [N, K/32], zero points packed two per byte
  uint8 [N, ceil(K/64)], outlier column indices int32 [n_out], outlier columns [N, n_out];
* ``nf4_b<block>_had<H>_csr`` (Format B, this build): packed uint8 [N, K/2], absmax fp16
  [N, K/block], CSR rowptr int32 [N+1], col int32 [nnz], val fp16 [nnz] -- exactly the
  kernel operands, so loading is a copy of the file's bytes to the device;
* ``lossless_<dtype>``: the raw tensor.

The writer streams to ``<file>.tmp`` and renames it when the manifest is in place
(compressor.py:421, :573-575).  The reader memory-maps the file (copy-on-write) and copies
each tensor straight from the mapping to its device; it checks the header like the
reference's loader (engine.py:799-813): a short file, a wrong magic, a manifest beyond the
end or a tensor outside the data region raise ``ValueError``.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Dict, Iterator, Optional, Tuple, Union

import numpy as np
import torch

from .kernels import validate_outliers

__all__ = ["MAGIC", "FORMAT_A", "nf4_type", "TrdcWriter", "TrdcReader", "FormatAWeight", "norm_vector_for",
           "prescan_norm_vectors", "stream_checkpoint", "compress_checkpoint", "nf4_concat", "select_csr_outliers"]

MAGIC = b"TRDC4B01"
HEADER_BYTES = 24
FORMAT_A = "q4_g32_hdsq"

_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32, "int64": torch.int64,
           "int32": torch.int32, "int16": torch.int16, "int8": torch.int8, "uint8": torch.uint8, "bool": torch.bool}


def nf4_type(block: int, hadamard_block: int) -> str:
    return f"nf4_b{block}_had{hadamard_block}_csr"


def _bytes(t: torch.Tensor) -> bytes:
    """Raw little-endian bytes of a tensor in memory order (any dtype, bf16 included)."""
    return t.detach().contiguous().cpu().reshape(-1).view(torch.uint8).numpy().tobytes()


def _dtype_name(t: torch.Tensor) -> str:
    return str(t.dtype).replace("torch.", "")


# ---------------------------------------------------------------------------
# writer
# ---------------------------------------------------------------------------
class TrdcWriter:
    """Streams tensors into a container; ``close()`` (or leaving the ``with`` block) writes
    the manifest and moves the file into place.  ``head`` is the manifest's leading part
    (the reference's keys: version, group_size, base_outlier_ratio, architecture, config)."""

    def __init__(self, path: Union[str, Path], head: Dict[str, Any]):
        self.path = Path(path)
        self.path.parent.mkdir(parents=True, exist_ok=True)
        self.tmp = self.path.with_suffix(".tmp")
        self.manifest = dict(head)
        self.manifest["tensors"] = {}
        self.f = open(self.tmp, "wb")
        self.f.write(MAGIC)
        self.f.write(struct.pack("<QQ", 0, 0))

    def _put(self, parts) -> Tuple[int, list]:
        off = self.f.tell()
        lens = []
        for b in parts:
            self.f.write(b)
            lens.append(len(b))
        return off, lens

    def add_format_a(self, name: str, shape, packed: torch.Tensor, scales: torch.Tensor, packed_zeros: torch.Tensor,
                     outlier_idx: torch.Tensor, outlier_w: torch.Tensor, ratio: float, kurtosis: float) -> None:
        """A ``q4_g32_hdsq`` entry with the reference's manifest keys in its order
        (compressor.py:496-515)."""
        idx = outlier_idx.to(torch.int32)
        off, (lp, ls, lz, li, lw) = self._put([_bytes(packed), _bytes(scales), _bytes(packed_zeros), _bytes(idx),
                                                _bytes(outlier_w)])
        self.manifest["tensors"][name] = {
            "type": FORMAT_A, "shape": list(shape), "offset": off,
            "packed_len": lp, "scale_len": ls, "zero_len": lz, "zero_packed": True,
            "outlier_idx_len": li, "outlier_idx_dtype": "int32",
            "outlier_w_len": lw, "outlier_w_dtype": _dtype_name(outlier_w),
            "num_outliers": idx.numel(), "outlier_ratio": round(ratio, 4), "kurtosis": round(kurtosis, 2),
            "marlin_layout": True, "total_len": lp + ls + lz + li + lw}

    def add_nf4(self, name: str, q, outlier_ratio: Optional[float] = None) -> None:
        """A Format B entry: the ``NF4Weight`` operands as they sit in device memory."""
        parts = [_bytes(q.packed), _bytes(q.absmax), _bytes(q.rowptr.to(torch.int32)), _bytes(q.col.to(torch.int32)),
                 _bytes(q.val.to(torch.float16))]
        off, (lp, la, lr, lc, lv) = self._put(parts)
        e = {"type": nf4_type(q.blocksize, q.hadamard_block), "shape": [q.n, q.k], "offset": off,
             "packed_len": lp, "absmax_len": la, "rowptr_len": lr, "col_len": lc, "val_len": lv,
             "block": q.blocksize, "hadamard_block": q.hadamard_block, "marlin_layout": bool(q.marlin_layout),
             "nnz": q.col.numel()}
        if outlier_ratio is not None:
            e["outlier_ratio"] = round(outlier_ratio, 6)
        e["total_len"] = lp + la + lr + lc + lv
        self.manifest["tensors"][name] = e

    def add_lossless(self, name: str, t: torch.Tensor) -> None:
        dt = _dtype_name(t)
        off, (ln,) = self._put([_bytes(t)])
        self.manifest["tensors"][name] = {"type": f"lossless_{dt}", "dtype": dt, "shape": list(t.shape),
                                          "offset": off, "total_len": ln}

    def close(self) -> Path:
        if self.f is None:
            return self.path
        moff = self.f.tell()
        mjson = json.dumps(self.manifest).encode("utf-8")
        self.f.write(mjson)
        self.f.seek(8)
        self.f.write(struct.pack("<QQ", moff, len(mjson)))
        self.f.close()
        self.f = None
        if self.path.exists():
            self.path.unlink()
        self.tmp.rename(self.path)
        return self.path

    def abort(self) -> None:
        if self.f is not None:
            self.f.close()
            self.f = None
            self.tmp.unlink(missing_ok=True)

    def __enter__(self):
        return self

    def __exit__(self, et, ev, tb):
        if et is None:
            self.close()
        else:
            self.abort()


# ---------------------------------------------------------------------------
# reader
# ---------------------------------------------------------------------------
@dataclass
class FormatAWeight:
    """Operands of a ``q4_g32_hdsq`` tensor as the reference's loader binds them
    (engine.py:1004-1025): zero points unpacked, outlier indices widened to int64."""
    packed: torch.Tensor          # uint8 [N, K/2]
    scales: torch.Tensor          # fp16 [N, K/32]
    zeros: torch.Tensor           # uint8 [N, K/32]
    outlier_idx: Optional[torch.Tensor]  # int64 [n_out]
    outlier_w: Optional[torch.Tensor]    # [N, n_out]
    k: int
    marlin_layout: bool = True

    @property
    def n(self) -> int:
        return self.packed.shape[0]


class TrdcReader:
    def __init__(self, path: Union[str, Path]):
        self.path = Path(path)
        size = self.path.stat().st_size
        if size < HEADER_BYTES:
            raise ValueError(f"TRDC container '{self.path.name}' is corrupted or empty ({size} bytes)")
        self._file = open(self.path, "rb")
        try:
            magic = self._file.read(8)
            if magic != MAGIC:
                raise ValueError(f"Invalid container header: {magic!r}")
            moff, mlen = struct.unpack("<QQ", self._file.read(16))
            if moff + mlen > size or moff < HEADER_BYTES:
                raise ValueError(f"Corrupted TRDC manifest table in '{self.path.name}': manifest offset ({moff}) + "
                                 f"length ({mlen}) exceeds file size ({size})")
            self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_COPY)
        except Exception:
            self._file.close()
            raise
        self.manifest = json.loads(bytes(self._map[moff:moff + mlen]).decode("utf-8"))
        self.tensors: Dict[str, Dict[str, Any]] = self.manifest["tensors"]
        self.config: Dict[str, Any] = self.manifest.get("config", {})
        self.group_size: int = self.manifest.get("group_size", 32)
        self._size = size
        for name, meta in self.tensors.items():
            if meta["offset"] < HEADER_BYTES or meta["offset"] + meta["total_len"] > moff:
                raise ValueError(f"tensor '{name}' lies outside the container's data region")

    def close(self) -> None:
        if self._map is not None:
            try:
                self._map.close()
            except BufferError:  # a caller still holds a view: the mapping goes with it
                pass
            self._file.close()
            self._map = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _parts(self, meta, keys) -> Iterator[memoryview]:
        pos = meta["offset"]
        for k in keys:
            n = meta.get(k, 0)
            yield memoryview(self._map)[pos:pos + n]
            pos += n

    @staticmethod
    def _tensor(buf: memoryview, dtype: torch.dtype, shape) -> torch.Tensor:
        if len(buf) == 0:
            return torch.empty(shape, dtype=dtype)
        return torch.frombuffer(buf, dtype=dtype).reshape(shape)

    def load(self, name: str, device: Optional[Union[str, torch.device]] = None):
        """The tensor ``name`` as kernel operands (on ``device``, copied straight from the
        mapping; CPU copies when None, independent of the reader's lifetime):
        ``FormatAWeight`` / ``NF4Weight`` / a plain tensor."""
        meta = self.tensors[name]
        ttype = meta["type"]
        mv = (lambda t: t.to(device)) if device is not None else (lambda t: t.clone())
        if ttype in (FORMAT_A, "q4_g32"):
            n, k = meta["shape"]
            g = self.group_size
            p_b, s_b, z_b, i_b, w_b = self._parts(meta, ["packed_len", "scale_len", "zero_len", "outlier_idx_len",
                                                         "outlier_w_len"])
            packed = mv(self._tensor(p_b, torch.uint8, (n, k // 2)))
            scales = mv(self._tensor(s_b, torch.float16, (n, k // g)))
            if meta.get("zero_packed", False):  # engine.py:1007-1012
                pz = self._tensor(z_b, torch.uint8, (n, -1)) if len(z_b) else torch.empty((n, 0), dtype=torch.uint8)
                z = torch.empty((n, pz.shape[1] * 2), dtype=torch.uint8)
                z[:, 0::2] = pz & 0x0F
                z[:, 1::2] = (pz >> 4) & 0x0F
                zeros = mv(z[:, : k // g].contiguous())
            else:
                zeros = mv(self._tensor(z_b, torch.uint8, (n, k // g)))
            idx = ow = None
            if meta.get("outlier_idx_len", 0) > 0:  # engine.py:1015-1025
                idt = meta.get("outlier_idx_dtype", "int64")
                if idt == "uint16":
                    idx = torch.from_numpy(np.frombuffer(i_b, dtype=np.uint16).astype(np.int64))
                elif idt == "int32":
                    idx = self._tensor(i_b, torch.int32, (-1,)).to(torch.int64)
                else:
                    idx = self._tensor(i_b, torch.int64, (-1,))
                wdt = _DTYPES.get(meta.get("outlier_w_dtype", "float16"), torch.float16)
                idx = mv(idx)
                ow = mv(self._tensor(w_b, wdt, (n, -1)))
                validate_outliers(n, k, idx=idx, ow=ow)
            return FormatAWeight(packed, scales, zeros, idx, ow, k, bool(meta.get("marlin_layout", False)))
        if ttype.startswith("nf4_"):
            from .compressor import NF4Weight
            n, k = meta["shape"]
            blk = meta["block"]
            p_b, a_b, r_b, c_b, v_b = self._parts(meta, ["packed_len", "absmax_len", "rowptr_len", "col_len", "val_len"])
            rowptr = mv(self._tensor(r_b, torch.int32, (n + 1,)))
            col = mv(self._tensor(c_b, torch.int32, (-1,)))
            val = mv(self._tensor(v_b, torch.float16, (-1,)))
            validate_outliers(n, k, rowptr=rowptr, col=col, val=val)
            return NF4Weight(mv(self._tensor(p_b, torch.uint8, (n, k // 2))),
                             mv(self._tensor(a_b, torch.float16, (n, k // blk))),
                             rowptr, col, val,
                             k, blk, int(meta["hadamard_block"]), bool(meta.get("marlin_layout", True)))
        if "lossless" in ttype:
            (raw,) = self._parts(meta, ["total_len"])
            dt = _DTYPES.get(meta.get("dtype", "float16"), torch.float16)
            return mv(self._tensor(raw, dt, meta["shape"]))
        raise ValueError(f"unknown tensor type {ttype!r} of '{name}'")


# ---------------------------------------------------------------------------
# checkpoint streaming and the compressor
# ---------------------------------------------------------------------------
_NORM_KEYWORDS = ("layernorm.weight", "norm.weight", "ln.weight", "ln_1.weight", "ln_2.weight", "ln_f.weight")


def _safetensor_files(model_dir: Path):
    index = model_dir / "model.safetensors.index.json"
    if index.exists():
        with open(index) as f:
            shards = sorted(set(json.load(f)["weight_map"].values()))
        return [model_dir / s for s in shards]
    return sorted(model_dir.glob("*.safetensors"))


def stream_checkpoint(model_dir: Union[str, Path]) -> Iterator[Tuple[str, torch.Tensor]]:
    """One tensor at a time from a local safetensors checkpoint, shards in sorted order and
    keys in file order (compressor.py:217-240)."""
    from safetensors import safe_open
    files = _safetensor_files(Path(model_dir))
    if not files:
        raise ValueError(f"no safetensors checkpoint in {model_dir}")
    for sf in files:
        with safe_open(str(sf), framework="pt", device="cpu") as f:
            for k in f.keys():
                yield k, f.get_tensor(k)


def prescan_norm_vectors(model_dir: Union[str, Path]) -> Dict[str, torch.Tensor]:
    """|gamma| of the 1-D normalisation weights (compressor.py:275-300)."""
    from safetensors import safe_open
    out = {}
    for sf in _safetensor_files(Path(model_dir)):
        with safe_open(str(sf), framework="pt", device="cpu") as f:
            for k in f.keys():
                if any(nk in k.lower() for nk in _NORM_KEYWORDS):
                    t = f.get_tensor(k)
                    if t.ndim == 1:
                        out[k] = t.detach().float().abs()
    return out


def norm_vector_for(name: str, norm_map: Dict[str, torch.Tensor], in_features: int) -> Optional[torch.Tensor]:
    """The norm that scales a projection's input (compressor.py:326-391): attention inputs ->
    the layer's attention pre-norm, MLP inputs -> its MLP pre-norm, nothing for output
    projections, embeddings and the head."""
    low = name.lower()
    attn_in = any(x in low for x in ("q_proj", "k_proj", "v_proj", "qkv_proj", "c_attn", "in_proj", "w_pack",
                                     "in_proj_weight"))
    mlp_in = any(x in low for x in ("gate_proj", "up_proj", "fc1", "c_fc", "w1", "w3", "gate_up_proj",
                                    "input_linear", "shared_mlp"))
    if not (attn_in or mlp_in):
        return None
    parts = name.split(".")
    prefix = None
    for i, p in enumerate(parts):
        if p in ("layers", "h", "blocks", "block") and i + 1 < len(parts) and parts[i + 1].isdigit():
            prefix = ".".join(parts[: i + 2])
            break
    if prefix is None:
        return None
    attn_c = ("input_layernorm", "attention_norm", "ln_1", "operator_norm", "norm1", "norm")
    mlp_c = ("post_attention_layernorm", "ffn_norm", "ln_2", "mlp_norm", "norm2", "norm", "shared_mlp_norm")
    for c in (attn_c if attn_in else mlp_c):
        key = f"{prefix}.{c}.weight"
        if key in norm_map and norm_map[key].numel() == in_features:
            return norm_map[key]
    for k, v in norm_map.items():
        if k.startswith(prefix) and v.numel() == in_features:
            kl = k.lower()
            if attn_in and any(x in kl for x in ("input", "ln_1", "attention", "norm1", "norm")):
                return v
            if mlp_in and any(x in kl for x in ("post", "ln_2", "ffn", "mlp", "norm2", "norm")):
                return v
    return None


def select_csr_outliers(w_rot: torch.Tensor, ratio: float) -> Optional[torch.Tensor]:
    """Format B outlier positions: in every row the round(ratio * K) entries of largest
    magnitude in the stored (rotated) basis, equal magnitudes lowest column first.
    Returns a boolean mask (None when no entry is kept)."""
    n, k = w_rot.shape
    per_row = int(round(ratio * k))
    if per_row <= 0:
        return None
    order = torch.sort(w_rot.float().abs(), dim=1, descending=True, stable=True).indices[:, :per_row]
    mask = torch.zeros((n, k), dtype=torch.bool, device=w_rot.device)
    mask.scatter_(1, order, True)
    return mask


def _rotation_block(name: str, k: int, hadamard_block: int) -> int:
    """Embedding rows are gathered, not multiplied, and the head shares them: no rotation."""
    low = name.lower()
    if hadamard_block <= 0 or "embed" in low or "lm_head" in low or k % hadamard_block:
        return 0
    return hadamard_block


def compress_checkpoint(model_dir: Union[str, Path], output_file: Union[str, Path], fmt: str = "nf4",
                        group_size: int = 32, base_outlier_ratio: float = 0.01, adaptive_kurtosis: bool = True,
                        nf4_block: int = 64, hadamard_block: int = 128, csr_ratio: float = 0.005,
                        config: Optional[Dict[str, Any]] = None,
                        device: Optional[torch.device] = None) -> Dict[str, Any]:
    """Compress a local safetensors checkpoint into a container (compressor.py:393-635).

    ``fmt="q4_g32"``: every 2-D tensor with K % 32 == 0 becomes ``q4_g32_hdsq`` exactly as the
    reference writes it (kurtosis-adaptive outlier columns with the layer's norm vector,
    group-32 quantization); the container is byte-identical to the reference's.
    ``fmt="nf4"``: Format B -- rows rotated by the blockwise FWHT (``hadamard_block``; not for
    the embedding / head), the ``csr_ratio`` largest magnitudes of every row kept as fp16 CSR
    outliers, NF4 with fp16 absmax per ``nf4_block``.  Other tensors are stored lossless.
    ``config`` overrides the model config read from ``config.json``."""
    from . import compressor as C
    from .kernels import fwht_rows
    model_dir = Path(model_dir)
    if fmt not in ("nf4", "q4_g32"):
        raise ValueError("fmt must be 'nf4' or 'q4_g32'")
    if config is None:
        from transformers import AutoConfig
        config = AutoConfig.from_pretrained(str(model_dir)).to_dict()
    dev = device or torch.device("cuda")
    head = {"version": MAGIC.decode(), "group_size": group_size if fmt == "q4_g32" else nf4_block,
            "base_outlier_ratio": base_outlier_ratio if fmt == "q4_g32" else csr_ratio,
            "architecture": config.get("architectures", ["AutoModelForCausalLM"])[0], "config": config}
    comp = C.SpectraCompressor(group_size=32, base_outlier_ratio=base_outlier_ratio,
                               adaptive_kurtosis=adaptive_kurtosis) if fmt == "q4_g32" else None
    norm_map = prescan_norm_vectors(model_dir) if fmt == "q4_g32" else {}
    n_in = n_q = 0
    with TrdcWriter(output_file, head) as wr:
        for name, param in stream_checkpoint(model_dir):
            n_in += param.numel() * param.element_size()
            gs = group_size if fmt == "q4_g32" else nf4_block
            if param.ndim == 2 and param.shape[1] >= gs and param.shape[1] % gs == 0:
                n, k = param.shape
                w = param.to(dev)
                if fmt == "q4_g32":
                    nv = norm_vector_for(name, norm_map, k)
                    w_dense, idx, ow, ratio, kurt = comp._isolate_hdsq_outliers(w, norm_vector=nv)
                    packed, scales, pz = C.compute_group32_quant(w, group_size, outlier_idx=idx)
                    wr.add_format_a(name, [n, k], packed, scales, pz, idx, ow, ratio, kurt)
                else:
                    had = _rotation_block(name, k, hadamard_block)
                    w_rot = fwht_rows(w.contiguous(), had, out_dtype=torch.float32) if had else w.float()
                    mask = select_csr_outliers(w_rot, csr_ratio)
                    q = C.quantize_nf4(w_rot, nf4_block, 0, mask, True)
                    q.hadamard_block = had
                    wr.add_nf4(name, q, outlier_ratio=q.col.numel() / float(n * k))
                n_q += 1
                del w
            else:
                wr.add_lossless(name, param)
    size = Path(output_file).stat().st_size
    return {"container": str(output_file), "format": fmt, "quantized_tensors": n_q, "uncompressed_bytes": n_in,
            "compressed_bytes": size, "compression_ratio": round(n_in / max(size, 1), 2)}


# ---------------------------------------------------------------------------
# Format B operand fusion along N (fused QKV / gate_up at load)
# ---------------------------------------------------------------------------
def nf4_concat(parts):
    """Row-concatenation of Format B weights with the same K, block, rotation and nibble
    order: every operand is row-local, so the fused weight is exact."""
    from .compressor import NF4Weight
    p0 = parts[0]
    for q in parts[1:]:
        if (q.k, q.blocksize, q.hadamard_block, q.marlin_layout) != (p0.k, p0.blocksize, p0.hadamard_block,
                                                                      p0.marlin_layout):
            raise ValueError("only Format B weights with equal K, block, rotation and layout concatenate")
    rowptrs, base = [], 0
    for i, q in enumerate(parts):
        rp = q.rowptr.to(torch.int64)
        rowptrs.append((rp if i == 0 else rp[1:]) + base)
        base += int(q.col.numel())
    return NF4Weight(torch.cat([q.packed for q in parts]), torch.cat([q.absmax for q in parts]),
                     torch.cat(rowptrs).to(torch.int32), torch.cat([q.col for q in parts]),
                     torch.cat([q.val for q in parts]), p0.k, p0.blocksize, p0.hadamard_block, p0.marlin_layout)
