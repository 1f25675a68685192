"""Writes the golden TRDC container of a tiny Llama-shaped checkpoint with the reference's
own compressor (reference spectra/compressor.py:393-635 ``SpectraCompressor.compress``:
header ``TRDC4B01`` + ``<QQ`` manifest location, raw tensors, JSON manifest; Format A
``q4_g32_hdsq`` for every compressible matrix, ``lossless_<dtype>`` otherwise).

Nothing in the reference's tests pins the container layout, so the bytes are taken from the
reference module itself, loaded by path in this (build) container on the CPU.  The
fixture is data only: ``tiny_llama_g32.trdc`` (the container bytes).  The checkpoint it
compresses is regenerated from a seed by ``make_checkpoint`` (the tests call it too).

    python tests/golden/make_trdc_golden.py /path/to/reference
"""
from __future__ import annotations

import importlib.util
import os
import shutil
import sys

sys.dont_write_bytecode = True  # loading the reference by path must leave no __pycache__ in its tree
import tempfile

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "tiny_llama_g32.trdc")

TINY = dict(hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, vocab_size=256, max_position_embeddings=128, tie_word_embeddings=True,
            rope_theta=10000.0, rms_norm_eps=1e-5, torch_dtype="float16")


def tiny_state_dict(seed: int = 7) -> dict:
    """HF Llama tensor names; fp16 weights N(0, 0.02) with a few heavy input columns per
    matrix (so the outlier selection has something to find); fp16 norms near 1."""
    g = torch.Generator().manual_seed(seed)
    h, inter, L, vocab = TINY["hidden_size"], TINY["intermediate_size"], TINY["num_hidden_layers"], TINY["vocab_size"]
    hd = h // TINY["num_attention_heads"]
    kvd = TINY["num_key_value_heads"] * hd

    def mat(n, k):
        w = torch.randn(n, k, generator=g) * 0.02
        cols = torch.randperm(k, generator=g)[:3]
        w[:, cols] *= 8.0
        return w.half()

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g)).half()

    sd = {"model.embed_tokens.weight": mat(vocab, h)}
    for i in range(L):
        p = f"model.layers.{i}."
        sd[p + "input_layernorm.weight"] = norm(h)
        sd[p + "self_attn.q_proj.weight"] = mat(h, h)
        sd[p + "self_attn.k_proj.weight"] = mat(kvd, h)
        sd[p + "self_attn.v_proj.weight"] = mat(kvd, h)
        sd[p + "self_attn.o_proj.weight"] = mat(h, h)
        sd[p + "post_attention_layernorm.weight"] = norm(h)
        sd[p + "mlp.gate_proj.weight"] = mat(inter, h)
        sd[p + "mlp.up_proj.weight"] = mat(inter, h)
        sd[p + "mlp.down_proj.weight"] = mat(h, inter)
    sd["model.norm.weight"] = norm(h)
    return sd


def make_checkpoint(directory: str, seed: int = 7) -> dict:
    """A local HF checkpoint (config.json + model.safetensors) of the tiny model."""
    from safetensors.torch import save_file
    from transformers import LlamaConfig
    os.makedirs(directory, exist_ok=True)
    cfg = LlamaConfig(**TINY)
    cfg.architectures = ["LlamaForCausalLM"]
    cfg.save_pretrained(directory)
    sd = tiny_state_dict(seed)
    save_file(sd, os.path.join(directory, "model.safetensors"))
    return sd


def load_reference_compressor(root: str):
    path = os.path.join(root, "spectra", "compressor.py")
    spec = importlib.util.spec_from_file_location("reference_compressor", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main(root: str) -> None:
    ref = load_reference_compressor(root)
    with tempfile.TemporaryDirectory() as d:
        ck = os.path.join(d, "tiny_llama")
        make_checkpoint(ck)
        out = os.path.join(d, "tiny_llama_g32.trdc")
        ref.SpectraCompressor(group_size=32, base_outlier_ratio=0.01).compress(ck, out, save_tokenizer=False)
        shutil.copyfile(out, GOLDEN)
    print(f"wrote {GOLDEN} ({os.path.getsize(GOLDEN)} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
