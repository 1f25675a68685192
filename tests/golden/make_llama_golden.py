"""Writes ``llama_hf_decode.npz``: logits and greedy tokens of Hugging Face's own
``LlamaForCausalLM`` (transformers 5.15.0, the model class the reference's engine builds the
decoder from: /root/reference/spectra/engine.py:919-939, modules swapped at :1044-1080) on a
tiny grouped-query Llama with float32 weights, run on the CPU in the build container.

It pins the fp32 decoder restatement in ``oracle/torch_ref.py`` (``Decoder``), the checker of
the GPU decoder, on what nothing else fixes: the residual and RMSNorm wiring of a layer, the
final norm, the rotate-half RoPE with its inverse-frequency table, grouped-query attention
and the KV-cache positions of decode steps.

Two RoPE tables are recorded:

* ``default``: ``rope_theta`` 500000, no scaling (the Llama-3.2 base frequencies);
* ``llama3``: the same weights with ``rope_type: llama3`` scaling as transformers applies it
  (factor 8, low / high frequency factors 1 / 4, original context 256, so that the
  96-token prompt reaches positions where the scaled low frequencies differ).

The reference's loader replaces every rotary module's table by
``compute_default_rope_parameters(config)`` whatever ``rope_type`` the config names
(engine.py:1170-1179); ``inv_reference_reinit`` records what that call returns for the
llama3 config (the unscaled table).

Weights come from ``llama_state_dict(seed)`` (seeded CPU generator; the tests regenerate
them and check ``weights_sha256``).  The fixture is data only.

    python tests/golden/make_llama_golden.py
"""
from __future__ import annotations

import hashlib
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "llama_hf_decode.npz")

TINY = dict(vocab_size=160, hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, max_position_embeddings=512, rms_norm_eps=1e-5, tie_word_embeddings=False)
THETA = 500000.0
LLAMA3 = dict(rope_type="llama3", factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
              original_max_position_embeddings=256)
PROMPT_LEN, DECODE_STEPS, SEED = 96, 4, 11


def llama_state_dict(seed: int = SEED) -> dict:
    """HF Llama tensor names, float32: q / k projections N(0, 0.25) (attention that depends on
    the positions), other matrices N(0, 0.08), norms 1 + 0.1 N(0, 1)."""
    g = torch.Generator().manual_seed(seed)
    h, inter, L, vocab = (TINY["hidden_size"], TINY["intermediate_size"], TINY["num_hidden_layers"],
                          TINY["vocab_size"])
    hd = h // TINY["num_attention_heads"]
    kvd = TINY["num_key_value_heads"] * hd

    def mat(n, k, std=0.08):
        return torch.randn(n, k, generator=g) * std

    def norm(n):
        return 1.0 + 0.1 * torch.randn(n, generator=g)

    sd = {"model.embed_tokens.weight": torch.randn(vocab, h, generator=g)}
    for i in range(L):
        p = f"model.layers.{i}."
        sd[p + "input_layernorm.weight"] = norm(h)
        sd[p + "self_attn.q_proj.weight"] = mat(h, h, 0.25)
        sd[p + "self_attn.k_proj.weight"] = mat(kvd, h, 0.25)
        sd[p + "self_attn.v_proj.weight"] = mat(kvd, h)
        sd[p + "self_attn.o_proj.weight"] = mat(h, h)
        sd[p + "post_attention_layernorm.weight"] = norm(h)
        sd[p + "mlp.gate_proj.weight"] = mat(inter, h)
        sd[p + "mlp.up_proj.weight"] = mat(inter, h)
        sd[p + "mlp.down_proj.weight"] = mat(h, inter)
    sd["model.norm.weight"] = norm(h)
    sd["lm_head.weight"] = mat(vocab, h)
    return sd


def weights_sha256(sd: dict) -> str:
    hsh = hashlib.sha256()
    for name in sorted(sd):
        hsh.update(name.encode())
        hsh.update(sd[name].contiguous().numpy().tobytes())
    return hsh.hexdigest()


def prompt_ids() -> torch.Tensor:
    return torch.randint(0, TINY["vocab_size"], (PROMPT_LEN,), generator=torch.Generator().manual_seed(SEED + 1))


def _run(rope_parameters: dict):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(**TINY, rope_parameters=rope_parameters, attn_implementation="eager")
    model = LlamaForCausalLM(cfg).float().eval()
    missing, unexpected = model.load_state_dict(llama_state_dict(), strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    ids = prompt_ids()
    logits, toks = [], []
    with torch.no_grad():
        out = model(input_ids=ids[None], use_cache=True)
        for _ in range(DECODE_STEPS + 1):
            lg = out.logits[0, -1].float()
            logits.append(lg.clone())
            tok = int(torch.argmax(lg))
            toks.append(tok)
            if len(toks) > DECODE_STEPS:
                break
            out = model(input_ids=torch.tensor([[tok]]), past_key_values=out.past_key_values, use_cache=True)
    inv = model.model.rotary_emb.inv_freq.detach().clone()
    reinit = model.model.rotary_emb.compute_default_rope_parameters(cfg)[0]  # engine.py:1172-1175
    return torch.stack(logits).numpy(), np.array(toks, np.int64), inv.numpy(), reinit.numpy()


def main() -> None:
    import transformers
    base = dict(rope_type="default", rope_theta=THETA)
    scaled = dict(LLAMA3, rope_theta=THETA)
    lg_d, tk_d, inv_d, _ = _run(base)
    lg_s, tk_s, inv_s, reinit = _run(scaled)
    # the llama3 table must move the logits at these positions far beyond the tests' 1e-4 bar
    assert np.abs(lg_d - lg_s).max() > 1e-2 * np.abs(lg_d).max()
    np.savez_compressed(
        GOLDEN, prompt=prompt_ids().numpy(), logits_default=lg_d, tokens_default=tk_d, inv_default=inv_d,
        logits_llama3=lg_s, tokens_llama3=tk_s, inv_llama3=inv_s, inv_reference_reinit=reinit,
        weights_sha256=np.array(weights_sha256(llama_state_dict())),
        transformers_version=np.array(transformers.__version__))
    print(f"wrote {GOLDEN}: tokens default {tk_d.tolist()}, llama3 {tk_s.tolist()}, "
          f"max |logit difference| {np.abs(lg_d - lg_s).max():.3f}")


if __name__ == "__main__":
    main()
