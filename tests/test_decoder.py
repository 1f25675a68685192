"""GPU tests of the embedding gather and the Llama-shaped decoder built on the quantized
linears (BASELINE configs[4] workload at a small shape).

* Embedding rows: bit-identical to the same rows of the bit-exact dequant (Format A with
  packed zero points, as engine.py:177-183 accepts, and Format B with CSR outliers).
* Decoder: prefill and graph-replayed greedy decode against an fp32 torch restatement that
  uses the dequantized weights (W_eff from the bit-exact dequant, the rotation from the
  bit-exact FWHT); logits within 1e-2 of the logit scale, identical greedy tokens, and the
  captured decode step identical bit for bit to the eager one.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from spectra_amd import compressor as C
from spectra_amd import kernels as K
from spectra_amd.engine import DecoderConfig, SpectraDecoder, SpectraFusedEmbedding

pytestmark = pytest.mark.gpu


def case(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.mark.parametrize("out_dt", [torch.float16, torch.float32])
def test_embedding_format_b_rows_bitexact(hip, out_dt):
    case(out_dt=out_dt)
    g = torch.Generator().manual_seed(3)
    n, k = 500, 1024
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    mask = torch.rand(n, k, generator=g) < 0.01
    q = C.quantize_nf4(w.cuda(), 64, 0, mask.cuda(), True)
    emb = SpectraFusedEmbedding(n, k, 64, True, codebook="nf4").cuda()
    emb.set_weights(q.packed, q.absmax, None, q.col, q.val, True, outlier_rowptr=q.rowptr)
    emb.target_dtype = out_dt
    ids = torch.tensor([[0, 499, 17], [17, 250, 3]], device="cuda")
    rows = emb(ids)
    assert rows.shape == (2, 3, k) and rows.dtype == out_dt
    full = K.w4_dequant(q.packed, q.absmax, None, out_dtype=out_dt, codebook="nf4", marlin_layout=True,
                        outlier_idx=q.col, outlier_w=q.val, outlier_rowptr=q.rowptr)
    assert torch.equal(rows.reshape(-1, k), full[ids.reshape(-1)])
    # ids outside [0, N) give zero rows
    bad = emb(torch.tensor([-1, n], device="cuda"))
    assert torch.equal(bad, torch.zeros_like(bad))


def test_embedding_format_a_packed_zeros(hip):
    """The reference's own module contract: Format A, packed zero points, outlier columns."""
    rng = np.random.default_rng(4)
    n, k = 300, 512
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    idx = np.sort(rng.permutation(k)[:7]).astype(np.int64)
    packed, scales, pz = O.compute_group32_quant(w.astype(np.float32), idx)
    emb = SpectraFusedEmbedding(n, k, 32, marlin_layout=True).cuda()
    emb.set_weights(torch.from_numpy(packed).cuda(), torch.from_numpy(scales).cuda(), torch.from_numpy(pz).cuda(),
                    torch.from_numpy(idx).cuda(), torch.from_numpy(w[:, idx].copy()).cuda(), marlin_layout=True)
    ids = torch.tensor([5, 0, 299, 5], device="cuda")
    rows = emb(ids)
    z = O.unpack_zeros(pz, k // 32)
    ref = O.apply_outlier_columns(O.dequant_group32(packed, scales, z, True, "float16"), idx, w[:, idx], "float16")
    assert np.array_equal(rows.cpu().numpy(), ref[ids.cpu().numpy()])


# ---------------------------------------------------------------------------
# decoder
# ---------------------------------------------------------------------------
SMALL = DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, inter=512, vocab=1000, max_seq=64,
                      hadamard_block=128, outlier_ratio=0.01, seed=7)


def _w_eff(q):
    col, val = q.outliers()
    return K.w4_dequant(q.packed, q.absmax, None, out_dtype=torch.float32, codebook="nf4", marlin_layout=True,
                        outlier_idx=col, outlier_w=val, outlier_rowptr=q.rowptr if col is not None else None)


class RefDecoder:
    """fp32 restatement of SpectraDecoder's math on the dequantized weights: the oracle's
    torch decoder (oracle/torch_ref.py) fed the bit-exact W_eff of every quantized weight."""

    def __init__(self, dec: SpectraDecoder):
        from oracle import torch_ref as TR
        c = dec.cfg
        self.c = c
        self.w = [[_w_eff(q) for q in layer] for layer in dec.layers_q]
        self.had = [[q.hadamard_block for q in layer] for layer in dec.layers_q]
        self.emb = _w_eff(dec.embed_q)
        self.head = _w_eff(dec.lm_q)
        self.norm = [w.float() for w in dec.norm_w]
        self.dec = TR.Decoder(self.w, self.had, self.norm, self.emb, self.head, heads=c.heads, kv_heads=c.kv_heads,
                              rope_theta=c.rope_theta, rms_eps=c.rms_eps, max_seq=c.max_seq,
                              rope_scaling=c.rope_scaling)

    def forward(self, ids, pos0):
        return self.dec.forward(ids, pos0)


def test_decoder_against_fp32_reference(hip):
    torch.manual_seed(0)
    dec = SpectraDecoder(SMALL)
    ref = RefDecoder(dec)
    prompt = torch.randint(0, SMALL.vocab, (9,), generator=torch.Generator().manual_seed(1)).cuda()
    case(stage="prefill", T=prompt.numel())
    lg = dec.prefill(prompt).float()
    lr = ref.forward(prompt, 0)
    scale = lr.abs().max().item()
    assert (lg - lr).abs().max().item() <= 1e-2 * scale, (lg - lr).abs().max().item() / scale
    toks = [int(torch.argmax(lr))]
    assert int(dec.cur_id) == toks[0]
    dec.capture_decode()
    for step in range(5):
        case(stage="decode", step=step)
        dec.graph.replay()
        lg = dec.graph_logits.float()
        lr = ref.forward(torch.tensor([toks[-1]], device="cuda"), prompt.numel() + step)
        assert (lg - lr).abs().max().item() <= 1e-2 * lr.abs().max().item()
        toks.append(int(torch.argmax(lr)))
        assert int(dec.cur_id) == toks[-1]
        assert int(dec.cur_pos) == prompt.numel() + step + 1


def _greedy_consistent(ours: int, lr: torch.Tensor, tol: float) -> None:
    """Our greedy token must be the reference's argmax, unless the reference's top two are
    closer than the logit tolerance allows to resolve (then ours must be within it of the max)."""
    top = torch.topk(lr.reshape(-1), 2).values
    if float(top[0] - top[1]) > 2 * tol:
        assert ours == int(torch.argmax(lr)), (ours, int(torch.argmax(lr)), float(top[0] - top[1]))
    else:
        assert float(lr.reshape(-1)[ours]) >= float(top[0]) - 2 * tol


def test_decoder_llama32_3b_shape_against_fp32_reference(hip):
    """BASELINE configs[4] at full size (engine.py:1801-1860, :1124-1168): 28 layers, hidden 3072,
    24 / 8 heads, intermediate 8192, vocab 128256, random init (seed 0), every linear NF4 +
    FWHT-128 + 0.5% CSR outliers, tied quantized embedding / lm_head (the fused-RMSNorm GEMV at
    N=128256, K=3072); a 512-token prompt, then 8 graph-replayed greedy steps, against the fp32
    restatement.  Greedy tokens equal (on a near-tie: within the logit tolerance of the
    reference's maximum, the reference then following our token); logits within 2e-2 of the
    logit scale.  The bar is 2e-2, not the single-layer 1e-2: every linear is held to 1e-3
    relative L2 (fp16 rotated activations and fp16 outputs, as in any fp16 implementation), and
    over 28 layers of a random-init residual stream those roundings compound -- measured
    0.16-0.3% of the logit scale after one layer, 0.5% after four, 0.8-1.3% after 28."""
    cfg = DecoderConfig(max_seq=640)
    dec = SpectraDecoder(cfg)
    ref = RefDecoder(dec)
    prompt = torch.randint(0, cfg.vocab, (512,), generator=torch.Generator().manual_seed(5)).cuda()

    def check(stage, lg, lr):
        scale = lr.abs().max().item()
        err = (lg - lr).abs().max().item()
        print(f"{stage}: max |dlogit| {err:.4e}, logit scale {scale:.4e} ({err / scale:.2e})", flush=True)
        assert err <= 2e-2 * scale
        _greedy_consistent(int(dec.cur_id), lr, 2e-2 * scale)

    case(stage="prefill", T=prompt.numel(), layers=cfg.layers, vocab=cfg.vocab)
    check("prefill", dec.prefill(prompt).float(), ref.forward(prompt, 0))
    dec.capture_decode()
    for step in range(8):
        case(stage="decode", step=step)
        tok = int(dec.cur_id)
        dec.graph.replay()
        check(f"step {step}", dec.graph_logits.float(),
              ref.forward(torch.tensor([tok], device="cuda"), prompt.numel() + step))
        assert int(dec.cur_pos) == prompt.numel() + step + 1


def test_decoder_graph_matches_eager(hip):
    """The captured decode step replays the eager computation bit for bit."""
    prompt = torch.randint(0, SMALL.vocab, (5,), generator=torch.Generator().manual_seed(2)).cuda()
    eager = SpectraDecoder(SMALL)
    eager.prefill(prompt)
    t_eager = eager.decode(6, use_graph=False)
    graphed = SpectraDecoder(SMALL)
    graphed.prefill(prompt)
    t_graph = graphed.decode(6, use_graph=True)
    assert torch.equal(t_eager, t_graph)
    assert torch.equal(eager.k_cache, graphed.k_cache) and torch.equal(eager.v_cache, graphed.v_cache)


def test_decoder_kv4_cache(hip):
    """The 4-bit cache: while every position is inside the fp16 window the decode is the fp16
    decoder's, bit for bit; the prompt's codes are the reference quantizer's codes of the
    fp16 decoder's keys / values; past the window the logits stay near the fp16 decoder's and
    graph replay equals eager decode."""
    import dataclasses
    import oracle as O
    prompt = torch.randint(0, SMALL.vocab, (24,), generator=torch.Generator().manual_seed(4)).cuda()
    full = SpectraDecoder(SMALL)
    wide = SpectraDecoder(dataclasses.replace(SMALL, kv_bits=4, kv_window=64))
    lf, lw = full.prefill(prompt), wide.prefill(prompt)
    assert torch.equal(lf, lw)
    assert torch.equal(full.decode(5, use_graph=False), wide.decode(5, use_graph=False))
    # prompt codes = the reference quantizer on the fp16 cache rows
    hd = SMALL.head_dim
    for li in range(SMALL.layers):
        for src, q4 in ((full.k_cache, wide.k4), (full.v_cache, wide.v4)):
            rows = src[li][:, :24].reshape(-1, hd).cpu().numpy()
            c, s, z = O.kv4_quantize(rows, "float16")
            assert np.array_equal(q4[0][li][:, :24].reshape(-1, hd // 2).cpu().numpy(), c.reshape(-1, hd // 2))
            assert np.array_equal(q4[1][li][:, :24].reshape(-1, hd // 32).cpu().numpy().view(np.uint16),
                                  s.reshape(-1, hd // 32).view(np.uint16))
            assert np.array_equal(q4[2][li][:, :24].reshape(-1, hd // 32).cpu().numpy(), z.reshape(-1, hd // 32))
    # a window of 8: the first decode step already reads 16 of its 25 positions from the codes
    narrow = dataclasses.replace(SMALL, kv_bits=4, kv_window=8)
    q4, ref = SpectraDecoder(narrow), SpectraDecoder(SMALL)
    q4.prefill(prompt), ref.prefill(prompt)
    lq = q4.forward_tokens(q4.cur_id, q4.cur_pos, None).float()
    lr = ref.forward_tokens(ref.cur_id, ref.cur_pos, None).float()
    assert (lq - lr).abs().max().item() <= 0.1 * lr.abs().max().item()
    eager, graphed = SpectraDecoder(narrow), SpectraDecoder(narrow)
    eager.prefill(prompt), graphed.prefill(prompt)
    assert torch.equal(eager.decode(6, use_graph=False), graphed.decode(6, use_graph=True))
    for a, b in zip(eager.cache_tensors(), graphed.cache_tensors()):
        assert torch.equal(a, b)
