"""TRDC container: layout parity with the reference's own writer, reader checks, Format B
round trip and the decoder built from a container.

Golden: ``golden/tiny_llama_g32.trdc`` was written by the reference's compressor
(``make_trdc_golden.py``) from the seeded checkpoint ``make_checkpoint`` regenerates.

* CPU: the reader decodes every tensor of the reference-written file to exactly what the
  oracle computes from the checkpoint (outlier columns with the layer's norm vector,
  group-32 quantization, the outlier columns, the lossless tensors); fed the same operands,
  the writer reproduces the reference's file byte for byte; corrupt files raise.
* GPU: the compressor (GPU quantizers) writes the reference's bytes for Format A; a Format B
  container round-trips to the quantizer's operands bit for bit, and the decoder loaded from
  it matches an fp32 restatement on the container's dequantized weights.
"""
import json
import os
import struct

import numpy as np
import pytest
import torch

import oracle as O
from spectra_amd import container as T
from spectra_amd.compressor import NF4Weight

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "tiny_llama_g32.trdc")

from golden.make_trdc_golden import TINY, make_checkpoint, tiny_state_dict  # noqa: E402


def _np16(t):
    return t.float().numpy()


def _norm_map(sd):
    return {k: v.float().abs() for k, v in sd.items() if v.ndim == 1 and "norm" in k}


def test_reference_container_reads_to_oracle_operands():
    sd = tiny_state_dict()
    nmap = _norm_map(sd)
    with T.TrdcReader(GOLDEN) as rd:
        assert rd.manifest["version"] == "TRDC4B01" and rd.group_size == 32
        assert set(rd.tensors) == set(sd)
        for name, w in sd.items():
            meta = rd.tensors[name]
            got = rd.load(name)
            if w.ndim == 1:
                assert meta["type"] == "lossless_float16" and torch.equal(got, w)
                continue
            assert meta["type"] == T.FORMAT_A and meta["shape"] == list(w.shape)
            n, k = w.shape
            nv = T.norm_vector_for(name, nmap, k)
            idx, ratio, kurt = O.select_outlier_columns(w.numpy(), "float16", nv.numpy() if nv is not None else None,
                                                        0.01, True)
            assert np.array_equal(got.outlier_idx.numpy(), idx.astype(np.int64)), name
            assert abs(meta["outlier_ratio"] - round(ratio, 4)) <= 1e-4 and abs(meta["kurtosis"] - round(kurt, 2)) <= 0.01
            packed, scales, pz = O.compute_group32_quant(_np16(w), idx)
            assert np.array_equal(got.packed.numpy(), packed) and np.array_equal(got.scales.numpy(), scales)
            assert np.array_equal(got.zeros.numpy(), O.unpack_zeros(pz, k // 32))
            assert torch.equal(got.outlier_w, w[:, torch.from_numpy(idx.astype(np.int64))])


def test_writer_reproduces_reference_bytes():
    """Same operands, same order, same manifest head -> the reference's file, byte for byte."""
    sd = tiny_state_dict()
    ref = open(GOLDEN, "rb").read()
    moff, mlen = struct.unpack("<QQ", ref[8:24])
    man = json.loads(ref[moff:moff + mlen])
    head = {k: man[k] for k in ("version", "group_size", "base_outlier_ratio", "architecture", "config")}
    out = os.path.join(os.environ.get("PYTEST_TMP", "/tmp"), f"trdc_cpu_{os.getpid()}.trdc")
    with T.TrdcWriter(out, head) as wr:
        for name in man["tensors"]:  # the reference's (safetensors) order
            w = sd[name]
            if w.ndim == 1:
                wr.add_lossless(name, w)
                continue
            meta = man["tensors"][name]
            with T.TrdcReader(GOLDEN) as rd:
                idx = rd.load(name).outlier_idx.numpy()
            packed, scales, pz = O.compute_group32_quant(_np16(w), idx)
            wr.add_format_a(name, list(w.shape), torch.from_numpy(packed), torch.from_numpy(scales),
                            torch.from_numpy(pz), torch.from_numpy(idx.astype(np.int32)),
                            w[:, torch.from_numpy(idx.astype(np.int64))], meta["outlier_ratio"], meta["kurtosis"])
    try:
        assert open(out, "rb").read() == ref
    finally:
        os.unlink(out)


def test_corrupt_containers_raise(tmp_path):
    good = open(GOLDEN, "rb").read()
    cases = {
        "short": good[:20],
        "magic": b"TRDC4B02" + good[8:],
        "manifest_past_end": good[:8] + struct.pack("<QQ", len(good) - 10, 100) + good[24:],
        "manifest_in_header": good[:8] + struct.pack("<QQ", 8, 16) + good[24:],
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.trdc"
        p.write_bytes(data)
        with pytest.raises(ValueError):
            T.TrdcReader(p)


def _small_nf4(n=4, k=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    rp = torch.tensor([0, 2, 2, 5, 6], dtype=torch.int32)[: n + 1]
    nnz = int(rp[-1])
    return NF4Weight(torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8),
                     torch.rand(n, k // 64, generator=g).half(), rp,
                     torch.tensor([3, 70, 0, 64, 127, 9], dtype=torch.int32)[:nnz],
                     torch.randn(nnz, generator=g).half(), k, 64, 128, True)


def test_corrupt_outlier_side_tensors_raise_at_load(tmp_path):
    """Side tensors the kernels use as addresses are checked when a tensor is loaded, before any
    launch: CSR rowptr must start at 0, never decrease and end at nnz, columns lie in [0, K);
    Format A outlier columns lie in [0, K)."""
    head = {"version": "TRDC4B01", "group_size": 32, "base_outlier_ratio": 0.01, "architecture": "LlamaForCausalLM",
            "config": {}}
    good = _small_nf4()
    bad = {
        "rowptr_decreasing": dict(rowptr=torch.tensor([0, 2, 1, 5, 6], dtype=torch.int32)),
        "rowptr_past_nnz": dict(rowptr=torch.tensor([0, 2, 2, 5, 7], dtype=torch.int32)),
        "rowptr_not_zero": dict(rowptr=torch.tensor([1, 2, 2, 5, 6], dtype=torch.int32)),
        "col_past_k": dict(col=torch.tensor([3, 70, 0, 128, 127, 9], dtype=torch.int32)),
        "col_negative": dict(col=torch.tensor([3, -1, 0, 64, 127, 9], dtype=torch.int32)),
    }
    p = tmp_path / "good.trdc"
    with T.TrdcWriter(p, head) as wr:
        wr.add_nf4("w", good)
    with T.TrdcReader(p) as rd:
        q = rd.load("w")
        assert torch.equal(q.rowptr, good.rowptr) and torch.equal(q.col, good.col)
    for name, repl in bad.items():
        f = {k: getattr(good, k) for k in ("packed", "absmax", "rowptr", "col", "val")} | repl
        q = NF4Weight(f["packed"], f["absmax"], f["rowptr"], f["col"], f["val"], good.k, 64, 128, True)
        p = tmp_path / f"{name}.trdc"
        with T.TrdcWriter(p, head) as wr:
            wr.add_nf4("w", q)
        with T.TrdcReader(p) as rd, pytest.raises(ValueError):
            rd.load("w")
    # Format A: an outlier column index past K
    n, k = 4, 64
    w = torch.randn(n, k, generator=torch.Generator().manual_seed(1)).half()
    idx = np.array([5, 64], dtype=np.int32)
    packed, scales, pz = O.compute_group32_quant(_np16(w), np.array([5, 63]))
    p = tmp_path / "fa.trdc"
    with T.TrdcWriter(p, head) as wr:
        wr.add_format_a("w", [n, k], torch.from_numpy(packed), torch.from_numpy(scales), torch.from_numpy(pz),
                        torch.from_numpy(idx), w[:, [5, 63]], 0.01, 3.0)
    with T.TrdcReader(p) as rd, pytest.raises(ValueError):
        rd.load("w")


def test_nf4_concat_rowptr_offsets():
    def q(n, nnz_rows, seed):
        g = torch.Generator().manual_seed(seed)
        rp = torch.zeros(n + 1, dtype=torch.int32)
        rp[1:] = torch.cumsum(torch.tensor(nnz_rows, dtype=torch.int32), 0)
        nnz = int(rp[-1])
        return NF4Weight(torch.randint(0, 256, (n, 64), generator=g, dtype=torch.uint8),
                         torch.rand(n, 2, generator=g).half(), rp, torch.randint(0, 128, (nnz,), generator=g,
                                                                                dtype=torch.int32),
                         torch.randn(nnz, generator=g).half(), 128, 64, 128, True)
    a, b, c = q(3, [1, 0, 2], 1), q(2, [0, 3], 2), q(1, [1], 3)
    f = T.nf4_concat([a, b, c])
    assert f.n == 6 and f.rowptr.tolist() == [0, 1, 1, 3, 3, 6, 7]
    assert torch.equal(f.col, torch.cat([a.col, b.col, c.col])) and torch.equal(f.packed[3:5], b.packed)
    with pytest.raises(ValueError):
        T.nf4_concat([a, NF4Weight(a.packed, a.absmax, a.rowptr, a.col, a.val, 128, 64, 0, True)])


# ---------------------------------------------------------------------------
# GPU: the compressor and the decoder from a container
# ---------------------------------------------------------------------------
@pytest.mark.gpu
def test_compressor_writes_reference_bytes(hip, tmp_path):
    ck = tmp_path / "ck"
    make_checkpoint(str(ck))
    out = tmp_path / "ours.trdc"
    T.compress_checkpoint(ck, out, fmt="q4_g32")
    ours, ref = out.read_bytes(), open(GOLDEN, "rb").read()
    mo, ml = struct.unpack("<QQ", ours[8:24])
    mr, mlr = struct.unpack("<QQ", ref[8:24])
    assert ours[:8] == ref[:8] and mo == mr and ours[24:mo] == ref[24:mr]  # magic and every tensor byte
    m_ours, m_ref = json.loads(ours[mo:mo + ml]), json.loads(ref[mr:mr + mlr])
    # the config records the checkpoint's (temporary) path
    m_ours["config"].pop("_name_or_path"), m_ref["config"].pop("_name_or_path")
    assert m_ours["config"] == m_ref["config"] and list(m_ours["tensors"]) == list(m_ref["tensors"])
    assert [m_ours[k] for k in ("version", "group_size", "base_outlier_ratio", "architecture")] == \
        [m_ref[k] for k in ("version", "group_size", "base_outlier_ratio", "architecture")]
    for name, e in m_ref["tensors"].items():
        o = m_ours["tensors"][name]
        for key, v in e.items():
            if key in ("outlier_ratio", "kurtosis"):  # the statistic agrees to 1 fp32 ulp before rounding
                assert abs(o[key] - v) <= (1e-4 if key == "outlier_ratio" else 0.01)
            else:
                assert o[key] == v, (name, key)


DEC = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, vocab_size=512, max_position_embeddings=256, tie_word_embeddings=True,
           rope_theta=10000.0, rms_norm_eps=1e-5, torch_dtype="float16")


@pytest.mark.gpu
def test_nf4_container_roundtrip_and_decoder(hip, tmp_path, monkeypatch):
    import golden.make_trdc_golden as G
    from spectra_amd import compressor as C
    from spectra_amd import kernels as K
    from spectra_amd.engine import SpectraDecoder
    from test_decoder import RefDecoder

    monkeypatch.setattr(G, "TINY", DEC)
    ck = tmp_path / "ck"
    sd = make_checkpoint(str(ck), seed=11)
    out = tmp_path / "b.trdc"
    summary = T.compress_checkpoint(ck, out, fmt="nf4", hadamard_block=128, csr_ratio=0.01)
    assert summary["quantized_tensors"] == 1 + 7 * DEC["num_hidden_layers"]
    with T.TrdcReader(out) as rd:
        for name, w in sd.items():
            got = rd.load(name, "cuda")
            if w.ndim == 1:
                assert torch.equal(got.cpu(), w)
                continue
            had = 0 if "embed" in name else 128
            assert rd.tensors[name]["type"] == T.nf4_type(64, had)
            w_rot = K.fwht_rows(w.cuda(), had, out_dtype=torch.float32) if had else w.cuda().float()
            q = C.quantize_nf4(w_rot, 64, 0, T.select_csr_outliers(w_rot, 0.01), True)
            for a, b in ((got.packed, q.packed), (got.absmax, q.absmax), (got.rowptr, q.rowptr), (got.col, q.col),
                         (got.val, q.val)):
                assert torch.equal(a, b), name
            assert got.hadamard_block == had and int(got.rowptr[-1]) == w.shape[0] * round(0.01 * w.shape[1])
    dec = SpectraDecoder.from_trdc(out, max_seq=64)
    assert dec.cfg.hidden == 256 and dec.cfg.kv_heads == 2 and dec.lm_q is dec.embed_q
    ref = RefDecoder(dec)
    prompt = torch.randint(0, DEC["vocab_size"], (7,), generator=torch.Generator().manual_seed(3)).cuda()
    lg = dec.prefill(prompt).float()
    lr = ref.forward(prompt, 0)
    assert (lg - lr).abs().max().item() <= 1e-2 * lr.abs().max().item()
    toks = [int(torch.argmax(lr))]
    assert int(dec.cur_id) == toks[0]
    dec.capture_decode()
    for step in range(4):
        dec.graph.replay()
        lr = ref.forward(torch.tensor([toks[-1]], device="cuda"), prompt.numel() + step)
        assert (dec.graph_logits.float() - lr).abs().max().item() <= 1e-2 * lr.abs().max().item()
        toks.append(int(torch.argmax(lr)))
        assert int(dec.cur_id) == toks[-1]


LLAMA3_ROPE = dict(rope_type="llama3", rope_theta=10000.0, factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                   original_max_position_embeddings=32)


@pytest.mark.gpu
@pytest.mark.parametrize("rope", ["reference", "config"])
def test_from_trdc_rope_scaling(hip, tmp_path, monkeypatch, rope):
    """A container whose config names llama3 RoPE scaling (original context 32, so a 48-token
    prompt reaches the scaled frequencies).  ``rope='reference'`` decodes with the unscaled
    table as the reference's loader does (engine.py:1170-1179) and warns; ``rope='config'``
    applies the scaling.  Each against the fp32 restatement with its table (the restatement's
    tables and wiring are pinned to transformers' LlamaForCausalLM on the CPU), and the two
    tables' logits apart by more than the bar."""
    import golden.make_trdc_golden as G
    from oracle import torch_ref as TR
    from spectra_amd.engine import SpectraDecoder
    from test_decoder import RefDecoder

    cfg = {k: v for k, v in DEC.items() if k != "rope_theta"}
    cfg["rope_parameters"] = dict(LLAMA3_ROPE)
    monkeypatch.setattr(G, "TINY", cfg)
    ck = tmp_path / "ck"
    make_checkpoint(str(ck), seed=12)
    out = tmp_path / "r.trdc"
    T.compress_checkpoint(ck, out, fmt="nf4", hadamard_block=128, csr_ratio=0.01)
    case = f"case: rope {rope}"
    print(case, flush=True)
    if rope == "reference":
        with pytest.warns(UserWarning, match="llama3"):
            dec = SpectraDecoder.from_trdc(out, max_seq=64)
        assert dec.cfg.rope_scaling is None
    else:
        dec = SpectraDecoder.from_trdc(out, max_seq=64, rope="config")
        assert dec.cfg.rope_scaling["rope_type"] == "llama3"
    ref = RefDecoder(dec)
    other = RefDecoder(dec)
    c = dec.cfg
    other.dec = TR.Decoder(other.w, other.had, other.norm, other.emb, other.head, heads=c.heads, kv_heads=c.kv_heads,
                           rope_theta=c.rope_theta, rms_eps=c.rms_eps, max_seq=c.max_seq,
                           rope_scaling=None if c.rope_scaling else dict(LLAMA3_ROPE))
    prompt = torch.randint(0, cfg["vocab_size"], (48,), generator=torch.Generator().manual_seed(4)).cuda()
    lg = dec.prefill(prompt).float()
    lr, lo = ref.forward(prompt, 0), other.forward(prompt, 0)
    tol = 1e-2 * lr.abs().max().item()
    assert (lg - lr).abs().max().item() <= tol
    assert (lo - lr).abs().max().item() > 3 * tol  # the tables are told apart at these positions
    dec.capture_decode()
    for step in range(2):
        tok = int(dec.cur_id)
        assert tok == int(torch.argmax(lr)) or (lr.max() - lr.reshape(-1)[tok]).item() <= 2 * tol
        dec.graph.replay()
        lr = ref.forward(torch.tensor([tok], device="cuda"), prompt.numel() + step)
        assert (dec.graph_logits.float() - lr).abs().max().item() <= 1e-2 * lr.abs().max().item()


def _format_a_w_eff(q, dtype="float32"):
    """W_eff of a Format A tensor: (q - z) * s, then the outlier columns (oracle dequant)."""
    w = O.dequant_group32(q.packed.cpu().numpy(), q.scales.cpu().numpy(), q.zeros.cpu().numpy(), q.marlin_layout,
                          dtype)
    if q.outlier_idx is not None:
        w = O.apply_outlier_columns(w, q.outlier_idx.cpu().numpy(), q.outlier_w.cpu().numpy(), dtype)
    return torch.from_numpy(np.ascontiguousarray(w)).float().cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("source", ["reference_golden", "compressor"])
def test_format_a_container_decoder(hip, tmp_path, monkeypatch, source):
    """A Format A (q4_g32_hdsq) container drives the decoder (engine.py:1004-1025 binds its
    tensors): q/k/v and gate/up stay separate Format A linears (the MFMA GEMM over the
    prompt, one GEMV per part in the captured decode step), the embedding gathers Format A
    rows and the tied lm_head is a Format A GEMV.  ``reference_golden`` is the file the
    reference's compressor wrote (head_dim 16); ``compressor`` is this package's compressor
    on a hidden-256 checkpoint (head_dim 64).  Against the fp32 restatement on the oracle's
    W_eff (the embedding rows in fp16, as the gather returns them): logits within 1e-2 of the
    logit scale, the greedy token the restatement's unless its top two are within that."""
    from oracle import torch_ref as TR
    from spectra_amd.engine import SpectraDecoder
    from test_decoder import _greedy_consistent

    if source == "reference_golden":
        path = GOLDEN
    else:
        import golden.make_trdc_golden as G
        monkeypatch.setattr(G, "TINY", DEC)
        ck = tmp_path / "ck"
        make_checkpoint(str(ck), seed=5)
        path = tmp_path / "a.trdc"
        T.compress_checkpoint(ck, path, fmt="q4_g32")
    dec = SpectraDecoder.from_trdc(path, max_seq=64)
    c = dec.cfg
    assert not dec.fused and dec.lm_q is dec.embed_q and len(dec.blocks[0]["qkv"]) == 3
    assert c.head_dim == (16 if source == "reference_golden" else 64)
    layers = [[torch.cat([_format_a_w_eff(p) for p in (q if isinstance(q, list) else [q])]) for q in layer]
              for layer in dec.layers_q]
    ref = TR.Decoder(layers, [[0, 0, 0, 0]] * c.layers, [w.float() for w in dec.norm_w],
                     _format_a_w_eff(dec.embed_q, "float16"), _format_a_w_eff(dec.lm_q), heads=c.heads,
                     kv_heads=c.kv_heads, rope_theta=c.rope_theta, rms_eps=c.rms_eps, max_seq=c.max_seq)
    prompt = torch.randint(0, c.vocab, (7,), generator=torch.Generator().manual_seed(2)).cuda()
    print("case: source", source, "prefill", flush=True)
    lg = dec.prefill(prompt).float()
    lr = ref.forward(prompt, 0)
    tol = 1e-2 * lr.abs().max().item()
    assert (lg - lr).abs().max().item() <= tol
    _greedy_consistent(int(dec.cur_id), lr, tol)
    dec.capture_decode()
    for step in range(6):
        print("case: source", source, "decode step", step, flush=True)
        tok = int(dec.cur_id)
        dec.graph.replay()
        lr = ref.forward(torch.tensor([tok], device="cuda"), prompt.numel() + step)
        tol = 1e-2 * lr.abs().max().item()
        assert (dec.graph_logits.float() - lr).abs().max().item() <= tol, step
        _greedy_consistent(int(dec.cur_id), lr, tol)
        assert int(dec.cur_pos) == prompt.numel() + step + 1
