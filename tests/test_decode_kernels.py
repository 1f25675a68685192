"""GPU tests of the decode-layer kernels between the quantized linears against fp32 torch
restatements of the same math:

* rmsnorm: residual add rounded to fp16 bit-exactly; the normalised row within fp16
  rounding plus the difference of summation order (1 fp16 ulp, rel 2e-3);
* rope_append: rotation bit-identical to the fp32 torch formula rounded to fp16 (the same
  operations in the same order), cache rows written exactly at the given positions and
  nowhere else;
* greedy_next: the index torch.argmax returns (ties: the first), history and position
  updated on the device;
* attend_decode: the rotated key and the value appended bit-exactly at the position (and
  nothing else written), the output within 2e-3 (times max|v|) of fp32 softmax attention
  over the cache prefix, at positions on and around the 64-position span edges and at the
  last slot, with one workspace reused across calls;
* silu_mul: within rel 2e-3 of fp32 silu(g) * u.
"""
import math
import os

import numpy as np

import pytest
import torch

from spectra_amd import kernels as K

pytestmark = pytest.mark.gpu


def case(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.mark.parametrize("rows,hidden", [(1, 3072), (3, 100), (5, 4097)])
@pytest.mark.parametrize("with_res", [False, True])
def test_rmsnorm(hip, rows, hidden, with_res):
    case(rows=rows, hidden=hidden, with_res=with_res)
    g = torch.Generator(device="cuda").manual_seed(rows * hidden)
    h = torch.randn(rows, hidden, device="cuda", generator=g).half()
    r = torch.randn(rows, hidden, device="cuda", generator=g).half() if with_res else None
    w = torch.rand(hidden, device="cuda", generator=g) + 0.5
    h_ref = (h + r) if with_res else h.clone()  # fp16 add, one rounding
    x = K.rmsnorm(h, w, 1e-5, residual=r)
    assert torch.equal(h, h_ref)
    hf = h_ref.float()
    ref = hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5) * w
    torch.testing.assert_close(x.float(), ref, rtol=2e-3, atol=1e-3)


def _rope_ref(x, cos, sin):
    h2 = x.shape[-1] // 2
    a, b = x[..., :h2].float(), x[..., h2:].float()
    return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1).half()


@pytest.mark.parametrize("heads,kv,hd,T", [(24, 8, 128, 1), (4, 2, 64, 9), (8, 8, 96, 3)])
def test_rope_append(hip, heads, kv, hd, T):
    case(heads=heads, kv=kv, hd=hd, T=T)
    L = 200
    g = torch.Generator(device="cuda").manual_seed(hd + T)
    qkv = torch.randn(T, (heads + 2 * kv) * hd + 8, device="cuda", generator=g).half()[:, 8:]  # strided rows
    pos = torch.randperm(L, device="cuda", generator=g)[:T].contiguous()
    inv = 1.0 / (5e5 ** (torch.arange(0, hd, 2, device="cuda", dtype=torch.float32) / hd))
    ang = torch.arange(L, device="cuda", dtype=torch.float32)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang), torch.sin(ang)
    kc = torch.full((kv, L, hd), 7.0, device="cuda", dtype=torch.float16)
    vc = torch.full((kv, L, hd), 7.0, device="cuda", dtype=torch.float16)
    q = K.rope_append(qkv, pos, cos, sin, heads, kv, kc, vc)
    c, s = cos[pos][:, None, :], sin[pos][:, None, :]
    q_ref = _rope_ref(qkv[:, : heads * hd].reshape(T, heads, hd), c, s)
    k_ref = _rope_ref(qkv[:, heads * hd: (heads + kv) * hd].reshape(T, kv, hd), c, s)
    v_ref = qkv[:, (heads + kv) * hd:].reshape(T, kv, hd)
    assert torch.equal(q, q_ref)
    assert torch.equal(kc[:, pos, :].permute(1, 0, 2), k_ref)
    assert torch.equal(vc[:, pos, :].permute(1, 0, 2), v_ref)
    keep = torch.ones(L, dtype=torch.bool, device="cuda")
    keep[pos] = False
    assert bool((kc[:, keep, :] == 7.0).all()) and bool((vc[:, keep, :] == 7.0).all())


def _tables(L, hd):
    inv = 1.0 / (5e5 ** (torch.arange(0, hd, 2, device="cuda", dtype=torch.float32) / hd))
    ang = torch.arange(L, device="cuda", dtype=torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang), torch.sin(ang)


@pytest.mark.parametrize("heads,kv,hd,L", [(24, 8, 128, 768), (4, 4, 64, 1000), (8, 2, 256, 130), (6, 3, 64, 64),
                                           (32, 4, 128, 300), (12, 2, 64, 200), (24, 8, 128, 1100),
                                           (4, 2, 16, 128), (4, 2, 16, 70), (8, 4, 32, 150),
                                           (20, 4, 64, 300), (14, 2, 128, 200), (16, 2, 256, 200)])
@pytest.mark.parametrize("rope", [True, False])
def test_attend_decode(hip, heads, kv, hd, L, rope):
    g = torch.Generator(device="cuda").manual_seed(heads * L + rope)
    kc = torch.randn(kv, L, hd, device="cuda", generator=g).half()
    vc = torch.randn(kv, L, hd, device="cuda", generator=g).half()
    cos, sin = _tables(L, hd) if rope else (None, None)
    ws = torch.zeros((K.attend_workspace_bytes(heads, hd, L),), device="cuda", dtype=torch.uint8)  # reused
    grp = heads // kv
    for p in sorted({0, 1, 62, 63, 64, 65, 511, 512, 513, L // 2, L - 2, L - 1}):
        if p >= L:
            continue
        case(heads=heads, kv=kv, hd=hd, L=L, rope=rope, pos=p)
        qkv = (torch.randn((heads + 2 * kv) * hd, device="cuda", generator=g) * 2).half()
        kc0, vc0 = kc.clone(), vc.clone()
        pos = torch.tensor([p], device="cuda", dtype=torch.int64)
        out = K.attend_decode(qkv, pos, cos, sin, heads, kv, kc, vc, ws)
        q = qkv[: heads * hd].reshape(1, heads, hd)
        k = qkv[heads * hd: (heads + kv) * hd].reshape(1, kv, hd)
        v = qkv[(heads + kv) * hd:].reshape(kv, hd)
        if rope:
            q, k = _rope_ref(q, cos[p][None, None, :], sin[p][None, None, :]), _rope_ref(k, cos[p][None, None, :],
                                                                                        sin[p][None, None, :])
        # the append: row p of both caches, nothing else
        kc0[:, p, :] = k[0]
        vc0[:, p, :] = v
        assert torch.equal(kc, kc0) and torch.equal(vc, vc0)
        kk = kc[:, : p + 1, :].float().transpose(1, 2).repeat_interleave(grp, dim=0)  # [heads, hd, n]
        vv = vc[:, : p + 1, :].float().repeat_interleave(grp, dim=0)  # [heads, n, hd]
        sc = torch.matmul(q[0].float()[:, None, :], kk.contiguous())[:, 0, :] / math.sqrt(hd)
        ref = torch.matmul(torch.softmax(sc, -1)[:, None, :], vv.contiguous())[:, 0, :]
        err = (out.float() - ref).abs().max().item()
        assert err <= 2e-3 * vc.abs().max().item(), (p, err)


def test_attend_workspace_shared_across_shapes(hip):
    """One zeroed workspace serves calls of different shapes in turn (the arrival counters sit
    at its start whatever the shape, and every call leaves them at zero): max_seq 1100 then
    100 then 700, head_dim 128 then 64, each against the fp32 reference."""
    heads, kv = 8, 2
    ws = torch.zeros(max(K.attend_workspace_bytes(heads, hd, L) for hd, L in ((128, 1100), (64, 700))),
                     device="cuda", dtype=torch.uint8)
    g = torch.Generator(device="cuda").manual_seed(11)
    for hd, L, p in ((128, 1100, 1000), (64, 100, 70), (128, 700, 650), (64, 700, 3), (128, 1100, 1099)):
        case(hd=hd, L=L, pos=p)
        kc = torch.randn(kv, L, hd, device="cuda", generator=g).half()
        vc = torch.randn(kv, L, hd, device="cuda", generator=g).half()
        qkv = torch.randn((heads + 2 * kv) * hd, device="cuda", generator=g).half()
        out = K.attend_decode(qkv, torch.tensor([p], device="cuda"), None, None, heads, kv, kc, vc, ws)
        q = qkv[: heads * hd].reshape(heads, hd).float()
        kk = kc[:, : p + 1, :].float().repeat_interleave(heads // kv, dim=0)  # [heads, n, hd]
        vv = vc[:, : p + 1, :].float().repeat_interleave(heads // kv, dim=0)
        sc = (kk @ q[:, :, None])[:, :, 0] / math.sqrt(hd)
        ref = (torch.softmax(sc, -1)[:, None, :] @ vv)[:, 0, :]
        assert (out.float() - ref).abs().max().item() <= 2e-3 * vc.abs().max().item()
    assert int(ws[: heads * 256].view(torch.int32).abs().sum()) == 0  # counters left at zero


@pytest.mark.parametrize("L", [600, 1100])
def test_attend_decode_ignores_rows_past_position(hip, L):
    """Cache rows past the position may hold anything (here NaN): the output and the rows
    up to the position are those of a cache with finite values there."""
    heads, kv, hd, p = 24, 8, 128, 300
    g = torch.Generator(device="cuda").manual_seed(L)
    kc = torch.randn(kv, L, hd, device="cuda", generator=g).half()
    vc = torch.randn(kv, L, hd, device="cuda", generator=g).half()
    cos, sin = _tables(L, hd)
    qkv = (torch.randn((heads + 2 * kv) * hd, device="cuda", generator=g) * 2).half()
    pos = torch.tensor([p], device="cuda", dtype=torch.int64)
    ws = torch.zeros((K.attend_workspace_bytes(heads, hd, L),), device="cuda", dtype=torch.uint8)
    kf, vf = kc.clone(), vc.clone()
    ref = K.attend_decode(qkv, pos, cos, sin, heads, kv, kf, vf, ws)
    kc[:, p + 1:, :] = float("nan")
    vc[:, p + 1:, :] = float("nan")
    out = K.attend_decode(qkv, pos, cos, sin, heads, kv, kc, vc, ws)
    assert torch.isfinite(out).all()
    assert torch.equal(out, ref)
    assert torch.equal(kc[:, : p + 1], kf[:, : p + 1]) and torch.equal(vc[:, : p + 1], vf[:, : p + 1])


@pytest.mark.parametrize("rows,inter", [(1, 8192), (7, 300)])
def test_silu_mul(hip, rows, inter):
    case(rows=rows, inter=inter)
    gen = torch.Generator(device="cuda").manual_seed(inter)
    gu = (torch.randn(rows, 2 * inter, device="cuda", generator=gen) * 3).half()
    act = K.silu_mul(gu)
    gf, uf = gu[:, :inter].float(), gu[:, inter:].float()
    ref = gf * torch.sigmoid(gf) * uf
    torch.testing.assert_close(act.float(), ref, rtol=2e-3, atol=1e-4)


@pytest.mark.parametrize("n", [128256, 1000, 5, 8])
def test_greedy_next(hip, n):
    case(n=n)
    gen = torch.Generator(device="cuda").manual_seed(n)
    logits = torch.randn(n, device="cuda", generator=gen).half()
    token = torch.zeros(1, dtype=torch.int64, device="cuda")
    K.greedy_next(logits, token)
    assert int(token) == int(torch.argmax(logits))
    # equal maxima: the first index, as torch.argmax
    logits[n // 3] = 100.0
    logits[n - 1] = 100.0
    hist = torch.full((10,), -1, dtype=torch.int64, device="cuda")
    pos = torch.tensor([3], dtype=torch.int64, device="cuda")
    K.greedy_next(logits, token, hist, pos)
    assert int(token) == n // 3 == int(torch.argmax(logits))
    assert int(pos) == 4 and int(hist[4]) == n // 3 and int((hist == -1).sum()) == 9


def _argmax_rule(x: torch.Tensor) -> int:
    """torch.argmax's rule, stated on the host: the first NaN, else the first maximum."""
    v = x.float().cpu()
    nan = torch.nonzero(torch.isnan(v))
    if nan.numel():
        return int(nan[0])
    return int(torch.nonzero(v == v.max())[0])


@pytest.mark.parametrize("n", [128256, 300001, 4097])
def test_greedy_next_ties_infinities_nans(hip, n):
    """Equal maxima across scan rounds and threads, all -inf, one finite value among -inf,
    NaNs (several), and the tail past the last 8-value chunk."""
    case(n=n)
    token = torch.zeros(1, dtype=torch.int64, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(n + 1)
    cases = []
    x = torch.full((n,), 2.0, device="cuda", dtype=torch.float16)
    cases.append(x.clone())  # all equal: index 0
    cases.append(torch.full((n,), float("-inf"), device="cuda", dtype=torch.float16))  # all -inf
    x = torch.full((n,), float("-inf"), device="cuda", dtype=torch.float16)
    x[n - 2] = -3.0
    cases.append(x)  # one finite value
    x = torch.randn(n, device="cuda", generator=gen).half()
    x[n - 1] = 50.0
    x[7] = 50.0
    x[n // 2 + 3] = 50.0
    cases.append(x)  # ties far apart (other rounds, other threads, the tail)
    x = torch.randn(n, device="cuda", generator=gen).half()
    x[n - 1] = float("nan")
    x[n // 3 + 5] = float("nan")
    x[2] = 60.0
    cases.append(x)  # NaNs: the first NaN
    for x in cases:
        K.greedy_next(x, token)
        assert int(token) == _argmax_rule(x)


# ---------------------------------------------------------------------------
# the GEMV with fused RMSNorm / SiLU-mul prologues and residual epilogue
# ---------------------------------------------------------------------------
from spectra_amd import compressor as C  # noqa: E402


def _nf4_ops(n, k, had, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).half()
    mask = torch.rand(n, k, device="cuda", generator=g) < 0.005
    w = torch.where(mask, (torch.randn(n, k, device="cuda", generator=g) * 0.2).half(), w)
    q = C.quantize_nf4(w, 64, 0, mask, True)
    col, val = q.outliers()
    ops = K.QWeightOperands(q.packed, q.absmax, None, k, codebook="nf4", group_size=64, hadamard_block=had,
                            marlin_layout=True, outlier_idx=col, outlier_w=val,
                            outlier_rowptr=q.rowptr if col is not None else None)
    w_eff = K.w4_dequant(q.packed, q.absmax, None, out_dtype=torch.float32, codebook="nf4", marlin_layout=True,
                         outlier_idx=col, outlier_w=val, outlier_rowptr=q.rowptr if col is not None else None)
    return ops, w_eff.double().cpu()


def _y_ref(x_eff, w_eff, had):
    """fp64 FWHT(x) @ W_eff^T of one fp32/fp64 row (the library FWHT is bit-exact to the reference)."""
    xr = K.fwht_rows(x_eff.float().reshape(1, -1).contiguous(), had, out_dtype=torch.float32) if had else x_eff
    return (xr.double().cpu().reshape(1, -1) @ w_eff.T).reshape(-1)


def _check(y, ref):
    yv = y.double().cpu().reshape(-1)
    ulp = torch.from_numpy(np.spacing(ref.abs().numpy().astype(np.float16)).astype(np.float64))
    err = (yv - ref).abs()
    assert bool((err <= torch.clamp(ulp, min=1e-2)).all()), float(err.max())
    assert float((yv - ref).norm() / ref.norm()) <= 1e-3


@pytest.mark.parametrize("n,k,had", [(640, 3072, 128), (16384, 3072, 128), (5000, 3072, 0), (512, 1024, 64),
                                     (128256, 3072, 128)])  # the decoder's tied lm_head
def test_gemv_rmsnorm_prologue(hip, n, k, had):
    case(n=n, k=k, had=had)
    ops, w_eff = _nf4_ops(n, k, had, seed=n + k)
    g = torch.Generator(device="cuda").manual_seed(k)
    h = (torch.randn(1, k, device="cuda", generator=g) * 3).half()
    nw = (torch.rand(k, device="cuda", generator=g) + 0.5).half()
    y = K.w4a16_gemv_fused(ops, h, prologue="rmsnorm", norm_weight=nw, eps=1e-5)
    hf = h.double()
    x_eff = hf * torch.rsqrt(hf.pow(2).mean() + 1e-5) * nw.double()
    _check(y, _y_ref(x_eff, w_eff, had))


@pytest.mark.parametrize("n,k,had", [(3072, 8192, 128), (700, 2048, 128)])
def test_gemv_silu_prologue_and_residual(hip, n, k, had):
    case(n=n, k=k, had=had)
    ops, w_eff = _nf4_ops(n, k, had, seed=n + 3 * k)
    g = torch.Generator(device="cuda").manual_seed(n)
    gu = (torch.randn(1, 2 * k, device="cuda", generator=g) * 2).half()
    act = K.silu_mul(gu)  # the prologue is bit-identical to the separate kernel
    ref = _y_ref(act.float(), w_eff, had)
    y = K.w4a16_gemv_fused(ops, gu, prologue="silu_mul")
    _check(y, ref)
    # residual epilogue, in place: h <- fp16(h + fp16(y)), bit-identical to the separate add
    h = (torch.randn(1, n, device="cuda", generator=g) * 4).half()
    h_sep = h + y
    out = K.w4a16_gemv_fused(ops, gu, prologue="silu_mul", residual=h, out=h)
    assert out.data_ptr() == h.data_ptr() and torch.equal(h, h_sep)


def test_gemv_residual_without_prologue(hip):
    case(n=1536, k=3072, had=128, m=3)
    ops, w_eff = _nf4_ops(1536, 3072, 128, seed=9)
    x = torch.randn(3, 3072, device="cuda", generator=torch.Generator(device="cuda").manual_seed(1)).half()
    res = torch.randn(3, 1536, device="cuda", generator=torch.Generator(device="cuda").manual_seed(2)).half()
    y = K.w4a16_gemv_fused(ops, x)  # plain
    assert torch.equal(y, K.w4a16_linear(ops, x))
    r = K.w4a16_gemv_fused(ops, x, residual=res)
    assert torch.equal(r, res + y)


def test_gemv_residual_several_rows_strided(hip):
    """Four rows on the row-owning kernel (down_proj's shape) with a residual whose rows are
    N + 40 apart (a padded view): out of place, then in place (out = the residual view, so
    the output rows are N + 40 apart too); both bit-identical to the separate add of the
    plain call."""
    n, k, m = 3072, 8192, 4
    case(n=n, k=k, had=128, m=m)
    ops, _ = _nf4_ops(n, k, 128, seed=21)
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(m, k, device="cuda", generator=g).half()
    y = K.w4a16_gemv_fused(ops, x)  # plain
    wide = (torch.randn(m, n + 40, device="cuda", generator=g) * 4).half()
    res = wide[:, 8:8 + n]
    sep = res + y
    pads = (wide[:, :8].clone(), wide[:, 8 + n:].clone())
    assert torch.equal(K.w4a16_gemv_fused(ops, x, residual=res), sep)
    out = K.w4a16_gemv_fused(ops, x, residual=res, out=res)
    assert out.data_ptr() == res.data_ptr() and torch.equal(res, sep)
    assert torch.equal(wide[:, :8], pads[0]) and torch.equal(wide[:, 8 + n:], pads[1]), "a store outside the rows"


@pytest.mark.parametrize("n,k,had,pro", [(128256, 3072, 0, "rmsnorm"),  # the decoder's lm_head
                                          (1000, 1024, 128, "none"), (257, 2048, 0, "rmsnorm")])
def test_gemv_fused_greedy_pick(hip, n, k, had, pro):
    """The greedy pick gathered in the GEMV epilogue (one atomic max per workgroup into 64
    slots) then read by greedy_finish: the same token, history and position update as
    greedy_next on the stored outputs, and the slots left at 0 for the next pick."""
    case(n=n, k=k, had=had, pro=pro)
    ops, _ = _nf4_ops(n, k, had, seed=n + 3)
    g = torch.Generator(device="cuda").manual_seed(n)
    nw = (torch.rand(k, device="cuda", generator=g) + 0.5).half()
    kw = dict(prologue="rmsnorm", norm_weight=nw) if pro == "rmsnorm" else {}
    pick = K.argmax_slots()
    for trial in range(3):
        h = (torch.randn(1, k, device="cuda", generator=g) * 3).half()
        y = K.w4a16_gemv_fused(ops, h, argmax_key=pick, **kw)
        # (the pick runs on one GEMV kernel; without it the planner may choose another, whose
        # fp32 summation order differs)
        y0 = K.w4a16_gemv_fused(ops, h, **kw)
        assert float((y.float() - y0.float()).abs().max()) <= 1e-2 * max(1.0, float(y0.float().abs().max()))
        tok, hist, pos = (torch.zeros(1, dtype=torch.int64, device="cuda"),
                          torch.full((8,), -1, dtype=torch.int64, device="cuda"),
                          torch.tensor([2], dtype=torch.int64, device="cuda"))
        K.greedy_finish(pick, tok, hist, pos)
        ref_tok, ref_hist, ref_pos = tok.clone(), hist.clone(), torch.tensor([2], dtype=torch.int64, device="cuda")
        ref_hist.fill_(-1)
        K.greedy_next(y.reshape(-1), ref_tok, ref_hist, ref_pos)
        assert int(tok) == int(ref_tok) == _argmax_rule(y.reshape(-1)), trial
        assert torch.equal(hist, ref_hist) and int(pos) == int(ref_pos) == 3
        assert int(pick.abs().sum()) == 0


def test_gemv_fused_greedy_pick_ties_and_nans(hip):
    """Equal outputs (every weight row the same): the lowest index; a NaN activation (every
    output NaN): index 0, as torch.argmax."""
    n, k = 3000, 1024
    case(n=n, k=k, rows="identical")
    g = torch.Generator(device="cuda").manual_seed(5)
    w = (torch.randn(1, k, device="cuda", generator=g) * 0.02).half().expand(n, k).contiguous()
    q = C.quantize_nf4(w, 64, 0, None, True)
    ops = K.QWeightOperands(q.packed, q.absmax, None, k, codebook="nf4", group_size=64, marlin_layout=True)
    pick = K.argmax_slots()
    tok = torch.zeros(1, dtype=torch.int64, device="cuda")
    h = torch.randn(1, k, device="cuda", generator=g).half()
    y = K.w4a16_gemv_fused(ops, h, argmax_key=pick)
    assert bool((y == y[0, 0]).all())
    K.greedy_finish(pick, tok)
    assert int(tok) == 0
    h[0, 17] = float("nan")
    y = K.w4a16_gemv_fused(ops, h, argmax_key=pick)
    assert bool(torch.isnan(y).all())
    K.greedy_finish(pick, tok)
    assert int(tok) == 0 and int(pick.abs().sum()) == 0


# ---------------------------------------------------------------------------
# the 4-bit KV cache (reference engine.py:614-700)
# ---------------------------------------------------------------------------
GOLD_KV4 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kv4_quant.npz")


@pytest.mark.parametrize("name", ["fp16_128", "fp16_64", "bf16_128", "bf16_96"])
def test_kv4_quantize_and_dequant_reference_vectors(hip, name):
    """Vectors from the reference's own _quantize / _dequantize (constant, zero and
    one-signed groups included): the kernel's codes, scales and zero points for fp16 rows
    and the dequant of the reference's codes, bit for bit."""
    case(name=name)
    g = np.load(GOLD_KV4)
    packed, scales, zeros = g[name + "_packed"], g[name + "_scales"], g[name + "_zeros"]
    rows, d = g[name + "_x"].shape
    if name.startswith("fp16"):
        x = torch.from_numpy(g[name + "_x"]).cuda()
        c, s, z = K.kv4_quantize(x)
        assert np.array_equal(c.cpu().numpy(), packed.reshape(rows, d // 2))
        assert np.array_equal(s.cpu().numpy().view(np.uint16), scales.reshape(rows, d // 32).view(np.uint16))
        assert np.array_equal(z.cpu().numpy(), zeros.reshape(rows, d // 32))
    deq = K.kv4_dequantize(torch.from_numpy(packed.reshape(rows, d // 2)).cuda(),
                           torch.from_numpy(scales.reshape(rows, d // 32)).cuda(),
                           torch.from_numpy(zeros.reshape(rows, d // 32)).cuda())
    assert np.array_equal(deq.cpu().view(torch.int16).numpy(), g[name + "_deq"])


@pytest.mark.gpu
@pytest.mark.parametrize("q4", [False, True])
def test_attend_decode_position_outside_cache(hip, q4):
    """A position outside [0, max_seq) appends nothing and gives NaN outputs; the next call
    at a valid position is unaffected (the merge counters were left at zero)."""
    heads, kv, hd, L, W = 8, 4, 64, 200, 32
    g = torch.Generator(device="cuda").manual_seed(77)
    cos, sin = _tables(L, hd)
    ws = torch.zeros(K.attend_workspace_bytes(heads, hd, L), device="cuda", dtype=torch.uint8)
    if q4:
        k4 = K.kv4_quantize(torch.randn(kv, L, hd, device="cuda", generator=g).half())
        v4 = K.kv4_quantize(torch.randn(kv, L, hd, device="cuda", generator=g).half())
        kc = torch.randn(kv, W, hd, device="cuda", generator=g).half()
        vc = torch.randn(kv, W, hd, device="cuda", generator=g).half()
        state = [kc, vc, *k4, *v4]
        run = lambda qkv, pos: K.attend_decode_q4(qkv, pos, cos, sin, heads, kv, kc, vc, k4, v4, ws)
    else:
        kc = torch.randn(kv, L, hd, device="cuda", generator=g).half()
        vc = torch.randn(kv, L, hd, device="cuda", generator=g).half()
        state = [kc, vc]
        run = lambda qkv, pos: K.attend_decode(qkv, pos, cos, sin, heads, kv, kc, vc, ws)
    for p in (L, L + 5, -1):
        case(q4=q4, pos=p)
        before = [t.clone() for t in state]
        qkv = torch.randn((heads + 2 * kv) * hd, device="cuda", generator=g).half()
        out = run(qkv, torch.tensor([p], device="cuda", dtype=torch.int64))
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(state, before)), f"pos={p}: the cache changed"
        assert torch.isnan(out.float()).all(), f"pos={p}: outputs are not NaN"
    # a valid position afterwards: the same outputs as on a fresh workspace
    case(q4=q4, pos=L - 1)
    qkv = torch.randn((heads + 2 * kv) * hd, device="cuda", generator=g).half()
    pos = torch.tensor([L - 1], device="cuda", dtype=torch.int64)
    before = [t.clone() for t in state]
    out = run(qkv, pos).clone()
    for t, b in zip(state, before):
        t.copy_(b)
    ws.zero_()
    ref = run(qkv, pos)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.equal(out, ref)


@pytest.mark.parametrize("heads,kv,hd,L,W", [(24, 8, 128, 300, 128), (8, 2, 64, 200, 16), (6, 3, 256, 130, 64),
                                              (8, 4, 32, 100, 16)])
def test_attend_decode_q4(hip, heads, kv, hd, L, W):
    import oracle as O
    g = torch.Generator(device="cuda").manual_seed(heads + L)
    kfull = torch.randn(kv, L, hd, device="cuda", generator=g).half()
    vfull = torch.randn(kv, L, hd, device="cuda", generator=g).half()
    cos, sin = _tables(L, hd)
    k4 = K.kv4_quantize(kfull)
    v4 = K.kv4_quantize(vfull)
    kw = torch.zeros(kv, W, hd, device="cuda", dtype=torch.float16)
    vw = torch.zeros_like(kw)
    ws = torch.zeros(K.attend_workspace_bytes(heads, hd, L), device="cuda", dtype=torch.uint8)
    grp = heads // kv
    p0 = L // 2
    last = torch.arange(max(0, p0 - W), p0, device="cuda")  # the window before the first step
    kw.index_copy_(1, last % W, kfull[:, last])
    vw.index_copy_(1, last % W, vfull[:, last])
    for p in range(p0, p0 + 4):
        case(heads=heads, kv=kv, hd=hd, L=L, W=W, pos=p)
        qkv = (torch.randn((heads + 2 * kv) * hd, device="cuda", generator=g) * 2).half()
        pos = torch.tensor([p], device="cuda", dtype=torch.int64)
        out = K.attend_decode_q4(qkv, pos, cos, sin, heads, kv, kw, vw, k4, v4, ws)
        q = _rope_ref(qkv[: heads * hd].reshape(1, heads, hd), cos[p][None, None, :], sin[p][None, None, :])
        k = _rope_ref(qkv[heads * hd: (heads + kv) * hd].reshape(1, kv, hd), cos[p][None, None, :],
                      sin[p][None, None, :])[0]
        v = qkv[(heads + kv) * hd:].reshape(kv, hd)
        # the append: fp16 ring slot p % W, and the codes of position p
        assert torch.equal(kw[:, p % W], k) and torch.equal(vw[:, p % W], v)
        kc, ks, kz = K.kv4_quantize(k.reshape(kv, 1, hd))
        assert torch.equal(k4[0][:, p], kc[:, 0]) and torch.equal(k4[1][:, p], ks[:, 0]) and torch.equal(k4[2][:, p], kz[:, 0])
        kfull[:, p], vfull[:, p] = k, v
        # reference: window positions in fp16, older ones through the reference's dequant
        kr = kfull[:, : p + 1].float().clone()
        vr = vfull[:, : p + 1].float().clone()
        old = p + 1 - W
        if old > 0:
            for src, dst in ((k4, kr), (v4, vr)):
                cn, sn_, zn = (t[:, :old].cpu().numpy() for t in src)
                deq = O.kv4_dequantize(cn.reshape(-1, hd // 32, 16), sn_.reshape(-1, hd // 32, 1),
                                       zn.reshape(-1, hd // 32, 1))
                dst[:, :old] = torch.from_numpy(O.bf16_bits_to_f32(deq).reshape(kv, old, hd)).cuda()
        kk = kr.transpose(1, 2).repeat_interleave(grp, dim=0)
        vv = vr.repeat_interleave(grp, dim=0)
        sc = torch.matmul(q[0].float()[:, None, :], kk.contiguous())[:, 0, :] / math.sqrt(hd)
        ref = torch.matmul(torch.softmax(sc, -1)[:, None, :], vv.contiguous())[:, 0, :]
        err = (out.float() - ref).abs().max().item()
        assert err <= 2e-3 * vfull.abs().max().item(), (p, err)
