#!/usr/bin/env python3
"""Benchmark of SPECTRA's W4A16 linear hot path on one MI355X.

Headline workload: the full SPECTRA linear at M=1 on
Llama-3.2-3B shapes -- fused QKV (K=3072, N=5120) and down_proj (K=8192, N=3072),
fp16 activations N(0,1) rotated by a blockwise FWHT-128, NF4 block-64 weights with
fp16 absmax, 0.5% fp16 CSR outliers of magnitude |N(0,0.2)|, seeded CPU generators.

One step = one QKV GEMV + one down_proj GEMV.  Weight copies rotate over a pool
larger than the 256 MB Infinity Cache so every launch streams from HBM; the K timed
steps are captured in one HIP graph (as the reference's engine captures its decode
step, engine.py:1813-1830) and replayed between synchronizations.

value = algorithmic bytes per step / time per step (GB/s); bytes are the stored
operand bytes (packed + absmax + CSR) + x + y of both launches.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from spectra_amd import _lib as L  # noqa: E402
from spectra_amd import compressor as C  # noqa: E402
from spectra_amd import kernels as K  # noqa: E402

METRIC = "W4A16 GEMV HBM GB/s (% of 8 TB/s peak) at M=1; decode tok/s, 3B-shape"
PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA
HAD = 128


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# synthetic Format B weights (seeded on the CPU: identical on every box)
# ---------------------------------------------------------------------------
def synth_nf4(n: int, k: int, seed: int, ratio: float = 0.005, dev="cuda") -> C.NF4Weight:
    gw = torch.Generator().manual_seed(seed + 1)
    w = (torch.randn(n, k, generator=gw) * 0.02).half()
    mask = None
    if ratio > 0:
        nnz = int(round(ratio * n * k))
        pos = torch.randperm(n * k, generator=torch.Generator().manual_seed(seed + 2))[:nnz]
        gv = torch.Generator().manual_seed(seed + 3)
        mag = torch.randn(nnz, generator=gv).abs() * 0.2
        sign = torch.where(torch.rand(nnz, generator=gv) < 0.5, -1.0, 1.0)
        w.view(-1)[pos] = (mag * sign).half()
        mask = torch.zeros(n * k, dtype=torch.bool)
        mask[pos] = True
        mask = mask.view(n, k).to(dev)
    # the synthetic matrix is taken as already stored in the rotated basis
    q = C.quantize_nf4(w.to(dev), 64, 0, mask, True)
    q.hadamard_block = HAD
    return q


def synth_nf4_gpu(n: int, k: int, seed: int, ratio: float = 0.005) -> C.NF4Weight:
    """Same distribution drawn with the GPU generator (for the 394M-weight lm_head)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).half()
    mask = torch.rand(n, k, generator=g, device="cuda") < ratio
    mag = (torch.randn(n, k, generator=g, device="cuda").abs() * 0.2).half()
    w = torch.where(mask, torch.where(torch.rand(n, k, generator=g, device="cuda") < 0.5, -mag, mag), w)
    q = C.quantize_nf4(w, 64, 0, mask, True)
    q.hadamard_block = HAD
    return q


def clone_nf4(q: C.NF4Weight) -> C.NF4Weight:
    return C.NF4Weight(q.packed.clone(), q.absmax.clone(), q.rowptr.clone(), q.col.clone(), q.val.clone(), q.k,
                       q.blocksize, q.hadamard_block, q.marlin_layout)


def operands(q: C.NF4Weight) -> K.QWeightOperands:
    col, val = q.outliers()
    return K.QWeightOperands(q.packed, q.absmax, None, q.k, codebook="nf4", group_size=q.blocksize,
                             hadamard_block=q.hadamard_block, marlin_layout=q.marlin_layout, outlier_idx=col,
                             outlier_w=val, outlier_rowptr=q.rowptr if col is not None else None)


def gemv_bytes(q: C.NF4Weight, m: int = 1) -> int:
    return q.nbytes() + m * q.k * 2 + m * q.n * 2


class Launcher:
    """Pre-bound linear call (descriptor, x, out[, workspace]) -> one ctypes call each.
    m = 1 uses the GEMV family, 2 <= m <= GEMV_MAX_M the dispatching entry
    (spectra_w4a16_linear: GEMV or small-batch family by shape), larger m the GEMM entry."""

    def __init__(self, lib, ops: K.QWeightOperands, x: torch.Tensor, out: torch.Tensor):
        m = x.shape[0]
        self.ops = ops
        if m == 1:
            self.name, self.fn = "spectra_w4a16_gemv", lib.spectra_w4a16_gemv
            self.args = (ctypes.byref(ops.desc), x.data_ptr(), x.stride(0), m, L.F16, out.data_ptr(), out.stride(0))
        else:
            ws = lib.spectra_w4a16_gemm_workspace(ctypes.byref(ops.desc), m, L.F16)
            self.ws = torch.empty(max(int(ws), 256), dtype=torch.uint8, device=x.device)
            if m <= K.GEMV_MAX_M:
                self.name, self.fn = "spectra_w4a16_linear", lib.spectra_w4a16_linear
            else:
                self.name, self.fn = "spectra_w4a16_gemm", lib.spectra_w4a16_gemm
            self.args = (ctypes.byref(ops.desc), x.data_ptr(), x.stride(0), m, L.F16, out.data_ptr(), out.stride(0),
                         self.ws.data_ptr(), self.ws.numel())

    def __call__(self, stream: int) -> None:
        st = self.fn(*self.args, stream)
        if st != L.OK:
            L.check(self.name, st)


def graph_of(calls, reps: int = 1) -> torch.cuda.CUDAGraph:
    for c in calls[: min(len(calls), 4)]:
        c(torch.cuda.current_stream().cuda_stream)  # eager warm-up before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream().cuda_stream
        for _ in range(reps):
            for c in calls:
                c(s)
    return g


def time_graph(g: torch.cuda.CUDAGraph, iters: int = 3) -> float:
    """Median seconds of one replay, measured with events on the replay stream."""
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / 1e3)
    return float(np.median(ts))


def pool_copies(bytes_per_copy: int, pool_bytes: float) -> int:
    return max(2, int(math.ceil(pool_bytes / bytes_per_copy)))


# ---------------------------------------------------------------------------
# CPU baseline: the oracle's torch restatement of the reference path, on the host cores
# ---------------------------------------------------------------------------
def _host_threads() -> int:
    """The host cores this process may use: the box's per-GPU share (OMP_NUM_THREADS, set by
    the box) when given, else every core."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(env))) if env and env.isdigit() else n


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _median_time(fn, min_runs: int, budget_s: float) -> float:
    fn()  # warm-up
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < min_runs or (time.perf_counter() < t_end and len(ts) < 1000):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_baseline(qs, xs, budget_s: float = 8.0) -> dict:
    """cfg2 step (QKV + down_proj GEMV) on the host with torch: variant A is the per-call
    reference path (NF4 dequant -> W_eff, FWHT-128 of x, float32 product; tests/test_kernels.py:31-46,
    engine.py:186-210), variant B the float32 product alone on pre-dequantized W_eff; medians
    of at least 20 runs."""
    from oracle import torch_ref as TR
    threads = _host_threads()
    torch.set_num_threads(threads)
    ops = [tuple(t.cpu() for t in (q.packed, q.absmax, q.rowptr, q.col, q.val)) for q in qs]
    hx = [x.cpu() for x in xs]
    step_bytes = sum(gemv_bytes(q) for q in qs)

    def step_a():
        for o, x in zip(ops, hx):
            TR.linear_a(x, *o, hadamard_block=HAD)

    w_eff = [TR.nf4_dequant(*o) for o in ops]

    def step_b():
        for w, x in zip(w_eff, hx):
            TR.linear_b(x, w, hadamard_block=HAD)

    ta = _median_time(step_a, 20, budget_s)
    tb = _median_time(step_b, 20, budget_s / 2)
    return {"value": round(step_bytes / ta / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"cfg2 steps (QKV + down_proj GEMV, M=1) with oracle/torch_ref.py: variant A (per-call NF4 "
                      f"dequant + FWHT-128 + fp32 matmul) {ta * 1e3:.2f} ms/step (median); variant B (fp32 matmul "
                      f"on pre-dequantized W_eff) {tb * 1e3:.3f} ms/step",
            "variant_b_value": round(step_bytes / tb / 1e9, 2), "cpu_model": _cpu_model(),
            "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}


def cpu_gemm_baseline(qs, a, budget_s: float = 10.0) -> dict:
    """cfg4's first prefill GEMM (M=2048, K=4096, N=14336) on the host: variant A (dequant +
    FWHT-128 of A + fp32 product) and variant B (fp32 product on pre-dequantized W_eff),
    medians of at least 20 runs, in TFLOP/s of the 2*M*K*N product."""
    from oracle import torch_ref as TR
    torch.set_num_threads(_host_threads())
    q = qs
    o = tuple(t.cpu() for t in (q.packed, q.absmax, q.rowptr, q.col, q.val))
    ha = a.cpu()
    flops = 2 * ha.shape[0] * q.k * q.n
    ta = _median_time(lambda: TR.linear_a(ha, *o, hadamard_block=q.hadamard_block), 20, budget_s)
    w = TR.nf4_dequant(*o)
    tb = _median_time(lambda: TR.linear_b(ha, w, hadamard_block=q.hadamard_block), 20, budget_s / 2)
    return {"cfg4_cpu_gemm_variant_a_TFLOPs": round(flops / ta / 1e12, 4),
            "cfg4_cpu_gemm_variant_b_TFLOPs": round(flops / tb / 1e12, 4),
            "cfg4_cpu_note": f"M=2048 K={q.k} N={q.n}, bf16 activations, medians: variant A {ta * 1e3:.0f} ms, "
                             f"variant B {tb * 1e3:.0f} ms"}


def cpu_decode_baseline(dev, prompt_len: int = 16, tokens: int = 4) -> dict:
    """cfg5 variant B on the host: the same random-init 28-layer decoder (seed 0), every
    weight dequantized once to float32 W_eff, then the oracle's float32 decoder
    (oracle/torch_ref.py) prefills ``prompt_len`` tokens and generates ``tokens`` greedy
    tokens; tok/s over the generated tokens."""
    from oracle import torch_ref as TR
    from spectra_amd.engine import DecoderConfig, SpectraDecoder
    torch.set_num_threads(_host_threads())
    dec = SpectraDecoder(DecoderConfig(max_seq=768))
    c = dec.cfg

    def w(q):  # dequantized on the GPU with the oracle's restatement, kept on the host
        col, val = q.outliers()
        return TR.nf4_dequant(q.packed, q.absmax, q.rowptr if col is not None else None, col, val,
                              marlin=q.marlin_layout, blocksize=q.blocksize).cpu()
    layers = [[w(q) for q in layer] for layer in dec.layers_q]
    had = [[q.hadamard_block for q in layer] for layer in dec.layers_q]
    emb, head = w(dec.embed_q), w(dec.lm_q)
    norms = [t.float().cpu() for t in dec.norm_w]
    del dec
    torch.cuda.empty_cache()
    ref = TR.Decoder(layers, had, norms, emb, head, heads=c.heads, kv_heads=c.kv_heads, rope_theta=c.rope_theta,
                     rms_eps=c.rms_eps, max_seq=c.max_seq)
    prompt = torch.randint(0, c.vocab, (prompt_len,), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        tok = int(torch.argmax(ref.forward(prompt, 0)))
        t0 = time.perf_counter()
        for i in range(tokens):
            tok = int(torch.argmax(ref.forward(torch.tensor([tok]), prompt_len + i)))
        dt = time.perf_counter() - t0
    return {"cfg5_cpu_decode_tok_s": round(tokens / dt, 3), "cfg5_cpu_decode_ms_per_token": round(dt * 1e3 / tokens, 1),
            "cfg5_cpu_note": f"variant B on {torch.get_num_threads()} host threads ({_cpu_model()}): float32 W_eff "
                             f"(13 GB), {prompt_len}-token prompt, {tokens} greedy tokens timed"}


# ---------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pool-gb", type=float, default=1.2, help="weight pool that defeats the 256 MB Infinity Cache")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-detail", action="store_true", help="skip the secondary configs")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="only run the dominant kernel's timing loop (for rocprofv3 runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run plain device copies of COPY_BYTES each (PMC traffic calibration)")
    ap.add_argument("--profile-gemm", action="store_true",
                    help="only run the cfg4 prefill GEMMs a few times (for rocprofv3 counter runs)")
    ap.add_argument("--profile-gemm-handwritten", action="store_true",
                    help="as --profile-gemm, on the hand-written MFMA GEMM instead of the library path")
    ap.add_argument("--profile-small-batch", action="store_true",
                    help="only run cfg3's small-batch calls (down_proj, gate_up) a few times (rocprofv3 runs)")
    ap.add_argument("--small-batch-m", type=int, default=16, choices=(2, 3, 4, 8, 16),
                    help="rows per call for --profile-small-batch (2-4: the row-owning GEMV; 8, 16: the MFMA family)")
    ap.add_argument("--decode-e2e", action="store_true",
                    help="only run the cfg5 end-to-end decode (for rocprofv3 runs); prints its JSON fields")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "sharding across GPUs is not built: each GPU would run these kernels at its shard's shape",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU", file=sys.stderr)
        sys.exit(1)
    lib = L.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        calibrate_copy(dev)
        return
    if args.decode_e2e:
        print(json.dumps(decode_e2e(dev)), flush=True)
        return
    if args.profile_gemm or args.profile_gemm_handwritten:
        print(json.dumps(profile_gemm(lib, dev, "dispatch" if args.profile_gemm else "handwritten")), flush=True)
        return
    if args.profile_small_batch:
        print(json.dumps(profile_small_batch(L.load(), dev, args.pool_gb, m=args.small_batch_m)), flush=True)
        return

    # ---- cfg2 operands
    log("bench: building cfg2 weights (QKV 3072->5120, down 8192->3072, NF4 b64, 0.5% CSR)")
    q_qkv = synth_nf4(5120, 3072, seed=0)
    q_down = synth_nf4(3072, 8192, seed=10)
    gx = torch.Generator().manual_seed(0)
    x_qkv = torch.randn(1, 3072, generator=gx).half().to(dev)
    x_down = torch.randn(1, 8192, generator=gx).half().to(dev)
    y_qkv = torch.empty(1, 5120, dtype=torch.float16, device=dev)
    y_down = torch.empty(1, 3072, dtype=torch.float16, device=dev)
    b_qkv, b_down = gemv_bytes(q_qkv), gemv_bytes(q_down)
    step_bytes = b_qkv + b_down
    P = pool_copies(q_qkv.nbytes() + q_down.nbytes(), args.pool_gb * 1e9)
    log(f"bench: pool of {P} weight copies ({P * (q_qkv.nbytes() + q_down.nbytes()) / 1e9:.2f} GB)")
    pool = [(q_qkv, q_down)] + [(clone_nf4(q_qkv), clone_nf4(q_down)) for _ in range(P - 1)]
    ops = [(operands(a), operands(b)) for a, b in pool]
    qkv_calls = [Launcher(lib, oa, x_qkv, y_qkv) for oa, _ in ops]
    down_calls = [Launcher(lib, ob, x_down, y_down) for _, ob in ops]

    # ---- dominant kernel timing (down_proj GEMV, HIP events over a graph of launches)
    nl = max(P, 100)
    g_down = graph_of([down_calls[i % P] for i in range(nl)])
    t_down = time_graph(g_down) / nl
    if args.profile_kernel:
        for _ in range(5):
            g_down.replay()
        torch.cuda.synchronize()
        log(f"bench: down_proj GEMV {t_down * 1e6:.2f} us/launch")
        return
    g_qkv = graph_of([qkv_calls[i % P] for i in range(nl)])
    t_qkv = time_graph(g_qkv) / nl

    # ---- the timed run: K steps, one graph, between synchronizations
    steps, warm = args.steps, args.warmup
    for i in range(warm):
        qkv_calls[i % P](torch.cuda.current_stream().cuda_stream)
        down_calls[i % P](torch.cuda.current_stream().cuda_stream)
    calls = []
    for i in range(steps):
        calls += [qkv_calls[i % P], down_calls[i % P]]
    g = graph_of(calls)
    g.replay()  # untimed replay
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / steps
    value = step_bytes / (wall / steps) / 1e9

    # correctness guard on the measured outputs (fp16 output of the last launched copy)
    y_chk = torch.empty_like(y_down)
    ref = K.fused_w4a16_gemv_hdsq(x_down, pool[(steps - 1) % P][1].packed, pool[(steps - 1) % P][1].absmax, None,
                                  outlier_idx=q_down.col, outlier_w=q_down.val, marlin_layout=True, codebook="nf4",
                                  hadamard_block=HAD, outlier_rowptr=q_down.rowptr, out=y_chk)
    assert torch.equal(ref, y_down), "graph replay output differs from an eager launch"

    achieved = b_down / t_down / 1e9
    traffic, traffic_note = measured_traffic()
    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic (seeded CPU generators; random NF4 weights, N(0,1) activations)",
        "config": {"workload": "cfg2: M=1 fused QKV (K=3072,N=5120) + down_proj (K=8192,N=3072) GEMV, NF4 block 64 "
                               "+ fp16 absmax + FWHT-128 activations + 0.5% fp16 CSR outliers",
                   "global_batch": 1, "seq_len": 1, "parallelism": "none (1 GPU)",
                   "bytes_per_step": step_bytes, "weight_pool_copies": P, "timing": "one HIP graph of all steps"},
        "roofline": {"bound": "hbm", "kernel": "gemv_rows_kernel (down_proj K=8192 N=3072)",
                     "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_note, "algorithmic_bytes_per_launch": b_down,
                     "avg_launch_us": round(t_down * 1e6, 3)},
        # the bars the -m gpu parity tests hold these kernels to (tests/test_gpu_parity.py)
        "parity": {"fp16_out": "max-abs <= max(1e-2, 1 fp16 ulp of |y|), rel-L2 <= 1e-3 vs fp64(x_rot) . fp64(W_eff)",
                   "bf16_out": "max-abs <= 1 bf16 ulp + 1e-2, rel-L2 <= 5e-3",
                   "w_eff_quantizers_fwht": "bit-exact", "replay_check": "graph output equals an eager launch"},
    }
    detail = {"qkv_gemv_us": round(t_qkv * 1e6, 3), "qkv_gemv_GBps": round(b_qkv / t_qkv / 1e9, 1),
              "down_gemv_us": round(t_down * 1e6, 3), "down_gemv_GBps": round(achieved, 1)}
    del g_down, g_qkv
    detail.update(ceilings(lib, dev, args.pool_gb, {"qkv": (b_qkv, t_qkv), "down": (b_down, t_down)}))
    if not args.no_detail:
        detail.update(secondary(lib, dev, args.pool_gb))
    result["detail"] = detail
    if not args.no_cpu_baseline:
        log("bench: timing the CPU restatement (bounded sample)")
        result["cpu_baseline"] = cpu_baseline([q_qkv, q_down], [x_qkv, x_down])
        if not args.no_detail:
            log("bench: cfg4 GEMM on the CPU")
            q4 = synth_nf4(14336, 4096, seed=40 + 4096)
            a4 = torch.randn(2048, 4096, generator=torch.Generator().manual_seed(4096)).bfloat16()
            result["cpu_baseline"].update(cpu_gemm_baseline(q4, a4))
            del q4, a4
            log("bench: cfg5 on the CPU (variant B, reduced token count)")
            result["cpu_baseline"].update(cpu_decode_baseline(dev))
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


def ceilings(lib, dev, pool_gb: float, gemvs: dict) -> dict:
    """The floor and ceiling of a one-launch stream on this GPU, timed like the GEMVs (a graph
    of 100 launches, HIP events on the replay stream), with the GEMVs' launch geometry (256
    workgroups of 1024 threads): an empty kernel (the fixed cost of a launch), and a plain
    streaming read of each GEMV's algorithmic bytes with its load pattern, rotating over a
    buffer larger than the Infinity Cache.  ``gemvs``: name -> (bytes, seconds per launch)."""
    grid, block, nl = 256, 1024, 100

    class Call:
        def __init__(self, fn, *args):
            self.fn, self.args = fn, args

        def __call__(self, stream):
            L.check(self.fn.__name__, self.fn(*self.args, stream))

    empty = Call(lib.spectra_measure_empty, grid, block)
    t_empty = time_graph(graph_of([empty] * nl)) / nl
    out = {"launch_floor_us": round(t_empty * 1e6, 3)}
    buf = torch.empty(int(pool_gb * 1e9) // 256 * 256, dtype=torch.uint8, device=dev)
    sink = torch.zeros(block, dtype=torch.int32, device=dev)
    for name, (nbytes, t_gemv) in gemvs.items():
        b16 = (nbytes + 15) // 16 * 16
        slot = (b16 + 4095) // 4096 * 4096
        copies = buf.numel() // slot
        calls = [Call(lib.spectra_measure_read, buf.data_ptr() + (i % copies) * slot, b16, grid, block,
                      sink.data_ptr()) for i in range(nl)]
        t_read = time_graph(graph_of(calls)) / nl
        out[f"read_ceiling_{name}_us"] = round(t_read * 1e6, 3)
        out[f"read_ceiling_{name}_GBps"] = round(nbytes / t_read / 1e9, 1)
        out[f"{name}_gemv_over_read_ceiling"] = round(t_gemv / t_read, 3)
    out["ceiling_note"] = (f"launch floor: an empty kernel of {grid} x {block} threads; read ceiling: a plain "
                           "16-byte-per-thread streaming read of the GEMV's algorithmic bytes with its load pattern "
                           f"and geometry, rotating over {buf.numel() / 1e9:.2f} GB; both in a graph of {nl} "
                           "launches, as the GEMVs are timed")
    del buf
    return out


COPY_BYTES = 16 << 20  # plain copy of known size: FETCH_SIZE / WRITE_SIZE scale factors

# The translation units that fix the measured kernel's memory traffic (the kernel's
# instantiation and its launch plan); the hash covers them and every header they include.
TRAFFIC_ROOTS = ("spectra_amd/csrc/gemv_rows_plain.hip", "spectra_amd/csrc/gemv.hip")


def include_closure(roots) -> list:
    """The files ``roots`` name and every local header they include, directly or through
    other headers (``#include "..."`` resolved next to the including file, else in
    ``include/``, the library's public header directory)."""
    import re
    seen, todo = [], list(roots)
    while todo:
        rel = os.path.normpath(todo.pop())
        if rel in seen:
            continue
        seen.append(rel)
        with open(os.path.join(ROOT, rel)) as f:
            for inc in re.findall(r'^\s*#\s*include\s+"([^"]+)"', f.read(), re.M):
                near = os.path.join(os.path.dirname(rel), inc)
                todo.append(near if os.path.exists(os.path.join(ROOT, near)) else os.path.join("include", inc))
    return sorted(seen)


TRAFFIC_SOURCES = tuple(include_closure(TRAFFIC_ROOTS))


def kernel_source_hash() -> str:
    import hashlib
    h = hashlib.sha256()
    for rel in TRAFFIC_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def measured_traffic():
    """HBM bytes per launch of the down_proj GEMV from the committed PMC summary, only when
    it was measured on the kernel these sources build (same sha256); else None."""
    tf = os.path.join(ROOT, "profiles", "traffic_gemv_cfg2_down.json")
    if not os.path.exists(tf):
        return None, "no PMC summary"
    with open(tf) as f:
        rec = json.load(f)
    if rec.get("kernel_source_sha256") != kernel_source_hash():
        return None, "PMC summary was measured on other kernel sources (sha256 differs): not reported"
    return rec.get("hbm_bytes_per_launch"), "profiles/traffic_gemv_cfg2_down.json (sha256 of the kernel sources matches)"


def calibrate_copy(dev) -> None:
    """Plain device-to-device copies of COPY_BYTES, rotating over a pool larger than the
    Infinity Cache so every copy reads from and writes to HBM.  The PMC counters of these
    dispatches give bytes per counted KiB for reads and writes."""
    n = 48
    src = [torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(i) for i in range(n)]
    dst = [torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev) for _ in range(n)]
    torch.cuda.synchronize()
    for rep in range(3):
        for i in range(n):
            dst[i].copy_(src[(i + rep) % n])
    torch.cuda.synchronize()
    log(f"bench: {3 * n} copies of {COPY_BYTES} bytes")


def secondary(lib, dev, pool_gb: float) -> dict:
    """cfg1 (plain NF4 GEMV), cfg3 (small-M), cfg4 (prefill GEMM) and the 28-layer
    per-token linear chain of cfg5 -- reported as detail, not as the headline."""
    out = {}
    # cfg1: plain NF4, K=N=4096, no rotation, no outliers
    q1 = synth_nf4(4096, 4096, seed=20, ratio=0.0)
    q1.hadamard_block = 0
    x1 = torch.randn(1, 4096, generator=torch.Generator().manual_seed(20)).half().to(dev)
    y1 = torch.empty(1, 4096, dtype=torch.float16, device=dev)
    P = pool_copies(q1.nbytes(), pool_gb * 1e9)
    pool = [q1] + [clone_nf4(q1) for _ in range(P - 1)]
    calls = [Launcher(lib, operands(q), x1, y1) for q in pool]
    t = time_graph(graph_of([calls[i % P] for i in range(max(P, 100))])) / max(P, 100)
    out["cfg1_gemv_us"] = round(t * 1e6, 3)
    out["cfg1_gemv_GBps"] = round(gemv_bytes(q1) / t / 1e9, 1)
    del pool, calls
    # cfg3: M=4 gate_up on the GEMV family; M=8/16 on the MFMA GEMM (weight pool rotated)
    q3 = synth_nf4(16384, 3072, seed=30)
    P = pool_copies(q3.nbytes(), pool_gb * 1e9)
    pool = [q3] + [clone_nf4(q3) for _ in range(P - 1)]
    pool_ops = [operands(q) for q in pool]
    for m in (4, 8, 16):
        xm = torch.randn(m, 3072, generator=torch.Generator().manual_seed(30 + m)).half().to(dev)
        ym = torch.empty(m, 16384, dtype=torch.float16, device=dev)
        calls = [Launcher(lib, o, xm, ym) for o in pool_ops]
        nl = max(P, 60)
        t = time_graph(graph_of([calls[i % P] for i in range(nl)])) / nl
        out[f"cfg3_gate_up_m{m}_us"] = round(t * 1e6, 2)
        out[f"cfg3_gate_up_m{m}_GBps"] = round(gemv_bytes(q3, m) / t / 1e9, 1)
    del q3, pool, pool_ops
    # cfg3 down_proj: K=8192 -> N=3072 at M=4/8/16
    q3d = synth_nf4(3072, 8192, seed=31)
    P = pool_copies(q3d.nbytes(), pool_gb * 1e9)
    pool = [q3d] + [clone_nf4(q3d) for _ in range(P - 1)]
    pool_ops = [operands(q) for q in pool]
    for m in (4, 8, 16):
        xm = torch.randn(m, 8192, generator=torch.Generator().manual_seed(31 + m)).half().to(dev)
        ym = torch.empty(m, 3072, dtype=torch.float16, device=dev)
        calls = [Launcher(lib, o, xm, ym) for o in pool_ops]
        nl = max(P, 100)
        t = time_graph(graph_of([calls[i % P] for i in range(nl)])) / nl
        out[f"cfg3_down_m{m}_us"] = round(t * 1e6, 2)
        out[f"cfg3_down_m{m}_GBps"] = round(gemv_bytes(q3d, m) / t / 1e9, 1)
    del q3d, pool, pool_ops
    out.update(host_overhead(lib, dev))
    # cfg4: prefill GEMM M=2048, (K,N) = (4096,14336) and (14336,4096), bf16: the dispatching
    # entry (the library path from 1024 rows) and the hand-written MFMA GEMM, whole calls
    for (kk, nn) in ((4096, 14336), (14336, 4096)):
        q4, a = cfg4_operands(dev, kk, nn)
        for family, tag in (("dispatch", ""), ("handwritten", "_handwritten")):
            t = _time_eager(cfg4_gemm(lib, dev, q4, a, family), iters=10)
            out[f"cfg4_gemm_k{kk}_n{nn}{tag}_us"] = round(t * 1e6, 1)
            out[f"cfg4_gemm_k{kk}_n{nn}{tag}_TFLOPs"] = round(2 * 2048 * kk * nn / t / 1e12, 1)
            out[f"cfg4_gemm_k{kk}_n{nn}{tag}_mfma_frac"] = round(2 * 2048 * kk * nn / t / 1e12 / PEAK_FP16_TFLOPS,
                                                                 4)
        del q4, a
    # cfg5 linear chain: 28 x (QKV, o_proj, gate_up, down) + lm_head GEMVs, distinct weights
    shapes = [(5120, 3072), (3072, 3072), (16384, 3072), (3072, 8192)]
    layer = [synth_nf4(n, k, seed=50 + i) for i, (n, k) in enumerate(shapes)]
    head = synth_nf4_gpu(128256, 3072, seed=60)
    xs = {k: torch.randn(1, k, generator=torch.Generator().manual_seed(k)).half().to(dev) for k in (3072, 8192)}
    ys = {n: torch.empty(1, n, dtype=torch.float16, device=dev) for n in (5120, 3072, 16384, 128256)}
    chain, keep = [], []
    for li in range(28):
        for q in (layer if li == 0 else [clone_nf4(q) for q in layer]):
            keep.append(q)
            chain.append(Launcher(lib, operands(q), xs[q.k], ys[q.n]))
    chain.append(Launcher(lib, operands(head), xs[3072], ys[128256]))
    t = time_graph(graph_of(chain))
    chain_bytes = sum(gemv_bytes(q) for q in keep) + gemv_bytes(head)
    out["cfg5_linear_chain_ms"] = round(t * 1e3, 4)
    out["cfg5_linear_chain_GBps"] = round(chain_bytes / t / 1e9, 1)
    out["cfg5_decode_tok_s_linears_only"] = round(1.0 / t, 1)
    out["cfg5_note"] = "113 GEMVs of one decode token (28 layers + lm_head) in one graph; attention/norms excluded"
    del chain, keep, layer, head
    out.update(decode_e2e(dev))
    return out


def host_overhead(lib, dev, n: int = 3000) -> dict:
    """Host time to issue one eager M=1 down_proj call (cfg2 shape), measured as the issue
    rate of ``n`` back-to-back calls: the C-ABI entry point through ctypes, the functional
    API (fused_w4a16_gemv_hdsq, cached descriptor), the module (SpectraFusedLinear, one
    call of the registered operator) and the operator called directly.
    Whichever exceeds the kernel's own time bounds an eager caller."""
    from spectra_amd.engine import SpectraFusedLinear
    q = synth_nf4(3072, 8192, seed=32)
    x = torch.randn(1, 8192, generator=torch.Generator().manual_seed(32)).half().to(dev)
    y = torch.empty(1, 3072, dtype=torch.float16, device=dev)
    raw = Launcher(lib, operands(q), x, y)
    stream = torch.cuda.current_stream().cuda_stream
    col, val = q.outliers()
    lin = SpectraFusedLinear(8192, 3072, q.blocksize, codebook="nf4", hadamard_block=HAD).to(dev)
    lin.set_weights(q.packed, q.absmax, None, outlier_idx=col, outlier_weight=val, marlin_layout=True,
                    outlier_rowptr=q.rowptr)

    def issue(fn):
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        return (t1 - t0) / n * 1e6

    with torch.no_grad():
        out = {"eager_m1_issue_us_c_abi": round(issue(lambda: raw(stream)), 2),
               "eager_m1_issue_us_functional": round(issue(lambda: K.fused_w4a16_gemv_hdsq(
                   x, q.packed, q.absmax, None, outlier_idx=col, outlier_w=val, marlin_layout=True,
                   out=y, **q.kernel_kwargs())), 2),
               "eager_m1_issue_us_module": round(issue(lambda: lin(x)), 2)}
        args = lin._op_args  # bound by the module's first call
        out["eager_m1_issue_us_torch_op"] = round(issue(lambda: torch.ops.spectra_hip.w4a16_linear(x, *args)), 2)
    out["eager_note"] = ("host issue time per eager M=1 down_proj call (3000 back-to-back calls); the kernel itself "
                         "takes down_gemv_us, so above that an eager caller is host-bound and a HIP graph is the remedy")
    return out


# the library path's own hipBLASLt workspace (spectra_amd/csrc/prefill.hip)
PREFILL_LT_WORKSPACE = 32 << 20


def cfg4_gemm(lib, dev, q4: C.NF4Weight, a: torch.Tensor, family: str):
    """One cfg4 GEMM through the C ABI on preallocated buffers (bf16 activations and output).
    family "dispatch": the workspace spectra_w4a16_gemm_workspace() asks for, so M >= 1024 runs
    the library path; "handwritten": the same buffer declared PREFILL_LT_WORKSPACE + 1 bytes
    short, which the library path does not fit, so the entry runs the hand-written MFMA GEMM
    (it holds that GEMM's own buffers)."""
    ops = operands(q4)
    m, n = a.shape[0], q4.n
    out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    need = int(lib.spectra_w4a16_gemm_workspace(ctypes.byref(ops.desc), m, L.BF16))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    ws_bytes = need if family == "dispatch" else need - PREFILL_LT_WORKSPACE - 1
    args = (ctypes.byref(ops.desc), a.data_ptr(), a.stride(0), m, L.BF16, out.data_ptr(), out.stride(0),
            ws.data_ptr(), ws_bytes)

    def call():
        L.check("spectra_w4a16_gemm", lib.spectra_w4a16_gemm(*args, torch.cuda.current_stream().cuda_stream))
    call.keep = (ops, out, ws)
    return call


def cfg4_operands(dev, kk: int, nn: int):
    q4 = synth_nf4(nn, kk, seed=40 + kk)
    a = torch.randn(2048, kk, generator=torch.Generator().manual_seed(kk)).bfloat16().to(dev)
    return q4, a


def profile_gemm(lib, dev, family: str = "dispatch", iters: int = 3) -> dict:
    """cfg4's two prefill GEMMs (M=2048, bf16), ``iters`` launches each after a warm-up, on the
    dispatching entry's path or on the hand-written GEMM (see cfg4_gemm)."""
    out = {}
    for kk, nn in ((4096, 14336), (14336, 4096)):
        q4, a = cfg4_operands(dev, kk, nn)
        t = _time_eager(cfg4_gemm(lib, dev, q4, a, family), iters)
        out[f"cfg4_gemm_k{kk}_n{nn}{'' if family == 'dispatch' else '_handwritten'}_us"] = round(t * 1e6, 1)
        del q4, a
    return out


def profile_small_batch(lib, dev, pool_gb: float, m: int = 16, reps: int = 3) -> dict:
    """cfg3 at M rows (16 by default): down_proj (K=8192, N=3072) and gate_up (K=3072,
    N=16384) through the module dispatch over a rotated weight pool, each graph replayed
    ``reps`` times."""
    out = {}
    for name, nn, kk, seed in (("down", 3072, 8192, 31), ("gate_up", 16384, 3072, 30)):
        q = synth_nf4(nn, kk, seed=seed)
        P = pool_copies(q.nbytes(), pool_gb * 1e9)
        pool = [q] + [clone_nf4(q) for _ in range(P - 1)]
        xm = torch.randn(m, kk, generator=torch.Generator().manual_seed(seed + m)).half().to(dev)
        ym = torch.empty(m, nn, dtype=torch.float16, device=dev)
        calls = [Launcher(lib, operands(o), xm, ym) for o in pool]
        nl = max(P, 60)
        g = graph_of([calls[i % P] for i in range(nl)])
        ts = [time_graph(g) / nl for _ in range(reps)]
        out[f"cfg3_{name}_m{m}_us"] = round(min(ts) * 1e6, 2)
        del q, pool, calls, g
    return out


def decode_e2e(dev) -> dict:
    """cfg5 end to end through the engine: random 512-token prompt, prefill, then 255 greedy
    decode steps, one captured decode step replayed per token (all linears NF4 + FWHT-128 +
    0.5% CSR outliers, fp16 KV cache); then the same with the 4-bit KV cache
    (kv_bits=4, 128-position fp16 window)."""
    out = _decode_run(dev, 16)
    q4 = _decode_run(dev, 4)
    out["cfg5_kv4_decode_ms_per_token"] = q4["cfg5_decode_ms_per_token"]
    out["cfg5_kv4_decode_tok_s"] = q4["cfg5_decode_tok_s"]
    out["cfg5_kv4_note"] = "same run with the 4-bit KV cache: positions older than 128 read through the 4-bit codes"
    return out


def _decode_run(dev, kv_bits: int) -> dict:
    from spectra_amd.engine import DecoderConfig, SpectraDecoder
    out = {}
    dec = SpectraDecoder(DecoderConfig(max_seq=768, kv_bits=kv_bits))
    prompt = torch.randint(0, dec.cfg.vocab, (512,), generator=torch.Generator().manual_seed(5)).to(dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    dec.prefill(prompt)  # first call: library set-up
    for t in dec.cache_tensors():
        t.zero_()
    ev[0].record()
    dec.prefill(prompt)
    ev[1].record()
    dec.capture_decode()
    ev[2].record()
    dec.decode(255)  # tokens 2..256 (the prefill yields the first)
    ev[3].record()
    ev[3].synchronize()
    dms = ev[2].elapsed_time(ev[3])
    out["cfg5_prefill_512_ms"] = round(ev[0].elapsed_time(ev[1]), 2)
    out["cfg5_decode_ms_per_token"] = round(dms / 255, 4)
    out["cfg5_decode_tok_s"] = round(255 / dms * 1e3, 1)
    out["cfg5_e2e_note"] = ("28-layer Llama-3.2-3B-shaped decoder (random init) through spectra_amd.engine: 512-token "
                            "prompt, 256 greedy tokens, fp16 KV cache, decode step replayed as one HIP graph")
    del dec
    torch.cuda.empty_cache()
    return out


def _time_eager(fn, iters: int = 20) -> float:
    """Per-call GPU time of ``fn`` at steady state: one untimed call is queued before the
    start event, so the host's issue latency after the synchronisation is not timed."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / 1e3 / iters


if __name__ == "__main__":
    main()
