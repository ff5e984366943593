"""bench.py -- W8A8 encode throughput on one MI355X (BERT-base, batch 64 x seq 512).

A step is one encode of one batch, resident on the device from token ids to pooled
embeddings (aikit_amd.bert_dev.DeviceBert: encoder/bert.go:260-371 and the mean pooling
+ L2 of encoder/pooling.go:84-105 / embed/pool.go:22-38): the embedding rows and their
LayerNorm, then 12 BERT-base layers -- fused QKV (768->2304, bias), attention, attention
output (768->768, bias), residual LayerNorm, FFN up (768->3072, bias + exact GELU), FFN
down (3072->768, bias), residual LayerNorm -- with every linear a W8A8 linear
(per-token int8 quantization + int8 MFMA GEMM + fused dequant epilogue), then mean pooling
and L2 normalisation of the 64 sequences. Inputs are synthetic and already resident in
HBM when the timed region starts: token ids uniform over the vocabulary, random N(0,0.02)
f32 weights quantized per output channel, random embedding tables.

`value` is 64 x steps / the wall time of the steps (torch.cuda.synchronize() on both
sides). A second region of the same steps records HIP events between the operations;
the per-kernel table and `roofline` (the W8A8 path's dominant kernel) come from it.
`linear_stack` re-times the 48 W8A8 linears alone, as the previous headline did.

Prints ONE JSON line on stdout (progress goes to stderr).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "W8A8 encode seqs/sec (BERT-base b64×s512) + int8 GEMM TOPS as % of peak"
PEAK_INT8_OPS = 5.0e15  # MI355X dense int8 MFMA (no sparsity)
PEAK_HBM_BPS = 8.0e12  # MI355X HBM3E
PEAK_FP32_FLOPS = 157.3e12  # MI355X dense fp32 MFMA
PEAK_BF16_FLOPS = 2.5e15  # MI355X dense bf16 MFMA


TRAFFIC_PROFILE = "profiles/bert_base_b64s512_hbm_traffic.md"


def gemv_kernel_name(K: int, act: int) -> str:
    """gemv_w8a8's instantiation for a weight of K columns (padded to 64): its fragments
    per wave and batch, as the library picks them."""
    per_wave = -(-(-(-K // 64) * 64 // 32) // 8)
    return f"enchip::gemv_w8a8<{1 + act}, {max(per_wave, 1) if per_wave <= 4 else 8}>"


def quant_kernel_name(K: int, frag: bool) -> str:
    """Name of the quantize kernel enchip launches for rows of K floats (aligned
    buffers, pitch K padded to 64): quant_rows_frag<ceil(Kp/256), rows per wave> for fragment-major
    codes (the persistent GEMM's), quant_rows_vec<ceil(K/256)> for row-major, up to
    4096."""
    Kp = (K + 63) // 64 * 64
    if frag:
        ch = (Kp + 255) // 256
        return f"enchip::quant_rows_frag<{ch}, {2 if ch <= 2 else 1}>" if 0 < Kp <= 4096 and K % 4 == 0 else "enchip::quant_rows_scalar<true>"
    return f"enchip::quant_rows_vec<{(K + 255) // 256}>" if 0 < K <= 4096 and K % 4 == 0 else "enchip::quant_rows_scalar<false>"


def ln_cpl(D: int) -> int:
    """Floats per lane of the LayerNorm kernels enchip launches for rows of D (multiple
    of 4, 16-byte aligned) floats."""
    return 4 if D <= 256 else 8 if D <= 512 else 12 if D <= 768 else 16 if D <= 1024 else 32 if D <= 2048 else 64


def measured_traffic() -> dict:
    """HBM bytes per launch for each linear and its quantizer, as measured by the two
    rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) recorded in TRAFFIC_PROFILE. The
    numbers are calibrated per counter against a 1 GiB copy kernel; that file gives the
    commands and the calibration. Empty when the file is absent."""
    path = os.path.join(ROOT, TRAFFIC_PROFILE)
    out = {}
    try:
        lines = open(path).read().split("traffic_bytes_per_launch", 1)[1].split("```", 1)[0].split()
    except (OSError, IndexError):
        return out
    for k, v in zip(lines[0::2], lines[1::2]):
        out[k] = int(v)
    return out


class HipEvents:
    """Timing events recorded on a raw HIP stream (the one the enchip kernels are
    launched on), through libamdhip64, the runtime torch has already loaded.
    torch.cuda.Event records only on torch's current stream."""

    def __init__(self):
        import ctypes

        self.ct = ctypes
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecordWithFlags.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.events = []

    def create(self):
        ev = self.ct.c_void_p()
        rc = self.lib.hipEventCreate(self.ct.byref(ev))
        if rc != 0:
            raise RuntimeError(f"hipEventCreate: {rc}")
        self.events.append(ev)
        return ev

    def record(self, ev, stream_ptr: int):
        rc = self.lib.hipEventRecordWithFlags(ev, self.ct.c_void_p(stream_ptr), 0)
        if rc != 0:
            raise RuntimeError(f"hipEventRecordWithFlags: {rc}")

    def elapsed_ms(self, e0, e1) -> float:
        ms = self.ct.c_float()
        rc = self.lib.hipEventElapsedTime(self.ct.byref(ms), e0, e1)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime: {rc}")
        return ms.value

    def close(self):
        for ev in self.events:
            self.lib.hipEventDestroy(ev)
        self.events = []


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(layer_w, cfg, seconds: float):
    """The reference's CPU encode on a bounded sample: one sequence (512 tokens) through
    one whole BERT-base layer, repeated for about `seconds`, scaled to seqs/s of the
    12-layer encode. The four linears run the C restatement of aikit's AVX2 W8A8 path
    (oracle/cpu_baseline.c, the column fan-out over the host threads), the attention the
    oracle's f32 attention with its heads over the host threads (bit-identical to
    orc_attention), and the two residual LayerNorms the oracle's, as encoder/bert.go
    composes them. Embeddings and pooling (under 0.1% of the forward) are left out."""
    import numpy as np

    import oracle
    from aikit_amd import workloads

    workers = host_threads()
    g = workloads.rng(99)
    L, D, I, H = cfg.seq, cfg.hidden, cfg.ffn, cfg.heads
    h0 = g.standard_normal((L, D), dtype=np.float32)
    ln = [((1 + g.standard_normal(D) * 0.02).astype(np.float32), (g.standard_normal(D) * 0.02).astype(np.float32))
          for _ in range(2)]
    bufs = {name: np.empty(L * N, np.float32) for name, _, N, _ in cfg.linears()}
    aq = np.empty(L * I, np.int8)
    asc = np.empty(L, np.float32)

    def lin(name, x):
        wq, ws, b, act = layer_w[name]
        K, N = wq.shape[1], wq.shape[0]
        return oracle.cpu_w8a8_linear(x, wq, ws, b, act, L, K, N, workers, dst=bufs[name], aq=aq, ascales=asc)

    times = {"linears": 0.0, "attention": 0.0, "layernorm": 0.0}

    def one_layer():
        t0 = time.perf_counter()
        qkv = lin("qkv", h0)
        t1 = time.perf_counter()
        ctxv = oracle.cpu_attention(np.ascontiguousarray(qkv[:, :D]), np.ascontiguousarray(qkv[:, D:2 * D]),
                                    np.ascontiguousarray(qkv[:, 2 * D:]), L, D, H, workers)
        t2 = time.perf_counter()
        out = lin("o", ctxv)
        t3 = time.perf_counter()
        h = oracle.layer_norm((h0 + out).astype(np.float32), *ln[0], L, D, 1e-12)
        t4 = time.perf_counter()
        ffn = lin("ffn_down", lin("ffn_up", h))
        t5 = time.perf_counter()
        oracle.layer_norm((h + ffn).astype(np.float32), *ln[1], L, D, 1e-12)
        t6 = time.perf_counter()
        times["linears"] += (t1 - t0) + (t3 - t2) + (t5 - t4)
        times["attention"] += t2 - t1
        times["layernorm"] += (t4 - t3) + (t6 - t5)

    one_layer()  # warm-up
    for k in times:
        times[k] = 0.0
    rounds, t0 = 0, time.perf_counter()
    while True:
        one_layer()
        rounds += 1
        el = time.perf_counter() - t0
        if el >= seconds or rounds >= 10000:
            break
    per_layer = el / rounds
    macs = sum(L * K * N for _, K, N, _ in cfg.linears())
    return {
        "value": 1.0 / (per_layer * cfg.layers),
        "unit": "seqs/s",
        "cores": workers,
        "kind": "port",
        "sample": (f"1 sequence (512 tokens) through one whole BERT-base layer (4 W8A8 linears, f32 attention, "
                   f"2 residual LayerNorms), {rounds} repetitions in {el:.1f} s, scaled x{cfg.layers} layers; "
                   f"linears: C restatement of aikit's Go AVX2 W8A8 path (oracle/cpu_baseline.c); attention: the "
                   f"oracle's f32 attention, heads over the threads; {workers} threads on {cpu_model()}"),
        "ms_per_layer": {k: v / rounds * 1e3 for k, v in times.items()},
        "linears_gmac_per_s": macs / (times["linears"] / rounds) / 1e9,
    }


def other_configs(ctx, torch, stream, ceilings):
    """Configs 2 and 3 (isolated linear, small-M GEMV), and ann.FlatI8 scoring, timed with HIP events on the
    launch stream.

    * config 2: the isolated W8A8 linear (M=4096, K=768 -> N=3072, bias + GELU), as
      quantize + GEMM per call. Judged on int8 TOPS.
    * config 3: the small-M GEMV (M=16, K=768 -> N=768 and N=3072). Each call reads a
      different registered copy of the weights, and the copies total > 2x the 256 MB
      MALL, so every call streams its weights from HBM. Judged on HBM GB/s over the
      algorithmic bytes N*K + M*K + 4M + 8N + 4MN.
    * ann.FlatI8 scoring: M in {1, 16, 256} queries against a 2^20 x 384 int8 index
      (403 MB, larger than the MALL), bias-free W8A8 scores. Judged on HBM GB/s over
      N*K + M*K + 4M + 4N + 4MN.
    """
    import numpy as np

    from aikit_amd import enchip, workloads

    import oracle

    out = {}
    sp = stream.cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def graph_us(fn, calls: int, replays: int = 3):
        """Device time per call of `calls` calls of fn captured as one HIP graph and replayed
        `replays` times (no host launch path between the calls); None if capture fails."""
        try:
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                for _ in range(calls):
                    fn()
            with torch.cuda.stream(stream):
                gr.replay()
                e0.record(stream)
                for _ in range(replays):
                    gr.replay()
                e1.record(stream)
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) * 1e-3 / (replays * calls)
            del gr
            return t * 1e6
        except Exception as exc:  # capture unsupported: the caller reports eager timing only
            log(f"graph capture failed ({exc})")
            torch.cuda.synchronize()
            return None

    def cpu_us(a, wq, ws, b, act, M, K, N, reps):
        oracle.cpu_w8a8_linear(a, wq, ws, b, act, M, K, N, host_threads())
        t0 = time.perf_counter()
        for _ in range(reps):
            oracle.cpu_w8a8_linear(a, wq, ws, b, act, M, K, N, host_threads())
        return (time.perf_counter() - t0) / reps * 1e6

    # the launch floor: an empty kernel (torch's spin kernel for 0 cycles) per call
    floor_us = graph_us(lambda: torch.cuda._sleep(0), 256, 3)

    c2 = workloads.LINEAR_CFG2
    M, K, N = c2["M"], c2["K"], c2["N"]
    g = workloads.rng(2)
    wq, ws = workloads.int8_weights(g, N, K)
    h = ctx.register_weight(wq, ws)
    ah = workloads.activations(g, M, K)
    bh = workloads.bias(g, N)
    with torch.cuda.stream(stream):
        a = torch.from_numpy(ah).cuda()
        b = torch.from_numpy(bh).cuda()
        dst = torch.empty((M, N), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    call = lambda: ctx.linear_dev(h, a.data_ptr(), M, b.data_ptr(), c2["act"], dst.data_ptr(), sp)
    for _ in range(5):
        call()
    reps = 50
    e0.record(stream)
    for _ in range(reps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    t_eager = e0.elapsed_time(e1) * 1e-3 / reps
    tg = graph_us(call, reps)
    t = tg * 1e-6 if tg is not None else t_eager
    ops = 2.0 * M * N * K
    # where a call's time goes: the same call without the GELU, and its two kernels alone
    # (the GEMM on the call's own fragment-major codes, with and without the GELU)
    _, ldq = ctx.frag_route(h, M)
    with torch.cuda.stream(stream):
        aq = torch.empty((M * ldq,), device="cuda", dtype=torch.int8)
        asc = torch.empty(M, device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    quant = lambda: ctx.quant_rows_frag_dev(a.data_ptr(), M, K, aq.data_ptr(), ldq, asc.data_ptr(), sp)
    quant()
    split = {
        "call_bias_only_us": graph_us(lambda: ctx.linear_dev(h, a.data_ptr(), M, b.data_ptr(), 0, dst.data_ptr(), sp),
                                      reps),
        "quantizer_us": graph_us(quant, reps),
        "gemm_gelu_us": graph_us(lambda: ctx.pre_frag_dev(h, aq.data_ptr(), ldq, M, asc.data_ptr(), b.data_ptr(),
                                                          c2["act"], dst.data_ptr(), sp), reps),
        "gemm_bias_only_us": graph_us(lambda: ctx.pre_frag_dev(h, aq.data_ptr(), ldq, M, asc.data_ptr(), b.data_ptr(),
                                                               0, dst.data_ptr(), sp), reps),
        "note": "HIP graph replay of 50 calls each; the GEMM legs run on the quantizer's codes of the same "
                "activations (enchip_w8a8_pre_frag_dev)"}
    out["config2_isolated_linear"] = {
        "split": split,
        "M": M, "K": K, "N": N, "act": "gelu", "us_per_call": t * 1e6, "int8_tops": ops / t / 1e12,
        "frac_int8_peak": ops / t / PEAK_INT8_OPS, "us_per_call_eager": t_eager * 1e6,
        "timing": "HIP graph replay" if tg is not None else "eager",
        "kernel": ctx.gemm_kernel_name(h, M, c2["act"]), "quant_kernel": quant_kernel_name(K, True),
        "cpu_port_us_per_call": cpu_us(ah, wq, ws, bh, c2["act"], M, K, N, 3), "cpu_port_threads": host_threads(),
        "note": "quantize + GEMM + fused epilogue per call (enchip_w8a8_linear_dev), activations resident in HBM; "
                "us_per_call from one captured graph of 50 calls (device time), us_per_call_eager from back-to-back "
                "eager calls; cpu_port = the C restatement of aikit's AVX2 W8A8 path on the host's threads"}
    ctx.release_weight(h)

    for c3 in workloads.GEMV_CFG3:
        M, K, N = c3["M"], c3["K"], c3["N"]
        g = workloads.rng(3)
        wq, ws = workloads.int8_weights(g, N, K)
        copies = max(2, int(np.ceil(600e6 / (N * K))))  # > 2 x 256 MB MALL of distinct weights
        hs = [ctx.register_weight(wq, ws) for _ in range(copies)]
        ah = workloads.activations(g, M, K)
        bh = workloads.bias(g, N)
        with torch.cuda.stream(stream):
            a = torch.from_numpy(ah).cuda()
            b = torch.from_numpy(bh).cuda()
            aq = torch.empty((M, K), device="cuda", dtype=torch.int8)
            asc = torch.empty(M, device="cuda", dtype=torch.float32)
            dst = torch.empty((M, N), device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        ctx.quant_rows_dev(a.data_ptr(), M, K, aq.data_ptr(), asc.data_ptr(), sp, ldq=K)
        it = iter(())

        def next_weight():
            nonlocal it
            try:
                return next(it)
            except StopIteration:
                it = iter(hs)
                return next(it)

        gemv = lambda: ctx.pre_dev(next_weight(), aq.data_ptr(), K, M, asc.data_ptr(), b.data_ptr(), c3["act"],
                                   dst.data_ptr(), sp)
        linear = lambda: ctx.linear_dev(next_weight(), a.data_ptr(), M, b.data_ptr(), c3["act"], dst.data_ptr(), sp)
        for _ in range(8):
            linear()
        e0.record(stream)
        for _ in range(len(hs)):
            linear()
        e1.record(stream)
        torch.cuda.synchronize()
        t_eager = e0.elapsed_time(e1) * 1e-3 / len(hs)
        t_lin = graph_us(linear, len(hs))
        t_gemv = graph_us(gemv, len(hs))
        nbytes = N * K + M * K + 4 * M + 8 * N + 4 * M * N
        qbytes = 5 * M * K + 4 * M
        tb = (t_lin * 1e-6) if t_lin is not None else t_eager
        out[f"config3_gemv_n{N}"] = {
            "M": M, "K": K, "N": N, "us_per_call": tb * 1e6,
            "hbm_gbps": (nbytes + qbytes) / tb / 1e9, "frac_hbm_peak": (nbytes + qbytes) / tb / PEAK_HBM_BPS,
            "frac_measured_read_ceiling": (nbytes + qbytes) / tb / 1e9 / ceilings["hbm_read_gbps"],
            "gemv_only_us_per_call": t_gemv, "gemv_only_kernel": gemv_kernel_name(K, c3["act"]),
            "launch_floor_us": floor_us,
            "us_per_call_eager": t_eager * 1e6, "timing": "HIP graph replay" if t_lin is not None else "eager",
            "weight_copies": len(hs), "weight_set_mb": len(hs) * N * K / 1e6,
            "kernel": ctx.gemm_kernel_name(hs[0], M, c3["act"]),
            "cpu_port_us_per_call": cpu_us(ah, wq, ws, bh, c3["act"], M, K, N, 20), "cpu_port_threads": host_threads(),
            "note": "one single-query W8A8 linear per call (enchip_w8a8_linear_dev: per-token quantization + small-M "
                    "GEMM), each call on a distinct registered weight copy (the copies exceed 2 x the 256 MB MALL, "
                    "so each call streams its weights from HBM; at M <= 32 the quantization runs inside the GEMV "
                    "kernel, one launch per call); bytes = weights + activations + scales + bias + "
                    "f32 output + the quantizer's; us_per_call from one captured graph of all calls (device time); "
                    "gemv_only = the GEMM on pre-quantized codes (enchip_w8a8_pre_dev); launch_floor = an empty "
                    "kernel per call in the same kind of graph"}
        for hh in hs:
            ctx.release_weight(hh)

    # ann.FlatI8 scoring: an int8 index of N rows x dim registered as a
    # weight (ann.Backend.NewI8Index), M queries scored as a bias-free W8A8 linear
    # (I8Index.Score / I8BatchIndex.ScoreBatch). The 403 MB index exceeds the 256 MB
    # MALL, so every call streams it from HBM.
    N, K = 1 << 20, 384
    g = workloads.rng(5)
    codes = g.integers(-127, 128, size=(N, K), dtype=np.int8)
    rscale = g.uniform(1e-3, 1e-2, size=N).astype(np.float32)
    hidx = ctx.register_weight(codes, rscale)
    for M in (1, 16, 256):
        with torch.cuda.stream(stream):
            a = torch.from_numpy(workloads.activations(g, M, K)).cuda()
            aq = torch.empty((M, K), device="cuda", dtype=torch.int8)
            asc = torch.empty(M, device="cuda", dtype=torch.float32)
            dst = torch.empty((M, N), device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        ctx.quant_rows_dev(a.data_ptr(), M, K, aq.data_ptr(), asc.data_ptr(), sp, ldq=K)
        for _ in range(3):
            ctx.pre_dev(hidx, aq.data_ptr(), K, M, asc.data_ptr(), 0, 0, dst.data_ptr(), sp)
        reps = 20
        e0.record(stream)
        for _ in range(reps):
            ctx.pre_dev(hidx, aq.data_ptr(), K, M, asc.data_ptr(), 0, 0, dst.data_ptr(), sp)
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        # I8TopKIndex.TopKBatch on the device: the same scores, then the k = 10 best per query
        kk = 10
        with torch.cuda.stream(stream):
            hi = torch.empty((M, kk), dtype=torch.int32, device="cuda")
            hs = torch.empty((M, kk), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        for _ in range(3):
            ctx.topk_rows_dev(dst.data_ptr(), N, M, N, kk, hi.data_ptr(), kk, hs.data_ptr(), kk, sp)
        e0.record(stream)
        for _ in range(reps):
            ctx.pre_dev(hidx, aq.data_ptr(), K, M, asc.data_ptr(), 0, 0, dst.data_ptr(), sp)
            ctx.topk_rows_dev(dst.data_ptr(), N, M, N, kk, hi.data_ptr(), kk, hs.data_ptr(), kk, sp)
        e1.record(stream)
        torch.cuda.synchronize()
        t_topk = e0.elapsed_time(e1) * 1e-3 / reps
        # the selection alone at larger k on the same device scores (256 queries): k = 64, the
        # top of the reference's device range, and k = 100, a retrieve-then-rerank depth
        t_sel = {}
        if M == 256:
            for kb in (10, 64, 100):
                with torch.cuda.stream(stream):
                    hib = torch.empty((M, kb), dtype=torch.int32, device="cuda")
                    hsb = torch.empty((M, kb), dtype=torch.float32, device="cuda")
                torch.cuda.synchronize()
                for _ in range(3):
                    ctx.topk_rows_dev(dst.data_ptr(), N, M, N, kb, hib.data_ptr(), kb, hsb.data_ptr(), kb, sp)
                e0.record(stream)
                for _ in range(reps):
                    ctx.topk_rows_dev(dst.data_ptr(), N, M, N, kb, hib.data_ptr(), kb, hsb.data_ptr(), kb, sp)
                e1.record(stream)
                torch.cuda.synchronize()
                t_sel[kb] = e0.elapsed_time(e1) * 1e3 / reps
                del hib, hsb
        # TopKBatch through its host entry point (enchip_ann_topk: host queries in, host hits
        # out, synchronous). Above the small-M limit with k <= 32 the selection runs in the
        # scoring pass and the M x N scores are never written (the fused route).
        qh = a.cpu().numpy()
        for _ in range(3):
            ctx.ann_topk(hidx, qh, kk)
        f0, b0 = ctx.ann_topk_stats()
        th = []
        for _ in range(reps):
            t0 = time.perf_counter()
            ctx.ann_topk(hidx, qh, kk)
            th.append(time.perf_counter() - t0)
        f1, b1 = ctx.ann_topk_stats()
        route = "two-pass" if f1 == f0 else ("fused" if b1 == b0 else "fused, fell back to two-pass")
        # the same at k = 64, the top of the reference's device range (gpu/anncuda/gemv_w8a8.cu:606-619)
        t64 = None
        if M > 1:
            for _ in range(3):
                ctx.ann_topk(hidx, qh, 64)
            t64 = []
            for _ in range(reps):
                t0 = time.perf_counter()
                ctx.ann_topk(hidx, qh, 64)
                t64.append(time.perf_counter() - t0)
        nbytes = N * K + M * K + 4 * M + 4 * N + 4 * M * N
        kname = ctx.gemm_kernel_name(hidx, M, 0)
        if "skinny" in kname:  # pre_dev's codes are row-major
            kname = kname.replace(", true>", ", false>")
        out[f"ann_flat_i8_m{M}"] = {
            "top10_us_per_call": t_topk * 1e6,
            "ann_topk_host_us_per_call": float(np.median(th)) * 1e6, "ann_topk_route": route,
            "ann_topk64_host_us_per_call": float(np.median(t64)) * 1e6 if t64 else None,
            "topk_rows_us_per_call": {str(kb): v for kb, v in t_sel.items()} or None,
            "M": M, "K": K, "N": N, "us_per_call": t * 1e6, "hbm_gbps": nbytes / t / 1e9,
            "frac_hbm_peak": nbytes / t / PEAK_HBM_BPS,
            "frac_measured_read_ceiling": nbytes / t / 1e9 / ceilings["hbm_read_gbps"],
            "int8_tops": 2.0 * M * N * K / t / 1e12, "kernel": kname,
            "note": "M queries against a 2^20 x 384 int8 index (403 MB > MALL), pre-quantized queries, "
                    "bias-free W8A8 scores (enchip_w8a8_pre_dev); bytes = index + queries + scales + M*N f32 scores; "
                    "top10_us_per_call = the same scores plus the device top-10 per query (enchip_topk_rows_dev); "
                    "ann_topk_host_us_per_call = enchip_ann_topk (host queries -> host top-10 hits, wall clock, "
                    "median), on the route ann_topk_route names; ann_topk64_host_us_per_call = the same at k = 64; "
                    "topk_rows_us_per_call = enchip_topk_rows_dev alone on the device scores, by k"}
        if M <= 16:
            # the reference's CPU path for the same scores: the C restatement of its AVX2
            # W8A8 linear (oracle/cpu_baseline.c), bias-free, on the host's cores
            import oracle

            qh = a.cpu().numpy()
            oracle.cpu_w8a8_linear(qh, codes, rscale, None, 0, M, K, N, host_threads())
            t0 = time.perf_counter()
            for _ in range(3):
                oracle.cpu_w8a8_linear(qh, codes, rscale, None, 0, M, K, N, host_threads())
            out[f"ann_flat_i8_m{M}"]["cpu_port_us_per_call"] = (time.perf_counter() - t0) / 3 * 1e6
            out[f"ann_flat_i8_m{M}"]["cpu_port_threads"] = host_threads()
        del a, aq, asc, dst, hi, hs
    del codes
    ctx.release_weight(hidx)

    # f32 attention products of one config-4 layer (encoder/attention.go:108,111) on the
    # device MatmulBT: QK^T and scores . V for all 64 sequences x 12 heads, each one
    # launch with the heads read in place from the fused [tokens, 3D] QKV rows.
    from aikit_amd.enchip import B_KN, B_NK

    S, L, H, hd = 64, 512, 12, 64
    D = H * hd
    with torch.cuda.stream(stream):
        qkv = torch.randn((S * L, 3 * D), device="cuda", generator=torch.Generator(device="cuda").manual_seed(9))
        scores = torch.empty((S, H, L, L), device="cuda")
        ctxv = torch.empty((S * L, D), device="cuda")
    torch.cuda.synchronize()
    base = qkv.data_ptr()

    def qk():
        ctx.matmul_bt_f32_dev(base, 3 * D, base + D * 4, 3 * D, B_NK, scores.data_ptr(), L, L, hd, L,
                              inner=(H, hd, hd, L * L), outer=(S, L * 3 * D, L * 3 * D, H * L * L), stream=sp)

    def pv():
        ctx.matmul_bt_f32_dev(scores.data_ptr(), L, base + 2 * D * 4, 3 * D, B_KN, ctxv.data_ptr(), D, L, L, hd,
                              inner=(H, L * L, hd, hd), outer=(S, H * L * L, L * 3 * D, L * D), stream=sp)

    flops = 2.0 * S * H * L * L * hd
    att = {}
    for name, fn, nbytes in (("qk", qk, 2 * S * L * D * 4 + S * H * L * L * 4),
                             ("pv", pv, S * H * L * L * 4 + 2 * S * L * D * 4)):
        for _ in range(3):
            fn()
        reps = 10
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        att[f"{name}_us"] = t * 1e6
        att[f"{name}_tflops"] = flops / t / 1e12
        att[f"{name}_frac_fp32_mfma_peak"] = flops / t / PEAK_FP32_FLOPS
        att[f"{name}_hbm_gbps"] = nbytes / t / 1e9
    # the fused form: both products and the softmax in one launch, scores kept on chip, with
    # its products on the f32 MFMA, on the bf16 MFMA over bfloat16-split operands, and (the
    # default) on the f16 MFMA over half-split operands
    for mode, tag in ((enchip.ATT_F32, "fused_f32"), (enchip.ATT_SPLIT_BF16, "fused_split_bf16"),
                      (enchip.ATT_FLASH_BF16, "fused_flash_bf16"), (enchip.ATT_FLASH_F16, "fused_flash_f16")):
        ctx.set_attention_products(mode)
        for _ in range(3):
            ctx.attention_f32_dev(base, base + D * 4, base + 2 * D * 4, 3 * D, ctxv.data_ptr(), D, S, L, H, hd, 0.125,
                                  sp)
        e0.record(stream)
        for _ in range(10):
            ctx.attention_f32_dev(base, base + D * 4, base + 2 * D * 4, 3 * D, ctxv.data_ptr(), D, S, L, H, hd, 0.125,
                                  sp)
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / 10
        att[f"{tag}_us"] = t * 1e6
        att[f"{tag}_tflops_f32_equivalent"] = 2 * flops / t / 1e12
        if mode == enchip.ATT_F32:
            att[f"{tag}_frac_fp32_mfma_peak"] = 2 * flops / t / PEAK_FP32_FLOPS
        else:  # three 16-bit products per f32 product (the bf16 and f16 dense peaks are equal)
            att[f"{tag}_frac_bf16_mfma_peak"] = 3 * 2 * flops / t / PEAK_BF16_FLOPS
    ctx.set_attention_products(enchip.ATT_DEFAULT)
    att.update({"S": S, "L": L, "heads": H, "head_dim": hd, "gflop_per_product": flops / 1e9,
                "kernels": "enchip::gemm_f32_bt_lds<2, 2, false> (QK^T), enchip::gemm_f32_bt_lds<4, 1, true> (PV), "
                           "enchip::attention_f32<64> (fused, f32 MFMA), enchip::attention_split_bf16<64, true> "
                           "(fused, split-bf16 MFMA), enchip::attention_flash<64, 8, true, false|true> (fused online softmax, "
                           "bfloat16 / half split products; the half split is the default)",
                "note": "one config-4 layer's attention products (qk, pv: f32 MatmulBT on v_mfma_f32_32x32x2_f32), all "
                        "768 (sequence, head) problems per launch, operands resident; bytes = operands read once + "
                        "output written once; softmax not included in qk/pv, included in the fused forms"})
    out["attention_f32_cfg4_layer"] = att
    del qkv, scores, ctxv

    # encoder.Q8Backend.MatmulBTQ8, the weight-only int8 seam (f32 activations never
    # quantized): a BERT-base layer's four linears at one 512-token sequence (the Go
    # forward's per-sequence calls) on device buffers and through the host entry point
    # (upload a, download dst), and at the config-4 batch of 32768 rows on the device;
    # the f32 MatmulBT on the widened weight (how enccuda serves this seam) beside it.
    g = np.random.default_rng(21)
    q8 = {}
    shapes = (("qkv", 768, 2304), ("o", 768, 768), ("ffn_up", 768, 3072), ("ffn_down", 3072, 768))
    for M in (512, 32768):
        tot_us = tot_host_us = tot_flop = 0.0
        for name, K, N in shapes:
            wq = g.integers(-127, 128, size=(N, K)).astype(np.int8)
            ws = (0.002 + (np.arange(N) % 13) * 1e-4).astype(np.float32)
            w = ctx.register_weight(wq, ws)
            with torch.cuda.stream(stream):
                da = torch.randn((M, K), device="cuda", generator=torch.Generator(device="cuda").manual_seed(M + K))
                dd = torch.empty((M, N), device="cuda")
            torch.cuda.synchronize()
            for _ in range(3):
                ctx.matmul_bt_q8_dev(w, da.data_ptr(), K, M, dd.data_ptr(), N, sp)
            reps = 10
            e0.record(stream)
            for _ in range(reps):
                ctx.matmul_bt_q8_dev(w, da.data_ptr(), K, M, dd.data_ptr(), N, sp)
            e1.record(stream)
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) * 1e-3 / reps
            q8[f"m{M}_{name}_us"] = t * 1e6
            tot_us += t * 1e6
            tot_flop += 2.0 * M * N * K
            if M == 512:
                ah = da.cpu().numpy()
                for _ in range(2):
                    ctx.matmul_bt_q8(w, ah)
                t0 = time.perf_counter()
                for _ in range(reps):
                    ctx.matmul_bt_q8(w, ah)
                th = (time.perf_counter() - t0) / reps
                q8[f"m{M}_{name}_host_us"] = th * 1e6
                tot_host_us += th * 1e6
            if M == 32768 and name == "ffn_up":
                wf = torch.from_numpy(wq.astype(np.float32) * ws[:, None]).cuda()  # float32(q) * scale
                for _ in range(2):
                    ctx.matmul_bt_f32_dev(da.data_ptr(), K, wf.data_ptr(), K, B_NK, dd.data_ptr(), N, M, K, N, stream=sp)
                e0.record(stream)
                for _ in range(3):
                    ctx.matmul_bt_f32_dev(da.data_ptr(), K, wf.data_ptr(), K, B_NK, dd.data_ptr(), N, M, K, N, stream=sp)
                e1.record(stream)
                torch.cuda.synchronize()
                q8["m32768_ffn_up_f32_matmul_bt_us"] = e0.elapsed_time(e1) * 1e3 / 3
                del wf
            ctx.release_weight(w)
            del da, dd
        q8[f"m{M}_layer_us"] = tot_us
        q8[f"m{M}_tflops"] = tot_flop / (tot_us * 1e-6) / 1e12
        q8[f"m{M}_frac_bf16_mfma_peak"] = 3 * tot_flop / (tot_us * 1e-6) / PEAK_BF16_FLOPS
        if tot_host_us:
            q8[f"m{M}_layer_host_us"] = tot_host_us
    q8.update({"kernels": "enchip::gemm_q8w<TM, TN, VEC> (LDS-staged split, 64 x 64 to 128 x 256 tiles), "
                          "enchip::gemm_q8w_small<TN, VEC> (K split over the workgroup's wavefronts)",
               "note": "TFLOP/s = 2MNK / time; each f32 activation is split exactly into three bf16 parts, so the "
                       "bf16 MFMA fraction counts 3 x 2MNK; host_us includes the upload of a and download of dst"})
    out["matmul_bt_q8_weight_only"] = q8
    return out


def weight_registration(ctx, layers_host):
    """Registering the 48 BERT-base weights from int8 codes (host swizzle + upload) against
    from pre-swizzled images (upload only; aikit_amd.weight_cache), wall time."""
    from aikit_amd import weight_cache

    ws = [(wq, s) for lw in layers_host for (wq, s, _, _) in lw.values()]
    images = [(weight_cache.frag_image(wq), s, wq.shape) for wq, s in ws]
    t0 = time.perf_counter()
    hs = [ctx.register_weight(wq, s) for wq, s in ws]
    t_codes = time.perf_counter() - t0
    for h in hs:
        ctx.release_weight(h)
    t0 = time.perf_counter()
    hs = [ctx.register_weight_image(img, s, N, K) for img, s, (N, K) in images]
    t_images = time.perf_counter() - t0
    for h in hs:
        ctx.release_weight(h)
    return {"weights": len(ws), "bytes": int(sum(img.size for img, _, _ in images)), "from_codes_s": t_codes,
            "from_images_s": t_images,
            "note": "enchip_weight_register (host swizzle + upload) vs enchip_weight_register_image (upload of a "
                    "pre-swizzled image, as loaded from a mapped weight_cache file)"}


def build_encoder(ctx, torch, stream, layers_host, cfg, head: str = "pool", seed: int = 77):
    """A whole encoder resident on the device (aikit_amd.bert_dev.DeviceBert) over one batch
    of cfg.batch x cfg.seq tokens, and a step() that runs one encode from token ids (already
    on the device, uniform over the vocabulary): the embedding rows and their LayerNorm
    (bert.go:299-323; XLM-R's position offset 2), every layer, then the head: "pool" = mean
    pooling + L2 (config 4, BERT-base embeddings), "rerank" = the cross-encoder head
    classifier(tanh(pooler(CLS))) with one label (config 5, encoder/crossencoder.go:219-238).
    Tables, LayerNorm parameters and weights are random-init. Returns (model, step, out)."""
    import numpy as np

    from aikit_amd import workloads
    from aikit_amd.bert_dev import DeviceBert

    g = workloads.rng(seed)
    D = cfg.hidden
    full = []
    for lw in layers_host:
        e = dict(lw)
        for name in ("attn_ln", "out_ln"):
            e[name] = ((1 + g.standard_normal(D) * 0.02).astype(np.float32),
                       (g.standard_normal(D) * 0.02).astype(np.float32))
        full.append(e)
    model = DeviceBert(ctx, full, D, cfg.heads, cfg.ffn)
    S, L = cfg.batch, cfg.seq
    sp = stream.cuda_stream
    with torch.cuda.stream(stream):
        gen = torch.Generator(device="cuda").manual_seed(5)
        rnd = lambda *shape: torch.randn(shape, device="cuda", generator=gen) * 0.02
        pos_off = 2 if head == "rerank" else 0  # XLM-R: pad_token_id + 1
        model.set_embeddings(rnd(cfg.vocab, D), rnd(512 + pos_off, D),
                             (1 + rnd(D), rnd(D)), typ=None if head == "rerank" else rnd(2, D), pos_off=pos_off)
        ids = torch.randint(0, cfg.vocab, (S * L,), device="cuda", dtype=torch.int32, generator=gen)
        h = torch.empty((S * L, D), device="cuda")
        if head == "rerank":
            dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
            pooler = (dev(g.standard_normal((D, D)) * 0.02), dev(g.standard_normal(D) * 0.02))
            classifier = (dev(g.standard_normal((1, D)) * 0.02), dev(g.standard_normal(1) * 0.02))
            out = torch.empty((S, 1), device="cuda")
        else:
            out = torch.empty((S, D), device="cuda")
    torch.cuda.synchronize()

    def step():
        model.embeddings(ids, S, L, h, stream=sp)
        if head == "rerank":
            model.rerank(h, S, L, pooler, classifier, out, sp)
        else:
            model.embed(h, S, L, out, sp)

    return model, step, out


def time_steps(torch, stream, step, steps: int, warmup: int) -> float:
    """Seconds for `steps` steps after `warmup` untimed ones, synchronised on both sides."""
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for _ in range(steps):
            step()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def time_ops(torch, stream, model, step, steps: int, hev, warmup: int = 1):
    """Per-operation device durations (ms lists by label) over `steps` steps, after `warmup`
    untimed steps with the same marks, and how they were timed: a HIP event recorded on the
    launch stream at each of the model's marks.

    An eager event pair also counts any time the GPU sits idle between the two records, as
    when a host stall lets the queue drain. So every event is created before the timed
    steps (the loop only records), and the stream starts with a ~20 ms device-side sleep:
    the host queues the steps far ahead of the GPU before the first timed kernel runs."""
    sp = stream.cuda_stream
    warm = []
    model.mark = lambda label: warm.append(hev.record(hev.create(), sp))
    with torch.cuda.stream(stream):
        for _ in range(max(1, warmup)):
            step()
    torch.cuda.synchronize()
    per_step = len(warm) // max(1, warmup)
    pool = iter([hev.create() for _ in range(per_step * steps + 1)])
    marks = []

    def mark(label):
        ev = next(pool)
        hev.record(ev, sp)
        marks.append((label, ev))

    model.mark = mark
    try:
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            torch.cuda._sleep(40_000_000)  # ~20 ms of shader clock: the host's head start
            for _ in range(steps):
                step()
        torch.cuda.synchronize()
    finally:
        model.mark = None
    per = {}
    for (lab, e0), (_, e1) in zip(marks, marks[1:]):
        if lab != "end":
            per.setdefault(lab, []).append(hev.elapsed_ms(e0, e1))
    return per, "eager launches, a HIP event recorded at each mark (events created beforehand, the host queued ahead)"


def fa_waves(ctx, S: int, L: int, H: int) -> int:
    """Wavefronts per workgroup of the library's flash attention launch (its dispatch rule)."""
    return 16 if L > 256 and (L != 512 if L <= 512 else -(-L // 512) * H * S >= ctx.device_info()["num_cus"]) else 8


def encode_units(ctx, model, cfg, per: dict, steps: int) -> dict:
    """Per-kernel table of one encode step: launches per step, mean device time per launch,
    algorithmic work per launch (2MNK ops and M*K + N*K + 4M + 8N +
    4MN bytes for a W8A8 GEMM; 5 B per element + 4 B per row for a quantizer; the fused
    residual LayerNorm + quantizer reads h and y and writes h and the codes, 13 B per
    element + 4 B per row; attention 4 L^2 hd flops per head and its Q, K, V, context
    bytes), and the kernel's name as rocprofv3 shows it."""
    M, D, I, H, L, S = cfg.tokens, cfg.hidden, cfg.ffn, cfg.heads, cfg.seq, cfg.batch
    hd = D // H
    lin = {name: (K, N, act) for name, K, N, act in cfg.linears()}
    wh = model.handles[0]
    table = {}
    for label, ms in per.items():
        n = len(ms)
        t = sum(ms) / n * 1e-3  # average launch
        u = {"launches_per_step": n / steps, "us_per_launch": t * 1e6, "us_per_launch_median": sorted(ms)[n // 2] * 1e3,
             "us_per_launch_min": min(ms) * 1e3, "us_per_launch_max": max(ms) * 1e3, "ops": 0.0, "bytes": 0.0}
        base = label.split(".")[0]
        if label.endswith(".gemm"):
            K, N, act = lin[base]
            if base == "ffn_up" and "ffn_down.gelu_quant" in per:
                act = 0  # the GELU runs in FFN-down's quantization
            u.update(kind="w8a8", ops=2.0 * M * N * K, bytes=float(M * K + N * K + 4 * M + 8 * N + 4 * M * N),
                     kernel=ctx.gemm_kernel_name(wh[base][0], M, act))
        elif label.endswith(".gelu_quant"):
            K = lin[base][0]
            u.update(kind="w8a8", bytes=float(5 * M * K + 4 * M),
                     kernel=f"enchip::quant_rows_frag_gelu<{((K + 63) // 64 * 64 + 255) // 256}>")
        elif label.endswith(".quant"):
            K = lin[base][0]
            u.update(kind="w8a8", bytes=float(5 * M * K + 4 * M), kernel=quant_kernel_name(K, True))
        elif label.endswith("+quant"):
            u.update(kind="w8a8", bytes=float(13 * M * D + 4 * M + 8 * D),
                     kernel=f"enchip::residual_layer_norm_quant<{ln_cpl(D)}>")
        elif label == "attention":
            mode = ctx.attention_products
            u.update(kind="attention", ops=4.0 * S * H * L * L * hd, bytes=float(4 * M * D * 4),
                     # the library's flash launch (fa_waves)
                     kernel=(f"enchip::attention_flash<{hd}, {fa_waves(ctx, S, L, H)}, true, {'true' if mode == 3 else 'false'}>"
                             if mode in (2, 3) else
                             f"enchip::attention_split_bf16<{hd}, {'true' if L == 512 else 'false'}>" if mode == 1
                             else f"enchip::attention_f32<{hd}>"))
        elif label == "embed_rows":
            u.update(kind="row", bytes=float(12 * M * D), kernel="enchip::embed_rows<true>")
        elif label in ("embed_ln", "attn_ln", "out_ln"):
            u.update(kind="row", bytes=float((8 if label == "embed_ln" else 12) * M * D),
                     kernel=f"enchip::residual_layer_norm<{ln_cpl(D)}, true>")
        else:
            u.update(kind="row", bytes=float(4 * M * D), kernel="enchip::pool_mean_cols + l2_normalize_rows")
        u["ms_per_step"] = u["us_per_launch"] * u["launches_per_step"] / 1e3
        if u["ops"] and u["kind"] == "w8a8":
            u["int8_tops"] = u["ops"] / t / 1e12
            u["frac_int8_peak"] = u["ops"] / t / PEAK_INT8_OPS
        if u["bytes"]:
            u["alg_gbps"] = u["bytes"] / t / 1e9
            u["frac_hbm_peak"] = u["bytes"] / t / PEAK_HBM_BPS
        if label == "attention":
            # split products: three 16-bit MFMA products per f32 product
            u["frac_mfma_peak"] = (u["ops"] / t / PEAK_FP32_FLOPS if ctx.attention_products == 0
                                   else 3 * u["ops"] / t / PEAK_BF16_FLOPS)
        table[label] = u
    return table


# VALU lane-operations per element of quant_rows_frag_gelu<12> in the BERT-base encode:
# SQ_INSTS_VALU = 76,243 wave-instructions per SIMD per launch x 1024 SIMDs x 64 lanes /
# (32768 x 3072 elements) = 49.6 (series, erf tails, absmax, codes, addressing).
GELU_QUANT_LANE_OPS = 50
GELU_QUANT_VALU_SOURCE = "profiles/int8_gemm_clock_mfma_busy_valu_bert_base_xlmr_large.md"


def traffic_key_of(label: str) -> str:
    """The row of TRAFFIC_PROFILE's table that measured the kernel of an encode label."""
    base = label.split(".")[0]
    if label.endswith(".gemm"):
        return base
    return ("gelu_quant_" if label.endswith(".gelu_quant") else "quant_") + base


def roofline_of(label: str, u: dict, ceilings: dict, traffic_key: str) -> dict:
    """The roofline entry of one kernel: MFMA-bound when its algorithmic intensity reaches
    the int8 ridge (peak ops / peak bytes), HBM-bound below it."""
    t = u["us_per_launch"] * 1e-6
    ops, nbytes = u["ops"], u["bytes"]
    ridge = PEAK_INT8_OPS / PEAK_HBM_BPS
    traffic = measured_traffic().get(traffic_key)
    if ops > 0 and ops / nbytes >= ridge:
        roof = {"bound": "mfma", "achieved": ops / t / 1e12, "peak": PEAK_INT8_OPS / 1e12, "unit": "TFLOP/s",
                "frac": ops / t / PEAK_INT8_OPS}
    else:
        roof = {"bound": "hbm", "achieved": nbytes / t / 1e9, "peak": PEAK_HBM_BPS / 1e9, "unit": "GB/s",
                "frac": nbytes / t / PEAK_HBM_BPS}
    return {
        **roof,
        "traffic": traffic,
        "kernel": u["kernel"],
        "unit_label": label,
        "launches_per_step": u["launches_per_step"],
        "avg_launch_us": u["us_per_launch"],
        "alg_bytes_per_launch": nbytes,
        "alg_ops_per_launch": ops,
        "arithmetic_intensity": (ops / nbytes) if ops else 0.0,
        "ridge_op_per_byte": ridge,
        "int8_frac_of_peak": ops / t / PEAK_INT8_OPS,
        "frac_of_measured_mfma_peak": ops / t / (ceilings["mfma_i8_tops"] * 1e12),
        "frac_of_measured_mfma_data_peak": ops / t / (ceilings["mfma_i8_data_tops"] * 1e12),
        "frac_of_measured_hbm_read": nbytes / t / 1e9 / ceilings["hbm_read_gbps"],
        "traffic_source": TRAFFIC_PROFILE if traffic is not None else None,
    }


def device_forward(ctx, torch, stream, layers_host, cfg, steps: int = 3, warmup: int = 1, head: str = "pool"):
    """`steps` encodes (build_encoder) timed back to back after `warmup`, in the current
    attention product mode."""
    from aikit_amd import enchip

    model, step, out = build_encoder(ctx, torch, stream, layers_host, cfg, head=head)
    try:
        el = time_steps(torch, stream, step, steps, warmup)
        finite = bool(torch.isfinite(out).all().item())
    finally:
        model.close()
    t = el / steps
    S = cfg.batch
    rate = "pairs_per_s" if head == "rerank" else "seqs_per_s"
    tail = "cross-encoder head (f32 pooler + tanh + classifier)" if head == "rerank" else "pooling + L2"
    products = ATT_NAMES[ctx.attention_products]
    return {rate: S / t, "ms_per_batch": t * 1e3, "batch": S, "seq_len": cfg.seq, "layers": cfg.layers,
            "hidden": cfg.hidden, "output_finite": finite, "attention_products": products, "steps": steps,
            "note": "%d encodes back to back from token ids (after %d warm-up): embedding rows + LayerNorm, W8A8 "
                    "linears, fused attention (%s MFMA products), LayerNorm, %s, all on the device"
                    % (steps, warmup, products, tail)}


def ffn_gelu_placement(ctx, torch, stream, reps: int = 5) -> dict:
    """Where FFN-up's exact GELU runs, measured at BERT-base's FFN shape (M = 32768,
    768 -> 3072 -> the codes of FFN-down's 3072-wide input) over pre-activations of several
    spreads: the GELU epilogue of FFN-up's GEMM followed by enchip_quant_rows_frag_dev,
    against a bias-only GEMM followed by enchip_quant_rows_frag_gelu_dev (what the device
    forward runs for K <= 3072). The weight scales set the pre-activations' standard
    deviation (int8 codes uniform over +-127 times N(0, 1) activations: ~2031 x the scale);
    `tails` is the fraction of arguments off ErfF32's series branch. Interleaved, the
    median of `reps` timings by HIP events on the launch stream; both codes and scales
    compared bit for bit."""
    import numpy as np

    from aikit_amd import enchip, workloads

    M, K, N = 32768, 768, 3072
    sp = stream.cuda_stream
    hev = HipEvents()
    g = workloads.rng(5)
    wq = g.integers(-127, 128, size=(N, K), dtype=np.int8)
    with torch.cuda.stream(stream):
        gen = torch.Generator(device="cuda").manual_seed(5)
        a = torch.randn((M, K), device="cuda", generator=gen)
        b = torch.from_numpy((g.standard_normal(N) * 0.05).astype(np.float32)).cuda()
        inter = torch.empty((M, N), device="cuda")
        s1, s2a, s2b = (torch.empty(M, device="cuda") for _ in range(3))
    out = {}
    try:
        for std in (0.28, 0.55, 1.1, 3.3):
            ws = (np.float32(std / 2031.0) * g.uniform(0.9, 1.1, N)).astype(np.float32)
            w = ctx.register_weight(wq, ws)
            try:
                ok, ldq = ctx.frag_route(w, M)
                if not ok:
                    return {"skipped": "no fragment-major route"}
                Mp = (M + 127) // 128 * 128
                with torch.cuda.stream(stream):
                    q1 = torch.zeros(Mp * ldq, dtype=torch.int8, device="cuda")
                    q2a = torch.zeros(Mp * N, dtype=torch.int8, device="cuda")
                    q2b = torch.zeros(Mp * N, dtype=torch.int8, device="cuda")
                ctx.quant_rows_frag_dev(a.data_ptr(), M, K, q1.data_ptr(), ldq, s1.data_ptr(), sp)
                legs = {
                    "gemm_gelu_us": lambda: ctx.pre_frag_dev(w, q1.data_ptr(), ldq, M, s1.data_ptr(), b.data_ptr(),
                                                             enchip.ACT_GELU, inter.data_ptr(), sp),
                    "quant_us": lambda: ctx.quant_rows_frag_dev(inter.data_ptr(), M, N, q2a.data_ptr(), N,
                                                                s2a.data_ptr(), sp),
                    "gemm_bias_us": lambda: ctx.pre_frag_dev(w, q1.data_ptr(), ldq, M, s1.data_ptr(), b.data_ptr(),
                                                             enchip.ACT_NONE, inter.data_ptr(), sp),
                    "gelu_quant_us": lambda: ctx.quant_rows_frag_gelu_dev(inter.data_ptr(), M, N, q2b.data_ptr(), N,
                                                                          s2b.data_ptr(), sp),
                }
                times = {k: [] for k in legs}
                for rep in range(reps + 1):
                    evs = []
                    for k, fn in legs.items():  # in this order: each quantizer reads the GEMM before it
                        e0, e1 = hev.create(), hev.create()
                        hev.record(e0, sp)
                        fn()
                        hev.record(e1, sp)
                        evs.append((k, e0, e1))
                    torch.cuda.synchronize()
                    if rep:
                        for k, e0, e1 in evs:
                            times[k].append(hev.elapsed_ms(e0, e1) * 1e3)
                    hev.close()
                pre = inter.cpu().numpy()
                tails = float(np.mean(~(np.abs(pre * np.float32(0.7071067811865476)) < 1)))
                same = bool(torch.equal(q2a, q2b)) and bool(torch.equal(s2a.view(torch.int32), s2b.view(torch.int32)))
                med = {k: float(np.median(v)) for k, v in times.items()}
                med.update(epilogue_pair_us=med["gemm_gelu_us"] + med["quant_us"],
                           quantizer_pair_us=med["gemm_bias_us"] + med["gelu_quant_us"], tails=tails,
                           codes_identical=same)
                out[str(std)] = med
                del q1, q2a, q2b
            finally:
                ctx.release_weight(w)
    finally:
        hev.close()
    out["note"] = ("FFN-up's GEMM (M 32768, 768 -> 3072) + FFN-down's quantizer: the GELU in the GEMM epilogue "
                   "(gemm_gelu + quant) vs in the quantizer (gemm_bias + gelu_quant), by pre-activation standard "
                   "deviation; median of HIP-event timings, interleaved")
    return out


def rerank_device(ctx, torch, stream, steps: int = 2):
    """Config 5: XLM-R-large (24 layers, D 1024, 16 heads, FFN 4096) cross-encoder scoring of
    128 (query, passage) pairs of 512 tokens, random-init weights quantized per channel."""
    from aikit_amd import workloads

    cfg = workloads.XLMR_LARGE_CE
    g = workloads.rng(2025)
    host = [workloads.encoder_layer_weights(g, cfg) for _ in range(cfg.layers)]
    return device_forward(ctx, torch, stream, host, cfg, steps=steps, head="rerank")


def linear_stack(ctx, torch, stream, cfg, layers_host, steps: int, warmup: int, ceilings: dict) -> dict:
    """The 48 W8A8 linears of one BERT-base b64xs512 forward alone (the previous headline):
    each linear's per-token quantization + GEMM + fused epilogue on seeded N(0,1) inputs
    resident in HBM (FFN-down reads FFN-up's output), `steps` steps timed back to back,
    then the same steps with HIP events around every launch for the per-kernel table."""
    import numpy as np

    M = cfg.tokens
    lin = cfg.linears()
    layers = []
    for lw in layers_host:
        layers.append({name: (ctx.register_weight(wq, ws), torch.from_numpy(b).cuda(), act)
                       for name, (wq, ws, b, act) in lw.items()})
    try:
        with torch.cuda.stream(stream):
            gen = torch.Generator(device="cuda").manual_seed(7)
            x_in = {n: torch.randn((M, K), generator=gen, device="cuda", dtype=torch.float32)
                    for n, K, _, _ in lin if n != "ffn_down"}
            outs = {n: torch.empty((M, N), device="cuda", dtype=torch.float32) for n, _, N, _ in lin}
            kmax = max(K for _, K, _, _ in lin)
            aq = torch.empty(((M + 127) // 128 * 128) * kmax, device="cuda", dtype=torch.int8)
            asc = torch.empty(M, device="cuda", dtype=torch.float32)
        torch.cuda.synchronize()
        sptr = stream.cuda_stream
        ldqs = {}
        for name, K, N, act in lin:
            ok, ldq = ctx.frag_route(layers[0][name][0], M)
            if not ok:
                raise SystemExit(f"bench: {name} has no fragment-major route")
            ldqs[name] = ldq
        hev = HipEvents()

        def run_step(evs=None):
            for li in range(cfg.layers):
                for j, (name, K, N, act) in enumerate(lin):
                    h, b, _ = layers[li][name]
                    x = outs["ffn_up"] if name == "ffn_down" else x_in[name]
                    if evs is not None:
                        hev.record(evs[li][j][0], sptr)
                    ctx.quant_rows_frag_dev(x.data_ptr(), M, K, aq.data_ptr(), ldqs[name], asc.data_ptr(), sptr)
                    if evs is not None:
                        hev.record(evs[li][j][1], sptr)
                    ctx.pre_frag_dev(h, aq.data_ptr(), ldqs[name], M, asc.data_ptr(), b.data_ptr(), act,
                                     outs[name].data_ptr(), sptr)
                    if evs is not None:
                        hev.record(evs[li][j][2], sptr)

        elapsed = time_steps(torch, stream, run_step, steps, warmup)
        events = [[[[hev.create() for _ in range(3)] for _ in lin] for _ in range(cfg.layers)] for _ in range(steps)]
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for st in range(steps):
                run_step(events[st])
        torch.cuda.synchronize()
        per = {name: {"quant_ms": [], "gemm_ms": []} for name, _, _, _ in lin}
        for st in range(steps):
            for li in range(cfg.layers):
                for j, (name, _, _, _) in enumerate(lin):
                    e0, e1, e2 = events[st][li][j]
                    per[name]["quant_ms"].append(hev.elapsed_ms(e0, e1))
                    per[name]["gemm_ms"].append(hev.elapsed_ms(e1, e2))
        hev.close()
        kernels = {}
        tot_ops = tot_gemm_s = 0.0
        for name, K, N, act in lin:
            gq = float(np.mean(per[name]["gemm_ms"])) * 1e-3
            qq = float(np.mean(per[name]["quant_ms"])) * 1e-3
            ops = 2.0 * M * N * K
            gbytes = M * K + N * K + 4 * M + 8 * N + 4 * M * N
            qbytes = 4 * M * K + M * K + 4 * M
            kernels[name] = {
                "M": M, "K": K, "N": N, "act": "gelu" if act else "none",
                "gemm_kernel": ctx.gemm_kernel_name(layers[0][name][0], M, act),
                "gemm_us": gq * 1e6, "gemm_tops": ops / gq / 1e12, "gemm_frac_int8_peak": ops / gq / PEAK_INT8_OPS,
                "gemm_alg_gbps": gbytes / gq / 1e9, "gemm_frac_hbm": gbytes / gq / PEAK_HBM_BPS,
                "quant_us": qq * 1e6, "quant_gbps": qbytes / qq / 1e9, "quant_frac_hbm": qbytes / qq / PEAK_HBM_BPS,
            }
            tot_ops += ops * cfg.layers
            tot_gemm_s += gq * cfg.layers
    finally:
        for entry in layers:
            for h, _, _ in entry.values():
                ctx.release_weight(h)
    return {
        "seqs_per_s": cfg.batch * steps / elapsed,
        "ms_per_step": elapsed * 1e3 / steps,
        "steps": steps,
        "gemm_tops": tot_ops / tot_gemm_s / 1e12,
        "gemm_frac_int8_peak": tot_ops / tot_gemm_s / PEAK_INT8_OPS,
        "int8_tops_per_step": tot_ops / 1e12,
        "kernels": kernels,
        "note": ("the 48 W8A8 linears of one BERT-base b64xs512 forward alone (12 layers x {QKV 768->2304 +bias, "
                 "O 768->768 +bias, FFN-up 768->3072 +bias+GELU, FFN-down 3072->768 +bias}), per-token int8 quant + "
                 "int8 MFMA GEMM + fused dequant epilogue each, on seeded N(0,1) inputs resident in HBM; kernel "
                 "times from HIP events around each launch in a second region of the same steps"),
    }


ATT_NAMES = {0: "f32 two-pass (ENCHIP_ATT_F32)", 1: "split-bf16 two-pass (ENCHIP_ATT_SPLIT_BF16)",
             2: "split-bf16 online-softmax (ENCHIP_ATT_FLASH_BF16)",
             3: "split-f16 online-softmax (ENCHIP_ATT_FLASH_F16)"}  # enchip_att_products

LINE_LIMIT = 8192  # bytes: the stdout line the driver parses stays well under this
DETAIL_PATH = os.path.join("gpurun_out", "bench_detail.json")


def write_detail(result: dict) -> str | None:
    """The full result (every kernel's figures, the linear stack, the other configs)
    goes to stderr and to DETAIL_PATH; the stdout line carries only its summary.
    Returns the path written, or None when it could not be written."""
    text = json.dumps(result)
    print(f"[bench] detail {text}", file=sys.stderr, flush=True)
    try:
        os.makedirs(os.path.dirname(DETAIL_PATH), exist_ok=True)
        with open(DETAIL_PATH, "w") as f:
            f.write(text + "\n")
        return DETAIL_PATH
    except OSError as e:
        log(f"could not write {DETAIL_PATH}: {e}")
        return None


def _r(x, nd: int = 4):
    """Round floats to nd significant digits for the compact line."""
    if isinstance(x, float):
        return float(f"{x:.{nd}g}")
    return x


def compact_result(result: dict, detail_path: str | None = None) -> dict:
    """The one JSON line bench.py prints: the contract's keys, a short config, the
    roofline of the W8A8 path's dominant kernel (with its VALU roof and measured HBM
    traffic), the step's dominant kernel, the measured ceilings, the CPU baseline, a
    {unit: [us per launch, fraction of its roof]} table of the encode's kernels and one
    figure per other config. Everything else stays in the detail file. The result is
    bounded by LINE_LIMIT whatever the number of kernels (the table is dropped first,
    then the other configs, if a line would exceed it)."""
    keep = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
            "scaling", "vs_baseline", "dtype", "data")
    out = {k: _r(result[k], 6) if k in ("value", "ms_per_step") else result[k] for k in keep if k in result}
    cfg = result.get("config", {})
    out["config"] = {
        "workload": "bert-base b64xs512 W8A8 encode (token ids -> pooled L2 embeddings), resident in HBM",
        **{k: cfg[k] for k in ("model", "global_batch", "seq_len", "parallelism", "attention_products", "launch")
           if k in cfg},
    }
    rf = result.get("roofline") or {}
    roof = {k: _r(rf[k]) for k in ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel", "unit_label",
                                    "avg_launch_us", "alg_bytes_per_launch", "alg_ops_per_launch",
                                    "int8_frac_of_peak", "traffic_source") if k in rf}
    if "valu" in rf:
        v = rf["valu"]
        roof["valu"] = {"frac": _r(v.get("frac")), "achieved_t_lane_ops": _r(v.get("achieved_t_lane_ops")),
                        "peak_t_lane_ops": _r(v.get("measured_peak_t_lane_ops")),
                        "lane_ops_per_output": v.get("lane_ops_per_output")}
    out["roofline"] = roof
    sd = result.get("roofline_step_dominant") or {}
    out["roofline_step_dominant"] = {k: _r(sd[k]) for k in ("unit_label", "kernel", "avg_launch_us", "share_of_step",
                                                            "bound", "unit", "achieved", "peak", "frac", "valu_frac")
                                     if k in sd}
    if result.get("measured_ceilings"):
        out["measured_ceilings"] = {k: _r(v) for k, v in result["measured_ceilings"].items()}
    cb = result.get("cpu_baseline")
    out["cpu_baseline"] = None if cb is None else {
        k: _r(cb[k]) if k != "sample" else str(cb[k])[:400] for k in ("value", "unit", "cores", "kind", "sample")
        if k in cb}
    kern = {}
    for label, u in (result.get("encode_kernels") or {}).items():
        frac = u.get("frac_int8_peak") if u.get("ops") else u.get("frac_hbm_peak")
        if label == "attention":
            frac = u.get("frac_mfma_peak", frac)
        kern[label] = [_r(u.get("us_per_launch"), 4), _r(frac, 3)]
    out["kernels_us_frac"] = kern
    other = {}
    oc = result.get("other_configs") or {}
    if "config2_isolated_linear" in oc:
        other["cfg2_us_per_call"] = _r(oc["config2_isolated_linear"].get("us_per_call"))
        sp2 = oc["config2_isolated_linear"].get("split") or {}
        for k in ("call_bias_only_us", "quantizer_us", "gemm_gelu_us", "gemm_bias_only_us"):
            if sp2.get(k) is not None:
                other[f"cfg2_{k}"] = _r(sp2[k])
    for n in ("768", "3072"):
        c = oc.get(f"config3_gemv_n{n}")
        if c:
            other[f"cfg3_n{n}_us_per_call"] = _r(c.get("us_per_call"))
            other[f"cfg3_n{n}_frac_hbm"] = _r(c.get("frac_hbm_peak"), 3)
    if "rerank_device_cfg5" in oc:
        other["cfg5_pairs_per_s"] = _r(oc["rerank_device_cfg5"].get("pairs_per_s"))
    fg = oc.get("ffn_gelu_placement") or {}
    if fg and "skipped" not in fg:
        # std: [GELU epilogue + quantizer, bias-only GEMM + GELU quantizer] in us, tail fraction
        other["ffn_gelu_epi_vs_quant_us"] = {k: [_r(v["epilogue_pair_us"], 4), _r(v["quantizer_pair_us"], 4),
                                                 _r(v["tails"], 3)]
                                             for k, v in fg.items() if isinstance(v, dict)}
    for m in ("1", "16", "256"):
        c = oc.get(f"ann_flat_i8_m{m}")
        if c:
            other[f"ann_m{m}_us"] = _r(c.get("us_per_call"))
            for kk in ("", "64"):
                if c.get(f"ann_topk{kk}_host_us_per_call") is not None:
                    other[f"ann_m{m}_topk{kk or '10'}_host_us"] = _r(c[f"ann_topk{kk}_host_us_per_call"])
            for kb, v in (c.get("topk_rows_us_per_call") or {}).items():
                other[f"ann_m{m}_select{kb}_us"] = _r(v)
    q8 = oc.get("matmul_bt_q8_weight_only")
    if q8:
        for k in ("m512_layer_us", "m512_layer_host_us", "m32768_layer_us", "m32768_tflops"):
            if q8.get(k) is not None:
                other[f"q8w_{k}"] = _r(q8[k])
    if "linear_stack" in result:
        other["linear_stack_ms"] = _r(result["linear_stack"].get("ms_per_step"))
    for k in ("encode_f32_products", "encode_split_bf16_two_pass", "encode_flash_bf16"):
        if k in result:
            other[f"{k}_ms"] = _r(result[k].get("ms_per_step"))
    out["other"] = other
    out["output_finite"] = result.get("output_finite")
    out["detail"] = detail_path or "stderr ([bench] detail ...)"
    for drop in ("kernels_us_frac", "other"):
        if len(json.dumps(out)) <= LINE_LIMIT:
            break
        out.pop(drop, None)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline sample length (0 = skip)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip everything but the headline encode (configs 2, 3, 5, ann, the linear stack)")
    ap.add_argument("--forward-only", nargs="?", const="cfg4", choices=["cfg4", "cfg5"], default=None,
                    help="only time the config-4 encode (cfg5: the config-5 cross-encoder instead) and print its "
                         "figures (a profiling mode: its kernels are then the only ones in a trace)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the W8A8 path is not sharded across GPUs; "
              "each GPU would take its own shard of the batch). Use --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from aikit_amd import enchip, workloads

    cfg = workloads.BERT_BASE
    log(f"torch {torch.__version__}, device {torch.cuda.get_device_name(0)}")
    ctx = enchip.Context(0)
    info = ctx.device_info()
    log(f"enchip device {info}")
    stream = torch.cuda.Stream()
    ceilings = ctx.probe_ceilings()
    log(f"measured ceilings {ceilings}")

    if args.forward_only == "cfg5":
        out = {"rerank_device_cfg5": rerank_device(ctx, torch, stream, steps=max(1, args.steps))}
        ctx.close()
        print(json.dumps(out), flush=True)
        return 0

    # ---- the encode: weights for 12 layers, random N(0,0.02) quantized per channel
    g = workloads.rng(2024)
    t0 = time.perf_counter()
    layers_host = [workloads.encoder_layer_weights(g, cfg) for _ in range(cfg.layers)]
    model, step, pooled = build_encoder(ctx, torch, stream, layers_host, cfg)
    log(f"encoder built ({cfg.layers * 4} weights registered) in {time.perf_counter() - t0:.1f}s")
    if args.forward_only == "cfg4":
        el = time_steps(torch, stream, step, max(1, args.steps), args.warmup)
        model.close()
        ctx.close()
        print(json.dumps({"encode_device_cfg4": {"seqs_per_s": cfg.batch * args.steps / el,
                                                 "ms_per_batch": el * 1e3 / args.steps}}), flush=True)
        return 0

    # Timed region 1 (value): K encodes back to back, nothing between the kernels.
    elapsed = time_steps(torch, stream, step, args.steps, args.warmup)
    ms_per_step = elapsed * 1e3 / args.steps
    seqs_per_s = cfg.batch * args.steps / elapsed
    finite = bool(torch.isfinite(pooled).all().item())
    log(f"timed {args.steps} encodes: {ms_per_step:.3f} ms/step, {seqs_per_s:.1f} seqs/s")

    # Timed region 2 (kernel durations): the same K encodes with a HIP event recorded on the
    # launch stream between consecutive operations.
    hev = HipEvents()
    per, op_timing = time_ops(torch, stream, model, step, args.steps, hev, args.warmup)
    hev.close()
    units = encode_units(ctx, model, cfg, per, args.steps)
    step_ms_events = sum(u["ms_per_step"] for u in units.values())
    w8a8 = {k: u for k, u in units.items() if u["kind"] == "w8a8"}
    key = max(w8a8, key=lambda k: w8a8[k]["ms_per_step"])
    traffic_key = traffic_key_of(key)
    roofline = roofline_of(key, w8a8[key], ceilings, traffic_key)
    u = w8a8[key]
    gelu_epi = key == "ffn_up.gemm" and "ffn_down.gelu_quant" not in units
    roofline["limiter"] = (
        "VALU issue: the GELU epilogue restates aikit's exact-erf GELUF32 with no FMA (~36 VALU per output in "
        "its branch-free pass), its largest fraction of any roof (roofline.valu); main loops and epilogues "
        "overlap only where a CU's two workgroups are in different phases"
        if gelu_epi else
        "the f32 output stores (4 B per output, most of its bytes) behind the main loop's MFMA issue; no GELU "
        "in this epilogue (FFN-down's quantization applies it)" if key == "ffn_up.gemm" else
        "MFMA issue in the main loop" if key.endswith(".gemm") else
        "VALU issue: the exact-erf GELU restated with no FMA (27 multiplies and adds per element in the "
        "series alone) plus the quantization, ~50 VALU lane-ops per element (roofline.valu), at 4 waves per "
        "SIMD" if key.endswith(".gelu_quant") else "HBM")
    roofline["scope"] = ("the W8A8 path's dominant kernel in the timed encode (by device time per step); "
                         "roofline_step_dominant covers the step's dominant kernel overall")
    if key.endswith(".gelu_quant"):
        # its binding roof: VALU lane-operations per element, measured (SQ_INSTS_VALU per
        # launch x 64 lanes / elements, GELU_QUANT_VALU_SOURCE) against the measured VALU rate
        elems = cfg.tokens * cfg.ffn
        valu_ops = float(GELU_QUANT_LANE_OPS) * elems
        t_l = u["us_per_launch"] * 1e-6
        roofline["valu"] = {"lane_ops_per_output": GELU_QUANT_LANE_OPS, "outputs_per_launch": elems,
                            "lane_ops_per_launch": valu_ops, "achieved_t_lane_ops": valu_ops / t_l / 1e12,
                            "measured_peak_t_lane_ops": ceilings["valu_f32_tops"],
                            "frac": valu_ops / t_l / 1e12 / ceilings["valu_f32_tops"],
                            "source": GELU_QUANT_VALU_SOURCE}
    if gelu_epi:
        # the third roof of this kernel: its epilogue's f32 VALU work (the exact-erf GELU with
        # no FMA: 36 VALU instructions per output in the branch-free pass, counted in the
        # kernel's gfx950 ISA) against the measured unfused f32 VALU rate
        outs = cfg.tokens * cfg.ffn
        valu_ops = 36.0 * outs
        t_l = u["us_per_launch"] * 1e-6
        roofline["valu"] = {"lane_ops_per_output": 36, "outputs_per_launch": outs, "lane_ops_per_launch": valu_ops,
                            "achieved_t_lane_ops": valu_ops / t_l / 1e12,
                            "measured_peak_t_lane_ops": ceilings["valu_f32_tops"],
                            "frac": valu_ops / t_l / 1e12 / ceilings["valu_f32_tops"]}
    dom = max(units, key=lambda k: units[k]["ms_per_step"])
    ud = units[dom]
    step_dom = {"unit_label": dom, "kernel": ud["kernel"], "avg_launch_us": ud["us_per_launch"],
                "launches_per_step": ud["launches_per_step"], "share_of_step": ud["ms_per_step"] / step_ms_events}
    if dom == "attention":
        f = ud["ops"] / (ud["us_per_launch"] * 1e-6)
        split = ctx.attention_products != enchip.ATT_F32
        step_dom.update({
            "bound": "mfma", "unit": "TFLOP/s", "achieved": f / 1e12,
            "alg_flops_per_launch": ud["ops"],
            "peak": (PEAK_BF16_FLOPS if split else PEAK_FP32_FLOPS) / 1e12,
            "frac": (3 * f / PEAK_BF16_FLOPS) if split else f / PEAK_FP32_FLOPS,
            "note": ("achieved = the f32 attention's algorithmic flops (4 L^2 hd per head) per second; with split "
                     "products each f32 product is three 16-bit MFMA products, so frac = 3 x achieved / the 2.5 PFLOP/s "
                     "bf16 dense peak (the MFMA work the kernel issues); the exact softmax's VALU work is not in it")
            if split else "achieved = algorithmic flops per second on the f32 MFMA"})
    elif dom in w8a8:
        # a W8A8 unit: the same roof as the roofline object (that object itself when the
        # two dominant kernels coincide)
        rd = roofline if dom == key else roofline_of(dom, ud, ceilings, traffic_key_of(dom))
        step_dom.update({f: rd[f] for f in ("bound", "unit", "achieved", "peak", "frac")})
        if "valu" in rd:
            step_dom["valu_frac"] = rd["valu"]["frac"]
    log(f"dominant W8A8 kernel {key}: {u['us_per_launch']:.1f} us, roofline frac {roofline['frac']:.3f}; "
        f"step-dominant {dom} ({step_dom['share_of_step']:.0%} of the step)")

    result = {
        "metric": METRIC,
        "value": seqs_per_s,
        "unit": "seqs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": ("bert-base b64xs512 W8A8 encode resident on the device: token ids -> embedding rows + "
                         "LayerNorm -> 12 layers x {W8A8 fused QKV 768->2304 +bias, fused attention "
                         "(online softmax, products on the f16 MFMA over half-split operands, within the f32 "
                         "MatmulBT gate), W8A8 O "
                         "768->768 +bias, "
                         "residual LayerNorm fused with the next quantization, W8A8 FFN-up 768->3072 +bias+GELU, "
                         "W8A8 FFN-down 3072->768 +bias, residual LayerNorm} -> mean pool + L2; every W8A8 "
                         "linear = per-token int8 quant + int8 MFMA GEMM + fused dequant epilogue"),
            "model": "bert-base (random-init weights, per-channel int8)",
            "global_batch": cfg.batch,
            "seq_len": cfg.seq,
            "tokens_per_step": cfg.tokens,
            "parallelism": "single GPU",
            "attention_products": ATT_NAMES[ctx.attention_products],
            "seeds": {"weights": 2024, "tables_and_ids": 5},
            "launch": "eager",
        },
        "output_finite": finite,
        "encode_kernels": units,
        "encode_kernels_timing": op_timing,
        "encode_ms_per_step_from_events": step_ms_events,
        "encode_int8_tops": sum(u_["ops"] * u_["launches_per_step"] for u_ in w8a8.values()) /
                            sum(u_["ms_per_step"] for k_, u_ in w8a8.items() if k_.endswith(".gemm")) / 1e9,
        "roofline": roofline,
        "roofline_step_dominant": step_dom,
        "measured_ceilings": ceilings,
        "device": info,
    }
    # the same encode with the attention's other product modes
    n2 = max(3, args.steps // 2)
    for mode, key, what in ((enchip.ATT_F32, "encode_f32_products",
                             "the two-pass attention with both products on the f32 MFMA"),
                            (enchip.ATT_SPLIT_BF16, "encode_split_bf16_two_pass",
                             "the two-pass attention (the reference's softmax steps) with split-bf16 products"),
                            (enchip.ATT_FLASH_BF16, "encode_flash_bf16",
                             "the online-softmax attention with bfloat16-split products")):
        ctx.set_attention_products(mode)
        el2 = time_steps(torch, stream, step, n2, 1)
        result[key] = {"seqs_per_s": cfg.batch * n2 / el2, "ms_per_step": el2 * 1e3 / n2, "steps": n2,
                       "note": f"the headline encode with {what} (enchip_set_attention_products)"}
        log(f"{key}: {result[key]['ms_per_step']:.3f} ms/step")
    ctx.set_attention_products(enchip.ATT_DEFAULT)
    model.close()

    if not args.no_other_configs:
        log("linear stack (the 48 W8A8 linears alone)")
        result["linear_stack"] = linear_stack(ctx, torch, stream, cfg, layers_host, args.steps, args.warmup, ceilings)
        log(f"  {result['linear_stack']['ms_per_step']:.3f} ms/step")
        log("configs 2 and 3 (isolated linear, small-M GEMV over a rotating > 2x MALL weight set), ann.FlatI8 scoring")
        result["other_configs"] = other_configs(ctx, torch, stream, ceilings)
        result["other_configs"]["weight_registration_cfg4"] = weight_registration(ctx, layers_host)
        log("FFN-up's GELU: in the GEMM epilogue or in FFN-down's quantizer, by pre-activation spread")
        result["other_configs"]["ffn_gelu_placement"] = ffn_gelu_placement(ctx, torch, stream)
        log("config 5 cross-encoder rerank resident on the device (XLM-R-large shape, 128 pairs x 512)")
        result["other_configs"]["rerank_device_cfg5"] = rerank_device(ctx, torch, stream)
        log(f"  {result['other_configs']['rerank_device_cfg5']['pairs_per_s']:.1f} pairs/s end to end")
    if args.cpu_seconds > 0:
        log(f"CPU baseline ({args.cpu_seconds:.0f}s sample, {host_threads()} threads)")
        result["cpu_baseline"] = cpu_baseline(layers_host[0], cfg, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    ctx.close()
    detail = write_detail(result)
    line = compact_result(result, detail)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
