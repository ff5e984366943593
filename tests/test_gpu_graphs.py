"""HIP graph capture of the device entry points that a serving loop would replay.

A caller that launches the same work every step can capture it once into a HIP graph and
replay it, with no host launch path between the kernels. These tests capture:
- `enchip_matmul_bt_q8_dev` in each of its kernel forms;
- `enchip_w8a8_linear_noalloc_dev` (the entry point for callers that cannot allocate);
- a whole device encode from token ids (embedding rows, every layer's linears, attention
  and LayerNorms, pooling; `aikit_amd.bert_dev.DeviceBert`).

Every test replays its graph several times. Between replays the program does its own
eager work (the captured inputs rewritten in place, then a synchronization). Each replay is
checked bit for bit against eager calls on the same inputs, so a captured operation that
behaves differently on a later replay (a memset node, a buffer the capture froze, scratch
grown during capture) fails.
"""
import numpy as np
import pytest

from aikit_amd import enchip, workloads

pytestmark = pytest.mark.gpu

REPLAYS = 4


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def test_graph_matmul_bt_q8_every_form(ctx):
    import torch

    # the K-split small form, 64 x 64, 128 x 128 and 128 x 256 tiles (the host's choice by
    # grid size on MI355X's 256 CUs)
    shapes = [(70, 768, 200), (512, 768, 3072), (4096 + 5, 768, 2304), (16384, 768, 2048)]
    g = workloads.rng(51)
    s = torch.cuda.Stream()
    items = []
    try:
        for M, K, N in shapes:
            w = ctx.register_weight(g.integers(-128, 128, size=(N, K)).astype(np.int8),
                                    (0.002 + (np.arange(N) % 13) * 1e-4).astype(np.float32))
            with torch.cuda.stream(s):
                a = torch.empty((M, K), device="cuda")
                d, e = torch.empty((M, N), device="cuda"), torch.empty((M, N), device="cuda")
            items.append((w, M, K, N, a, d, e))
        torch.cuda.synchronize()

        def run(out_index):
            for w, M, K, N, a, d, e in items:
                ctx.matmul_bt_q8_dev(w, a.data_ptr(), K, M, (d, e)[out_index].data_ptr(), N, s.cuda_stream)

        for _, M, K, N, a, _, _ in items:
            a.normal_()
        run(1)  # eager once before capture
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            run(0)
        say(f"matmul_bt_q8_dev: {len(shapes)} calls captured, {REPLAYS} replays")
        for r in range(REPLAYS):
            with torch.cuda.stream(s):
                for _, M, K, N, a, _, _ in items:
                    a.normal_()
            torch.cuda.synchronize()
            gr.replay()
            torch.cuda.synchronize()
            run(1)
            torch.cuda.synchronize()
            for _, M, K, N, _, d, e in items:
                assert np.array_equal(bits(d), bits(e)), f"replay {r}, M={M} K={K} N={N}"
        del gr
    finally:
        for it in items:
            ctx.release_weight(it[0])


def test_graph_linear_noalloc(ctx):
    import torch

    # the one-launch small-M route and the quantize + persistent GEMM route, with GELU
    shapes = [(16, 768, 3072), (4096, 768, 3072)]
    g = workloads.rng(52)
    s = torch.cuda.Stream()
    items = []
    try:
        for M, K, N in shapes:
            wq, ws = workloads.int8_weights(g, N, K)
            w = ctx.register_weight(wq, ws)
            with torch.cuda.stream(s):
                a = torch.empty((M, K), device="cuda")
                b = torch.from_numpy(workloads.bias(g, N)).cuda()
                d, e = torch.empty((M, N), device="cuda"), torch.empty((M, N), device="cuda")
            items.append((w, M, K, N, a, b, d, e))
        torch.cuda.synchronize()

        def run(out_index):
            for w, M, K, N, a, b, d, e in items:
                ctx.linear_noalloc_dev(w, a.data_ptr(), M, b.data_ptr(), enchip.ACT_GELU, (d, e)[out_index].data_ptr(),
                                       s.cuda_stream)

        for it in items:
            it[4].normal_()
        run(1)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            run(0)
        say(f"linear_noalloc_dev: {len(shapes)} calls captured, {REPLAYS} replays")
        for r in range(REPLAYS):
            with torch.cuda.stream(s):
                for it in items:
                    it[4].normal_().mul_(1.0 + r)
            torch.cuda.synchronize()
            gr.replay()
            torch.cuda.synchronize()
            run(1)
            torch.cuda.synchronize()
            for _, M, K, N, _, _, d, e in items:
                assert np.array_equal(bits(d), bits(e)), f"replay {r}, M={M} K={K} N={N}"
        del gr
    finally:
        for it in items:
            ctx.release_weight(it[0])


def test_graph_device_encode(ctx):
    import torch

    from aikit_amd.bert_dev import DeviceBert

    cfg = workloads.MINILM_L6
    S, L, D = 4, 128, cfg.hidden
    g = workloads.rng(53)
    layers = []
    for _ in range(cfg.layers):
        lw = workloads.encoder_layer_weights(g, cfg)
        for name in ("attn_ln", "out_ln"):
            lw[name] = ((1 + g.standard_normal(D) * 0.02).astype(np.float32),
                        (g.standard_normal(D) * 0.02).astype(np.float32))
        layers.append(lw)
    model = DeviceBert(ctx, layers, D, cfg.heads, cfg.ffn)
    try:
        rnd = lambda *shape: (g.standard_normal(shape) * 0.02).astype(np.float32)
        model.set_embeddings(rnd(cfg.vocab, D), rnd(512, D), (1 + rnd(D), rnd(D)), typ=rnd(2, D))
        s = torch.cuda.Stream()
        sp = s.cuda_stream
        with torch.cuda.stream(s):
            ids = torch.empty(S * L, device="cuda", dtype=torch.int32)
            h = torch.empty((S * L, D), device="cuda")
            pooled, eager = torch.empty((S, D), device="cuda"), torch.empty((S, D), device="cuda")
        torch.cuda.synchronize()

        def encode(out):
            model.embeddings(ids, S, L, h, stream=sp)
            model.embed(h, S, L, out, sp)

        ids.copy_(torch.from_numpy(g.integers(0, cfg.vocab, size=S * L).astype(np.int32)))
        torch.cuda.synchronize()
        encode(eager)  # eager once before capture: the model's buffers, the kernels' LDS limits
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            encode(pooled)
        say(f"{cfg.name} encode of {S} x {L} captured, {REPLAYS} replays")
        for r in range(REPLAYS):
            ids.copy_(torch.from_numpy(g.integers(0, cfg.vocab, size=S * L).astype(np.int32)))
            torch.cuda.synchronize()
            gr.replay()
            torch.cuda.synchronize()
            encode(eager)
            torch.cuda.synchronize()
            assert np.array_equal(bits(pooled), bits(eager)), f"replay {r}"
            assert torch.isfinite(pooled).all()
        del gr
    finally:
        model.close()
