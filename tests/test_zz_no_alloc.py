"""enchip_w8a8_linear_noalloc_dev: the allocation-free variant of enchip_w8a8_linear_dev,
through the C ABI, against that entry point's output (bit for bit) on two calls in a row
per kernel route, the second with a smaller input, and with device memory unchanged by
its calls on a fresh context."""
import ctypes

import numpy as np
import pytest

from aikit_amd import enchip, workloads

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# (K, N, act, [M first, M second]): the persistent GEMM on fragment-major codes (N % 4 == 0,
# M > 32), the one-launch small-M kernel (M <= 32, K <= 4096), the general GEMM on row-major
# codes (N % 4 != 0)
ROUTES = [(768, 3072, 1, [4096, 300]), (3072, 768, 0, [8192, 1000]), (768, 768, 1, [32, 16]),
          (768, 3072, 0, [16, 1]), (3072, 768, 1, [24, 9]), (384, 1001, 1, [777, 64])]


def test_noalloc_matches_linear_dev_on_two_calls():
    import torch

    lib = enchip.load()
    ctx = enchip.Context(0)  # fresh: its own growable scratch is still empty
    g = workloads.rng(4242)
    cases, weights = [], []
    try:
        # every weight, input and output exists before the first no-alloc call
        for K, N, act, Ms in ROUTES:
            wq, ws = workloads.int8_weights(g, N, K)
            w = ctx.register_weight(wq, ws)
            weights.append(w)
            b = torch.from_numpy(workloads.bias(g, N)).cuda()
            for M in Ms:  # the second call of a route has the smaller input
                a = torch.from_numpy(workloads.activations(g, M, K)).cuda()
                a[M // 2] = 0
                cases.append((w, b, act, M, K, N, a, torch.full((M, N), 7.0, device="cuda"),
                              torch.full((M, N), 7.0, device="cuda")))
        w0, b0, act0, _, K0, _, a0, got0, _ = cases[0]
        rc = lib.enchip_w8a8_linear_noalloc_dev(ctx.handle, w0.handle, a0.data_ptr(), 1, b0.data_ptr(), act0,
                                                got0.data_ptr(), None)  # warms the launch path
        assert rc == enchip.OK, lib.enchip_last_error(ctx.handle).decode()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for w, b, act, M, K, N, a, got, _ in cases:
            say(f"no-alloc linear M={M} K={K} N={N} act={act} ({ctx.gemm_kernel_name(w, M, act)})")
            rc = lib.enchip_w8a8_linear_noalloc_dev(ctx.handle, w.handle, a.data_ptr(), M, b.data_ptr(), act,
                                                    got.data_ptr(), None)
            assert rc == enchip.OK, lib.enchip_last_error(ctx.handle).decode()
            torch.cuda.synchronize()
            assert torch.cuda.mem_get_info()[0] == free0, "a no-alloc call changed the device's free memory"
        # the existing entry point (which grows the context's scratch) on the same inputs
        for w, b, act, M, K, N, a, got, want in cases:
            ctx.linear_dev(w, a.data_ptr(), M, b.data_ptr(), act, want.data_ptr())
            torch.cuda.synchronize()
            assert np.array_equal(bits(got.cpu().numpy()), bits(want.cpu().numpy())), (M, K, N)
    finally:
        for w in weights:
            ctx.release_weight(w)
        ctx.close()


def test_noalloc_declines_beyond_its_scratch():
    import torch

    lib = enchip.load()
    ctx = enchip.Context(0)
    try:
        g = workloads.rng(4243)
        K, N = 768, 1024
        w = ctx.register_weight(*workloads.int8_weights(g, N, K))
        try:
            M = 45000  # 45056 rows x 768 = 33 MiB of codes > 32 MiB
            a = torch.zeros((M, K), device="cuda")
            d = torch.full((M, N), 7.0, device="cuda")
            torch.cuda.synchronize()
            say(f"no-alloc linear M={M} K={K}: past the scratch")
            rc = lib.enchip_w8a8_linear_noalloc_dev(ctx.handle, w.handle, a.data_ptr(), M, None, 0, d.data_ptr(), None)
            assert rc == enchip.ERR_ARG
            assert "no-alloc scratch" in lib.enchip_last_error(ctx.handle).decode()
            rc = lib.enchip_w8a8_linear_noalloc_dev(ctx.handle, w.handle, a.data_ptr(), (1 << 18) + 1, None, 0,
                                                    d.data_ptr(), None)
            assert rc == enchip.ERR_ARG
            torch.cuda.synchronize()
            assert bool((d == 7.0).all().item()), "a declined call wrote dst"
        finally:
            ctx.release_weight(w)
    finally:
        ctx.close()


def test_noalloc_calls_on_two_streams_and_contexts_stay_exact():
    """Calls enqueued back to back on two streams of two contexts share the device's
    array; the library's per-device event orders them, so each output equals
    enchip_w8a8_linear_dev's bit for bit (without it, the next call's quantizer would
    overwrite codes a running GEMM still reads)."""
    import torch

    lib = enchip.load()
    ctxs = [enchip.Context(0), enchip.Context(0)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    g = workloads.rng(4244)
    K, N, M, n_calls = 3072, 768, 4096, 6
    wq, ws = workloads.int8_weights(g, N, K)
    ws_h = [c.register_weight(wq, ws) for c in ctxs]
    try:
        b = torch.from_numpy(workloads.bias(g, N)).cuda()
        acts = [torch.from_numpy(workloads.activations(g, M, K)).cuda() for _ in range(n_calls)]
        outs = [torch.full((M, N), 7.0, device="cuda") for _ in range(n_calls)]
        torch.cuda.synchronize()
        say(f"no-alloc linear M={M} K={K} N={N}: {n_calls} calls alternating over 2 streams / 2 contexts")
        for i in range(n_calls):
            c, w, s = ctxs[i % 2], ws_h[i % 2], streams[i % 2]
            rc = lib.enchip_w8a8_linear_noalloc_dev(c.handle, w.handle, acts[i].data_ptr(), M, b.data_ptr(), 0,
                                                    outs[i].data_ptr(), ctypes.c_void_p(s.cuda_stream))
            assert rc == enchip.OK, lib.enchip_last_error(c.handle).decode()
        torch.cuda.synchronize()
        for i in range(n_calls):
            want = torch.empty((M, N), device="cuda")
            ctxs[0].linear_dev(ws_h[0], acts[i].data_ptr(), M, b.data_ptr(), 0, want.data_ptr())
            torch.cuda.synchronize()
            assert np.array_equal(bits(outs[i].cpu().numpy()), bits(want.cpu().numpy())), i
    finally:
        for c, w in zip(ctxs, ws_h):
            c.release_weight(w)
            c.close()
