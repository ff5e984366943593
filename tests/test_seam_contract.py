"""The seam contract libenchip keeps for aikit's encoder, exercised through the C ABI.

aikit routes each linear to a backend and, when the backend declines, runs its CPU
path unchanged (encoder/scratch.go:186-218; encoder/backend_use.go:59-83). The Go leaf
(gpu/enchip) maps every non-zero enchip status to that decline. These tests mirror the
reference's wiring tests on the W8A8 capability:

* decline == no backend, bit for bit (TestQ8Backend_declineFallsBackExactly,
  encoder/backend_wiring_test.go:294-315);
* a backend that computes something else moves the output (TestQ8Backend_isLoadBearing,
  :317-334), so the comparison would catch a silently wrong device;
* every decline path (bad activation code, unknown handle, oversize shape, a failed
  device allocation -- forced with a scratch cap, as enccuda degrades on OOM,
  gpu/enccuda/backend.go:141-153) returns non-zero before touching dst;
* one context called from 8 threads at once (encoder.EncodeBatch's workers,
  encoder/model.go:214), each result bit-exact, each failing thread reading its own
  message;
* host calls and device-resident calls on different streams sharing the context's
  quantization scratch.

The CPU path of the mirrored dispatch is the oracle's AVX2 restatement of aikit's W8A8
linear (bit-identical to the scalar oracle, tests/test_oracle.py) -- test
infrastructure standing in for the Go caller, not part of the product.
"""
import ctypes
import threading

import numpy as np
import pytest

import oracle
from aikit_amd import enchip, workloads

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


class EnchipW8A8:
    """The Go leaf's W8A8Backend.MatmulBTW8A8 restated over the raw ABI: weights
    registered once per (array identity), any non-zero status is a decline."""

    def __init__(self, ctx, perturb=False):
        self.ctx, self.lib, self.perturb = ctx, enchip.load(), perturb
        self.handles = {}
        self.calls = self.declines = 0

    def __call__(self, dst, a, wq, ws, bias, act, M, K, N):
        self.calls += 1
        key = id(wq)
        if key not in self.handles:
            w = wq.copy()
            if self.perturb:  # a wrong backend: one weight code off by one
                w[0, 0] = w[0, 0] + 1 if w[0, 0] < 127 else w[0, 0] - 1
            self.handles[key] = self.ctx.register_weight(w, ws)
        h = self.handles[key]
        rc = self.lib.enchip_w8a8_linear(self.ctx.handle, h.handle, a.ctypes.data, M,
                                         None if bias is None else bias.ctypes.data, act, dst.ctypes.data, None)
        if rc != enchip.OK:
            self.declines += 1
            return False
        return True

    def close(self):
        for h in self.handles.values():
            self.ctx.release_weight(h)
        self.handles = {}


class Decline:
    def __call__(self, *args):
        return False


def mmw8a8(backend, dst, a, wq, ws, bias, act, M, K, N, workers):
    """encoder/scratch.go:211-218's dispatch on the W8A8 capability: the backend, or
    on decline the reference's CPU W8A8 path."""
    if backend is not None and backend(dst, a, wq, ws, bias, act, M, K, N):
        return
    dst[:] = oracle.cpu_w8a8_linear(a, wq, ws, bias, act, M, K, N, workers=workers)


def run_mlp(backend, x, layers, workers):
    """Two BERT FFN blocks (up + GELU, down, residual) through the seam."""
    M, D = x.shape
    h = x.copy()
    for up, down in layers:
        I = up[0].shape[0]
        inter = np.empty((M, I), np.float32)
        mmw8a8(backend, inter, h, up[0], up[1], up[2], enchip.ACT_GELU, M, D, I, workers)
        out = np.empty((M, D), np.float32)
        mmw8a8(backend, out, inter, down[0], down[1], down[2], enchip.ACT_NONE, M, I, D, workers)
        h = (h + out).astype(np.float32)
    return h


@pytest.fixture(scope="module")
def mlp():
    g = workloads.rng(31)
    M, D, I = 200, 384, 1536
    x = workloads.activations(g, M, D)
    layers = []
    for _ in range(2):
        up = workloads.quantize_weights((g.standard_normal((I, D)) * 0.02).astype(np.float32)) + (workloads.bias(g, I),)
        down = workloads.quantize_weights((g.standard_normal((D, I)) * 0.02).astype(np.float32)) + (workloads.bias(g, D),)
        layers.append((up, down))
    return x, layers


def test_decline_is_bit_identical_to_no_backend(ctx, workers, mlp):
    x, layers = mlp
    base = run_mlp(None, x, layers, workers)
    declined = run_mlp(Decline(), x, layers, workers)
    assert np.array_equal(bits(base), bits(declined))
    be = EnchipW8A8(ctx)
    try:
        dev = run_mlp(be, x, layers, workers)
        say(f"enchip handled {be.calls - be.declines} of {be.calls} linears")
        assert be.calls == 4 and be.declines == 0
    finally:
        be.close()
    # the device linears are bit-exact, so the seam's output is unchanged by them
    assert np.array_equal(bits(base), bits(dev))


def test_wrong_backend_moves_the_output(ctx, workers, mlp):
    x, layers = mlp
    base = run_mlp(None, x, layers, workers)
    be = EnchipW8A8(ctx, perturb=True)
    try:
        bad = run_mlp(be, x, layers, workers)
    finally:
        be.close()
    assert be.declines == 0
    assert not np.array_equal(bits(base), bits(bad)), "a wrong W8A8 backend changed nothing"


def test_forced_oom_declines_and_falls_back_exactly(ctx, workers, mlp):
    x, layers = mlp
    base = run_mlp(None, x, layers, workers)
    be = EnchipW8A8(ctx)
    ctx.set_scratch_limit(4096)  # far below one linear's quantized activations
    try:
        out = run_mlp(be, x, layers, workers)
        assert be.declines == be.calls == 4
        assert "scratch limit" in ctx._lib.enchip_last_error(ctx.handle).decode()
    finally:
        ctx.set_scratch_limit(0)
        be.close()
    assert np.array_equal(bits(base), bits(out))
    # with the cap lifted the same context serves the calls again
    be = EnchipW8A8(ctx)
    try:
        again = run_mlp(be, x, layers, workers)
        assert be.declines == 0
    finally:
        be.close()
    assert np.array_equal(bits(base), bits(again))


def test_every_decline_leaves_dst_untouched(ctx):
    lib = enchip.load()
    g = workloads.rng(32)
    M, K, N = 64, 768, 1024
    a = workloads.activations(g, M, K)
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    sentinel = np.float32(1234.5)
    try:
        def call(handle=w.handle, act=0, m=M, bias=b):
            dst = np.full((M, N), sentinel, np.float32)
            rc = lib.enchip_w8a8_linear(ctx.handle, handle, a.ctypes.data, m, None if bias is None else bias.ctypes.data,
                                        act, dst.ctypes.data, None)
            return rc, dst, lib.enchip_last_error(ctx.handle).decode()

        cases = {
            "bad act": (dict(act=7), enchip.ERR_ARG, "act"),
            "unknown handle": (dict(handle=w.handle + 999), enchip.ERR_HANDLE, "handle"),
            "negative M": (dict(m=-1), enchip.ERR_ARG, "M="),
            "oversize M": (dict(m=(1 << 31)), enchip.ERR_ARG, "M="),
        }
        for name, (kw, code, text) in cases.items():
            rc, dst, msg = call(**kw)
            say(f"decline {name}: rc={rc} '{msg}'")
            assert rc == code, name
            assert text in msg, (name, msg)
            assert (dst == sentinel).all(), f"{name}: dst was written"
        ctx.set_scratch_limit(4096)
        try:
            rc, dst, msg = call()
        finally:
            ctx.set_scratch_limit(0)
        assert rc == enchip.ERR_OOM and "scratch limit" in msg and (dst == sentinel).all()
        # batch: an op with the wrong K is refused before any op runs
        w2 = ctx.register_weight(*workloads.int8_weights(g, 256, 512))
        try:
            d1 = np.full((M, N), sentinel, np.float32)
            d2 = np.full((M, 256), sentinel, np.float32)
            ops = (enchip.EnchipOp * 2)(enchip.EnchipOp(w.handle, None, 0, d1.ctypes.data),
                                        enchip.EnchipOp(w2.handle, None, 0, d2.ctypes.data))
            rc = lib.enchip_w8a8_batch(ctx.handle, a.ctypes.data, M, K, ctypes.cast(ops, ctypes.c_void_p), 2)
            assert rc == enchip.ERR_ARG and "K=512" in lib.enchip_last_error(ctx.handle).decode()
            assert (d1 == sentinel).all() and (d2 == sentinel).all()
        finally:
            ctx.release_weight(w2)
        # and a valid call on the same context still works, bit-exact
        rc, dst, _ = call()
        assert rc == enchip.OK
        assert np.array_equal(bits(dst), bits(oracle.w8a8_linear(a, wq, ws, b, 0, M, K, N)))
    finally:
        ctx.release_weight(w)


def test_eight_threads_on_one_context(ctx, workers):
    # encoder.EncodeBatch calls the backend from worker goroutines (encoder/model.go:214);
    # ctypes drops the GIL around each foreign call, so these calls overlap in the library.
    lib = enchip.load()
    g = workloads.rng(33)
    K = 768
    shapes = [(37 + 61 * t, 512 + 256 * (t % 4)) for t in range(8)]
    wts = [workloads.int8_weights(g, N, K) for _, N in shapes]
    hs = [ctx.register_weight(wq, ws) for wq, ws in wts]
    inputs = [workloads.activations(g, M, K) for M, _ in shapes]
    biases = [workloads.bias(g, N) for _, N in shapes]
    results, errors = {}, {}
    start = threading.Barrier(8)

    def worker(t):
        try:
            M, N = shapes[t]
            start.wait()
            outs = []
            for it in range(6):
                dst = np.empty((M, N), np.float32)
                rc = lib.enchip_w8a8_linear(ctx.handle, hs[t].handle, inputs[t].ctypes.data, M,
                                            biases[t].ctypes.data, it % 2, dst.ctypes.data, None)
                assert rc == enchip.OK, lib.enchip_last_error(ctx.handle).decode()
                outs.append(dst)
                # a failing call of this thread's own: its message must be its own
                bad_act = 40 + t
                dummy = np.empty(1, np.float32)
                rc = lib.enchip_w8a8_linear(ctx.handle, hs[t].handle, inputs[t].ctypes.data, M, None, bad_act,
                                            dummy.ctypes.data, None)
                msg = lib.enchip_last_error(ctx.handle).decode()
                assert rc == enchip.ERR_ARG and f"bad act {bad_act}" in msg, msg
            results[t] = outs
        except BaseException as exc:  # reported by the main thread
            errors[t] = exc

    try:
        threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
        say("8 threads x 6 linears (+ 6 failing calls) on one context")
        for th in threads:
            th.start()
        for th in threads:
            th.join(timeout=100)
        assert not errors, errors
        for t, (M, N) in enumerate(shapes):
            wq, ws = wts[t]
            want = [oracle.cpu_w8a8_linear(inputs[t], wq, ws, biases[t], act, M, K, N, workers=workers)
                    for act in (0, 1)]
            for it, got in enumerate(results[t]):
                assert np.array_equal(bits(got), bits(want[it % 2])), f"thread {t} call {it}"
    finally:
        for h in hs:
            ctx.release_weight(h)


def test_host_and_device_calls_on_different_streams(ctx, workers):
    # enchip_w8a8_linear_dev on a caller stream quantizes into the context scratch and
    # returns before its GEMM has read the codes; a host call (the context stream)
    # issued right after reuses that scratch. The library orders the two on the device.
    import torch

    g = workloads.rng(34)
    M, K, N = 32768, 3072, 768
    a = workloads.activations(g, M, K)
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    a2 = workloads.activations(g, 4096, K)
    w = ctx.register_weight(wq, ws)
    try:
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
            dd = torch.empty((M, N), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        say("linear_dev M=32768 K=3072 on a caller stream, then a host linear on the context stream")
        for _ in range(3):
            ctx.linear_dev(w, da.data_ptr(), M, db.data_ptr(), 0, dd.data_ptr(), st.cuda_stream)
            host = ctx.linear(w, a2, bias=b, act=1)
        torch.cuda.synchronize()
        rows = np.concatenate([np.arange(256), np.arange(M - 256, M)])
        want = oracle.cpu_w8a8_linear(a[rows], wq, ws, b, 0, len(rows), K, N, workers=workers)
        assert np.array_equal(bits(dd.cpu().numpy()[rows]), bits(want))
        want2 = oracle.cpu_w8a8_linear(a2, wq, ws, b, 1, 4096, K, N, workers=workers)
        assert np.array_equal(bits(host), bits(want2))
    finally:
        ctx.release_weight(w)


# ---- the weight-only seam, encoder.Q8Backend.MatmulBTQ8 (encoder/backend_use.go:59-83)

MIN_GPU_FLOPS = 1 << 20  # gpu/enccuda/backend.go:75, the threshold the Go leaf keeps


class EnchipQ8:
    """The Go leaf's MatmulBTQ8 restated over the raw ABI (gpu/enchip/backend.go): small
    shapes decline, weights are registered once per weight array (the leaf keys by
    (ptr, len); here by the array object), activations are passed on every call, any
    non-zero status is a decline."""

    def __init__(self, ctx):
        self.ctx, self.lib = ctx, enchip.load()
        self.handles = {}

    def __call__(self, dst, a, wq, ws, M, K, N):
        if 2 * M * K * N < MIN_GPU_FLOPS or M <= 0 or K <= 0 or N <= 0:
            return False
        key = id(wq)
        if key not in self.handles:
            try:
                self.handles[key] = self.ctx.register_weight(wq, ws)
            except enchip.EnchipError:
                return False
        rc = self.lib.enchip_matmul_bt_q8(self.ctx.handle, self.handles[key].handle, a.ctypes.data, M,
                                          dst.ctypes.data)
        return rc == enchip.OK

    def close(self):
        for h in self.handles.values():
            self.ctx.release_weight(h)
        self.handles = {}


def mmq8(backend, dst, a, wq, ws, M, K, N):
    """encoder/scratch.go:211-218: the backend, or on decline matmulBTQ8Into's CPU path
    (widen with DequantizeRowsInt8Into, then an f32 product; numpy's f32 product stands
    in for matmulBTInto's loop order here)."""
    if backend is not None and backend(dst, a, wq, ws, M, K, N):
        return True
    with np.errstate(invalid="ignore"):  # an infinite scale widens zero codes to NaN
        dst[:] = a @ oracle.dequant_rows_i8(wq, ws, N, K).T
    return False


def test_q8_weight_residency_and_activations_never_cached(ctx):
    # gpu/enccuda/backend_test.go:291-369 (TestEncCUDA_q8WeightResidency): one
    # registration per distinct weight, a re-used weight hits, two weights give two
    # results, and a new activation against the cached weight changes the result and
    # meets the gate.
    g = workloads.rng(12)
    M, K, N = 128, 768, 768
    a1 = g.standard_normal((M, K)).astype(np.float32)
    a2 = g.standard_normal((M, K)).astype(np.float32)
    w1 = g.integers(-127, 128, size=(N, K)).astype(np.int8)
    w2 = g.integers(-127, 128, size=(N, K)).astype(np.int8)
    ws = np.full(N, 0.003, np.float32)
    be = EnchipQ8(ctx)
    try:
        d1, d2, d3, d4 = (np.empty((M, N), np.float32) for _ in range(4))
        assert mmq8(be, d1, a1, w1, ws, M, K, N) and len(be.handles) == 1
        assert mmq8(be, d2, a1, w2, ws, M, K, N) and len(be.handles) == 2
        assert mmq8(be, d3, a1, w1, ws, M, K, N) and len(be.handles) == 2
        assert np.array_equal(bits(d1), bits(d3))
        assert not np.array_equal(d1, d2)
        assert mmq8(be, d4, a2, w1, ws, M, K, N)
        assert not np.array_equal(d1, d4), "a new activation gave the cached result"
        worst = oracle.matmul_bt_worst_rel(d4, oracle.matmul_bt_q8_f64(a2, w1, ws, M, K, N))
        say(f"  new activation against the cached weight: worst {worst:.3g}")
        assert worst <= 2e-4
    finally:
        be.close()


def test_q8_declines_leave_dst_to_the_cpu_path(ctx):
    # below the threshold (backend_test.go:250, "tiny/declined") and for a weight with an
    # infinite scale (whose zero codes the CPU path turns into NaN) the backend declines
    # without writing dst, and the CPU path's result is what the caller gets.
    g = workloads.rng(13)
    be = EnchipQ8(ctx)
    try:
        M, K, N = 8, 32, 32
        a = g.standard_normal((M, K)).astype(np.float32)
        wq = g.integers(-127, 128, size=(N, K)).astype(np.int8)
        ws = np.full(N, 0.002, np.float32)
        dst = np.full((M, N), 7.0, np.float32)
        assert not be(dst, a, wq, ws, M, K, N) and np.all(dst == 7.0) and not be.handles
        assert not mmq8(be, dst, a, wq, ws, M, K, N)
        assert np.array_equal(bits(dst), bits(a @ oracle.dequant_rows_i8(wq, ws, N, K).T))

        M, K, N = 64, 256, 128
        a = g.standard_normal((M, K)).astype(np.float32)
        wq = g.integers(-127, 128, size=(N, K)).astype(np.int8)
        wq[0, 3] = 0
        ws = np.full(N, 0.002, np.float32)
        ws[0] = np.inf
        dst = np.full((M, N), 7.0, np.float32)
        assert not be(dst, a, wq, ws, M, K, N) and np.all(dst == 7.0)
        assert not mmq8(be, dst, a, wq, ws, M, K, N)
        assert np.all(np.isnan(dst[:, 0]))  # 0 * inf in the CPU path's widened weight
    finally:
        be.close()


def test_q8_eight_threads_on_one_context(ctx):
    # encoder.EncodeBatch's workers (encoder/model.go:214) on the weight-only seam: 8
    # threads, each alternating weight-only and W8A8 calls on its own weight through one
    # context. Every weight-only result is bit-identical to the same call made alone
    # (the kernels' sums run in a fixed order) and within the gate, and the W8A8 calls in
    # between, which share the context's device buffers, leave them undisturbed.
    lib = enchip.load()
    g = workloads.rng(35)
    shapes = [(64 + 96 * t, 768 if t % 2 else 3072, 256 * (1 + t % 3)) for t in range(8)]
    wts = [(g.integers(-127, 128, size=(N, K)).astype(np.int8), np.full(N, 0.002, np.float32))
           for _, K, N in shapes]
    hs = [ctx.register_weight(wq, ws) for wq, ws in wts]
    inputs = [g.standard_normal((M, K)).astype(np.float32) for M, K, _ in shapes]
    alone = [ctx.matmul_bt_q8(h, a) for h, a in zip(hs, inputs)]
    results, errors = {}, {}
    start = threading.Barrier(8)

    def worker(t):
        try:
            M, K, N = shapes[t]
            start.wait()
            outs = []
            for it in range(6):
                dst = np.empty((M, N), np.float32)
                rc = lib.enchip_matmul_bt_q8(ctx.handle, hs[t].handle, inputs[t].ctypes.data, M, dst.ctypes.data)
                assert rc == enchip.OK, lib.enchip_last_error(ctx.handle).decode()
                outs.append(dst)
                d8 = np.empty((M, N), np.float32)
                rc = lib.enchip_w8a8_linear(ctx.handle, hs[t].handle, inputs[t].ctypes.data, M, None, 0,
                                            d8.ctypes.data, None)
                assert rc == enchip.OK, lib.enchip_last_error(ctx.handle).decode()
            results[t] = outs
        except BaseException as exc:  # reported by the main thread
            errors[t] = exc

    try:
        threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
        say("8 threads x 6 weight-only + 6 W8A8 calls on one context")
        for th in threads:
            th.start()
        for th in threads:
            th.join(timeout=100)
        assert not errors, errors
        for t, (M, K, N) in enumerate(shapes):
            for it, got in enumerate(results[t]):
                assert np.array_equal(bits(got), bits(alone[t])), f"thread {t} call {it}"
            wq, ws = wts[t]
            rows = slice(0, 32)
            ref = oracle.matmul_bt_q8_f64(np.ascontiguousarray(inputs[t][rows]), wq, ws, 32, K, N)
            assert oracle.matmul_bt_worst_rel(alone[t][rows], ref) <= 2e-4
    finally:
        for h in hs:
            ctx.release_weight(h)
