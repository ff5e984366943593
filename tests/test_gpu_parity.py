"""GPU parity: libenchip.so on the MI355X against the CPU oracle, through the C ABI.

The bar: quantized activations and int32 accumulators
bit-exact; dequantized f32 outputs within 1e-5 max relative error per GEMM. The
epilogue restates the reference's float32 operation order, so the f32 outputs
are also asserted bit-identical, which is stronger.

Mirrors the reference's device tests: TestCUDA_vitQuantRows (byte-exact incl. the
zero row, gpu/cuda_vit_test.go:154-226), TestCUDA_vitGEMMs (exact int reference,
:228-310), TestCUDA_gemmTiledMatchesUntiled (bit-identical across shapes,
:720-800), TestW8A8Batch_bitIdenticalToPerOp and TestW8A8Reblock_matchesPerRow
(linalg/batch_test.go:13-66,102-135).
"""
import os

import numpy as np
import pytest

import oracle
from aikit_amd import enchip, workloads

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "w8a8_golden.npz")
REL_TOL = 1e-5  # the W8A8 parity bar: dequantized f32 outputs, max relative error per GEMM


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def assert_f32_parity(got, want, what):
    """Bit-identical (NaN payloads aside), and the 1e-5 max rel error bar (REL_TOL) over
    the finite values (infinities must match exactly)."""
    assert got.shape == want.shape, what
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all(), f"{what}: NaN mismatch"
    g, w = got[~nan], want[~nan]
    fin = np.isfinite(w)
    assert (g[~fin] == w[~fin]).all(), f"{what}: infinity mismatch"
    gf, wf = g[fin], w[fin]
    denom = np.maximum(np.abs(wf), np.finfo(np.float32).tiny)
    rel = float(np.max(np.abs(gf.astype(np.float64) - wf) / denom)) if gf.size else 0.0
    assert rel <= REL_TOL, f"{what}: max rel err {rel:.3g} > {REL_TOL}"
    mism = np.flatnonzero(bits(g) != bits(w))
    assert mism.size == 0, f"{what}: {mism.size} elements differ in bits (first at {mism[:5]})"


# ------------------------------------------------------------------ quantization
def test_quant_rows_golden(ctx):
    d = np.load(GOLDEN, allow_pickle=False)
    names, off, rows = d["quant_names"], d["quant_offsets"], d["quant_rows"]
    for i, name in enumerate(names):
        r = rows[off[i]:off[i + 1]][None, :]
        say(f"quant golden {name} K={r.shape[1]}")
        q, s = ctx.quant_rows(r)
        assert (q[0] == d["quant_codes_act"][off[i]:off[i + 1]]).all(), name
        assert bits(s) [0] == bits(d["quant_scales_act"][i:i + 1])[0], name


@pytest.mark.parametrize("K", [1, 3, 4, 64, 97, 384, 768, 1000, 1024, 1536, 3072, 4096, 4100, 5000])
def test_quant_rows_matches_oracle(ctx, K):
    # gpu/cuda_vit_test.go:154-226 shape family, plus the vector/scalar kernel edges.
    g = workloads.rng(100 + K)
    M = 37
    a = workloads.activations(g, M, K)
    a[5] = 0
    a[7] *= np.float32(1e-3)
    a[9, : min(K, 4)] = [127, -2.5, 0.5, 1.5][: min(K, 4)]
    say(f"quant M={M} K={K}")
    q, s = ctx.quant_rows(a)
    wq, ws = oracle.quantize_activations(a, M, K)
    assert (q == wq).all()
    assert (bits(s) == bits(ws)).all()
    assert s[5] == 0 and (q[5] == 0).all()


def test_quant_rows_dev_matches_host(ctx):
    import torch

    g = workloads.rng(7)
    M, K = 1000, 768
    a = workloads.activations(g, M, K)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        da = torch.from_numpy(a).cuda()
        dq = torch.empty((M, K), dtype=torch.int8, device="cuda")
        ds = torch.empty(M, dtype=torch.float32, device="cuda")
        say("quant_rows_dev M=1000 K=768")
        ctx.quant_rows_dev(da.data_ptr(), M, K, dq.data_ptr(), ds.data_ptr(), st.cuda_stream)
    torch.cuda.synchronize()
    wq, ws = oracle.quantize_activations(a, M, K)
    assert (dq.cpu().numpy() == wq).all()
    assert (bits(ds.cpu().numpy()) == bits(ws)).all()


# ------------------------------------------------------------------ GEMM + epilogue
def _linear_case(ctx, M, K, N, act, with_bias, seed, small_m=32, zero_rows=(0,)):
    g = workloads.rng(seed)
    a = workloads.activations(g, M, K)
    for r in zero_rows:
        if r < M:
            a[r] = 0
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N) if with_bias else None
    w = ctx.register_weight(wq, ws)
    try:
        ctx.set_small_m(small_m)
        dst, acc = ctx.linear(w, a, bias=b, act=act, want_acc=True)
    finally:
        ctx.set_small_m(32)
        ctx.release_weight(w)
    return a, wq, ws, b, dst, acc


REF_SHAPES = [(1, 1, 1), (16, 16, 16), (17, 47, 33), (64, 129, 96), (129, 1152, 65),  # gpu/cuda_vit_test.go:720-800
              (1, 16, 8), (16, 32, 32), (17, 65, 33),  # gpu/cuda_vit_test.go:233 (M,K,N)
              (33, 768, 300), (257, 200, 513), (300, 3072, 768), (1000, 96, 1000)]


@pytest.mark.parametrize("M,K,N", REF_SHAPES)
@pytest.mark.parametrize("act,with_bias", [(0, False), (1, True)])
def test_linear_matches_oracle(ctx, M, K, N, act, with_bias):
    say(f"linear M={M} K={K} N={N} act={act} bias={with_bias}")
    a, wq, ws, b, dst, acc = _linear_case(ctx, M, K, N, act, with_bias, seed=M * 7 + K * 3 + N)
    aq, a_s = oracle.quantize_activations(a, M, K)
    want_acc = (aq.astype(np.int64) @ wq.astype(np.int64).T).astype(np.int32)
    assert np.array_equal(acc, want_acc), "int32 accumulators differ"
    want = oracle.w8a8_linear(a, wq, ws, b, act, M, K, N)
    assert_f32_parity(dst, want, f"linear {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(1, 384, 131104), (7, 100, 140001), (32, 200, 131200), (3, 768, 40000)])
@pytest.mark.parametrize("act,with_bias", [(0, False), (1, True)])
def test_wide_small_m_kernel_matches_oracle(ctx, M, K, N, act, with_bias):
    # N wide enough (>= 8 32-channel groups per CU, or >= 4 with K <= 1024, on MI355X) for the
    # one-wavefront-per-group small-M kernel; ragged N and K below one 12-fragment batch.
    g = workloads.rng(M * 11 + K + N)
    wq, ws = workloads.int8_weights(g, 64, K)
    w = ctx.register_weight(np.resize(wq, (N, K)), np.resize(ws, N))
    name = ctx.gemm_kernel_name(w, M, act)
    ctx.release_weight(w)
    say(f"wide small-M linear M={M} K={K} N={N} act={act} via {name}")
    assert name.startswith("enchip::gemv_w8a8_wide<"), name
    a, wq, ws, b, dst, acc = _linear_case(ctx, M, K, N, act, with_bias, seed=M * 13 + K + N)
    aq, _ = oracle.quantize_activations(a, M, K)
    want_acc = (aq.astype(np.int64) @ wq.astype(np.int64).T).astype(np.int32)
    assert np.array_equal(acc, want_acc), "int32 accumulators differ"
    assert_f32_parity(dst, oracle.w8a8_linear(a, wq, ws, b, act, M, K, N), f"wide linear {M}x{K}x{N}")


@pytest.mark.parametrize("M", [1, 2, 5, 16, 31, 32])
@pytest.mark.parametrize("K,N", [(768, 768), (768, 3072), (100, 50)])
def test_small_m_kernel_matches_gemm_kernel(ctx, M, K, N):
    # Kernel choice is numerically inert (cf. TestParallelWidth_bitIdentical,
    # linalg/width_test.go:13): the small-M path and the tiled GEMM give the same bits.
    say(f"small-M vs GEMM M={M} K={K} N={N}")
    _, _, _, _, d1, acc1 = _linear_case(ctx, M, K, N, 1, True, seed=M + K + N, small_m=32)
    a, wq, ws, b, d2, acc2 = _linear_case(ctx, M, K, N, 1, True, seed=M + K + N, small_m=0)
    assert np.array_equal(acc1, acc2)
    assert np.array_equal(bits(d1), bits(d2))
    assert_f32_parity(d1, oracle.w8a8_linear(a, wq, ws, b, 1, M, K, N), "small-M")


def test_batch_bit_identical_to_per_op(ctx, workers):
    # linalg/batch_test.go:13-66: a shared-activation batch equals one call per op, and
    # each op equals the reference's MatmulBTW8A8Batch op (linalg/quant.go:319-370): the
    # oracle's W8A8 linear, bit for bit; ops with and without a bias, one with GELU.
    g = workloads.rng(21)
    for M, K, Ns in [(300, 768, (768, 768, 768, 3072)), (16, 768, (768, 3072)), (2048, 384, (1152, 1536))]:
        a = workloads.activations(g, M, K)
        a[min(3, M - 1)] = 0
        wts = [workloads.int8_weights(g, N, K) for N in Ns]
        bs = [workloads.bias(g, N) if i % 2 == 0 else None for i, N in enumerate(Ns)]
        acts = [1 if i == len(Ns) - 1 else 0 for i in range(len(Ns))]
        handles = [ctx.register_weight(wq, s_) for wq, s_ in wts]
        try:
            say(f"batch of {len(Ns)} ops M={M} K={K} N={Ns}")
            ops = list(zip(handles, bs, acts))
            outs = ctx.batch(a, ops)
            for i, ((h, b, act), (wq, ws)) in enumerate(zip(ops, wts)):
                # the AVX2 restatement, bit-identical to the scalar oracle (test_oracle.py)
                want = oracle.cpu_w8a8_linear(a, wq, ws, b, act, M, K, h.N, workers=workers)
                assert_f32_parity(outs[i], want, f"batch op {i}")
                single = ctx.linear(h, a, bias=b, act=act)
                assert np.array_equal(bits(outs[i]), bits(single)), f"op {i}"
        finally:
            for h in handles:
                ctx.release_weight(h)


def test_row_invariance(ctx):
    # linalg/batch_test.go:102-135: a row's output does not depend on the other rows.
    g = workloads.rng(22)
    M, K, N = 777, 768, 1024
    a = workloads.activations(g, M, K)
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    try:
        say("row invariance")
        full = ctx.linear(w, a, bias=b, act=1)
        for lo, hi in [(0, 1), (5, 37), (300, 777)]:
            part = ctx.linear(w, a[lo:hi], bias=b, act=1)
            assert np.array_equal(bits(part), bits(full[lo:hi]))
    finally:
        ctx.release_weight(w)


def test_linear_dev_matches_host(ctx):
    import torch

    g = workloads.rng(23)
    M, K, N = 2048, 768, 2304
    a = workloads.activations(g, M, K)
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    try:
        host = ctx.linear(w, a, bias=b, act=1)
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
            dd = torch.empty((M, N), dtype=torch.float32, device="cuda")
            say("linear_dev 2048x768x2304")
            ctx.linear_dev(w, da.data_ptr(), M, db.data_ptr(), 1, dd.data_ptr(), st.cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(bits(dd.cpu().numpy()), bits(host))
    finally:
        ctx.release_weight(w)


def test_golden_linears(ctx):
    d = np.load(GOLDEN, allow_pickle=False)
    for i in range(3):
        a, wq, ws = d[f"lin{i}_a"], d[f"lin{i}_wq"], d[f"lin{i}_ws"]
        b = d[f"lin{i}_bias"]
        b = b if b.size else None
        w = ctx.register_weight(wq, ws)
        try:
            say(f"golden linear {i}")
            got = ctx.linear(w, a, bias=b, act=int(d[f"lin{i}_act"]))
        finally:
            ctx.release_weight(w)
        assert np.array_equal(bits(got), bits(d[f"lin{i}_dst"]))


# ------------------------------------------------------------------ benchmark configs at full size
def _full_config(ctx, workers, M, K, N, act, seed, sample_rows=None):
    g = workloads.rng(seed)
    a = workloads.activations(g, M, K)
    a[1] = 0
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    try:
        say(f"full config M={M} K={K} N={N} act={act}")
        dst = ctx.linear(w, a, bias=b, act=act)
    finally:
        ctx.release_weight(w)
    rows = np.arange(M) if sample_rows is None else sample_rows
    want = oracle.cpu_w8a8_linear(a[rows], wq, ws, b, act, len(rows), K, N, workers=workers)
    assert_f32_parity(dst[rows], want, f"config {M}x{K}x{N}")


def test_config2_isolated_linear(ctx, workers):
    c = workloads.LINEAR_CFG2
    _full_config(ctx, workers, c["M"], c["K"], c["N"], c["act"], seed=2)


@pytest.mark.parametrize("N", [768, 3072])
def test_config3_small_m(ctx, workers, N):
    _full_config(ctx, workers, 16, 768, N, 0, seed=3)


@pytest.mark.parametrize("name,K,N,act", workloads.BERT_BASE.linears())
def test_config4_bert_base_linears(ctx, workers, name, K, N, act):
    # Full M = 64*512 rows; every row is checked.
    _full_config(ctx, workers, workloads.BERT_BASE.tokens, K, N, act, seed=40 + N + K)


@pytest.mark.parametrize("name,K,N,act", workloads.XLMR_LARGE_CE.linears())
def test_config5_xlmr_linears(ctx, workers, name, K, N, act):
    # M = 128*512 = 65536 rows computed on the device; 1024 rows (the first 512
    # and 512 random) are checked -- each output row depends only on its own
    # input row (row invariance, tested above).
    M = workloads.XLMR_LARGE_CE.tokens
    g = np.random.Generator(np.random.PCG64(5))
    rows = np.concatenate([np.arange(512), np.sort(g.choice(np.arange(512, M), 512, replace=False))])
    _full_config(ctx, workers, M, K, N, act, seed=50 + N + K, sample_rows=rows)


def test_device_ceilings_coherent(ctx):
    # gpu/roofline_test.go:57-140 asserts the probes are coherent, not that the
    # device is fast: each ceiling is positive and below the nameplate with margin.
    say("roofline probes")
    c = ctx.probe_ceilings()
    print(f"[ceilings] {c}", flush=True)
    assert 1000 < c["hbm_read_gbps"] < 12000
    assert 1000 < c["hbm_write_gbps"] < 12000
    assert 500 < c["mfma_i8_tops"] < 6000
    # operands that switch the multipliers cannot issue faster than constant ones, and each
    # probe's shader clock is within the part's range (MI355X: up to 2.4 GHz)
    assert 500 < c["mfma_i8_data_tops"] < 1.05 * c["mfma_i8_tops"]
    assert 300 < c["mfma_i8_data_mhz"] < 1.05 * c["mfma_i8_mhz"] and c["mfma_i8_mhz"] < 3000
    # the rate follows the clock: 2048 int8 ops per clock per SIMD at the measured clock
    # bounds each probe (4 SIMDs per CU)
    cus = ctx.device_info()["num_cus"]
    for tops, mhz in ((c["mfma_i8_tops"], c["mfma_i8_mhz"]), (c["mfma_i8_data_tops"], c["mfma_i8_data_mhz"])):
        assert tops < 1.05 * 2048 * 4 * cus * mhz * 1e6 / 1e12
    # non-packed f32 lane-operations: at most two wavefronts' instructions per SIMD per
    # 4-cycle issue slot, 32 lanes per clock x 1024 SIMDs x 2.4 GHz = 78.6 T
    assert 5 < c["valu_f32_tops"] < 80


@pytest.mark.parametrize("M,K,Ns,small_m", [(1500, 768, (2304, 768), 32), (300, 1024, (2304, 768), 32),
                                             (77, 1536, (2304, 768), 32), (16, 768, (768, 3072), 32),
                                             (16, 768, (768, 3072), 0), (256, 384, (16384,), 32)])
def test_pre_quantized_matches_oracle(ctx, workers, M, K, Ns, small_m):
    # linalg/quant.go:215-234 MatmulBTW8A8Pre: quantize once (QuantizeActivationsInto)
    # and reuse the codes across weights. pre_dev takes row-major codes: the persistent
    # kernel without AF for M above the small-M limit, the small-M kernels at config 3's
    # M=16 (and, with the limit lowered to 0, the persistent kernel at M=16), the
    # persistent kernel at an ann.FlatI8 M=256 batch. Each output is checked against
    # the oracle's W8A8 linear and against the fused call.
    import torch

    g = workloads.rng(24 + K + M)
    a = workloads.activations(g, M, K)
    a[3] = 0
    wts = [workloads.int8_weights(g, N, K) for N in Ns]
    bs = [workloads.bias(g, N) for N in Ns]
    acts = [i % 2 for i in range(len(Ns))]
    hs = [ctx.register_weight(wq, s) for wq, s in wts]
    ctx.set_small_m(small_m)
    try:
        for h in hs:
            name = ctx.gemm_kernel_name(h, M, 0)
            assert ("gemv" in name) == (M <= small_m), name
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            da = torch.from_numpy(a).cuda()
            ldq = (K + 63) // 64 * 64
            dq = torch.zeros((M, ldq), dtype=torch.int8, device="cuda")
            ds = torch.empty(M, dtype=torch.float32, device="cuda")
            say(f"quant_rows_dev + pre_dev M={M} K={K} N={Ns} small_m={small_m}")
            ctx.quant_rows_dev(da.data_ptr(), M, K, dq.data_ptr(), ds.data_ptr(), st.cuda_stream, ldq=ldq)
            outs = []
            for h, b, act in zip(hs, bs, acts):
                db = torch.from_numpy(b).cuda()
                dd = torch.empty((M, h.N), dtype=torch.float32, device="cuda")
                ctx.pre_dev(h, dq.data_ptr(), ldq, M, ds.data_ptr(), db.data_ptr(), act, dd.data_ptr(), st.cuda_stream)
                outs.append((dd, db))
        torch.cuda.synchronize()
        aq, asc = oracle.quantize_activations(a, M, K)
        assert np.array_equal(dq.cpu().numpy()[:, :K].reshape(-1), aq.reshape(-1))
        assert np.array_equal(bits(ds.cpu().numpy()), bits(asc))
        for (dd, _), (wq, ws), h, b, act in zip(outs, wts, hs, bs, acts):
            got = dd.cpu().numpy()
            want = oracle.cpu_w8a8_linear(a, wq, ws, b, act, M, K, h.N, workers=workers)
            assert_f32_parity(got, want, f"pre_dev N={h.N}")
            assert np.array_equal(bits(got), bits(ctx.linear(h, a, bias=b, act=act)))
    finally:
        ctx.set_small_m(32)
        for h in hs:
            ctx.release_weight(h)


# ------------------------------------------------------------------ epilogue branches and dispatch
# (M, N) pairs that route to each GEMM kernel (K = 768): M <= 32 runs gemv_w8a8;
# otherwise gemm_w8a8_pt (fragment-major activations) when N % 4 == 0, gemm_w8a8 when
# not.
KERNEL_ROUTES = [(8, 1024, "gemv"), (20, 1001, "gemv"), (300, 1024, "gemm_w8a8_pt<64, 256, 64, 2,"),
                 (300, 1001, "gemm_w8a8<")]


def _gelu_spread_scales(a, wq, target_std=3.0):
    """Per-channel weight scales that put the pre-GELU values of every column at
    std ~target_std, so ErfF32's three branches (|u| < 1, 1 <= |u| <= 4, |u| > 4,
    u = x / sqrt(2)) all occur many times."""
    M, K = a.shape
    aq, a_s = oracle.quantize_activations(a, M, K)
    y0 = (aq.astype(np.float64) @ wq.astype(np.float64).T) * a_s[:, None]
    sd = np.maximum(y0.std(axis=0), 1e-6)
    return (target_std / sd).astype(np.float32)


@pytest.mark.parametrize("M,N,route", KERNEL_ROUTES)
@pytest.mark.parametrize("spread", [3.0, 40.0])
def test_gelu_every_branch(ctx, M, N, route, spread):
    # spread 40: most arguments on ErfF32's sign branch, so the persistent kernel's
    # epilogue also takes its chunk-wide sign-branch pass
    g = workloads.rng(31 + M + N)
    K = 768
    a = workloads.activations(g, M, K)
    a[M // 2] = 0  # an all-zero row (scale 0 -> +0 before bias)
    wq, _ = workloads.int8_weights(g, N, K)
    ws = _gelu_spread_scales(a, wq, spread)
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    try:
        assert route in ctx.gemm_kernel_name(w, M, enchip.ACT_GELU)
        say(f"GELU branches M={M} N={N} via {route}, pre-activation spread {spread}")
        got = ctx.linear(w, a, bias=b, act=enchip.ACT_GELU)
    finally:
        ctx.release_weight(w)
    # the inputs exercise every branch (checked on the oracle's pre-GELU values)
    u = np.abs(oracle.w8a8_linear(a, wq, ws, b, 0, M, K, N).astype(np.float64)) / np.sqrt(2.0)
    n = u.size
    assert (u < 1).sum() > 0.01 * n and ((u >= 1) & (u <= 4)).sum() > 0.05 * n and (u > 4).sum() > 0.01 * n
    if spread > 10:
        assert (u > 4).sum() > 0.5 * n
    else:
        # over a quarter of the arguments off the series branch: a persistent-kernel chunk
        # (32 rows x 64 columns per wavefront) then holds more tail values than its 512-cell
        # list, so the per-lane rounds for the rest run too
        assert (u >= 1).sum() > 0.4 * n
    assert_f32_parity(got, oracle.w8a8_linear(a, wq, ws, b, 1, M, K, N), f"GELU {route}")


@pytest.mark.parametrize("M,N,route", KERNEL_ROUTES)
@pytest.mark.parametrize("act", [0, 1])
def test_special_weight_scales(ctx, M, N, route, act):
    # Scales the quantizer never produces but the ABI accepts: inf, NaN, negative,
    # zero, subnormal, huge. With zero activation rows these reach the reference's
    # "+0 when aScale == 0" rule (linalg/quant.go:291-293) with every sign of wS.
    g = workloads.rng(41 + M + N + act)
    K = 768
    a = workloads.activations(g, M, K)
    a[0] = 0
    a[M - 1] = 0
    wq, ws = workloads.int8_weights(g, N, K)
    special = np.array([np.inf, -np.inf, np.nan, -1e-3, 0.0, -0.0, 1e-40, 3e38, -3e38], np.float32)
    ws[:special.size] = special
    ws[N - special.size:] = special
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    try:
        say(f"special scales M={M} N={N} act={act} via {route}")
        got = ctx.linear(w, a, bias=b, act=act)
    finally:
        ctx.release_weight(w)
    assert_f32_parity(got, oracle.w8a8_linear(a, wq, ws, b, act, M, K, N), f"special scales {route}")


@pytest.mark.parametrize("M,N,K,bm", [(300, 1024, 768, 64), (4096, 3072, 256, 64), (16384, 1024, 128, 128)])
@pytest.mark.parametrize("act", [0, 1])
def test_persistent_tile_heights_match_oracle(ctx, M, N, K, bm, act):
    # gemm_w8a8_pt runs 64-row tiles (3 workgroups per CU) when 128-row tiles would leave
    # workgroup slots idle (fewer than 2 per CU: 512 on MI355X), else 128-row tiles (M =
    # 16384, N = 1024: exactly 512). Both bit-identical to the oracle, with and without
    # GELU; the GELU case at config 2's wide pre-activations.
    g = workloads.rng(61 + M + N + K + act)
    a = workloads.activations(g, M, K)
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    try:
        name = ctx.gemm_kernel_name(w, M, act)
        cus = ctx.device_info()["num_cus"]
        tiles128 = -(-M // 128) * -(-N // 256)
        assert name.startswith(f"enchip::gemm_w8a8_pt<{bm if cus == 256 else (64 if tiles128 < 2 * cus else 128)}, "), name
        say(f"persistent GEMM M={M} N={N} K={K} act={act} via {name}")
        got = ctx.linear(w, a, bias=b, act=act)
    finally:
        ctx.release_weight(w)
    assert_f32_parity(got, oracle.w8a8_linear(a, wq, ws, b, act, M, K, N), f"tile height {bm}")


def test_kernel_name_matches_dispatch(ctx):
    g = workloads.rng(51)
    for M, N, route in KERNEL_ROUTES:
        wq, ws = workloads.int8_weights(g, N, 768)
        w = ctx.register_weight(wq, ws)
        try:
            for act in (0, 1):
                name = ctx.gemm_kernel_name(w, M, act)
                assert route in name, (M, N, name)
        finally:
            ctx.release_weight(w)


# ------------------------------------------------------------------ fragment-major codes
def frag_to_rows(buf, M, ldq):
    """Row-major [M][ldq] view of codes in the documented fragment-major layout:
    byte (r, k) at ((r/32)*(ldq/32) + k/32)*1024 + ((r%32) + 32*((k/16)%2))*16 + k%16."""
    r = np.arange(M)[:, None]
    k = np.arange(ldq)[None, :]
    off = ((r // 32) * (ldq // 32) + k // 32) * 1024 + ((r % 32) + 32 * ((k // 16) % 2)) * 16 + k % 16
    return buf[off]


@pytest.mark.parametrize("M,K,N,act", [(1500, 768, 2304, 0), (300, 3072, 768, 1), (129, 200, 64, 1), (33, 768, 3072, 1)])
def test_frag_twins_match_linear(ctx, M, K, N, act):
    # enchip_quant_rows_frag_dev + enchip_w8a8_pre_frag_dev: codes byte-exact against the
    # oracle under the documented layout (zero K padding), outputs bit-identical to the
    # fused linear and to the row-major pre_dev path.
    import torch

    g = workloads.rng(61 + M + K + N)
    a = workloads.activations(g, M, K)
    a[M // 3] = 0
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    try:
        ok, ldq = ctx.frag_route(w, M)
        assert ok and ldq == (K + 63) // 64 * 64
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            da = torch.from_numpy(a).cuda()
            db = torch.from_numpy(b).cuda()
            Mp = (M + 127) // 128 * 128
            dq = torch.full((Mp * ldq,), 99, dtype=torch.int8, device="cuda")  # padding rows: any content
            ds = torch.empty(M, dtype=torch.float32, device="cuda")
            dd = torch.empty((M, N), dtype=torch.float32, device="cuda")
            say(f"frag twins M={M} K={K} N={N} act={act}")
            ctx.quant_rows_frag_dev(da.data_ptr(), M, K, dq.data_ptr(), ldq, ds.data_ptr(), st.cuda_stream)
            ctx.pre_frag_dev(w, dq.data_ptr(), ldq, M, ds.data_ptr(), db.data_ptr(), act, dd.data_ptr(), st.cuda_stream)
        torch.cuda.synchronize()
        want_q, want_s = oracle.quantize_activations(a, M, K)
        codes = frag_to_rows(dq.cpu().numpy(), M, ldq)
        assert np.array_equal(codes[:, :K], want_q), "codes differ"
        assert (codes[:, K:] == 0).all(), "K padding not zero"
        assert np.array_equal(bits(ds.cpu().numpy()), bits(want_s))
        got = dd.cpu().numpy()
        assert np.array_equal(bits(got), bits(ctx.linear(w, a, bias=b, act=act)))
        assert_f32_parity(got, oracle.w8a8_linear(a, wq, ws, b, act, M, K, N), "frag twins")
    finally:
        ctx.release_weight(w)


def test_frag_route_rejects_other_shapes(ctx):
    import torch

    g = workloads.rng(71)
    for M, N, why in [(16, 768, "small M"), (300, 1001, "N % 4")]:
        wq, ws = workloads.int8_weights(g, N, 768)
        w = ctx.register_weight(wq, ws)
        try:
            ok, ldq = ctx.frag_route(w, M)
            assert not ok and ldq == 768, why
            dq = torch.zeros(((M + 127) // 128 * 128) * ldq, dtype=torch.int8, device="cuda")
            ds = torch.ones(M, dtype=torch.float32, device="cuda")
            dd = torch.empty((M, N), dtype=torch.float32, device="cuda")
            with pytest.raises(enchip.EnchipError):
                ctx.pre_frag_dev(w, dq.data_ptr(), ldq, M, ds.data_ptr(), 0, 0, dd.data_ptr())
        finally:
            ctx.release_weight(w)
    # a pitch other than the padded K is refused
    wq, ws = workloads.int8_weights(g, 768, 768)
    w = ctx.register_weight(wq, ws)
    try:
        dq = torch.zeros(512 * 1024, dtype=torch.int8, device="cuda")
        ds = torch.ones(300, dtype=torch.float32, device="cuda")
        dd = torch.empty((300, 768), dtype=torch.float32, device="cuda")
        with pytest.raises(enchip.EnchipError):
            ctx.pre_frag_dev(w, dq.data_ptr(), 1024, 300, ds.data_ptr(), 0, 0, dd.data_ptr())
    finally:
        ctx.release_weight(w)
    torch.cuda.synchronize()


# ------------------------------------------------------------------ ann.FlatI8 scoring
@pytest.mark.parametrize("M,N,K", [(1, 5000, 384), (16, 4099, 384), (40, 3000, 768)])
def test_ann_flat_i8_scores(ctx, M, N, K):
    # ann.Backend (ann/backend.go:16-60): NewI8Index = a registered weight (int8 codes +
    # per-row scales), I8Index.Score / I8BatchIndex.ScoreBatch = the bias-free W8A8
    # linear, "the same W8A8 value linalg.MatmulBTW8A8 computes on the CPU".
    g = workloads.rng(81 + M + N)
    q = workloads.activations(g, M, K)
    codes = g.integers(-127, 128, size=(N, K), dtype=np.int8)
    scales = g.uniform(1e-3, 1e-2, size=N).astype(np.float32)
    w = ctx.register_weight(codes, scales)
    try:
        say(f"ann scores M={M} N={N} K={K} via {ctx.gemm_kernel_name(w, M, 0)}")
        got = ctx.linear(w, q)
    finally:
        ctx.release_weight(w)
    assert_f32_parity(got, oracle.w8a8_linear(q, codes, scales, None, 0, M, K, N), "ann scores")


@pytest.mark.parametrize("M,N,K,with_bias", [(40, 32772, 100, True), (129, 65540, 384, False), (256, 40000, 512, True),
                                              (100, 33000, 256, False), (250, 32768, 384, True)])
def test_skinny_scores_match_oracle(ctx, M, N, K, with_bias):
    # gemm_w8a8_skinny (33..256 rows, Kp / 32 in {4, 8, 12, 16}, N >= 32768: ann scoring):
    # all rows' codes in LDS, weights streamed per 32-channel group. Bit-identical to the
    # oracle through the library's own fragment-major quantization (linear) and on
    # row-major codes at a padded pitch (pre_dev), with ragged N, ragged row blocks and
    # a bias.
    import torch

    g = workloads.rng(97 + M + N + K)
    q = workloads.activations(g, M, K)
    codes = g.integers(-127, 128, size=(N, K), dtype=np.int8)
    scales = g.uniform(1e-3, 1e-2, size=N).astype(np.float32)
    bias = workloads.bias(g, N) if with_bias else None
    want = oracle.w8a8_linear(q, codes, scales, bias, 0, M, K, N)
    w = ctx.register_weight(codes, scales)
    try:
        name = ctx.gemm_kernel_name(w, M, 0)
        say(f"skinny scores M={M} N={N} K={K} bias={with_bias} via {name}")
        assert "gemm_w8a8_skinny" in name, name
        assert_f32_parity(ctx.linear(w, q, bias), want, "skinny linear")
        ldq = (K + 63) // 64 * 64 + 64  # a pitch past Kp
        qc, qs = oracle.quantize_activations(q, M, K)
        aq = np.zeros((M, ldq), np.int8)
        aq[:, :K] = qc
        da = torch.from_numpy(aq).cuda()
        ds = torch.from_numpy(np.ascontiguousarray(qs, np.float32)).cuda()
        db = torch.from_numpy(bias).cuda() if with_bias else None
        dd = torch.empty((M, N), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        ctx.pre_dev(w, da.data_ptr(), ldq, M, ds.data_ptr(), db.data_ptr() if with_bias else 0, 0, dd.data_ptr())
        torch.cuda.synchronize()
        assert_f32_parity(dd.cpu().numpy(), want, "skinny pre_dev")
    finally:
        ctx.release_weight(w)


# ------------------------------------------------------------------ pre-swizzled weight images
def test_weight_image_export_and_register(ctx, tmp_path):
    # enchip_weight_export gives the image weight_cache.frag_image builds on the host;
    # registering that image (directly, or from a memory-mapped safetensors file) gives a
    # weight whose linears are bit-identical to the normally registered one.
    from aikit_amd import weight_cache

    g = workloads.rng(91)
    M, K, N = 300, 200, 520
    a = workloads.activations(g, M, K)
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    w0 = ctx.register_weight(wq, ws)
    w1 = w2 = None
    try:
        image, scales = ctx.export_weight(w0)
        assert image.size == ctx.weight_image_bytes(N, K)
        assert np.array_equal(image, weight_cache.frag_image(wq))
        assert np.array_equal(bits(scales), bits(ws))
        w1 = ctx.register_weight_image(weight_cache.frag_image(wq), ws, N, K)
        path = str(tmp_path / "w.safetensors")
        weight_cache.save(path, {"w": (wq, ws)})
        w2 = weight_cache.load(ctx, path)["w"]
        want = ctx.linear(w0, a, bias=b, act=1)
        for w in (w1, w2):
            assert np.array_equal(bits(ctx.linear(w, a, bias=b, act=1)), bits(want))
        with pytest.raises(enchip.EnchipError):
            ctx.register_weight_image(image[:-1], ws, N, K)
    finally:
        for w in (w0, w1, w2):
            if w is not None:
                ctx.release_weight(w)


# ------------------------------------------------------------------ ann top-k on the device
def _check_topk(hi, hs, scores, k, what):
    for r in range(scores.shape[0]):
        idx, sc = oracle.top_hits(scores[r], k)
        got_i, got_s = hi[r], hs[r]
        assert got_i[:idx.size].tolist() == idx.tolist(), f"{what} row {r}: indices differ"
        assert np.array_equal(bits(got_s[:idx.size]), bits(sc)), f"{what} row {r}: scores differ"
        assert (got_i[idx.size:] == -1).all() and np.isnan(got_s[idx.size:]).all(), f"{what} row {r}: padding"


@pytest.mark.parametrize("rows,n,k", [(3, 10000, 10), (2, 4096, 1024), (5, 1000, 1000), (1, 1, 5), (4, 50000, 100),
                                      (2, 8193, 7), (1, 300000, 64), (2, 0, 5), (3, 70000, 32), (2, 16384, 10),
                                      (1, 16385, 1), (2, 40000, 33), (3, 70000, 48), (2, 1100003, 64),
                                      (1, 5000000, 10), (2, 2100000, 16)])
def test_topk_rows_matches_reference_selection(ctx, rows, n, k):
    # FlatI8.topHits' order (score desc, index asc; NaN skipped) on scores full of ties
    # (a coarse grid), signed zeros and NaNs, across chunk boundaries.
    import torch

    g = workloads.rng(rows * n + k)
    s = (g.integers(-50, 51, size=(rows, n)) * 0.25).astype(np.float32)
    s[g.random((rows, n)) < 0.02] = np.nan
    s[g.random((rows, n)) < 0.02] = -0.0
    say(f"topk rows={rows} n={n} k={k}")
    ds = torch.from_numpy(s).cuda()
    di = torch.empty((rows, k), dtype=torch.int32, device="cuda")
    dv = torch.empty((rows, k), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.topk_rows_dev(ds.data_ptr(), n, rows, n, k, di.data_ptr(), k, dv.data_ptr(), k)
    torch.cuda.synchronize()
    _check_topk(di.cpu().numpy(), dv.cpu().numpy(), s, k, "topk")


def _fast_top_hits(s, k):
    # oracle.top_hits for long rows: every score above the k-th largest, plus the ties at
    # it, sorted by (score desc, index asc), first k. Checked against oracle.top_hits below.
    idx = np.flatnonzero(~np.isnan(s))
    if idx.size <= k:
        return oracle.top_hits(s, k)
    v = s[idx]
    kth = np.partition(v, v.size - k)[v.size - k]
    keep = idx[v >= kth]
    order = np.lexsort((keep, -s[keep].astype(np.float64)))
    keep = keep[order[:k]]
    return keep, s[keep]


@pytest.mark.parametrize("kind,k", [("normal", 10), ("grid", 10), ("grid", 32), ("normal", 1), ("increasing", 10),
                                    ("decreasing", 10), ("constant", 10), ("nan_head", 10), ("normal", 64),
                                    ("grid", 48), ("increasing", 64), ("constant", 64), ("nan_head", 40),
                                    ("normal", 100), ("grid", 200), ("increasing", 100), ("constant", 128),
                                    ("decreasing", 100), ("nan_head", 100)])
def test_topk_rows_threshold_filter(ctx, kind, k):
    # 64 rows of 2^20 + 3 scores (129 chunks of 8192, the last ragged): stage 1 runs on each
    # row's first 4 chunks, takes the k-th largest of their keys as the row's bound, and the
    # other chunks keep only their keys at or above it when they are at most k. Exact for
    # any data: ties at the bound break by index (grid, constant), a rising row exceeds the
    # bound in every chunk (full selection everywhere), a falling one in none, and rows
    # whose first chunks are NaN have no bound. For 32 < k <= 64 the rows but "normal" are
    # 2^20 scores, so the merge's 128 k candidates take its 8192-key register form; "normal"
    # keeps 129 chunks and the merge's radix form. Past k = 64 the chunks are 4096 scores
    # (257 per row) and the bound comes from topk_thresh_radix.
    import torch

    rows, n = 64, (1 << 20) + 3 if k <= 32 or k > 64 or kind == "normal" else 1 << 20
    g = workloads.rng(1000 + k + len(kind))
    if kind == "normal":
        s = g.standard_normal((rows, n), dtype=np.float32)
    elif kind == "grid":
        s = (g.integers(-50, 51, size=(rows, n)) * 0.25).astype(np.float32)
        s[g.random((rows, n)) < 0.02] = np.nan
        s[g.random((rows, n)) < 0.02] = -0.0
    elif kind in ("increasing", "decreasing"):
        ramp = np.arange(n, dtype=np.float32)
        s = np.tile(ramp if kind == "increasing" else -ramp, (rows, 1))
    elif kind == "constant":
        s = np.full((rows, n), 0.5, np.float32)
    else:
        s = g.standard_normal((rows, n), dtype=np.float32)
        s[: rows // 2, : 4 * 8192] = np.nan
    say(f"topk threshold filter {kind} rows={rows} n={n} k={k}")
    ds = torch.from_numpy(s).cuda()
    di = torch.empty((rows, k), dtype=torch.int32, device="cuda")
    dv = torch.empty((rows, k), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.topk_rows_dev(ds.data_ptr(), n, rows, n, k, di.data_ptr(), k, dv.data_ptr(), k)
    torch.cuda.synchronize()
    hi, hs = di.cpu().numpy(), dv.cpu().numpy()
    for r in range(rows):
        idx, sc = _fast_top_hits(s[r], k)
        if r < 2:
            oi, osc = oracle.top_hits(s[r], k)
            assert np.array_equal(idx, oi) and np.array_equal(bits(sc), bits(osc)), "fast reference != oracle"
        assert hi[r, : idx.size].tolist() == idx.tolist(), f"{kind} row {r}: indices differ"
        assert np.array_equal(bits(hs[r, : idx.size]), bits(sc)), f"{kind} row {r}: scores differ"
        assert (hi[r, idx.size:] == -1).all() and np.isnan(hs[r, idx.size:]).all(), f"{kind} row {r}: padding"


@pytest.mark.parametrize("k", [1, 10, 32, 64])
def test_topk_rows_concentrated_winners(ctx, k):
    # Every large score sits at positions one thread of a chunk holds (index = 5 mod 256),
    # so that thread's maximum alone clears the bound and its 64 keys (more than a
    # wavefront) are gathered for the final selection; ties among them break by index.
    import torch

    rows, n = 2, 50000
    g = workloads.rng(900 + k)
    s = (g.standard_normal((rows, n)) * 0.01).astype(np.float32)
    hot = np.arange(5, n, 256)
    s[:, hot] = (10 + g.integers(0, 3, size=(rows, hot.size))).astype(np.float32)
    say(f"topk concentrated rows={rows} n={n} k={k}")
    ds = torch.from_numpy(s).cuda()
    di = torch.empty((rows, k), dtype=torch.int32, device="cuda")
    dv = torch.empty((rows, k), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.topk_rows_dev(ds.data_ptr(), n, rows, n, k, di.data_ptr(), k, dv.data_ptr(), k)
    torch.cuda.synchronize()
    _check_topk(di.cpu().numpy(), dv.cpu().numpy(), s, k, "topk")


@pytest.mark.parametrize("M,N,K,k", [(1, 140001, 384, 10), (16, 50000, 384, 100), (40, 3000, 768, 1000)])
def test_ann_topk_matches_score_batch_plus_top_hits(ctx, M, N, K, k):
    # I8TopKIndex.TopKBatch is "rank-identical to ScoreBatch + topHits"
    # (ann/backend.go:46-55): the oracle's W8A8 scores, then the reference's selection.
    g = workloads.rng(83 + M + N)
    q = workloads.activations(g, M, K)
    codes = g.integers(-127, 128, size=(N, K), dtype=np.int8)
    scales = g.uniform(1e-3, 1e-2, size=N).astype(np.float32)
    w = ctx.register_weight(codes, scales)
    try:
        say(f"ann top-k M={M} N={N} K={K} k={k}")
        hi, hs = ctx.ann_topk(w, q, k)
    finally:
        ctx.release_weight(w)
    _check_topk(hi, hs, oracle.w8a8_linear(q, codes, scales, None, 0, M, K, N), k, "ann_topk")


@pytest.mark.parametrize("kind,M,k,K", [("normal", 64, 10, 256), ("normal", 40, 32, 256), ("normal", 33, 1, 256),
                                        ("ties", 64, 10, 256), ("constant", 40, 5, 256), ("rising", 48, 10, 256),
                                        ("normal", 300, 10, 256), ("normal", 64, 10, 600), ("normal", 40, 10, 500),
                                        ("normal", 16, 10, 384), ("normal", 8, 32, 256), ("ties", 9, 10, 256),
                                        ("rising", 8, 10, 256), ("normal", 64, 64, 256), ("ties", 40, 48, 256),
                                        ("constant", 40, 40, 256), ("rising", 48, 64, 256), ("normal", 16, 64, 384),
                                        ("normal", 64, 64, 600)])
def test_ann_topk_fused_route(ctx, kind, M, k, K):
    # Above the small-M limit, with k <= 64 and at least 131072 index rows, TopKBatch keeps
    # the scores on the chip: each query's bound is the k-th best key among the first
    # 32768 rows' scores, one scoring pass (gemm_w8a8_pt's EPI_TOPK epilogue) lists only
    # the scores at or above it, and a merge selects from the lists. Identical to
    # ScoreBatch + topHits on the oracle's scores:
    #   (8 <= M <= 32, the small-M limit: the codes are quantized fragment-major for this
    #   route and the candidate pass holds one 32-row block)
    #   normal: random codes, a ragged last tile (N % 256 = 244), ragged last row-block;
    #     300 queries: three candidate launches of up to 128 queries; K = 600 (Kp = 640, 20
    #     K steps, past the skinny kernel's 16): the persistent kernel's candidate
    #     epilogue; K = 500: the skinny kernel's one-deep ring (16 K steps);
    #   ties: every non-zero score negative and the best ones zeros of both signs (index
    #     rows of zero codes, scales of either sign), NaN scores from NaN scales: the
    #     bound is a zero and ties at it break by index, -0 comes back as -0;
    #   constant: all scores equal, so exactly k clear the bound;
    #   rising: scores grow along the index, every row past the sample clears the bound,
    #     the lists overflow and the call runs the two-pass route instead;
    #   k > 32: lists of up to 8192 candidates and their merge's 32-per-thread form.
    N = 150004
    g = workloads.rng(4000 + M + k + K + len(kind))
    q = workloads.activations(g, M, K)
    if kind == "normal":
        codes = g.integers(-127, 128, size=(N, K), dtype=np.int8)
        scales = g.uniform(1e-3, 1e-2, size=N).astype(np.float32)
    elif kind == "ties":
        q = np.abs(q) + np.float32(0.01)
        codes = g.integers(-3, 1, size=(N, K), dtype=np.int8)
        scales = g.choice(np.array([0.25, 0.5], np.float32), size=N)
        zero = g.random(N) < 0.002
        codes[zero] = 0
        scales[zero] *= g.choice(np.array([1, -1], np.float32), size=int(zero.sum()))
        scales[(g.random(N) < 0.002) & ~zero] = np.nan
    else:
        q = np.abs(q) + np.float32(0.01)
        codes = np.ones((N, K), np.int8)
        scales = (np.full(N, 1e-3, np.float32) if kind == "constant"
                  else np.linspace(1e-3, 2e-3, N, dtype=np.float32))
    want_fallback = kind == "rising"
    w = ctx.register_weight(codes, scales)
    try:
        f0, b0 = ctx.ann_topk_stats()
        say(f"ann top-k fused route {kind} M={M} N={N} K={K} k={k}")
        hi, hs = ctx.ann_topk(w, q, k)
        f1, b1 = ctx.ann_topk_stats()
    finally:
        ctx.release_weight(w)
    assert (f1 - f0, b1 - b0) == (1, 1 if want_fallback else 0), "route"
    scores = oracle.w8a8_linear(q, codes, scales, None, 0, M, K, N)
    if kind == "ties":
        assert np.signbit(scores[:, zero]).any() and (scores[:, zero] == 0).all(), "signed zeros present"
    _check_topk(hi, hs, scores, k, f"ann_topk fused {kind}")


# ------------------------------------------------------------------ fused small-M quantize + GEMV
@pytest.mark.parametrize("M,K,N,act", [(1, 768, 768, 0), (16, 768, 3072, 1), (16, 768, 768, 0), (16, 1024, 768, 1),
                                       (5, 64, 1001, 1), (7, 1000, 96, 0), (9, 384, 1024, 0), (3, 36, 40, 1),
                                       (32, 1024, 768, 1), (32, 768, 3072, 0), (8, 768, 768, 1), (13, 512, 96, 0),
                                       (1, 256, 64, 1), (4, 260, 200, 0), (31, 700, 160, 1),
                                       (16, 3072, 768, 0), (5, 4096, 1024, 1), (32, 1536, 384, 1), (7, 2000, 100, 0),
                                       (1, 4096, 96, 0)])
def test_fused_small_m_matches_two_kernels_and_oracle(ctx, M, K, N, act):
    # At M <= 32 a self-quantizing linear is one launch (gemv_w8a8_q: each workgroup
    # quantizes its group of 8 rows into on-chip memory, one wavefront per row, held in 1-16
    # float4 per lane by K <= 4096); with want_acc the same call runs the separate quantizer +
    # gemv_w8a8. Same bits, and the oracle's, including an all-zero row (scale 0), an Inf
    # row (scale Inf: codes 0) and a row with NaNs (ignored by the absmax), across every
    # row group (M = 1 .. 32, ragged last groups).
    import torch

    g = workloads.rng(900 + M + K + N)
    a = workloads.activations(g, M, K)
    a[0] = 0
    if M > 2:
        a[1, 3] = np.inf
        a[2, ::7] = np.nan
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    w = ctx.register_weight(wq, ws)
    try:
        name = ctx.gemm_kernel_name(w, M, act)
        assert "gemv_w8a8_q<" in name, name
        say(f"fused small-M linear M={M} K={K} N={N} act={act} ({name})")
        fused = ctx.linear(w, a, bias=b, act=act)
        split, _ = ctx.linear(w, a, bias=b, act=act, want_acc=True)
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
            dd = torch.empty((M, N), dtype=torch.float32, device="cuda")
            ctx.linear_dev(w, da.data_ptr(), M, db.data_ptr(), act, dd.data_ptr(), st.cuda_stream)
        torch.cuda.synchronize()
    finally:
        ctx.release_weight(w)
    assert np.array_equal(bits(fused), bits(split))
    assert np.array_equal(bits(dd.cpu().numpy()), bits(fused))
    assert_f32_parity(fused, oracle.w8a8_linear(a, wq, ws, b, act, M, K, N), "fused small-M")
