"""GPU parity for the weight-only int8 product (encoder.Q8Backend.MatmulBTQ8,
encoder/backend_use.go:59-83) on the MI355X bf16 MFMA, through the C ABI.

The contract is the reference's own gate for this seam, TestEncCUDA_q8Parity
(gpu/enccuda/backend_test.go:234-289): against the float64 ground truth cpuQ8Ref
(oracle.matmul_bt_q8_f64), worst |dst - ref| / max(|ref|, 1) <= 2e-4, on its shapes and
its weight scales. That test also pins what this path must NOT do, quantize the
activations: the W8A8 entry point on the same registered weight misses the gate by
orders of magnitude here, the weight-only one meets it. Beyond the tolerance:
integer-valued activations with power-of-two scales, whose every partial sum is exact in
f32, must come out exact (a wrong k permutation between the operands, a wrong channel's
scale or a transposed operand fails bit for bit); one-hot weights must return single
full-significand activations exactly (a dropped part of the three-way split fails); the
full int8 range including -128 (linalg/dequant_i8_test.go:46-75); non-finite
activations give the ground truth's inf / NaN pattern; both tile forms, ragged M, K and
N, pitched device buffers whose padding must stay untouched.
"""
import numpy as np
import pytest

import oracle
from aikit_amd import enchip, workloads

pytestmark = pytest.mark.gpu

GATE = 2e-4  # gpu/enccuda/backend_test.go:280


def say(msg):
    print(f"[case] {msg}", flush=True)


def ref_scales(N):
    # backend_test.go:258-261
    return (0.002 + (np.arange(N) % 13) * 0.0001).astype(np.float32)


def rand_q8(g, N, K, lo=-127):
    # backend_test.go:226-232 (randQ8: [-127, 127]); lo=-128 covers the full int8 range
    return g.integers(lo, 128, size=(N, K)).astype(np.int8)


def worst(got, a, q, s):
    M, K = a.shape
    N = q.shape[0]
    return oracle.matmul_bt_worst_rel(got, oracle.matmul_bt_q8_f64(a, q, s, M, K, N))


# backend_test.go:250-254, and the forward_q8 linears of linalg_q8_test.go:111-117
REF_SHAPES = [(8, 32, 32), (128, 768, 768), (128, 768, 3072), (80, 768, 2304), (80, 3072, 768), (512, 768, 3072)]
EDGE_SHAPES = [(1, 1, 1), (1, 768, 768), (31, 7, 33), (33, 31, 17), (65, 64, 300), (200, 100, 1), (513, 33, 257),
               (64, 4096, 64), (3, 1000, 130), (256 + 17, 768, 3072 + 50), (256 + 17, 1001, 3072 + 50)]


@pytest.mark.parametrize("M,K,N", REF_SHAPES + EDGE_SHAPES)
def test_matmul_bt_q8_gate(ctx, M, K, N):
    say(f"matmul_bt_q8 M={M} K={K} N={N}")
    g = workloads.rng(11 + M + 3 * K + 7 * N)
    a = g.standard_normal((M, K)).astype(np.float32)
    q = rand_q8(g, N, K, lo=-128)
    s = ref_scales(N)
    w = ctx.register_weight(q, s)
    try:
        got = ctx.matmul_bt_q8(w, a)
        wr = worst(got, a, q, s)
        say(f"  worst relative delta {wr:.3g}")
        assert wr <= GATE
        assert np.array_equal(ctx.matmul_bt_q8(w, a).view(np.uint32), got.view(np.uint32))  # deterministic
    finally:
        ctx.release_weight(w)


@pytest.mark.parametrize("M,K,N", [(96, 64, 160), (33, 511, 70), (128, 1024, 64), (5, 6, 7), (300, 4096, 33),
                                   (200, 1000, 3000), (200, 1001, 3000)])
def test_matmul_bt_q8_exact_on_integers(ctx, M, K, N):
    # |a| <= 16, |q| <= 128, K <= 4096: every product and partial sum is an integer below
    # 2^24, exact in f32 in any order; power-of-two scales keep the final multiply exact.
    g = workloads.rng(M * K + N)
    ai = g.integers(-16, 17, size=(M, K))
    qi = rand_q8(g, N, K, lo=-128)
    s = np.ldexp(1.0, g.integers(-3, 3, size=N)).astype(np.float32)
    say(f"matmul_bt_q8 integers M={M} K={K} N={N}")
    w = ctx.register_weight(qi, s)
    try:
        got = ctx.matmul_bt_q8(w, ai.astype(np.float32))
        want = ((ai.astype(np.float64) @ qi.astype(np.float64).T) * s.astype(np.float64)).astype(np.float32)
        assert np.array_equal(got, want)
    finally:
        ctx.release_weight(w)


@pytest.mark.parametrize("M,K,N", [(70, 100, 90), (513, 768, 300), (256 + 17, 300, 3072 + 50),
                                   (4096 + 37, 200, 2048 + 100), (16384 + 37, 200, 2048 + 100)])
def test_matmul_bt_q8_one_hot_selects_activations_exactly(ctx, M, K, N):
    # Channel n has one nonzero code, c_n in {1, -1, 2, -128}, at k = p_n, and a
    # power-of-two scale: dst[m, n] = a[m, p_n] * c_n * s_n exactly, for activations with
    # full 24-bit significands over 1e-30 .. 1e30 (so that even the third part, 2^-16 of
    # a, is a normal number: 2^-126 and up). Only a split that keeps
    # all three bf16 parts (a dropped third part is 2^-17 relative, inside the gate),
    # feeds both operands in the same k order and scales the right channel gets every bit.
    g = workloads.rng(M + K + N)
    x = g.standard_normal((M, K))
    x = np.where(np.abs(x) < 0.1, 0.5, x)
    a = (x * 10.0 ** g.integers(-29, 30, size=(M, K))).astype(np.float32)
    p = g.integers(0, K, size=N)
    c = g.choice(np.array([1, -1, 2, -128]), size=N)
    q = np.zeros((N, K), np.int8)
    q[np.arange(N), p] = c
    s = np.ldexp(1.0, g.integers(-4, 4, size=N)).astype(np.float32)
    say(f"matmul_bt_q8 one-hot M={M} K={K} N={N}")
    w = ctx.register_weight(q, s)
    try:
        got = ctx.matmul_bt_q8(w, a)
    finally:
        ctx.release_weight(w)
    want = (a[:, p].astype(np.float64) * (c * s.astype(np.float64))).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,N", [(4096 + 37, 2048 + 100), (16384 + 37, 2048 + 100)])
def test_matmul_bt_q8_wide_tiles_ragged(ctx, M, N):
    # enough 128 x 128 (then 128 x 256) tiles to take the wide forms, M and N not multiples
    # of the tile; checked exactly on integers over the whole output, and against the gate
    # on the first and last rows (the float64 truth of every row would take the oracle
    # minutes)
    K = 768
    g = workloads.rng(77)
    say(f"matmul_bt_q8 wide tiles M={M} K={K} N={N}")
    ai = g.integers(-16, 17, size=(M, K))
    qi = rand_q8(g, N, K, lo=-128)
    s = np.ldexp(1.0, g.integers(-3, 3, size=N)).astype(np.float32)
    w = ctx.register_weight(qi, s)
    try:
        got = ctx.matmul_bt_q8(w, ai.astype(np.float32))
        want = ((ai.astype(np.float64) @ qi.astype(np.float64).T) * s.astype(np.float64)).astype(np.float32)
        assert np.array_equal(got, want)
    finally:
        ctx.release_weight(w)
    a = g.standard_normal((M, K)).astype(np.float32)
    s = ref_scales(N)
    w = ctx.register_weight(qi, s)
    try:
        got = ctx.matmul_bt_q8(w, a)
        rows = np.r_[0:64, M - 64:M]
        assert worst(got[rows], np.ascontiguousarray(a[rows]), qi, s) <= GATE
    finally:
        ctx.release_weight(w)


def test_matmul_bt_q8_does_not_quantize_activations(ctx):
    # backend_test.go:237-242: a quantized-activation kernel cannot fit inside 2e-4. The
    # same registered weight through the W8A8 entry point misses it; MatmulBTQ8 meets it.
    M, K, N = 128, 768, 768
    g = workloads.rng(12)
    a = g.standard_normal((M, K)).astype(np.float32)
    q = rand_q8(g, N, K)
    s = ref_scales(N)
    w = ctx.register_weight(q, s)
    try:
        w8a8 = worst(ctx.linear(w, a), a, q, s)
        q8 = worst(ctx.matmul_bt_q8(w, a), a, q, s)
        say(f"  W8A8 worst {w8a8:.3g}, weight-only worst {q8:.3g}")
        assert q8 <= GATE < w8a8
    finally:
        ctx.release_weight(w)


def test_matmul_bt_q8_non_finite(ctx):
    # An infinite activation gives +-inf, or NaN against a zero code or an inf of the other
    # sign, as the float64 truth does; NaN gives NaN; a NaN scale gives a NaN channel, a
    # zero scale zeros. Finite rows stay within the gate.
    M, K, N = 40, 200, 96
    g = workloads.rng(13)
    a = g.standard_normal((M, K)).astype(np.float32)
    a[1, 5] = np.inf
    a[2, 199] = -np.inf
    a[3, 0] = np.nan
    a[4, 7], a[4, 9] = np.inf, -np.inf
    a[5, :] = np.float32(3e30)  # large but finite: every partial sum stays finite
    q = rand_q8(g, N, K, lo=-128)
    q[:, 5] = 0
    q[::2, 5] = 1  # channels with a zero code at k = 5 get NaN from row 1's inf
    s = ref_scales(N)
    s[10] = np.nan
    s[11] = 0.0
    say("matmul_bt_q8 non-finite activations and scales")
    w = ctx.register_weight(q, s)
    try:
        got = ctx.matmul_bt_q8(w, a).astype(np.float64)
    finally:
        ctx.release_weight(w)
    ref = oracle.matmul_bt_q8_f64(a, q, s, M, K, N)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf])
    fin = np.isfinite(ref)
    assert np.all(np.isfinite(got[fin]))
    den = np.maximum(np.abs(ref[fin]), 1.0)
    assert np.max(np.abs(got[fin] - ref[fin]) / den) <= GATE


def test_matmul_bt_q8_refuses_infinite_scale_and_bad_args(ctx):
    g = workloads.rng(14)
    q = rand_q8(g, 64, 32)
    s = ref_scales(64)
    s[3] = np.inf
    w = ctx.register_weight(q, s)
    try:
        with pytest.raises(enchip.EnchipError, match="infinite scale"):
            ctx.matmul_bt_q8(w, g.standard_normal((4, 32)).astype(np.float32))
    finally:
        ctx.release_weight(w)
    w = ctx.register_weight(q, ref_scales(64))
    try:
        with pytest.raises(ValueError):
            ctx.matmul_bt_q8(w, g.standard_normal((4, 31)).astype(np.float32))
        import torch

        d = torch.zeros(64 * 64, device="cuda")
        with pytest.raises(enchip.EnchipError):  # lda below K
            ctx.matmul_bt_q8_dev(w, d.data_ptr(), 31, 4, d.data_ptr(), 64)
        with pytest.raises(enchip.EnchipError):  # ldd below N
            ctx.matmul_bt_q8_dev(w, d.data_ptr(), 32, 4, d.data_ptr(), 63)
        with pytest.raises(enchip.EnchipError):  # null output
            ctx.matmul_bt_q8_dev(w, d.data_ptr(), 32, 4, 0, 64)
        assert ctx.matmul_bt_q8(w, np.zeros((0, 32), np.float32)).shape == (0, 64)
    finally:
        ctx.release_weight(w)


def test_matmul_bt_q8_empty_k(ctx):
    # K = 0: the empty sum, zeros whatever the scales (NaN included)
    s = ref_scales(40)
    s[0] = np.nan
    w = ctx.register_weight(np.zeros((40, 0), np.int8), s)
    try:
        got = ctx.matmul_bt_q8(w, np.zeros((7, 0), np.float32))
        assert got.shape == (7, 40) and np.array_equal(got, np.zeros((7, 40), np.float32))
    finally:
        ctx.release_weight(w)


@pytest.mark.parametrize("K,lda_pad", [(768, 4), (100, 3), (33, 0)])
def test_matmul_bt_q8_dev_pitches(ctx, K, lda_pad):
    # the device form on pitched buffers: bit-identical to the host form, and the pitch
    # padding of the output left as it was (lda_pad = 3 takes the unaligned loads)
    import torch

    M, N = 70, 200
    lda, ldd = K + lda_pad, N + 5
    g = workloads.rng(15 + K)
    a = g.standard_normal((M, K)).astype(np.float32)
    q = rand_q8(g, N, K, lo=-128)
    w = ctx.register_weight(q, ref_scales(N))
    say(f"matmul_bt_q8_dev K={K} lda={lda} ldd={ldd}")
    try:
        host = ctx.matmul_bt_q8(w, a)
        da = torch.full((M, lda), float("nan"), device="cuda")
        da[:, :K] = torch.from_numpy(a).cuda()
        dd = torch.full((M, ldd), -7.0, device="cuda")
        s = torch.cuda.Stream()
        ctx.matmul_bt_q8_dev(w, da.data_ptr(), lda, M, dd.data_ptr(), ldd, stream=s.cuda_stream)
        s.synchronize()
        got = dd.cpu().numpy()
        assert np.array_equal(got[:, :N].view(np.uint32), host.view(np.uint32))
        assert np.all(got[:, N:] == -7.0)
    finally:
        ctx.release_weight(w)


def test_matmul_bt_q8_image_round_trip(ctx):
    # a weight registered from its exported fragment-major image gives the same bits
    M, K, N = 50, 300, 90
    g = workloads.rng(16)
    a = g.standard_normal((M, K)).astype(np.float32)
    w = ctx.register_weight(rand_q8(g, N, K, lo=-128), ref_scales(N))
    try:
        image, scales = ctx.export_weight(w)
        w2 = ctx.register_weight_image(image, scales, N, K)
        try:
            assert np.array_equal(ctx.matmul_bt_q8(w, a).view(np.uint32), ctx.matmul_bt_q8(w2, a).view(np.uint32))
        finally:
            ctx.release_weight(w2)
    finally:
        ctx.release_weight(w)
