"""GPU parity of enchip_quant_rows_frag_gelu_dev: the quantization of GELU(a) from the
pre-activations a, against the CPU oracle, through the C ABI.

The bar is that of the quantizer (TestCUDA_vitQuantRows, gpu/cuda_vit_test.go:154-226):
codes byte-exact and scales bit-exact, here against quantizeRowInt8Core
(linalg/quant.go:43-71) applied to GELUF32 (linalg/exp.go:260-263) of every element, both
restated in the oracle. The distributions cover every branch of ErfF32 in bulk: the series
branch (|u| < 1), the A&S tail with the reference's exp (1 <= |u| <= 4) and the sign
branch (|u| > 4), from ~1% tails (a random-init encoder's FFN) to nearly all of them.
"""
import numpy as np
import pytest

import oracle
from aikit_amd import enchip, workloads

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def frag_to_rows(buf, M, ldq):
    """Row-major [M][ldq] view of codes in the fragment-major layout of the header:
    byte (r, k) at ((r/32)*(ldq/32) + k/32)*1024 + ((r%32) + 32*((k/16)%2))*16 + k%16."""
    r = np.arange(M)[:, None]
    k = np.arange(ldq)[None, :]
    off = ((r // 32) * (ldq // 32) + k // 32) * 1024 + ((r % 32) + 32 * ((k // 16) % 2)) * 16 + k % 16
    return buf[off]


def gelu_quant_dev(ctx, a, M, K, ldq, fill=99):
    import torch

    Mp = (M + 127) // 128 * 128
    da = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    dq = torch.full((Mp * ldq,), fill, dtype=torch.int8, device="cuda")
    ds = torch.full((M,), -7.0, dtype=torch.float32, device="cuda")
    ctx.quant_rows_frag_gelu_dev(da.data_ptr(), M, K, dq.data_ptr(), ldq, ds.data_ptr())
    torch.cuda.synchronize()
    return frag_to_rows(dq.cpu().numpy(), M, ldq), ds.cpu().numpy()


def check_against_oracle(ctx, a, M, K, what):
    ldq = (K + 63) // 64 * 64
    codes, scales = gelu_quant_dev(ctx, a, M, K, ldq)
    g = oracle.gelu(a)
    want_q, want_s = oracle.quantize_activations(g, M, K)
    bad = np.flatnonzero((codes[:, :K] != want_q).any(axis=1))
    assert bad.size == 0, f"{what}: codes differ in rows {bad[:8]}"
    assert (codes[:, K:] == 0).all(), f"{what}: K padding not zero"
    sb = np.flatnonzero(bits(scales) != bits(want_s))
    assert sb.size == 0, f"{what}: scales differ in rows {sb[:8]}"


def tail_fraction(a):
    u = np.abs(a.astype(np.float32) * np.float32(0.7071067811865476))
    return float(np.mean(~(u < 1)))


@pytest.mark.parametrize("M,K,std", [(257, 3072, 0.5), (130, 3072, 1.1), (64, 3072, 3.3), (40, 768, 22.0),
                                     (33, 4096, 1.1), (17, 1000, 1.0), (100, 1536, 0.55), (9, 64, 2.0),
                                     (70, 200, 1.5), (48, 2048, 0.28)])
def test_gelu_quant_matches_oracle(ctx, M, K, std):
    g = workloads.rng(1000 + M + K)
    a = (g.standard_normal((M, K)) * std).astype(np.float32)
    say(f"gelu quant M={M} K={K} std={std} tails={tail_fraction(a):.3f}")
    check_against_oracle(ctx, a, M, K, f"M={M} K={K} std={std}")


def test_gelu_quant_special_rows(ctx):
    # zero rows (GELU(0) = 0: codes 0, scale 0), rows whose GELU is all -0 (every input
    # below -5.66: scale 0), NaN and infinities (NaN ignored by the absmax, coded 0;
    # GELU(+inf) = +inf, GELU(-inf) = NaN), subnormals, values on the branch edges
    # (|u| = 1 and 4 exactly, and their neighbours), and a row that is all tails.
    M, K = 24, 3072
    g = workloads.rng(4242)
    a = (g.standard_normal((M, K)) * 0.6).astype(np.float32)
    a[0] = 0
    a[1] = -(6 + np.abs(g.standard_normal(K))).astype(np.float32)
    a[2, ::7] = np.nan
    a[3, 5], a[3, 9] = np.inf, -np.inf
    a[4] = np.float32(1e-40) * g.standard_normal(K).astype(np.float32)
    edge = np.array([1.0, 4.0], np.float32) / np.float32(0.7071067811865476)
    for j, e in enumerate(np.concatenate([edge, -edge])):
        a[5, 64 * j: 64 * j + 32] = np.nextafter(e, np.float32(np.inf), dtype=np.float32)
        a[5, 64 * j + 32: 64 * j + 64] = np.nextafter(e, np.float32(-np.inf), dtype=np.float32)
        a[6, 16 * j] = e
    a[7] = (g.standard_normal(K) * 40).astype(np.float32)  # nearly every value a tail
    a[8] = np.nan
    a[9, :] = 0
    a[9, 3000] = -1.5  # the one nonzero code comes from a tail value
    # subnormal row scales: maxAbs/127 underflows to 0 (inv = inf, the lone value codes to
    # 127 by the clamp) or to a subnormal (v * inv can exceed 127, clamped)
    a[10] = 0
    a[10, 7] = np.float32(2.8e-45)
    a[11] = 0
    a[11, 100], a[11, 2000] = np.float32(1e-39), np.float32(-3e-40)
    a[12] = (np.float32(1e-37) * g.standard_normal(K)).astype(np.float32)
    say(f"gelu quant special rows M={M} K={K}")
    check_against_oracle(ctx, a, M, K, "special rows")


@pytest.mark.parametrize("M", [1, 7, 8, 9, 4100])
def test_gelu_quant_row_counts(ctx, M):
    # blocks of 8 rows: partial last blocks, and rows past M never written
    K = 768
    g = workloads.rng(77 + M)
    a = (g.standard_normal((M, K)) * 1.3).astype(np.float32)
    say(f"gelu quant M={M} K={K}")
    check_against_oracle(ctx, a, M, K, f"M={M}")


def test_gelu_quant_equals_gelu_linear_then_quant(ctx):
    # The pair it replaces: a linear with the GELU epilogue, then enchip_quant_rows_frag_dev
    # of its output, against the same linear with a bias-only epilogue, then this call:
    # the same codes and scales for the next linear, and the same outputs from it.
    import torch

    M, K, N, N2 = 600, 768, 3072, 768
    g = workloads.rng(9001)
    a = workloads.activations(g, M, K)
    wq, ws = workloads.int8_weights(g, N, K)
    b = workloads.bias(g, N)
    wq2, ws2 = workloads.int8_weights(g, N2, N)
    b2 = workloads.bias(g, N2)
    w, w2 = ctx.register_weight(wq, ws), ctx.register_weight(wq2, ws2)
    try:
        ok, ldq = ctx.frag_route(w2, M)
        assert ok and ldq == N
        da = torch.from_numpy(a).cuda()
        db, db2 = torch.from_numpy(b).cuda(), torch.from_numpy(b2).cuda()
        Mp = (M + 127) // 128 * 128
        outs = []
        for fused in (False, True):
            inter = torch.empty((M, N), device="cuda")
            dq = torch.zeros(Mp * ldq, dtype=torch.int8, device="cuda")
            ds = torch.empty(M, device="cuda")
            dst = torch.empty((M, N2), device="cuda")
            say(f"gelu linear + quant vs bias linear + gelu quant, fused={fused}")
            ctx.linear_dev(w, da.data_ptr(), M, db.data_ptr(), enchip.ACT_NONE if fused else enchip.ACT_GELU,
                           inter.data_ptr())
            if fused:
                ctx.quant_rows_frag_gelu_dev(inter.data_ptr(), M, N, dq.data_ptr(), ldq, ds.data_ptr())
            else:
                ctx.quant_rows_frag_dev(inter.data_ptr(), M, N, dq.data_ptr(), ldq, ds.data_ptr())
            ctx.pre_frag_dev(w2, dq.data_ptr(), ldq, M, ds.data_ptr(), db2.data_ptr(), enchip.ACT_NONE,
                             dst.data_ptr())
            torch.cuda.synchronize()
            outs.append((frag_to_rows(dq.cpu().numpy(), M, ldq), bits(ds.cpu().numpy()), bits(dst.cpu().numpy())))
        assert np.array_equal(outs[0][0], outs[1][0]), "codes differ"
        assert np.array_equal(outs[0][1], outs[1][1]), "scales differ"
        assert np.array_equal(outs[0][2], outs[1][2]), "next linear's outputs differ"
    finally:
        ctx.release_weight(w)
        ctx.release_weight(w2)


def test_gelu_quant_declines_unsupported_shapes(ctx):
    import torch

    buf = torch.zeros(4096 * 8, device="cuda")
    q = torch.zeros(8 * 8192, dtype=torch.int8, device="cuda")
    s = torch.zeros(8, device="cuda")
    for M, K, ldq, off in [(8, 766, 768, 0), (8, 768, 704, 0), (8, 4100, 4160, 0), (8, 768, 768, 4), (-1, 768, 768, 0),
                           (8, 0, 64, 0)]:
        with pytest.raises(enchip.EnchipError) as ei:
            ctx.quant_rows_frag_gelu_dev(buf.data_ptr() + off, M, K, q.data_ptr(), ldq, s.data_ptr())
        assert ei.value.code == enchip.ERR_ARG, (M, K, ldq, off)
