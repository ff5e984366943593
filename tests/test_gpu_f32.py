"""GPU parity for the f32 MatmulBT (encoder.Backend.MatmulBT, encoder/backend.go:19-28)
on the MI355X f32 MFMA, through the C ABI.

The contract is the reference's own backend gate, TestEncCUDA_parity
(gpu/enccuda/backend_test.go:47-86): against the float64 ground truth refMatmulBT
(oracle.matmul_bt_f64), worst |dst - ref| / max(|ref|, 1) <= 2e-4, over the same
shapes. TestEncCUDA_noStaleOperands (:88-130) is mirrored as is. Beyond the
tolerance, integer-valued operands whose every partial sum is exact in f32 must come
out exact: any wrong index, dropped k block or transposed operand fails that bit for
bit. The batched, strided device form is checked against per-head host calls on the
attention shapes it exists for (encoder/attention.go:95-111).
"""
import numpy as np
import pytest

import oracle
from aikit_amd import enchip, workloads

pytestmark = pytest.mark.gpu

GATE = 2e-4  # gpu/enccuda/backend_test.go:81


def say(msg):
    print(f"[case] {msg}", flush=True)


def randf(g, *shape):
    return g.standard_normal(shape).astype(np.float32)


REF_SHAPES = [(8, 32, 32), (80, 64, 80), (128, 768, 768), (128, 768, 3072), (512, 768, 3072)]  # backend_test.go:55-61
EDGE_SHAPES = [(1, 1, 1), (33, 7, 65), (100, 3, 130), (65, 64, 1), (1, 4096, 257), (300, 20, 64), (64, 17, 300)]


@pytest.mark.parametrize("M,K,N", REF_SHAPES + EDGE_SHAPES)
def test_matmul_bt_f32_gate(ctx, M, K, N):
    say(f"matmul_bt_f32 M={M} K={K} N={N}")
    g = workloads.rng(3 + M + K + N)
    a, b = randf(g, M, K), randf(g, N, K)
    got = ctx.matmul_bt_f32(a, b)
    worst = oracle.matmul_bt_worst_rel(got, oracle.matmul_bt_f64(a, b, M, K, N))
    say(f"  worst relative delta {worst:.3g}")
    assert worst <= GATE


@pytest.mark.parametrize("M,K,N", [(96, 64, 160), (33, 511, 70), (128, 1024, 64), (5, 6, 7)])
def test_matmul_bt_f32_exact_on_integers(ctx, M, K, N):
    # |a|, |b| <= 16 and K <= 1024: every product and partial sum is an integer below
    # 2^24, so f32 is exact in any order and the result must equal the integer product.
    g = workloads.rng(M * K + N)
    ai = g.integers(-16, 17, size=(M, K))
    bi = g.integers(-16, 17, size=(N, K))
    say(f"matmul_bt_f32 integers M={M} K={K} N={N}")
    got = ctx.matmul_bt_f32(ai.astype(np.float32), bi.astype(np.float32))
    assert np.array_equal(got, (ai @ bi.T).astype(np.float32))


def test_matmul_bt_f32_no_stale_operands(ctx):
    # backend_test.go:88-130: the same host buffer rewritten in place must be re-read.
    g = workloads.rng(4)
    M, K, N = 128, 768, 768
    a, w = randf(g, M, K), randf(g, N, K)
    d1 = ctx.matmul_bt_f32(a, w)
    w[...] = randf(g, N, K)
    d2 = ctx.matmul_bt_f32(a, w)
    assert not np.array_equal(d1, d2), "in-place operand rewrite was not observed"
    assert oracle.matmul_bt_worst_rel(d2, oracle.matmul_bt_f64(a, w, M, K, N)) <= GATE


def test_matmul_bt_f32_empty_and_bad_args(ctx):
    g = workloads.rng(5)
    got = ctx.matmul_bt_f32(np.zeros((3, 0), np.float32), np.zeros((4, 0), np.float32))
    assert got.shape == (3, 4) and not got.any()  # the empty dot product
    assert ctx.matmul_bt_f32(np.zeros((0, 5), np.float32), randf(g, 4, 5)).shape == (0, 4)
    import torch

    d = torch.zeros(64, device="cuda")
    p = d.data_ptr()
    with pytest.raises(enchip.EnchipError):  # unknown b layout
        ctx.matmul_bt_f32_dev(p, 4, p, 4, 2, p, 4, 4, 4, 4)
    with pytest.raises(enchip.EnchipError):  # ldb shorter than a row of b
        ctx.matmul_bt_f32_dev(p, 4, p, 3, enchip.B_NK, p, 4, 4, 4, 4)
    with pytest.raises(enchip.EnchipError):  # negative batch stride
        ctx.matmul_bt_f32_dev(p, 4, p, 4, enchip.B_NK, p, 4, 4, 4, 4, inner=(2, 16, -16, 16))
    ctx.matmul_bt_f32_dev(p, 4, p, 4, enchip.B_NK, p, 4, 4, 4, 4, inner=(0, 16, 16, 16))  # no problems: no-op
    torch.cuda.synchronize()


def _heads(x, L, D, H):
    """[L, D] interleaved heads -> [H, L, D/H] (encoder/attention.go:96-104 extracts)."""
    return np.ascontiguousarray(x.reshape(L, H, D // H).transpose(1, 0, 2))


@pytest.mark.parametrize("S,L,H,hd", [(2, 128, 12, 64), (1, 77, 4, 64), (3, 40, 6, 32)])
def test_batched_attention_products_match_per_head_calls(ctx, S, L, H, hd):
    # One strided launch per product over every (head, sequence): QK^T reads Q and K
    # heads in place from the fused [L, 3D] QKV rows, scores . V reads V in place
    # (ENCHIP_B_KN). Both must equal the per-head host calls bit for bit (same kernel,
    # same k order) and pass the float64 gate.
    import torch

    D = H * hd
    g = workloads.rng(S * L + H)
    qkv = randf(g, S, L, 3 * D)
    say(f"attention products S={S} L={L} H={H} hd={hd}")
    dq = torch.from_numpy(qkv).cuda()
    scores = torch.empty((S, H, L, L), device="cuda")
    ctxv = torch.empty((S, L, D), device="cuda")
    base = dq.data_ptr()
    # one launch: inner level = heads (hd floats apart), outer level = sequences. The
    # calls run on the context stream, so torch's work is synchronized before each.
    torch.cuda.synchronize()
    ctx.matmul_bt_f32_dev(base, 3 * D, base + D * 4, 3 * D, enchip.B_NK, scores.data_ptr(), L, L, hd, L,
                          inner=(H, hd, hd, L * L), outer=(S, L * 3 * D, L * 3 * D, H * L * L))
    torch.cuda.synchronize()
    sc = scores.cpu().numpy()
    for s in range(S):
        Q = _heads(qkv[s, :, :D], L, D, H)
        K = _heads(qkv[s, :, D:2 * D], L, D, H)
        for h in range(H):
            want = ctx.matmul_bt_f32(Q[h], K[h])
            assert np.array_equal(sc[s, h], want), f"QK^T s={s} h={h} differs from the per-head call"
            assert oracle.matmul_bt_worst_rel(sc[s, h], oracle.matmul_bt_f64(Q[h], K[h], L, hd, L)) <= GATE
    # scores . V with V read in place as [K=L, N=hd] rows of pitch 3D
    p = torch.softmax(scores, dim=-1).contiguous()
    torch.cuda.synchronize()
    ctx.matmul_bt_f32_dev(p.data_ptr(), L, base + 2 * D * 4, 3 * D, enchip.B_KN, ctxv.data_ptr(), D, L, L, hd,
                          inner=(H, L * L, hd, hd), outer=(S, H * L * L, L * 3 * D, L * D))
    torch.cuda.synchronize()
    pn, cv = p.cpu().numpy(), ctxv.cpu().numpy()
    for s in range(S):
        V = _heads(qkv[s, :, 2 * D:], L, D, H)
        for h in range(H):
            vht = np.ascontiguousarray(V[h].T)  # vHT[d, i] = V[i, head, d] (attention.go:100-103)
            got = cv[s][:, h * hd:(h + 1) * hd]
            assert np.array_equal(got, ctx.matmul_bt_f32(pn[s, h], vht)), f"PV s={s} h={h} differs from the per-head call"
            assert oracle.matmul_bt_worst_rel(got, oracle.matmul_bt_f64(pn[s, h], vht, L, L, hd)) <= GATE
