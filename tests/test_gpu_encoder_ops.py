"""GPU parity for the encoder row operations (softmax, residual + LayerNorm, mean pool +
L2), through the C ABI, against the oracle's restatements of the reference
(linalg/exp_scalar.go:9-35,84-89; encoder/layernorm.go:18-38; encoder/pooling.go:84-105;
embed/pool.go:22-38).

Pooling keeps the reference's summation order and must match bit for bit. Softmax and
LayerNorm add their float64 partial sums as a tree, so a result may differ from the
oracle by one f32 ulp where the float64 sum lands differently; the tests allow exactly
that (and require NaN patterns and special rows to match exactly).
"""
import numpy as np
import pytest

import oracle
from aikit_amd import workloads

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def ordered(x):
    """float32 -> int64 keys whose differences count ulps across the sign boundary."""
    i = np.ascontiguousarray(x, np.float32).view(np.int32).astype(np.int64)
    return np.where(i < 0, -(i & 0x7FFFFFFF), i)


def assert_ulps(got, want, max_ulps, what):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all(), f"{what}: NaN pattern differs"
    d = np.abs(ordered(got[~nan]) - ordered(want[~nan]))
    assert d.size == 0 or d.max() <= max_ulps, f"{what}: {int(d.max())} ulps apart (allowed {max_ulps})"
    return int((d > 0).sum())


def _dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


@pytest.mark.parametrize("cols", [1, 7, 64, 77, 128, 512, 1000, 4096])
def test_softmax_rows_scaled_matches_oracle(ctx, cols):
    import torch

    g = workloads.rng(300 + cols)
    rows = 67
    x = (g.standard_normal((rows, cols)) * 6).astype(np.float32)
    if cols > 3:
        x[1, 0] = np.nan            # NaN first: maxV NaN, every e 0 -> uniform row
        x[2, 2] = np.nan            # later NaN: skipped by the max; expF32Core(NaN) is 0 (Go's int32 conversion)
        x[3, :] = -np.inf           # all -inf: v - maxV is NaN -> e 0 -> uniform
        x[4, 0] = -np.inf           # -inf first, then finite values
        x[5, :] = 0                 # all equal
        x[6, 1] = 200.0             # one dominant value, the rest underflow to 0
    scale = np.float32(0.125)
    say(f"softmax rows={rows} cols={cols}")
    d = _dev(torch, x)
    torch.cuda.synchronize()
    ctx.softmax_rows_scaled_dev(d.data_ptr(), cols, rows, cols, float(scale))
    torch.cuda.synchronize()
    got = d.cpu().numpy()
    want = np.stack([oracle.softmax_row_scaled(r, scale) for r in x])
    n = assert_ulps(got, want, 1, f"softmax cols={cols}")
    say(f"  {n} of {got.size} values one ulp apart")
    if cols > 3:
        for r in (1, 3, 5):  # uniform rows and the all-equal row: sums of integers, exact in any order
            assert np.array_equal(got[r], want[r]), f"special row {r}"


def test_softmax_two_column_rows_pin_exp_bits(ctx):
    # Rows [0, x], x <= 0: the max is the first element, and the float64 sum of the two
    # exponentials (1 + e) is exact in any order, so every output must equal the oracle's
    # bit for bit: this pins the device expF32Core (its non-positive-argument form) on
    # ~200k arguments across its range, into the underflow to 0 and at NaN.
    import torch

    g = workloads.rng(321)
    xs = np.concatenate([-np.abs(g.standard_normal(100000) * 30), -g.uniform(80, 110, 50000),
                         -g.uniform(0, 1e-3, 50000), [0.0, -0.0, -np.inf, np.nan, -87.33654, -88.72283, -103.97]])
    x = np.zeros((xs.size, 2), np.float32)
    x[:, 1] = xs
    d = _dev(torch, x)
    torch.cuda.synchronize()
    ctx.softmax_rows_scaled_dev(d.data_ptr(), 2, xs.size, 2, 1.0)
    torch.cuda.synchronize()
    got = d.cpu().numpy()
    want = np.stack([oracle.softmax_row_scaled(r, np.float32(1.0)) for r in x])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_softmax_pitched_rows(ctx):
    # ld > cols: only the first cols of each row are touched.
    import torch

    g = workloads.rng(310)
    rows, cols, ld = 40, 300, 320
    x = g.standard_normal((rows, ld)).astype(np.float32)
    d = _dev(torch, x)
    torch.cuda.synchronize()
    ctx.softmax_rows_scaled_dev(d.data_ptr(), ld, rows, cols, 0.5)
    torch.cuda.synchronize()
    got = d.cpu().numpy()
    assert np.array_equal(got[:, cols:], x[:, cols:])
    want = np.stack([oracle.softmax_row_scaled(r[:cols], np.float32(0.5)) for r in x])
    assert_ulps(got[:, :cols], want, 1, "pitched softmax")


@pytest.mark.parametrize("D,with_res", [(384, True), (768, True), (768, False), (1024, True), (100, True),
                                        (4096, True)])
def test_residual_layer_norm_matches_oracle(ctx, D, with_res):
    import torch

    g = workloads.rng(400 + D)
    rows = 130
    h = (g.standard_normal((rows, D)) * 3 + 0.5).astype(np.float32)
    y = g.standard_normal((rows, D)).astype(np.float32)
    h[7] = 1.25  # constant row: variance 0, output = shift
    w = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    b = (g.standard_normal(D) * 0.1).astype(np.float32)
    say(f"layer norm rows={rows} D={D} residual={with_res}")
    dh, dy, dw, db = (_dev(torch, v) for v in (h, y, w, b))
    torch.cuda.synchronize()
    ctx.residual_layer_norm_dev(dh.data_ptr(), D, dy.data_ptr() if with_res else 0, D, rows, D, dw.data_ptr(),
                                db.data_ptr(), 1e-12)
    torch.cuda.synchronize()
    x = (h + y).astype(np.float32) if with_res else h  # the f32 residual add, element by element
    want = oracle.layer_norm(x, w, b, rows, D, 1e-12)
    n = assert_ulps(dh.cpu().numpy(), want, 1, f"layer norm D={D}")
    say(f"  {n} of {rows * D} values one ulp apart")


@pytest.mark.parametrize("S,L,D", [(3, 128, 384), (2, 512, 768), (1, 1, 5), (4, 77, 1024)])
def test_pool_mean_l2_bit_exact(ctx, S, L, D):
    import torch

    g = workloads.rng(500 + S * L + D)
    h = g.standard_normal((S * L, D)).astype(np.float32)
    say(f"pool S={S} L={L} D={D}")
    dh = _dev(torch, h)
    out = torch.empty((S, D), device="cuda")
    torch.cuda.synchronize()
    ctx.pool_mean_l2_dev(dh.data_ptr(), D, S, L, D, out.data_ptr(), D)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for s in range(S):
        want = oracle.l2_normalize(oracle.pool_mean(h[s * L:(s + 1) * L], L, D))
        assert np.array_equal(got[s].view(np.uint32), want.view(np.uint32)), f"sequence {s}"


def test_pool_zero_and_empty_sequences(ctx):
    import torch

    D = 64
    h = np.zeros((4, D), np.float32)
    dh = _dev(torch, h)
    out = torch.full((2, D), 7.0, device="cuda")
    torch.cuda.synchronize()
    ctx.pool_mean_l2_dev(dh.data_ptr(), D, 2, 2, D, out.data_ptr(), D)  # all-zero rows: norm < 1e-12 -> zeros
    ctx.pool_mean_l2_dev(dh.data_ptr(), D, 1, 0, D, out.data_ptr(), D)  # L = 0: the zero vector
    torch.cuda.synchronize()
    assert not out.cpu().numpy().any()


# ------------------------------------------------------------------ fused attention
def _attention_f64(qkv, S, L, H, hd, scale):
    """float64 ground truth of attentionCore's context (encoder/attention.go:95-116)."""
    D = H * hd
    out = np.empty((S, L, D), np.float64)
    for s in range(S):
        x = qkv[s].astype(np.float64)
        for h in range(H):
            Q, K, V = (x[:, o + h * hd:o + (h + 1) * hd] for o in (0, D, 2 * D))
            sc = (Q @ K.T) * float(scale)
            e = np.exp(sc - sc.max(axis=1, keepdims=True))
            out[s, :, h * hd:(h + 1) * hd] = (e / e.sum(axis=1, keepdims=True)) @ V
    return out


PRODUCT_MODES = {"f32": 0, "split_bf16": 1, "flash_bf16": 2, "flash_f16": 3}  # enchip_att_products
FLASH_MODES = [2, 3]  # the online-softmax kernel with bfloat16 / half split products


@pytest.mark.parametrize("products", list(PRODUCT_MODES))
@pytest.mark.parametrize("S,L,H,hd", [(2, 128, 12, 64), (1, 512, 4, 64), (3, 77, 6, 32), (2, 40, 2, 64),
                                      (1, 1, 3, 64), (2, 512, 2, 32), (1, 33, 2, 64), (1, 511, 1, 32)])
def test_fused_attention_matches_f64_and_unfused(ctx, S, L, H, hd, products):
    # Gate: the f32 MatmulBT statistic (gpu/enccuda/backend_test.go:71-81) against a
    # float64 attention, for the fused kernel (both product modes) and for the unfused
    # chain (two batched MatmulBT calls around the softmax), and between the two.
    import torch

    from aikit_amd import enchip

    ctx.set_attention_products(PRODUCT_MODES[products])

    D = H * hd
    g = workloads.rng(700 + S * L + H + hd)
    qkv = g.standard_normal((S, L, 3 * D)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(hd))
    say(f"fused attention S={S} L={L} H={H} hd={hd} products {products}")
    dq = torch.from_numpy(qkv).cuda()
    fused = torch.full((S * L, D), np.nan, device="cuda")
    unfused = torch.full((S * L, D), np.nan, device="cuda")
    scores = torch.empty((S, H, L, L), device="cuda")
    torch.cuda.synchronize()
    q = dq.data_ptr()
    ctx.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, fused.data_ptr(), D, S, L, H, hd, float(scale))
    ctx.matmul_bt_f32_dev(q, 3 * D, q + D * 4, 3 * D, enchip.B_NK, scores.data_ptr(), L, L, hd, L,
                          inner=(H, hd, hd, L * L), outer=(S, L * 3 * D, L * 3 * D, H * L * L))
    ctx.softmax_rows_scaled_dev(scores.data_ptr(), L, S * H * L, L, float(scale))
    ctx.matmul_bt_f32_dev(scores.data_ptr(), L, q + 2 * D * 4, 3 * D, enchip.B_KN, unfused.data_ptr(), D, L, L, hd,
                          inner=(H, L * L, hd, hd), outer=(S, H * L * L, L * 3 * D, L * D))
    torch.cuda.synchronize()
    f, u = fused.cpu().numpy().reshape(S, L, D), unfused.cpu().numpy().reshape(S, L, D)
    want = _attention_f64(qkv, S, L, H, hd, scale)
    wf, wu, fu = (oracle.matmul_bt_worst_rel(a, b) for a, b in ((f, want), (u, want), (f, u)))
    say(f"  worst rel: fused {wf:.3g}, unfused {wu:.3g}, fused vs unfused {fu:.3g}")
    assert wf <= 2e-4 and wu <= 2e-4 and fu <= 2e-4
    # and the CPU restatement of the reference's attention for the first sequence
    ref = oracle.attention(qkv[0, :, :D], qkv[0, :, D:2 * D], qkv[0, :, 2 * D:], L, D, H)
    assert oracle.matmul_bt_worst_rel(f[0], ref) <= 2e-4
    ctx.set_attention_products(enchip.ATT_DEFAULT)


@pytest.mark.parametrize("mode", [1, 2, 3])
def test_split_bf16_attention_error_is_bounded_by_the_split(ctx, mode):
    # The split-bfloat16 products against the f64 attention on inputs of larger and mixed
    # magnitude (V spanning 6 decades), each output's error measured against the scale of
    # its terms, sum_j P_j |V_j|, rather than max(|ref|, 1): bf16 alone (2^-9 per product)
    # or a dropped or mis-signed lo part fails 2e-4 there; the 3-product split (3 * 2^-18
    # per product, also through the scores into the softmax) passes.
    import torch

    from aikit_amd import enchip

    S, L, H, hd = 2, 200, 3, 64
    D = H * hd
    g = workloads.rng(7070)
    qkv = g.standard_normal((S, L, 3 * D)).astype(np.float32)
    qkv[..., :2 * D] *= 1.5
    qkv[..., 2 * D:] *= np.float32(10.0) ** g.integers(-3, 3, size=(S, L, D))
    scale = np.float32(1.0 / np.sqrt(hd))
    dq = torch.from_numpy(qkv).cuda()
    out = torch.full((S * L, D), np.nan, device="cuda")
    torch.cuda.synchronize()
    q = dq.data_ptr()
    try:
        ctx.set_attention_products(mode)
        ctx.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, out.data_ptr(), D, S, L, H, hd, float(scale))
        torch.cuda.synchronize()
    finally:
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    got = out.cpu().numpy().reshape(S, L, D).astype(np.float64)
    want = _attention_f64(qkv, S, L, H, hd, scale)
    # |ctx| <= sum_j P_j |V_j|: the scale of the P.V sum's terms per output
    x = qkv.astype(np.float64)
    mag = np.empty_like(want)
    for s in range(S):
        for h in range(H):
            sl = slice(h * hd, (h + 1) * hd)
            sc = (x[s, :, sl] @ x[s, :, D:2 * D][:, sl].T) * float(scale)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            mag[s, :, sl] = p @ np.abs(x[s, :, 2 * D:][:, sl])
    err = np.abs(got - want) / mag
    say(f"  split-bf16 attention: worst error / sum|terms| {err.max():.3g}")
    assert err.max() <= 2e-4


@pytest.mark.parametrize("mode", FLASH_MODES)
def test_flash_attention_wide_and_narrow_workgroups_agree(ctx, mode):
    # The flash kernel runs 16 wavefronts per workgroup (512 queries) for 256 < L < 512 and
    # for L > 512 on a grid of at least as many workgroups as CUs; else 8. Each query's
    # arithmetic is the same in both, so the same sequences give the same bits whether they
    # run in a batch large enough for the 16-wavefront form or alone (the 8-wavefront
    # form); both against float64.
    import torch

    from aikit_amd import enchip

    H, hd, L = 12, 64, 700
    D = H * hd
    cus = ctx.device_info()["num_cus"]
    S_wide = -(-cus // (2 * H))  # ceil(L / 512) = 2 workgroups per (head, sequence)
    g = workloads.rng(7400)
    qkv = g.standard_normal((S_wide, L, 3 * D)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(hd))
    dq = torch.from_numpy(qkv).cuda()
    wide = torch.full((S_wide * L, D), np.nan, device="cuda")
    narrow = torch.full((2 * L, D), np.nan, device="cuda")
    torch.cuda.synchronize()
    q = dq.data_ptr()
    ctx.set_attention_products(mode)
    say(f"flash attention (mode {mode}) L={L}: {S_wide} sequences (16 wavefronts) and 2 sequences (8 wavefronts)")
    try:
        ctx.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, wide.data_ptr(), D, S_wide, L, H, hd, float(scale))
        ctx.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, narrow.data_ptr(), D, 2, L, H, hd, float(scale))
        torch.cuda.synchronize()
    finally:
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    w = wide.cpu().numpy().reshape(S_wide, L, D)
    n = narrow.cpu().numpy().reshape(2, L, D)
    assert np.array_equal(w[:2].view(np.uint32), n.view(np.uint32))
    want = _attention_f64(qkv[[0, S_wide - 1]], 2, L, H, hd, scale)
    wf = oracle.matmul_bt_worst_rel(w[[0, S_wide - 1]], want)
    say(f"  worst rel {wf:.3g}")
    assert wf <= 2e-4


@pytest.mark.parametrize("mode", FLASH_MODES)
@pytest.mark.parametrize("L", [77, 300])
@pytest.mark.parametrize("scale", [-0.2, 0.0, 0.4])
def test_flash_attention_any_scale(ctx, L, scale, mode):
    # The online softmax runs in base 2 on c = |scale| log2 e with Q negated for a negative
    # scale (an exact negation), so the running maximum stays that of the scaled scores;
    # scale 0 gives the mean of V, including over the padded keys of the last tile. Both
    # workgroup widths (8 wavefronts up to L = 256, 16 above).
    import torch

    from aikit_amd import enchip

    S, H, hd = 2, 3, 64
    D = H * hd
    g = workloads.rng(7300 + L)
    qkv = g.standard_normal((S, L, 3 * D)).astype(np.float32)
    dq = torch.from_numpy(qkv).cuda()
    out = torch.full((S * L, D), np.nan, device="cuda")
    torch.cuda.synchronize()
    q = dq.data_ptr()
    ctx.set_attention_products(mode)
    try:
        ctx.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, out.data_ptr(), D, S, L, H, hd, float(scale))
        torch.cuda.synchronize()
    finally:
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    got = out.cpu().numpy().reshape(S, L, D)
    want = _attention_f64(qkv, S, L, H, hd, np.float32(scale))
    wf = oracle.matmul_bt_worst_rel(got, want)
    say(f"flash attention L={L} scale={scale}: worst rel {wf:.3g}")
    assert np.isfinite(got).all() and wf <= 2e-4
    if scale == 0.0:  # every query attends uniformly: the mean of V over the L keys
        mean_v = qkv[:, :, 2 * D:].astype(np.float64).mean(axis=1, keepdims=True)
        assert np.abs(got - mean_v).max() <= 1e-5


@pytest.mark.parametrize("mode", FLASH_MODES)
@pytest.mark.parametrize("S,L,H,hd", [(1, 1000, 2, 64), (2, 700, 3, 32)])
def test_flash_attention_beyond_512_keys(ctx, S, L, H, hd, mode):
    # The online-softmax kernel has no key limit (the two-pass kernels hold a row of
    # scores in LDS, L <= 512): longer sequences against float64 at the same gate.
    import torch

    from aikit_amd import enchip

    D = H * hd
    g = workloads.rng(7100 + L)
    qkv = g.standard_normal((S, L, 3 * D)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(hd))
    say(f"flash attention S={S} L={L} H={H} hd={hd}")
    dq = torch.from_numpy(qkv).cuda()
    out = torch.full((S * L, D), np.nan, device="cuda")
    torch.cuda.synchronize()
    q = dq.data_ptr()
    try:
        ctx.set_attention_products(mode)
        ctx.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, out.data_ptr(), D, S, L, H, hd, float(scale))
        torch.cuda.synchronize()
    finally:
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    wf = oracle.matmul_bt_worst_rel(out.cpu().numpy().reshape(S, L, D), _attention_f64(qkv, S, L, H, hd, scale))
    say(f"  worst rel {wf:.3g}")
    assert wf <= 2e-4


@pytest.mark.parametrize("std", [2.0, 4.0])
@pytest.mark.parametrize("products", ["flash_f16", "f32"])
def test_attention_gate_at_realistic_magnitudes(ctx, std, products):
    # The reference's f32 MatmulBT gate (gpu/enccuda/backend_test.go:71-81: worst
    # |got - ref| / max(|ref|, 1) <= 2e-4) against a float64 attention on Q, K, V of
    # standard deviation 2 and 4 (scores of standard deviation 4 and 16 at head_dim 64,
    # trained-model magnitudes), for the default mode (half split products) and the f32
    # products. The bfloat16 split's figure on the same inputs is printed beside them: it
    # exceeds the gate here (measured 1.8-3.0e-4 at standard deviation 2), which is why it
    # is not the default.
    import torch

    from aikit_amd import enchip

    S, L, H, hd = 2, 512, 4, 64
    D = H * hd
    g = workloads.rng(7500 + int(std))
    qkv = (g.standard_normal((S, L, 3 * D)) * std).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(hd))
    dq = torch.from_numpy(qkv).cuda()
    q = dq.data_ptr()
    want = _attention_f64(qkv, S, L, H, hd, scale)
    got = {}
    try:
        for name in (products, "flash_bf16"):
            out = torch.full((S * L, D), np.nan, device="cuda")
            torch.cuda.synchronize()
            ctx.set_attention_products(PRODUCT_MODES[name])
            ctx.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, out.data_ptr(), D, S, L, H, hd, float(scale))
            torch.cuda.synchronize()
            got[name] = oracle.matmul_bt_worst_rel(out.cpu().numpy().reshape(S, L, D), want)
    finally:
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    say(f"attention std={std}: worst rel {products} {got[products]:.3g} (flash_bf16 {got['flash_bf16']:.3g})")
    assert got[products] <= 2e-4


def test_flash_f16_out_of_range_operand_gives_nan(ctx):
    # The half split is finite only for operands below 65520 in magnitude; a larger one
    # makes inf - inf in its products, so the rows that use it come out NaN (never a finite
    # wrong value), while the bfloat16 split (any finite operand) stays finite and within
    # the gate there.
    import torch

    from aikit_amd import enchip

    S, L, H, hd = 1, 64, 2, 64
    D = H * hd
    g = workloads.rng(7600)
    qkv = g.standard_normal((S, L, 3 * D)).astype(np.float32)
    qkv[0, 5, 3] = 1e5  # query 5 of head 0
    scale = np.float32(1.0 / np.sqrt(hd))
    dq = torch.from_numpy(qkv).cuda()
    q = dq.data_ptr()
    outs = {}
    try:
        for mode in (enchip.ATT_FLASH_F16, enchip.ATT_FLASH_BF16):
            out = torch.zeros((S * L, D), device="cuda")
            torch.cuda.synchronize()
            ctx.set_attention_products(mode)
            ctx.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, out.data_ptr(), D, S, L, H, hd, float(scale))
            torch.cuda.synchronize()
            outs[mode] = out.cpu().numpy().reshape(S, L, D)
    finally:
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    f16 = outs[enchip.ATT_FLASH_F16]
    assert np.isnan(f16[0, 5, :hd]).all()  # the row of head 0 whose query overflowed
    ok = np.ones((S, L, D), bool)
    ok[0, 5, :hd] = False
    assert np.isfinite(f16[ok]).all()  # every other row: finite
    bf = outs[enchip.ATT_FLASH_BF16]
    assert np.isfinite(bf).all()
    assert oracle.matmul_bt_worst_rel(bf, _attention_f64(qkv, S, L, H, hd, scale)) <= 2e-4


def test_fused_attention_rejects_unsupported(ctx):
    import torch

    from aikit_amd import enchip

    d = torch.zeros(4096, device="cuda")
    p = d.data_ptr()
    with pytest.raises(enchip.EnchipError):  # head_dim 48
        ctx.attention_f32_dev(p, p, p, 48, p, 48, 1, 8, 1, 48, 0.1)
    with pytest.raises(enchip.EnchipError):  # row pitch past the flash kernel's 32-bit tile offsets
        ctx.attention_f32_dev(p, p, p, (1 << 25) + 4, p, 64, 1, 8, 1, 64, 0.1)
    ctx.set_attention_products(enchip.ATT_SPLIT_BF16)
    try:
        with pytest.raises(enchip.EnchipError):  # L above 512 in a two-pass mode
            ctx.attention_f32_dev(p, p, p, 64, p, 64, 1, 513, 1, 64, 0.1)
    finally:
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    torch.cuda.synchronize()


def test_bias_tanh_matches_oracle(ctx):
    # encoder/crossencoder.go:229-236 addBias + TanhInto: bit-identical to the oracle's
    # TanhF32 restatement (both branches, the saturation above 9, signed zeros, NaN).
    import torch

    from aikit_amd import enchip

    g = workloads.rng(880)
    rows, cols = 37, 300
    x = (g.standard_normal((rows, cols)) * 4).astype(np.float32)
    x[0, :6] = [0.0, -0.0, 0.6249, 0.625, 9.5, np.nan]
    b = (g.standard_normal(cols) * 0.5).astype(np.float32)
    b[:6] = 0
    dx, db = _dev(torch, x), _dev(torch, b)
    torch.cuda.synchronize()
    ctx.bias_act_rows_dev(dx.data_ptr(), cols, rows, cols, db.data_ptr(), enchip.ACT_TANH)
    torch.cuda.synchronize()
    want = oracle.tanh((x + b).astype(np.float32))
    got = dx.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(want)].view(np.uint32), want[~np.isnan(want)].view(np.uint32))


@pytest.mark.parametrize("type_vocab,pos_off,with_segs,D", [(2, 0, False, 96), (2, 2, True, 96), (0, 2, False, 96),
                                                           (2, 1, True, 75)])
def test_embed_rows_bit_exact(ctx, type_vocab, pos_off, with_segs, D):
    # encoder/bert.go:299-322: word[clampTokenID(id)] + pos[i + posOff] (+ type[seg]),
    # f32 adds in that order; ids outside the vocabulary read row 0 (forward.go:15-20),
    # segments outside [0, type_vocab) read type row 0.
    import torch

    g = workloads.rng(4040 + type_vocab + pos_off)
    S, L, vocab, npos = 3, 37, 500, 64  # D = 75: the scalar path
    word = g.standard_normal((vocab, D)).astype(np.float32)
    pos = g.standard_normal((npos, D)).astype(np.float32)
    typ = g.standard_normal((max(type_vocab, 1), D)).astype(np.float32)
    ids = g.integers(-5, vocab + 5, size=S * L).astype(np.int32)
    ids[:4] = [-1, vocab, 0, vocab - 1]
    segs = g.integers(-1, 4, size=S * L).astype(np.int32)
    want = np.empty((S * L, D), np.float32)
    for r in range(S * L):
        i, t = r % L, ids[r]
        w = word[t if 0 <= t < vocab else 0]
        row = (w + pos[i + pos_off]).astype(np.float32)
        if type_vocab > 0:
            sg = segs[r] if with_segs else 0
            row = (row + typ[sg if 0 <= sg < type_vocab else 0]).astype(np.float32)
        want[r] = row
    dv = {k: torch.from_numpy(v).cuda() for k, v in dict(word=word, pos=pos, typ=typ, ids=ids, segs=segs).items()}
    h = torch.full((S * L, D + 8), np.nan, device="cuda")
    torch.cuda.synchronize()
    ctx.embed_rows_dev(dv["ids"].data_ptr(), dv["segs"].data_ptr() if with_segs else 0, S, L, dv["word"].data_ptr(),
                       vocab, dv["pos"].data_ptr(), npos, pos_off, dv["typ"].data_ptr() if type_vocab else 0,
                       type_vocab, D, h.data_ptr(), D + 8)
    torch.cuda.synchronize()
    got = h.cpu().numpy()
    assert np.array_equal(got[:, :D].view(np.uint32), want.view(np.uint32))
    assert np.isnan(got[:, D:]).all()  # the pitch's padding untouched


def test_embed_rows_rejects_positions_past_the_table(ctx):
    import torch

    from aikit_amd import enchip

    d = torch.zeros(4096, device="cuda")
    ids = torch.zeros(64, dtype=torch.int32, device="cuda")
    p = d.data_ptr()
    with pytest.raises(enchip.EnchipError):  # L + pos_off = 34 > 32 position rows
        ctx.embed_rows_dev(ids.data_ptr(), 0, 1, 32, p, 10, p, 32, 2, 0, 0, 8, p, 8)
    torch.cuda.synchronize()


def _frag_codes(buf, rows, ldq):
    """The [rows, ldq] code matrix from its fragment-major layout (include/enchip.h)."""
    r = np.arange(rows)[:, None]
    k = np.arange(ldq)[None, :]
    off = ((r // 32) * (ldq // 32) + k // 32) * 1024 + ((r % 32) + 32 * ((k // 16) % 2)) * 16 + k % 16
    return buf[off]


@pytest.mark.parametrize("rows,D,ldq,zero", [(300, 768, 768, False), (77, 384, 384, False), (64, 1024, 1024, False),
                                             (50, 320, 384, False), (33, 768, 768, True), (9, 2048, 2048, False)])
def test_residual_layer_norm_quant_matches_unfused(ctx, rows, D, ldq, zero):
    # One kernel = enchip_residual_layer_norm_dev then enchip_quant_rows_frag_dev on the
    # stored rows: the same h bits, the same codes (columns [D, ldq) zero) and scales;
    # zero: gain and shift 0, so every normalised row is 0 (scale 0, codes 0).
    import torch

    g = workloads.rng(5050 + rows + D)
    h0 = (g.standard_normal((rows, D)) * 2).astype(np.float32)
    y = g.standard_normal((rows, D)).astype(np.float32)
    w = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    b = (g.standard_normal(D) * 0.1).astype(np.float32)
    if zero:
        w[:] = 0
        b[:] = 0
    Mp = (rows + 127) // 128 * 128
    dh1, dh2, dy, dw, db = (_dev(torch, x) for x in (h0, h0, y, w, b))
    q1 = torch.zeros(Mp * ldq, dtype=torch.int8, device="cuda")
    q2 = torch.zeros(Mp * ldq, dtype=torch.int8, device="cuda")
    s1 = torch.full((rows,), np.nan, device="cuda")
    s2 = torch.full((rows,), np.nan, device="cuda")
    torch.cuda.synchronize()
    ctx.residual_layer_norm_quant_dev(dh1.data_ptr(), D, dy.data_ptr(), D, rows, D, dw.data_ptr(), db.data_ptr(),
                                      1e-12, q1.data_ptr(), ldq, s1.data_ptr())
    ctx.residual_layer_norm_dev(dh2.data_ptr(), D, dy.data_ptr(), D, rows, D, dw.data_ptr(), db.data_ptr(), 1e-12)
    ctx.quant_rows_frag_dev(dh2.data_ptr(), rows, D, q2.data_ptr(), ldq, s2.data_ptr())
    torch.cuda.synchronize()
    h1, h2 = dh1.cpu().numpy(), dh2.cpu().numpy()
    assert np.array_equal(h1.view(np.uint32), h2.view(np.uint32))
    c1, c2 = _frag_codes(q1.cpu().numpy(), rows, ldq), _frag_codes(q2.cpu().numpy(), rows, ldq)
    assert np.array_equal(c1, c2)
    assert (c1[:, D:] == 0).all()
    assert np.array_equal(s1.cpu().numpy().view(np.uint32), s2.cpu().numpy().view(np.uint32))
    if zero:
        assert (c1 == 0).all() and (s1.cpu().numpy() == 0).all()
