"""End-to-end W8A8 encoder forward: pooled embeddings from the device linears vs the
CPU reference composition (the bar: final pooled embeddings at cosine >= 0.9999).

The forward follows encoder/bert.go:300-368 operation for operation:
  1. embeddings word + position (+ token type 0), then LayerNorm (eps 1e-12);
  2. per layer:
     - Q, K, V = h W + b;
     - per-head scaled-dot-product attention (encoder/attention.go:81-130);
     - O projection + bias, residual, LayerNorm;
     - FFN-up + bias, then GELU;
     - FFN-down + bias, residual, LayerNorm;
  3. mean pooling (encoder/pooling.go:84-105) and L2Normalize (embed/pool.go:22-38).

Each `s.mm(W) + addBias (+ gelu)` is one W8A8 linear: per-token int8 activations and
per-channel int8 weights, the composition of the BERT / MiniLM / XLM-R encoders
(vision/encoder.go:234-255 is the in-tree precedent). Q, K and V share one
quantization of h and run as a single N = 3D linear (linalg.MatmulBTW8A8Batch,
bit-identical to per-op).

The two arms differ only in who computes the linears:
  * reference: oracle.cpu_w8a8_linear, the C restatement of aikit's Go path;
  * device: libenchip.so on the GPU, through the C ABI.
The glue (attention, LayerNorm, pooling) is the oracle's in both arms, so any difference
in the embeddings comes from the linears.
"""
import numpy as np
import pytest

import oracle
from aikit_amd import enchip, workloads

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999  # the encoder parity bar: cosine against the reference composition
ATT_MODES = {"flash_f16": 3, "flash_bf16": 2, "split_bf16": 1, "f32": 0}  # enchip_att_products


def say(msg):
    print(f"[case] {msg}", flush=True)


def model_weights(cfg, seed, max_pos=512, type_vocab=2):
    g = workloads.rng(seed)
    D = cfg.hidden
    w = {
        "word": (g.standard_normal((cfg.vocab, D)) * 0.02).astype(np.float32),
        "pos": (g.standard_normal((max_pos, D)) * 0.02).astype(np.float32),
        "type": (g.standard_normal((type_vocab, D)) * 0.02).astype(np.float32),
        "emb_ln": ((1 + g.standard_normal(D) * 0.02).astype(np.float32), (g.standard_normal(D) * 0.02).astype(np.float32)),
        "layers": [],
    }
    for _ in range(cfg.layers):
        lw = workloads.encoder_layer_weights(g, cfg)
        lw["attn_ln"] = ((1 + g.standard_normal(D) * 0.02).astype(np.float32), (g.standard_normal(D) * 0.02).astype(np.float32))
        lw["out_ln"] = ((1 + g.standard_normal(D) * 0.02).astype(np.float32), (g.standard_normal(D) * 0.02).astype(np.float32))
        w["layers"].append(lw)
    return w


def encode(ids, w, cfg, linear):
    """bert.go forward + mean pool + L2 for one sequence. linear(x, li, name) returns
    act(W8A8(x, W_name) + b_name) as an f32 [M, N] array."""
    L, D = len(ids), cfg.hidden
    eps = 1e-12
    h = np.empty((L, D), np.float32)
    for i, t in enumerate(ids):
        row = (w["word"][t] + w["pos"][i]).astype(np.float32)
        h[i] = (row + w["type"][0]).astype(np.float32)
    h = oracle.layer_norm(h, *w["emb_ln"], L, D, eps)
    for li in range(cfg.layers):
        qkv = linear(h, li, "qkv")
        Q = np.ascontiguousarray(qkv[:, :D])
        K = np.ascontiguousarray(qkv[:, D:2 * D])
        V = np.ascontiguousarray(qkv[:, 2 * D:])
        ctx = oracle.attention(Q, K, V, L, D, cfg.heads)
        out = linear(ctx, li, "o")
        h = oracle.layer_norm((h + out).astype(np.float32), *w["layers"][li]["attn_ln"], L, D, eps)
        inter = linear(h, li, "ffn_up")
        ffn = linear(inter, li, "ffn_down")
        h = oracle.layer_norm((h + ffn).astype(np.float32), *w["layers"][li]["out_ln"], L, D, eps)
    return oracle.l2_normalize(oracle.pool_mean(h, L, D))


def run_both(ctx, workers, cfg, seqs, seed):
    w = model_weights(cfg, seed)
    handles = [{n: ctx.register_weight(v[0], v[1]) for n, v in lw.items() if n in ("qkv", "o", "ffn_up", "ffn_down")}
               for lw in w["layers"]]
    try:
        def ref_linear(x, li, name):
            wq, ws, b, act = w["layers"][li][name]
            M, K = x.shape
            return oracle.cpu_w8a8_linear(x, wq, ws, b, act, M, K, wq.shape[0], workers=workers).reshape(M, -1)

        def dev_linear(x, li, name):
            _, _, b, act = w["layers"][li][name]
            return ctx.linear(handles[li][name], np.ascontiguousarray(x), bias=b, act=act)

        for s, ids in enumerate(seqs):
            say(f"{cfg.name} sequence {s} (L={len(ids)})")
            ref = encode(ids, w, cfg, ref_linear)
            dev = encode(ids, w, cfg, dev_linear)
            cos = float(np.dot(ref.astype(np.float64), dev.astype(np.float64)) /
                        (np.linalg.norm(ref.astype(np.float64)) * np.linalg.norm(dev.astype(np.float64))))
            assert cos >= COS_MIN, f"{cfg.name} seq {s}: cosine {cos}"
            # the linears are bit-exact, so the whole forward is too
            assert np.array_equal(ref.view(np.uint32), dev.view(np.uint32)), f"{cfg.name} seq {s}: embeddings differ in bits"
    finally:
        for hs in handles:
            for h in hs.values():
                ctx.release_weight(h)


def test_config1_minilm_l6_embeddings(ctx, workers):
    # Config 1: MiniLM-L6 shape, batch 8 x seq 128, ids uniform in [1000, 30000)
    cfg = workloads.MINILM_L6
    g = workloads.rng(11)
    seqs = [g.integers(1000, 30000, size=cfg.seq) for _ in range(cfg.batch)]
    run_both(ctx, workers, cfg, seqs, seed=101)


def test_config4_bert_base_embedding(ctx, workers):
    # Config 4 shape at full sequence length, one sequence (each sequence's
    # forward is independent of the others in the batch; the full b64 linears are
    # checked row by row in test_gpu_parity.py)
    cfg = workloads.BERT_BASE
    g = workloads.rng(12)
    seqs = [g.integers(1000, 30000, size=cfg.seq)]
    run_both(ctx, workers, cfg, seqs, seed=102)


def embeddings_in(ids, w, cfg):
    """bert.go:299-323 for one sequence: word + position + token type 0, then LayerNorm."""
    L, D = len(ids), cfg.hidden
    h = np.empty((L, D), np.float32)
    for i, t in enumerate(ids):
        row = (w["word"][t] + w["pos"][i]).astype(np.float32)
        h[i] = (row + w["type"][0]).astype(np.float32)
    return oracle.layer_norm(h, *w["emb_ln"], L, D, 1e-12)


@pytest.mark.parametrize("fused", ["flash_f16", "flash_bf16", "split_bf16", "f32", False])
def test_config1_device_resident_forward(ctx, workers, fused):
    # The whole forward on the device (aikit_amd.bert_dev: W8A8 linears, f32 attention
    # products, softmax, residual + LayerNorm, pooling), every activation resident,
    # against the CPU reference composition of the same model. Attention and LayerNorm
    # sum in a different order on the device, so the bar is the encoder parity cosine (COS_MIN).
    import torch

    from aikit_amd.bert_dev import DeviceBert

    cfg = workloads.MINILM_L6
    g = workloads.rng(11)
    seqs = [g.integers(1000, 30000, size=cfg.seq) for _ in range(cfg.batch)]
    w = model_weights(cfg, seed=101)

    def ref_linear(x, li, name):
        wq, ws, b, act = w["layers"][li][name]
        M, K = x.shape
        return oracle.cpu_w8a8_linear(x, wq, ws, b, act, M, K, wq.shape[0], workers=workers).reshape(M, -1)

    S, L, D = cfg.batch, cfg.seq, cfg.hidden
    h0 = np.concatenate([embeddings_in(ids, w, cfg) for ids in seqs])
    from aikit_amd import enchip

    model = DeviceBert(ctx, w["layers"], D, cfg.heads, cfg.ffn, fused=bool(fused))
    ctx.set_attention_products(ATT_MODES[fused] if fused else enchip.ATT_DEFAULT)
    try:
        say(f"{cfg.name} device-resident forward, {S} sequences of {L}, fused attention {fused}")
        h = torch.from_numpy(h0).cuda()
        pooled = torch.empty((S, D), device="cuda")
        torch.cuda.synchronize()
        model.embed(h, S, L, pooled)
        torch.cuda.synchronize()
        dev = pooled.cpu().numpy()
    finally:
        model.close()
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    worst = 1.0
    for s, ids in enumerate(seqs):
        ref = encode(ids, w, cfg, ref_linear)
        cos = float(np.dot(ref.astype(np.float64), dev[s].astype(np.float64)) /
                    (np.linalg.norm(ref.astype(np.float64)) * np.linalg.norm(dev[s].astype(np.float64))))
        worst = min(worst, cos)
        assert cos >= COS_MIN, f"{cfg.name} seq {s}: cosine {cos}"
    say(f"  worst cosine {worst:.9f}")


def test_config5_shaped_cross_encoder_on_device(ctx, workers):
    # Config 5's architecture (XLM-R-large widths: D=1024, 16 heads, FFN 4096) at 2 layers
    # and 2 pairs of 128 tokens, scored as a cross-encoder (encoder/crossencoder.go:219-238)
    # entirely on the device, against the CPU reference composition (the reference's W8A8
    # linears, the oracle's attention / LayerNorm / TanhF32, the f32 head in float64).
    # Attention and LayerNorm sum in another order on the device; a last-bit difference
    # can move one per-token int8 code in the next linear, so the chain is held to the
    # encoder parity cosine (COS_MIN) on the [CLS] hidden state, and the head alone (f32 MatmulBT,
    # bias, TanhF32, classifier) to 1e-5 on the device's own [CLS] rows.
    import torch

    from aikit_amd import enchip
    from aikit_amd.bert_dev import DeviceBert

    cfg = workloads.EncoderConfig("xlmr-shaped-2l", layers=2, hidden=1024, heads=16, ffn=4096, batch=2, seq=128,
                                  vocab=1000)
    w = model_weights(cfg, seed=505)
    g = workloads.rng(506)
    seqs = [g.integers(0, cfg.vocab, size=cfg.seq) for _ in range(cfg.batch)]
    D, labels = cfg.hidden, 1
    pw = (g.standard_normal((D, D)) * 0.02).astype(np.float32)
    pb = (g.standard_normal(D) * 0.02).astype(np.float32)
    cw = (g.standard_normal((labels, D)) * 0.02).astype(np.float32)
    cb = (g.standard_normal(labels) * 0.02).astype(np.float32)

    def ref_linear(x, li, name):
        wq, ws, b, act = w["layers"][li][name]
        M, K = x.shape
        return oracle.cpu_w8a8_linear(x, wq, ws, b, act, M, K, wq.shape[0], workers=workers).reshape(M, -1)

    def ref_cls(ids):
        L = len(ids)
        h = embeddings_in(ids, w, cfg)
        for li in range(cfg.layers):
            qkv = ref_linear(h, li, "qkv")
            ctxv = oracle.attention(np.ascontiguousarray(qkv[:, :D]), np.ascontiguousarray(qkv[:, D:2 * D]),
                                    np.ascontiguousarray(qkv[:, 2 * D:]), L, D, cfg.heads)
            h = oracle.layer_norm((h + ref_linear(ctxv, li, "o")).astype(np.float32), *w["layers"][li]["attn_ln"],
                                  L, D, 1e-12)
            ffn = ref_linear(ref_linear(h, li, "ffn_up"), li, "ffn_down")
            h = oracle.layer_norm((h + ffn).astype(np.float32), *w["layers"][li]["out_ln"], L, D, 1e-12)
        return h[0]

    def head(cls):
        pooled = oracle.tanh((cls.astype(np.float64) @ pw.T.astype(np.float64) + pb).astype(np.float32))
        return pooled.astype(np.float64) @ cw.T.astype(np.float64) + cb

    ref_cls_rows = np.array([ref_cls(ids) for ids in seqs])

    S, L = cfg.batch, cfg.seq
    h0 = np.concatenate([embeddings_in(ids, w, cfg) for ids in seqs])
    model = DeviceBert(ctx, w["layers"], D, cfg.heads, cfg.ffn)
    try:
        say(f"{cfg.name} cross-encoder on the device, {S} pairs of {L}")
        dv = {k: torch.from_numpy(v).cuda() for k, v in dict(h=h0, pw=pw, pb=pb, cw=cw, cb=cb).items()}
        logits = torch.empty((S, labels), device="cuda")
        torch.cuda.synchronize()
        model.rerank(dv["h"], S, L, (dv["pw"], dv["pb"]), (dv["cw"], dv["cb"]), logits)
        torch.cuda.synchronize()
        got = logits.cpu().numpy().astype(np.float64)
        dev_cls = dv["h"].cpu().numpy().reshape(S, L, D)[:, 0]
    finally:
        model.close()
    head_err = np.abs(got - np.array([head(c) for c in dev_cls])).max()
    say(f"  head on the device's [CLS] rows: worst abs error {head_err:.3g}")
    assert head_err <= 1e-5
    for s_ in range(S):
        a, b = ref_cls_rows[s_].astype(np.float64), dev_cls[s_].astype(np.float64)
        cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))
        say(f"  pair {s_}: [CLS] cosine {cos:.9f}, logit {got[s_, 0]:.6f} vs {head(ref_cls_rows[s_])[0]:.6f}")
        assert cos >= COS_MIN


def test_config1_device_forward_from_token_ids(ctx, workers):
    # The whole encode on the device from token ids: embedding rows + LayerNorm
    # (DeviceBert.embeddings), the layers, pooling; against the CPU reference composition
    # from the same ids (encode), to the encoder parity cosine (COS_MIN).
    import torch

    from aikit_amd.bert_dev import DeviceBert

    cfg = workloads.MINILM_L6
    g = workloads.rng(12)
    seqs = [g.integers(1000, 30000, size=cfg.seq) for _ in range(cfg.batch)]
    w = model_weights(cfg, seed=102)

    def ref_linear(x, li, name):
        wq, ws, b, act = w["layers"][li][name]
        M, K = x.shape
        return oracle.cpu_w8a8_linear(x, wq, ws, b, act, M, K, wq.shape[0], workers=workers).reshape(M, -1)

    S, L, D = cfg.batch, cfg.seq, cfg.hidden
    model = DeviceBert(ctx, w["layers"], D, cfg.heads, cfg.ffn)
    try:
        model.set_embeddings(w["word"], w["pos"], w["emb_ln"], typ=w["type"])
        say(f"{cfg.name} device forward from token ids, {S} sequences of {L}")
        ids = torch.from_numpy(np.concatenate(seqs).astype(np.int32)).cuda()
        h = torch.empty((S * L, D), device="cuda")
        pooled = torch.empty((S, D), device="cuda")
        torch.cuda.synchronize()
        model.embeddings(ids, S, L, h)
        model.embed(h, S, L, pooled)
        torch.cuda.synchronize()
        dev = pooled.cpu().numpy()
    finally:
        model.close()
    for s_, ids_ in enumerate(seqs):
        ref = encode(ids_, w, cfg, ref_linear).astype(np.float64)
        d = dev[s_].astype(np.float64)
        cos = float(ref @ d / (np.linalg.norm(ref) * np.linalg.norm(d)))
        say(f"  seq {s_}: cosine {cos:.9f}")
        assert cos >= COS_MIN


def test_device_forward_ln_quant_fusion_is_bit_identical(ctx):
    # DeviceBert with the LayerNorm + next-linear quantization fused (the default) and
    # unfused: identical pooled bits (the fused kernel reproduces both halves exactly).
    import torch

    from aikit_amd.bert_dev import DeviceBert

    cfg = workloads.MINILM_L6
    g = workloads.rng(13)
    w = model_weights(cfg, seed=103)
    S, L, D = cfg.batch, cfg.seq, cfg.hidden
    h0 = torch.from_numpy(np.concatenate([embeddings_in(g.integers(1000, 30000, size=L), w, cfg)
                                          for _ in range(S)])).cuda()
    got = []
    for fuse in (True, False):
        model = DeviceBert(ctx, w["layers"], D, cfg.heads, cfg.ffn, fuse_ln_quant=fuse)
        try:
            h = h0.clone()
            pooled = torch.empty((S, D), device="cuda")
            torch.cuda.synchronize()
            model.embed(h, S, L, pooled)
            torch.cuda.synchronize()
            got.append(pooled.cpu().numpy())
        finally:
            model.close()
    say(f"{cfg.name}: fused LN + quantization vs unfused, pooled bits equal")
    assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32))


@pytest.mark.parametrize("up_scale", [1.0, 8.0])
def test_device_forward_gelu_in_quant_is_bit_identical(ctx, up_scale):
    # DeviceBert with FFN-up's GELU applied by FFN-down's quantization (the default) and in
    # FFN-up's epilogue: identical pooled bits. up_scale widens FFN-up's weight scales so
    # that many pre-activations take ErfF32's tail and sign branches (random-init weights
    # put ~1% there).
    import torch

    from aikit_amd import enchip
    from aikit_amd.bert_dev import DeviceBert

    cfg = workloads.MINILM_L6
    g = workloads.rng(14)
    w = model_weights(cfg, seed=104)
    for lw in w["layers"]:
        wq, ws, b, act = lw["ffn_up"]
        lw["ffn_up"] = (wq, (ws * np.float32(up_scale)).astype(np.float32), b, act)
    S, L, D = cfg.batch, cfg.seq, cfg.hidden
    h0 = torch.from_numpy(np.concatenate([embeddings_in(g.integers(1000, 30000, size=L), w, cfg)
                                          for _ in range(S)])).cuda()
    got = []
    for gq in (True, False):
        model = DeviceBert(ctx, w["layers"], D, cfg.heads, cfg.ffn, gelu_in_quant=gq)
        try:
            assert bool(model.gelu_quant_route(enchip.ACT_GELU, model.handles[0]["ffn_down"][0], S * L)) == gq
            h = h0.clone()
            pooled = torch.empty((S, D), device="cuda")
            torch.cuda.synchronize()
            model.embed(h, S, L, pooled)
            torch.cuda.synchronize()
            got.append(pooled.cpu().numpy())
        finally:
            model.close()
    say(f"{cfg.name} (FFN-up scales x{up_scale}): GELU in FFN-down's quantization vs in FFN-up, pooled bits equal")
    assert np.isfinite(got[0]).all()
    assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32))


# ------------------------------------------------------------------ full depth at L = 512
def _cos(a, b):
    a, b = np.asarray(a, np.float64).reshape(-1), np.asarray(b, np.float64).reshape(-1)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def _ref_linear_fn(w, workers):
    def ref_linear(x, li, name):
        wq, ws, b, act = w["layers"][li][name]
        M, K = x.shape
        return oracle.cpu_w8a8_linear(x, wq, ws, b, act, M, K, wq.shape[0], workers=workers).reshape(M, -1)
    return ref_linear


@pytest.fixture(scope="module")
def bert_base_full(workers):
    """Config 4's model (BERT-base: 12 layers, D 768, 12 heads, FFN 3072) on two
    512-token sequences, and the CPU reference composition's pooled embeddings."""
    cfg = workloads.BERT_BASE
    w = model_weights(cfg, seed=104)
    g = workloads.rng(14)
    seqs = [g.integers(1000, 30000, size=cfg.seq) for _ in range(2)]
    say(f"{cfg.name}: CPU reference for {len(seqs)} sequences of {cfg.seq} through {cfg.layers} layers")
    refs = [encode(ids, w, cfg, _ref_linear_fn(w, workers)) for ids in seqs]
    return cfg, w, seqs, refs


@pytest.mark.parametrize("mode", list(ATT_MODES))
def test_config4_full_depth_device_encode(ctx, bert_base_full, mode):
    # The forward bench.py times, at config 4's full depth and sequence length: token ids
    # -> device embedding rows + LayerNorm -> 12 resident layers (W8A8 linears, fused
    # attention with the given product mode, residual LayerNorms) -> mean pool + L2, as
    # DeviceBert.embeddings + DeviceBert.embed; against the reference composition
    # (encoder/bert.go:260-371, the whole-model cosine gate of encoder/bert_test.go:14-72).
    import torch

    from aikit_amd.bert_dev import DeviceBert

    cfg, w, seqs, refs = bert_base_full
    S, L, D = len(seqs), cfg.seq, cfg.hidden
    model = DeviceBert(ctx, w["layers"], D, cfg.heads, cfg.ffn)
    ctx.set_attention_products(ATT_MODES[mode])
    try:
        model.set_embeddings(w["word"], w["pos"], w["emb_ln"], typ=w["type"])
        say(f"{cfg.name} device encode from token ids, {S} x {L}, {cfg.layers} layers, products {mode}")
        ids = torch.from_numpy(np.concatenate(seqs).astype(np.int32)).cuda()
        h = torch.empty((S * L, D), device="cuda")
        pooled = torch.empty((S, D), device="cuda")
        torch.cuda.synchronize()
        model.embeddings(ids, S, L, h)
        model.embed(h, S, L, pooled)
        torch.cuda.synchronize()
        dev = pooled.cpu().numpy()
    finally:
        model.close()
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    for s_, ref in enumerate(refs):
        cos = _cos(ref, dev[s_])
        say(f"  seq {s_}: cosine {cos:.9f}")
        assert cos >= COS_MIN


def _attention_f64(Q, K, V, L, D, heads):
    """The attention of encoder/attention.go:81-121 in float64, rounded to f32 once: the
    reference composition with only its attention's rounding changed."""
    hd = D // heads
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    out = np.empty((L, D))
    for h in range(heads):
        c = slice(h * hd, (h + 1) * hd)
        s = Q[:, c].astype(np.float64) @ K[:, c].astype(np.float64).T * scale
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, c] = p @ V[:, c].astype(np.float64)
    return out.astype(np.float32)


@pytest.fixture(scope="module")
def xlmr_large_full(workers):
    """Config 5's architecture (24 layers, D 1024, 16 heads, FFN 4096) on one 512-token
    pair and the head's weights, with the reference composition's final hidden state
    computed twice: with the oracle's f32 attention, and with the same attention in
    float64 (rounded to f32). The second run measures how far the W8A8 composition drifts
    from itself when only the f32 rounding of its glue changes -- every per-token
    requantization turns a last-bit difference into a code step, and 24 layers compound
    it -- which sets the scale of agreement an exact-in-f32 device forward can reach. The
    vocabulary is cut to 30522 rows: the table's size does not enter the arithmetic."""
    cfg = workloads.EncoderConfig("xlmr-large-24l", layers=24, hidden=1024, heads=16, ffn=4096, batch=1, seq=512,
                                  vocab=30522)
    w = model_weights(cfg, seed=507)
    g = workloads.rng(508)
    ids = g.integers(0, cfg.vocab, size=cfg.seq)
    D = cfg.hidden
    head = dict(pw=(g.standard_normal((D, D)) * 0.02).astype(np.float32),
                pb=(g.standard_normal(D) * 0.02).astype(np.float32),
                cw=(g.standard_normal((1, D)) * 0.02).astype(np.float32),
                cb=(g.standard_normal(1) * 0.02).astype(np.float32))
    ref_linear = _ref_linear_fn(w, workers)
    L = cfg.seq

    def forward(attention):
        h = embeddings_in(ids, w, cfg)
        for li in range(cfg.layers):
            qkv = ref_linear(h, li, "qkv")
            ctxv = attention(np.ascontiguousarray(qkv[:, :D]), np.ascontiguousarray(qkv[:, D:2 * D]),
                             np.ascontiguousarray(qkv[:, 2 * D:]), L, D, cfg.heads)
            h = oracle.layer_norm((h + ref_linear(ctxv, li, "o")).astype(np.float32), *w["layers"][li]["attn_ln"],
                                  L, D, 1e-12)
            ffn = ref_linear(ref_linear(h, li, "ffn_up"), li, "ffn_down")
            h = oracle.layer_norm((h + ffn).astype(np.float32), *w["layers"][li]["out_ln"], L, D, 1e-12)
        return h

    say(f"{cfg.name}: CPU reference for one pair of {cfg.seq} through {cfg.layers} layers (f32 and float64 attention)")
    ref = forward(lambda Q, K, V, L_, D_, H_: oracle.cpu_attention(Q, K, V, L_, D_, H_, workers))
    ref64 = forward(_attention_f64)
    return cfg, w, ids, head, ref, ref64


def _head_logit(cls, head):
    """encoder/crossencoder.go:229-236 in float64 over f32 inputs: classifier(tanh(pooler(CLS)))."""
    pooled = oracle.tanh((cls.astype(np.float64) @ head["pw"].T.astype(np.float64) + head["pb"]).astype(np.float32))
    return float((pooled.astype(np.float64) @ head["cw"].T.astype(np.float64) + head["cb"])[0])


@pytest.mark.parametrize("mode", list(ATT_MODES))
def test_config5_full_depth_device_rerank(ctx, xlmr_large_full, mode):
    # Config 5's cross-encoder forward (DeviceBert.embeddings + DeviceBert.rerank, as the
    # bench runs it) at its full depth and length on one pair, against the reference
    # composition. Bars:
    #  * the mean-pooled final hidden state at the encoder parity cosine >= 0.9999;
    #  * the [CLS] row (what the head reads): its distance from the reference, 1 - cosine,
    #    at most twice the reference's own drift when only its attention's rounding
    #    changes (f32 vs float64; ~4e-4 at 24 layers, measured live) -- a single token's
    #    state cannot agree more closely than the composition agrees with itself;
    #  * the device head on the device's own [CLS] row within 1e-5;
    #  * the device logit against the reference's within twice the reference's own logit
    #    drift (its logit with float64 attention against its logit with f32 attention)
    #    plus 0.01 (1.6% of this head's logit): a fixed bar set by the reference alone,
    #    not by the device's own [CLS] error.
    import torch

    from aikit_amd.bert_dev import DeviceBert

    cfg, w, ids, head, ref, ref64 = xlmr_large_full
    L, D = cfg.seq, cfg.hidden
    model = DeviceBert(ctx, w["layers"], D, cfg.heads, cfg.ffn)
    ctx.set_attention_products(ATT_MODES[mode])
    try:
        model.set_embeddings(w["word"], w["pos"], w["emb_ln"], typ=w["type"])
        say(f"{cfg.name} device rerank from token ids, 1 x {L}, {cfg.layers} layers, products {mode}")
        dv = {k: torch.from_numpy(v).cuda() for k, v in head.items()}
        d_ids = torch.from_numpy(ids.astype(np.int32)).cuda()
        h = torch.empty((L, D), device="cuda")
        logits = torch.empty((1, 1), device="cuda")
        torch.cuda.synchronize()
        model.embeddings(d_ids, 1, L, h)
        model.rerank(h, 1, L, (dv["pw"], dv["pb"]), (dv["cw"], dv["cb"]), logits)
        torch.cuda.synchronize()
        got = float(logits.cpu().numpy()[0, 0])
        dev_h = h.cpu().numpy()
    finally:
        model.close()
        ctx.set_attention_products(enchip.ATT_DEFAULT)
    dev_cls, ref_cls = dev_h[0], ref[0]
    pooled_cos = _cos(dev_h.astype(np.float64).mean(axis=0), ref.astype(np.float64).mean(axis=0))
    cos = _cos(ref_cls, dev_cls)
    self_cos = _cos(ref_cls, ref64[0])
    head_err = abs(got - _head_logit(dev_cls, head))
    ref_logit = _head_logit(ref_cls, head)
    self_drift = abs(_head_logit(ref64[0], head) - ref_logit)
    bar = 2 * self_drift + 0.01
    say(f"  pooled cosine {pooled_cos:.9f}; [CLS] cosine {cos:.9f} (reference vs itself with float64 attention "
        f"{self_cos:.9f}); logit {got:.6f} vs {ref_logit:.6f} (reference's own logit drift {self_drift:.3g}, bar "
        f"{bar:.3g}); head error {head_err:.3g}")
    assert pooled_cos >= COS_MIN
    assert 1 - cos <= 2 * (1 - self_cos)
    assert head_err <= 1e-5
    assert abs(got - ref_logit) <= bar
