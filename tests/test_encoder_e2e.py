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

COS_MIN = 0.9999  # north_star


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


@pytest.mark.parametrize("fused", ["split_bf16", "f32", False])
def test_config1_device_resident_forward(ctx, workers, fused):
    # The whole forward on the device (aikit_amd.bert_dev: W8A8 linears, f32 attention
    # products, softmax, residual + LayerNorm, pooling), every activation resident,
    # against the CPU reference composition of the same model. Attention and LayerNorm
    # sum in a different order on the device, so the bar is the north star's cosine.
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
    ctx.set_attention_products(enchip.ATT_F32 if fused == "f32" else enchip.ATT_SPLIT_BF16)
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
        ctx.set_attention_products(enchip.ATT_SPLIT_BF16)  # the default
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
    # north star's cosine on the [CLS] hidden state, and the head alone (f32 MatmulBT,
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
    # from the same ids (encode), to the north star's cosine.
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
