"""A BERT encoder forward resident on the device, composed from libenchip's entry points.

It follows encoder/bert.go:324-368 layer for layer, with every activation kept in device
memory between operations (the residency the reference names as the next step after the
matmul seam, docs/task-native-gpu.md:418-427):

  qkv   = W8A8(h, Wqkv) + b            enchip_w8a8_linear_dev (Q, K, V fused: one N = 3D
                                        weight sharing one activation quantization,
                                        linalg.MatmulBTW8A8Batch)
  ctx_h = softmax(Q_h.K_h^T/sqrt(hd)).V_h
                                        enchip_attention_f32_dev: every (head, sequence) in
                                        one launch, heads read in place from qkv, scores
                                        kept on chip (head_dim 32/64; any L with the default
                                        online-softmax mode, L <= 512 otherwise); otherwise
                                        enchip_matmul_bt_f32_dev, enchip_softmax_rows_scaled_dev,
                                        enchip_matmul_bt_f32_dev through an [S, H, L, L] buffer
  out   = W8A8(ctx, Wo) + b             enchip_w8a8_linear_dev
  h     = LN(h + out)                   enchip_residual_layer_norm_dev
  inter = GELU(W8A8(h, Wi) + b)         enchip_w8a8_linear_dev (fused epilogue), or, when
                                        FFN-down takes fragment-major codes of K <= 4096,
                                        W8A8(h, Wi) + b alone, the GELU applied by FFN-down's
                                        quantization (enchip_quant_rows_frag_gelu_dev): the
                                        same codes
  ffn   = W8A8(inter, Wd) + b           enchip_w8a8_linear_dev
  h     = LN(h + ffn)                   enchip_residual_layer_norm_dev

A linear that takes fragment-major codes (enchip_frag_route) runs as
enchip_quant_rows_frag_dev + enchip_w8a8_pre_frag_dev into this object's code buffer: the
kernels enchip_w8a8_linear_dev launches, as two calls that can be timed apart. When the
linear after a LayerNorm (FFN-up, and the next layer's QKV) takes fragment-major
codes, the LayerNorm and that linear's quantization run as one kernel
(enchip_residual_layer_norm_quant_dev, then enchip_w8a8_pre_frag_dev): the same bits, and
the normalised rows are not read back to be quantized.

and pools with enchip_pool_mean_l2_dev (encoder/pooling.go:84-105, embed/pool.go:22-38),
or, as a cross-encoder, scores each sequence with classifier(tanh(pooler(CLS)))
(encoder/crossencoder.go:219-238): the f32 MatmulBT on the CLS rows read in place, then
enchip_bias_act_rows_dev for the bias + TanhF32 and the classifier's bias.
forward() takes the [S*L, D] f32 hidden state after the embedding LayerNorm; embeddings()
computes that state on the device from token ids (bert.go:299-323: enchip_embed_rows_dev,
then enchip_residual_layer_norm_dev with no residual). Every sequence of a batch has the
same L.

This module holds no arithmetic of its own; torch provides device buffers and the stream.
"""
from __future__ import annotations

import math
from typing import Dict, List, Sequence, Tuple

import numpy as np

from . import enchip

LN_EPS = 1e-12  # BERT's layer_norm_eps (encoder/bert.go)


class DeviceBert:
    """Weights registered once; forward() runs the layers on device tensors.

    layers: per layer {"qkv"|"o"|"ffn_up"|"ffn_down": (wq int8 [N,K], ws f32 [N],
    bias f32 [N], act), "attn_ln"|"out_ln": (gain f32 [D], shift f32 [D])}.
    """

    def __init__(self, ctx: enchip.Context, layers: Sequence[Dict], hidden: int, heads: int, ffn: int,
                 fused: bool = True, fuse_ln_quant: bool = True, gelu_in_quant: bool = True):
        import torch

        self.fused = fused
        self.fuse_ln_quant = fuse_ln_quant
        self.gelu_in_quant = gelu_in_quant
        self.torch = torch
        self.ctx, self.D, self.H, self.I = ctx, hidden, heads, ffn
        self.hd = hidden // heads
        if self.hd * heads != hidden:
            raise ValueError(f"hidden {hidden} is not a multiple of heads {heads}")
        self.handles: List[Dict[str, Tuple]] = []
        dev = torch.device("cuda")
        for lw in layers:
            entry = {}
            for name in ("qkv", "o", "ffn_up", "ffn_down"):
                wq, ws, b, act = lw[name]
                entry[name] = (ctx.register_weight(wq, ws), torch.from_numpy(np.ascontiguousarray(b)).to(dev), act)
            for name in ("attn_ln", "out_ln"):
                g, s = lw[name]
                entry[name] = (torch.from_numpy(np.ascontiguousarray(g)).to(dev),
                               torch.from_numpy(np.ascontiguousarray(s)).to(dev))
            self.handles.append(entry)
        self._bufs = {}
        self._emb = None
        # Optional callback mark(label) called before each device operation this object
        # enqueues (and with "end" after the last), for per-operation timing; None: off.
        self.mark = None

    def _m(self, label: str) -> None:
        if self.mark is not None:
            self.mark(label)

    def set_embeddings(self, word, pos, ln, typ=None, pos_off: int = 0) -> None:
        """The embedding tables: word [vocab, D], pos [npos, D], optional token types
        [type_vocab, D], the embedding LayerNorm (gain [D], shift [D]), as numpy arrays
        (uploaded) or f32 device tensors; pos_off is the position-id offset (0 for BERT,
        pad_token_id + 1 for RoBERTa / XLM-R)."""
        t, dev = self.torch, self.torch.device("cuda")

        def up(a):  # numpy arrays are uploaded; f32 device tensors are used as they are
            if isinstance(a, t.Tensor):
                if a.device.type != "cuda" or a.dtype != t.float32 or not a.is_contiguous():
                    raise ValueError("set_embeddings: tensors must be contiguous f32 on the device")
                return a
            return t.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)

        self._emb = dict(word=up(word), pos=up(pos), type=None if typ is None else up(typ),
                         ln=(up(ln[0]), up(ln[1])), pos_off=int(pos_off))

    def embeddings(self, ids, S: int, L: int, h, segs=None, stream: int = 0) -> None:
        """h [S*L, D] = LayerNorm(word[id] + pos[i + pos_off] (+ type[seg])) for int32 device ids
        [S*L] (and optional int32 segment ids), bert.go:299-323."""
        e, D = self._emb, self.D
        if e is None:
            raise ValueError("embeddings: call set_embeddings first")
        typ = e["type"]
        self._m("embed_rows")
        self.ctx.embed_rows_dev(ids.data_ptr(), 0 if segs is None else segs.data_ptr(), S, L, e["word"].data_ptr(),
                                e["word"].shape[0], e["pos"].data_ptr(), e["pos"].shape[0], e["pos_off"],
                                0 if typ is None else typ.data_ptr(), 0 if typ is None else typ.shape[0], D,
                                h.data_ptr(), D, stream)
        g, b = e["ln"]
        self._m("embed_ln")
        self.ctx.residual_layer_norm_dev(h.data_ptr(), D, 0, D, S * L, D, g.data_ptr(), b.data_ptr(), LN_EPS, stream)

    def close(self) -> None:
        for entry in self.handles:
            for name in ("qkv", "o", "ffn_up", "ffn_down"):
                self.ctx.release_weight(entry[name][0])
        self.handles = []
        self._bufs = {}

    def fused_attention(self, L: int) -> bool:
        if not self.fused or self.hd not in (32, 64):
            return False
        return L <= 512 or self.ctx.attention_products in (enchip.ATT_FLASH_BF16, enchip.ATT_FLASH_F16)

    # Widest FFN-down input whose GELU moves into the quantization: every width the
    # quantizer takes (enchip_quant_rows_frag_gelu_dev: ldq <= 4096). Measured on MI355X,
    # same process, identical outputs: BERT-base (K = 3072) 8.81 -> 8.52 ms per encode,
    # XLM-R-large (K = 4096) 53.5 -> 51.8 ms per rerank batch.
    GELU_QUANT_MAX_K = 4096

    def gelu_quant_route(self, up_act: int, down: "enchip.Weight", M: int) -> int:
        """The padded K of FFN-down's codes when FFN-up's GELU moves into FFN-down's
        quantization (enchip_quant_rows_frag_gelu_dev: FFN-up stores its pre-activations, the
        quantizer applies the GELU; the same codes, scales and outputs), else 0."""
        if not self.gelu_in_quant or up_act != enchip.ACT_GELU or down.K % 4 != 0:
            return 0
        ok, ldq = self.ctx.frag_route(down, M)
        return ldq if ok and ldq <= self.GELU_QUANT_MAX_K else 0

    def _buffers(self, S: int, L: int):
        key = (S, L)
        if key not in self._bufs:
            t, M = self.torch, S * L
            f = dict(device="cuda", dtype=t.float32)
            sc = (1,) if self.fused_attention(L) else (S, self.H, L, L)
            Mp = (M + 127) // 128 * 128  # fragment-major codes are read up to a multiple of 128 rows
            kp = (max(self.D, self.I) + 63) // 64 * 64  # the widest padded K of the layer's linears
            self._bufs = {key: dict(qkv=t.empty((M, 3 * self.D), **f), scores=t.empty(sc, **f),
                                    ctx=t.empty((M, self.D), **f), out=t.empty((M, self.D), **f),
                                    inter=t.empty((M, self.I), **f), ffn=t.empty((M, self.D), **f),
                                    codes=t.empty(Mp * kp, device="cuda", dtype=t.int8),
                                    ascale=t.empty(M, **f))}
        return self._bufs[key]

    def forward(self, h, S: int, L: int, stream: int = 0) -> None:
        """Runs every layer on h ([S*L, D] f32 on the device), in place, on `stream`."""
        c, D, H, hd, M = self.ctx, self.D, self.H, self.hd, S * L
        if tuple(h.shape) != (M, D) or not h.is_contiguous():
            raise ValueError(f"h must be a contiguous [{M}, {D}] tensor")
        b = self._buffers(S, L)
        qkv, scores, ctxv, out, inter, ffn = b["qkv"], b["scores"], b["ctx"], b["out"], b["inter"], b["ffn"]
        codes, ascale = b["codes"].data_ptr(), b["ascale"].data_ptr()
        q = qkv.data_ptr()
        scale = float(np.float32(1.0 / math.sqrt(hd)))  # encoder/attention.go:86

        def route(w):  # the padded K when LN + quantization can run fused before w, else 0
            if not self.fuse_ln_quant:
                return 0
            ok, ldq = c.frag_route(w, M)
            return ldq if ok and ldq <= D else 0

        def linear(name, w, x, bias, act, dst):  # one W8A8 linear on x [M, K]
            ok, ldq = c.frag_route(w, M)
            if ok:  # the kernels enchip_w8a8_linear_dev launches, as two timed calls
                self._m(name + ".quant")
                c.quant_rows_frag_dev(x.data_ptr(), M, w.K, codes, ldq, ascale, stream)
                self._m(name + ".gemm")
                c.pre_frag_dev(w, codes, ldq, M, ascale, bias.data_ptr(), act, dst.data_ptr(), stream)
            else:
                self._m(name)
                c.linear_dev(w, x.data_ptr(), M, bias.data_ptr(), act, dst.data_ptr(), stream)

        def ln_then(g, s_, y, nxt, label):  # h = LN(h + y); codes for weight nxt when it takes them
            ldq = route(nxt) if nxt is not None else 0
            self._m(label + ("+quant" if ldq else ""))
            if ldq:
                c.residual_layer_norm_quant_dev(h.data_ptr(), D, y.data_ptr(), D, M, D, g.data_ptr(), s_.data_ptr(),
                                                LN_EPS, codes, ldq, ascale, stream)
            else:
                c.residual_layer_norm_dev(h.data_ptr(), D, y.data_ptr(), D, M, D, g.data_ptr(), s_.data_ptr(), LN_EPS,
                                          stream)
            return ldq

        pending = 0  # padded K of codes already quantized for this layer's QKV
        for li, e in enumerate(self.handles):
            w, bias, act = e["qkv"]
            if pending:
                self._m("qkv.gemm")
                c.pre_frag_dev(w, codes, pending, M, ascale, bias.data_ptr(), act, q, stream)
            else:
                linear("qkv", w, h, bias, act, qkv)
            self._m("attention")
            if self.fused_attention(L):
                c.attention_f32_dev(q, q + D * 4, q + 2 * D * 4, 3 * D, ctxv.data_ptr(), D, S, L, H, hd, scale, stream)
            else:
                c.matmul_bt_f32_dev(q, 3 * D, q + D * 4, 3 * D, enchip.B_NK, scores.data_ptr(), L, L, hd, L,
                                    inner=(H, hd, hd, L * L), outer=(S, L * 3 * D, L * 3 * D, H * L * L),
                                    stream=stream)
                c.softmax_rows_scaled_dev(scores.data_ptr(), L, S * H * L, L, scale, stream)
                c.matmul_bt_f32_dev(scores.data_ptr(), L, q + 2 * D * 4, 3 * D, enchip.B_KN, ctxv.data_ptr(), D, L, L,
                                    hd, inner=(H, L * L, hd, hd), outer=(S, H * L * L, L * 3 * D, L * D),
                                    stream=stream)
            w, bias, act = e["o"]
            linear("o", w, ctxv, bias, act, out)
            g, s = e["attn_ln"]
            w, bias, act = e["ffn_up"]
            gq = self.gelu_quant_route(act, e["ffn_down"][0], M)
            up_act = enchip.ACT_NONE if gq else act
            ldq = ln_then(g, s, out, w, "attn_ln")
            if ldq:
                self._m("ffn_up.gemm")
                c.pre_frag_dev(w, codes, ldq, M, ascale, bias.data_ptr(), up_act, inter.data_ptr(), stream)
            else:
                linear("ffn_up", w, h, bias, up_act, inter)
            w, bias, act = e["ffn_down"]
            if gq:  # inter holds FFN-up's pre-activations: GELU them while quantizing
                self._m("ffn_down.gelu_quant")
                c.quant_rows_frag_gelu_dev(inter.data_ptr(), M, w.K, codes, gq, ascale, stream)
                self._m("ffn_down.gemm")
                c.pre_frag_dev(w, codes, gq, M, ascale, bias.data_ptr(), act, ffn.data_ptr(), stream)
            else:
                linear("ffn_down", w, inter, bias, act, ffn)
            g, s = e["out_ln"]
            nxt = self.handles[li + 1]["qkv"][0] if li + 1 < len(self.handles) else None
            pending = ln_then(g, s, ffn, nxt, "out_ln")

    def embed(self, h, S: int, L: int, pooled, stream: int = 0) -> None:
        """forward(), then mean pooling + L2 normalisation of each sequence into pooled [S, D]."""
        self.forward(h, S, L, stream)
        self._m("pool")
        self.ctx.pool_mean_l2_dev(h.data_ptr(), self.D, S, L, self.D, pooled.data_ptr(), self.D, stream)
        self._m("end")

    def rerank(self, h, S: int, L: int, pooler, classifier, logits, stream: int = 0) -> None:
        """forward(), then the cross-encoder head on each sequence's [CLS] row (row 0):
        logits [S, labels] = classifier(tanh(pooler(CLS))). pooler = (W [D, D], b [D]),
        classifier = (W [labels, D], b [labels]), f32 device tensors (PyTorch [out, in])."""
        c, D = self.ctx, self.D
        pw, pb = pooler
        cw, cb = classifier
        labels = cw.shape[0]
        if tuple(pw.shape) != (D, D) or tuple(cw.shape) != (labels, D) or tuple(logits.shape) != (S, labels):
            raise ValueError("rerank: pooler [D, D], classifier [labels, D], logits [S, labels]")
        self.forward(h, S, L, stream)
        self._m("head")
        pooled = self._bufs[(S, L)].setdefault("pooled", self.torch.empty((S, D), device="cuda"))
        # CLS rows are every L-th row of h: pitch L*D
        c.matmul_bt_f32_dev(h.data_ptr(), L * D, pw.data_ptr(), D, enchip.B_NK, pooled.data_ptr(), D, S, D, D,
                            stream=stream)
        c.bias_act_rows_dev(pooled.data_ptr(), D, S, D, pb.data_ptr(), enchip.ACT_TANH, stream)
        c.matmul_bt_f32_dev(pooled.data_ptr(), D, cw.data_ptr(), D, enchip.B_NK, logits.data_ptr(), labels, S, D,
                            labels, stream=stream)
        c.bias_act_rows_dev(logits.data_ptr(), labels, S, labels, cb.data_ptr(), enchip.ACT_NONE, stream)
        self._m("end")
