"""The benchmark workloads: shapes and seeded synthetic inputs.

Shared by bench.py and the tests. Generators use numpy's PCG64 with fixed seeds
(recorded in bench output), so inputs are reproducible across machines.

Config 2 ("isolated W8A8 linear") and config 3 ("small-M GEMV") inputs follow
the benchmark definition: activations ~N(0,1) with 1% of elements x20, int8
weights uniform in [-127,127], per-channel scales uniform in [1e-3,1e-2], bias
~N(0,0.1). The encoder configs use random-init N(0,0.02) f32 weights quantized
per output channel (quantize_weights, the QuantizeRowsInt8 scheme of
linalg/quant.go:24-35) and N(0,0.02) biases.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import numpy as np

ACT_NONE, ACT_GELU = 0, 1


@dataclass(frozen=True)
class EncoderConfig:
    name: str
    layers: int
    hidden: int
    heads: int
    ffn: int
    batch: int
    seq: int
    vocab: int = 30522

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    def linears(self, fused_qkv: bool = True) -> List[Tuple[str, int, int, int]]:
        """(name, K, N, act) of one layer's W8A8 linears in encoder/bert.go:343-368
        order. Q,K,V share one activation quantization (linalg.MatmulBTW8A8Batch),
        so they run as one N=3*hidden GEMM when fused_qkv."""
        D, I = self.hidden, self.ffn
        qkv = [("qkv", D, 3 * D, ACT_NONE)] if fused_qkv else [
            ("q", D, D, ACT_NONE), ("k", D, D, ACT_NONE), ("v", D, D, ACT_NONE)]
        return qkv + [("o", D, D, ACT_NONE), ("ffn_up", D, I, ACT_GELU), ("ffn_down", I, D, ACT_NONE)]

    def int8_ops_per_forward(self) -> int:
        """2*M*N*K summed over every W8A8 linear of the forward."""
        return sum(2 * self.tokens * K * N for _, K, N, _ in self.linears()) * self.layers


MINILM_L6 = EncoderConfig("minilm-l6", layers=6, hidden=384, heads=12, ffn=1536, batch=8, seq=128)
BERT_BASE = EncoderConfig("bert-base", layers=12, hidden=768, heads=12, ffn=3072, batch=64, seq=512)
XLMR_LARGE_CE = EncoderConfig("xlm-r-large-ce", layers=24, hidden=1024, heads=16, ffn=4096, batch=128, seq=512,
                              vocab=250002)

# Config 2 and 3 shapes.
LINEAR_CFG2 = dict(M=4096, K=768, N=3072, act=ACT_GELU)
GEMV_CFG3 = [dict(M=16, K=768, N=768, act=ACT_NONE), dict(M=16, K=768, N=3072, act=ACT_NONE)]


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def activations(g: np.random.Generator, M: int, K: int, outlier_frac: float = 0.01,
                outlier_mult: float = 20.0) -> np.ndarray:
    a = g.standard_normal((M, K), dtype=np.float32)
    if outlier_frac > 0 and M * K > 0:
        n = int(round(outlier_frac * M * K))
        idx = np.unique(g.integers(0, M * K, size=n))  # ~1% of positions, each scaled once
        a.reshape(-1)[idx] *= np.float32(outlier_mult)
    return a


def int8_weights(g: np.random.Generator, N: int, K: int):
    wq = g.integers(-127, 128, size=(N, K), dtype=np.int8)
    ws = g.uniform(1e-3, 1e-2, size=N).astype(np.float32)
    return wq, ws


def bias(g: np.random.Generator, N: int, std: float = 0.1) -> np.ndarray:
    return (g.standard_normal(N) * std).astype(np.float32)


def quantize_weights(w: np.ndarray):
    """QuantizeRowsInt8 (linalg/quant.go:24-35, :43-71) for load-time weight
    preparation of synthetic f32 weights: scale = maxAbs/127 in f32, codes =
    round-half-away-from-zero(v * (1/scale)) clamped to +-127, all-zero row ->
    scale 1. A load-time utility for the harness; the device path receives int8."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    maxabs = np.max(np.abs(w), axis=1)
    safe = np.where(maxabs == 0, np.float32(127), maxabs).astype(np.float32)
    s = (safe / np.float32(127)).astype(np.float32)
    inv = (np.float32(1) / s).astype(np.float32)
    x = (w * inv[:, None]).astype(np.float32).astype(np.float64)
    q = np.trunc(x + np.copysign(0.5, x))
    q = np.clip(q, -127, 127).astype(np.int8)
    q[maxabs == 0] = 0
    s = np.where(maxabs == 0, np.float32(1), s).astype(np.float32)
    return q, s


def encoder_layer_weights(g: np.random.Generator, cfg: EncoderConfig, fused_qkv: bool = True):
    """One layer's quantized weights: {name: (wq[N,K], ws[N], bias[N], act)}."""
    out = {}
    for name, K, N, act in cfg.linears(fused_qkv):
        w = (g.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        wq, ws = quantize_weights(w)
        out[name] = (wq, ws, bias(g, N, 0.02), act)
    return out
