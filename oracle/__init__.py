"""CPU oracle for the W8A8 linear path -- TEST INFRASTRUCTURE, not the product.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or, for the baseline, as
the timed CPU restatement). The product path (``aikit_amd``) never calls it.

``liboracle.so`` is built from ``oracle.c`` (a scalar restatement of aikit's Go
``linalg``/``encoder`` arithmetic, each function citing the reference file:line)
and ``cpu_baseline.c`` (the reference's AVX2 W8A8 CPU path) by ``Makefile``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_quantize_row": (ctypes.c_float, [_f32p, _i8p, _i64, ctypes.c_float]),
            "orc_quantize_rows_weights": (None, [_f32p, _i64, _i64, _i8p, _f32p]),
            "orc_quantize_activations": (None, [_f32p, _i64, _i64, _i8p, _f32p]),
            "orc_dot_i8": (ctypes.c_int32, [_i8p, _i8p, _i64]),
            "orc_acc_i32": (None, [_i8p, _i8p, _i32p, _i64, _i64, _i64]),
            "orc_w8a8_span": (None, [_i8p, _f32p, _i8p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64]),
            "orc_matmul_bt_w8a8": (None, [_f32p, _i8p, _f32p, _f32p, _i64, _i64, _i64]),
            "orc_add_bias": (None, [_f32p, ctypes.c_void_p, _i64, _i64]),
            "orc_exp_f32_core": (ctypes.c_float, [ctypes.c_float]),
            "orc_exp_f32": (ctypes.c_float, [ctypes.c_float]),
            "orc_erf_f32": (ctypes.c_float, [ctypes.c_float]),
            "orc_gelu_f32": (ctypes.c_float, [ctypes.c_float]),
            "orc_tanh_f32": (ctypes.c_float, [ctypes.c_float]),
            "orc_gelu_into": (None, [_f32p, _i64]),
            "orc_tanh_into": (None, [_f32p, _i64]),
            "orc_erf_into": (None, [_f32p, _i64]),
            "orc_exp_into": (None, [_f32p, _i64]),
            "orc_w8a8_linear": (None, [_f32p, _i64, _i64, _i8p, _f32p, _i64, ctypes.c_void_p, ctypes.c_int, _f32p]),
            "orc_layer_norm": (None, [_f32p, _f32p, _f32p, _i64, _i64, ctypes.c_double]),
            "orc_softmax_row_scaled": (None, [_f32p, _i64, ctypes.c_float]),
            "orc_attention": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64]),
            "orc_matmul_bt_f64": (None, [_f32p, _f32p, _i64, _i64, _i64,
                                         np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")]),
            "orc_dequant_rows_i8": (None, [_i8p, _f32p, _i64, _i64, _f32p]),
            "orc_matmul_bt_q8_f64": (None, [_f32p, _i8p, _f32p, _i64, _i64, _i64,
                                            np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")]),
            "orc_pool_mean": (None, [_f32p, _i64, _i64, _f32p]),
            "orc_l2_normalize": (None, [_f32p, _i64]),
            "cpub_dot_i8": (ctypes.c_int32, [_i8p, _i8p, _i64]),
            "cpub_attention": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, ctypes.c_int]),
            "cpub_matmul_bt_w8a8": (None, [_f32p, _i8p, _f32p, _f32p, _i64, _i64, _i64, ctypes.c_int, _i8p, _f32p]),
            "cpub_w8a8_linear": (None, [_f32p, _i64, _i64, _i8p, _f32p, _i64, ctypes.c_void_p, ctypes.c_int,
                                        _f32p, ctypes.c_int, _i8p, _f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _c(x, dt):
    return np.ascontiguousarray(x, dtype=dt)


def _ptr_or_null(x):
    return None if x is None else x.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- quantization
def quantize_row(row, zero_scale: float):
    row = _c(row, np.float32)
    q = np.empty(row.size, np.int8)
    s = lib().orc_quantize_row(row, q, row.size, zero_scale)
    return q, np.float32(s)


def quantize_rows_weights(w, rows: int, cols: int):
    """QuantizeRowsInt8 (linalg/quant.go:24-35): all-zero row -> scale 1."""
    w = _c(w, np.float32).reshape(-1)
    q = np.empty(rows * cols, np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_quantize_rows_weights(w, rows, cols, q, s)
    return q.reshape(rows, cols), s


def quantize_activations(a, M: int, K: int):
    """QuantizeActivationsInto (linalg/quant.go:206-213): all-zero row -> scale 0."""
    a = _c(a, np.float32).reshape(-1)
    q = np.empty(max(M * K, 1), np.int8)
    s = np.empty(max(M, 1), np.float32)
    lib().orc_quantize_activations(a, M, K, q, s)
    return q[: M * K].reshape(M, K), s[:M]


# ---------------------------------------------------------------- integer GEMM
def dot_i8(a, b) -> int:
    a, b = _c(a, np.int8), _c(b, np.int8)
    return int(lib().orc_dot_i8(a, b, a.size))


def acc_i32(aq, bq, M: int, K: int, N: int):
    out = np.empty(max(M * N, 1), np.int32)
    lib().orc_acc_i32(_c(aq, np.int8).reshape(-1), _c(bq, np.int8).reshape(-1), out, M, K, N)
    return out[: M * N].reshape(M, N)


def w8a8_span(aq, ascales, bq, bscales, M, K, N):
    dst = np.empty(max(M * N, 1), np.float32)
    lib().orc_w8a8_span(_c(aq, np.int8).reshape(-1), _c(ascales, np.float32), _c(bq, np.int8).reshape(-1),
                        _c(bscales, np.float32), dst, M, K, N, 0, N)
    return dst[: M * N].reshape(M, N)


def matmul_bt_w8a8(a, bq, bscales, M, K, N):
    dst = np.empty(max(M * N, 1), np.float32)
    lib().orc_matmul_bt_w8a8(_c(a, np.float32).reshape(-1), _c(bq, np.int8).reshape(-1),
                             _c(bscales, np.float32), dst, M, K, N)
    return dst[: M * N].reshape(M, N)


def w8a8_linear(a, bq, bscales, bias, act: int, M: int, K: int, N: int):
    """MatmulBTW8A8Into + addBias + (act==1) GELU, the BERT composition."""
    dst = np.empty(max(M * N, 1), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().orc_w8a8_linear(_c(a, np.float32).reshape(-1), M, K, _c(bq, np.int8).reshape(-1),
                          _c(bscales, np.float32), N, _ptr_or_null(b), act, dst)
    return dst[: M * N].reshape(M, N)


def add_bias(dst, bias, M, N):
    dst = _c(dst, np.float32).copy().reshape(-1)
    b = None if bias is None else _c(bias, np.float32)
    lib().orc_add_bias(dst, _ptr_or_null(b), M, N)
    return dst.reshape(M, N)


# ---------------------------------------------------------------- elementwise
def gelu(x):
    x = _c(x, np.float32).copy()
    flat = x.reshape(-1)
    lib().orc_gelu_into(flat, flat.size)
    return x


def tanh(x):
    x = _c(x, np.float32).copy()
    flat = x.reshape(-1)
    lib().orc_tanh_into(flat, flat.size)
    return x


def erf_vec(x):
    x = _c(x, np.float32).copy()
    lib().orc_erf_into(x.reshape(-1), x.size)
    return x


def exp_vec(x):
    x = _c(x, np.float32).copy()
    lib().orc_exp_into(x.reshape(-1), x.size)
    return x


def exp_f32(x: float) -> np.float32:
    return np.float32(lib().orc_exp_f32(float(x)))


def exp_f32_core(x: float) -> np.float32:
    return np.float32(lib().orc_exp_f32_core(float(x)))


def erf_f32(x: float) -> np.float32:
    return np.float32(lib().orc_erf_f32(float(x)))


# ---------------------------------------------------------------- encoder glue
def layer_norm(x, w, b, L, D, eps):
    x = _c(x, np.float32).copy().reshape(-1)
    lib().orc_layer_norm(x, _c(w, np.float32), _c(b, np.float32), L, D, eps)
    return x.reshape(L, D)


def softmax_row_scaled(row, scale):
    row = _c(row, np.float32).copy()
    lib().orc_softmax_row_scaled(row, row.size, scale)
    return row


def attention(Q, K, V, L, D, heads):
    ctx = np.empty(L * D, np.float32)
    lib().orc_attention(_c(Q, np.float32).reshape(-1), _c(K, np.float32).reshape(-1),
                        _c(V, np.float32).reshape(-1), ctx, L, D, heads)
    return ctx.reshape(L, D)


def matmul_bt_f64(a, b, M: int, K: int, N: int):
    """refMatmulBT (gpu/enccuda/backend_test.go:32-44): float64 a[M,K] . b[N,K]^T."""
    dst = np.empty(max(M * N, 1), np.float64)
    lib().orc_matmul_bt_f64(_c(a, np.float32).reshape(-1), _c(b, np.float32).reshape(-1), M, K, N, dst)
    return dst[: M * N].reshape(M, N)


def dequant_rows_i8(q, scales, rows: int, cols: int):
    """DequantizeRowsInt8Into (linalg/dequant_i8.go:20-43): float32(q) * scale per row."""
    dst = np.empty(max(rows * cols, 1), np.float32)
    lib().orc_dequant_rows_i8(_c(q, np.int8).reshape(-1), _c(scales, np.float32).reshape(-1), rows, cols, dst)
    return dst[: rows * cols].reshape(rows, cols)


def matmul_bt_q8_f64(a, q, scales, M: int, K: int, N: int):
    """cpuQ8Ref (gpu/enccuda/backend_test.go:208-224): float64 a[M,K] . (q[N,K] * scales[N])^T."""
    dst = np.empty(max(M * N, 1), np.float64)
    lib().orc_matmul_bt_q8_f64(_c(a, np.float32).reshape(-1), _c(q, np.int8).reshape(-1),
                               _c(scales, np.float32).reshape(-1), M, K, N, dst)
    return dst[: M * N].reshape(M, N)


def matmul_bt_worst_rel(got, ref) -> float:
    """The f32 MatmulBT gate's statistic (gpu/enccuda/backend_test.go:71-80): the worst
    |got - ref| / max(|ref|, 1) over all elements; the gate is <= 2e-4."""
    ref = np.asarray(ref, np.float64)
    den = np.maximum(np.abs(ref), 1.0)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref) / den)) if ref.size else 0.0


def pool_mean(seq, L, D):
    out = np.empty(D, np.float32)
    lib().orc_pool_mean(_c(seq, np.float32).reshape(-1), L, D, out)
    return out


def l2_normalize(v):
    v = _c(v, np.float32).copy()
    lib().orc_l2_normalize(v, v.size)
    return v


# ---------------------------------------------------------------- CPU baseline
def cpu_w8a8_linear(a, bq, bscales, bias, act, M, K, N, workers: int, dst=None, aq=None, ascales=None):
    """The reference's AVX2 W8A8 path (cpu_baseline.c) over `workers` threads."""
    if dst is None:
        dst = np.empty(M * N, np.float32)
    if aq is None:
        aq = np.empty(max(M * K, 1), np.int8)
    if ascales is None:
        ascales = np.empty(max(M, 1), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().cpub_w8a8_linear(_c(a, np.float32).reshape(-1), M, K, _c(bq, np.int8).reshape(-1),
                           _c(bscales, np.float32), N, _ptr_or_null(b), act, dst.reshape(-1), workers,
                           aq, ascales)
    return dst.reshape(M, N)


def cpu_attention(Q, K, V, L, D, heads, workers: int):
    """orc_attention over `workers` threads (cpu_baseline.c), bit-identical to attention()."""
    ctx = np.empty(max(L * D, 1), np.float32)
    lib().cpub_attention(_c(Q, np.float32).reshape(-1), _c(K, np.float32).reshape(-1),
                         _c(V, np.float32).reshape(-1), ctx, L, D, heads, workers)
    return ctx[: L * D].reshape(L, D)


def cpu_dot_i8(a, b) -> int:
    a, b = _c(a, np.int8), _c(b, np.int8)
    return int(lib().cpub_dot_i8(a, b, a.size))


# ---------------------------------------------------------------- top-k (ann)
def top_hits_selector(scores, k: int):
    """FlatI8.topHits (ann/flat_i8.go:208-242) for k < len(scores), as the reference runs
    it: topk.Selector (topk/topk.go:44-48,85-125: a min-heap on (score asc, seq desc),
    NaN rejected, a candidate kept only if strictly above the minimum, pushed in index
    order with the hoisted threshold), then sorted by topk.Cmp (topk/cmp.go:15-27: score
    descending, index ascending). Pure Python: for small inputs. Returns [(index, score)]."""
    import heapq

    heap = []  # entries (score, -seq, index): heapq's minimum is the reference's heap[0]
    seq = 0
    for i, s in enumerate(np.asarray(scores, np.float32).tolist()):
        if s != s:
            continue
        if len(heap) < k:
            heapq.heappush(heap, (s, -seq, i))
        elif s > heap[0][0]:
            heapq.heapreplace(heap, (s, -seq, i))
        seq += 1
    return sorted(((i, s) for s, _, i in heap), key=lambda t: (-t[1], t[0]))


def top_hits(scores, k: int):
    """The same selection in closed form (numpy): the k largest non-NaN scores, ordered
    by score descending then index ascending (float32 -0 equals +0). Returns
    (index int64 [<=k], score float32 [<=k])."""
    s = np.asarray(scores, np.float32)
    idx = np.flatnonzero(~np.isnan(s))
    order = np.lexsort((idx, -s[idx].astype(np.float64)))
    keep = idx[order[:k]]
    return keep, s[keep]
