"""ctypes binding of libenchip.so (the C ABI in include/enchip.h).

This is the Python twin of what the Go leaf ``gpu/enchip`` binds with purego: it
loads the in-tree ``libenchip.so`` and exposes each entry point one to one. It
has no compute path of its own -- when the library is missing, or no device is
present, calls raise; nothing here falls back to the CPU.

torch is imported (when installed) before the library is loaded, so that the
process has one HIP runtime: libenchip.so's ``libamdhip64.so.7`` dependency then
resolves to the runtime torch already loaded, and device pointers from torch
tensors are valid in both.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libenchip.so")

OK, ERR_NO_DEVICE, ERR_ARG, ERR_HIP, ERR_OOM, ERR_HANDLE = range(6)
ACT_NONE, ACT_GELU, ACT_TANH = 0, 1, 2
ATT_F32, ATT_SPLIT_BF16, ATT_FLASH_BF16, ATT_FLASH_F16 = 0, 1, 2, 3  # enchip_att_products
ATT_DEFAULT = ATT_FLASH_F16  # the library's default
B_NK, B_KN = 0, 1  # enchip_matmul_bt_f32_dev b layouts: b[N,K] rows, b[K,N] rows
ABI_VERSION = 3

# Every symbol include/enchip.h declares, with (restype, argtypes).
_vp, _i64, _int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
_SIGNATURES = {
    "enchip_abi_version": (_int, []),
    "enchip_open": (_int, [_int, ctypes.POINTER(_vp)]),
    "enchip_close": (_int, [_vp]),
    "enchip_last_error": (ctypes.c_char_p, [_vp]),
    "enchip_device_info": (_int, [_vp, ctypes.POINTER(_int), ctypes.POINTER(_int), ctypes.c_char_p, _int]),
    "enchip_quant_rows": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "enchip_weight_register": (_int, [_vp, _vp, _vp, _i64, _i64, ctypes.POINTER(ctypes.c_uint64)]),
    "enchip_weight_release": (_int, [_vp, ctypes.c_uint64]),
    "enchip_weight_shape": (_int, [_vp, ctypes.c_uint64, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "enchip_w8a8_linear": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _vp, _int, _vp, _vp]),
    "enchip_w8a8_batch": (_int, [_vp, _vp, _i64, _i64, _vp, _int]),
    "enchip_quant_rows_dev": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "enchip_w8a8_pre_dev": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _i64, _vp, _vp, _int, _vp, _vp]),
    "enchip_w8a8_linear_dev": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _vp, _int, _vp, _vp]),
    "enchip_quant_rows_frag_dev": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "enchip_quant_rows_frag_gelu_dev": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "enchip_matmul_bt_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64]),
    "enchip_weight_image_bytes": (_i64, [_i64, _i64]),
    "enchip_topk_rows_dev": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "enchip_ann_topk": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _i64, _vp, _vp]),
    "enchip_ann_topk_stats": (_int, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "enchip_weight_export": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _vp]),
    "enchip_weight_register_image": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, ctypes.POINTER(ctypes.c_uint64)]),
    "enchip_softmax_rows_scaled_dev": (_int, [_vp, _vp, _i64, _i64, _i64, ctypes.c_float, _vp]),
    "enchip_residual_layer_norm_dev": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp, ctypes.c_double,
                                              _vp]),
    "enchip_pool_mean_l2_dev": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "enchip_bias_act_rows_dev": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp]),
    "enchip_set_attention_products": (_int, [_vp, _int]),
    "enchip_residual_layer_norm_quant_dev": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp, ctypes.c_double,
                                                    _vp, _i64, _vp, _vp]),
    "enchip_embed_rows_dev": (_int, [_vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp,
                                     _i64, _vp]),
    "enchip_attention_f32_dev": (_int, [_vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
                                        _vp]),
    "enchip_matmul_bt_f32_dev": (_int, [_vp, _vp, _i64, _vp, _i64, _int, _vp, _i64, _i64, _i64, _i64, _vp, _vp,
                                        _vp]),
    "enchip_w8a8_pre_frag_dev": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _i64, _vp, _vp, _int, _vp, _vp]),
    "enchip_frag_route": (_int, [_vp, ctypes.c_uint64, _i64, ctypes.POINTER(_i64)]),
    "enchip_gemm_kernel_name": (_int, [_vp, ctypes.c_uint64, _i64, _int, ctypes.c_char_p, _int]),
    "enchip_probe_ceilings": (_int, [_vp, _vp]),
    "enchip_set_small_m": (_int, [_vp, _i64]),
    "enchip_set_scratch_limit": (_int, [_vp, _i64]),
    "enchip_w8a8_linear_noalloc_dev": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _vp, _int, _vp, _vp]),
    "enchip_matmul_bt_q8": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _vp]),
    "enchip_matmul_bt_q8_dev": (_int, [_vp, ctypes.c_uint64, _vp, _i64, _i64, _vp, _i64, _vp]),
}
SYMBOLS = tuple(_SIGNATURES)


class EnchipOp(ctypes.Structure):
    """``enchip_op`` of include/enchip.h."""
    _fields_ = [("w", ctypes.c_uint64), ("bias", _vp), ("act", _int), ("dst", _vp)]


class EnchipCeilings(ctypes.Structure):
    """``enchip_ceilings`` of include/enchip.h."""
    _fields_ = [("hbm_read_gbps", ctypes.c_double), ("hbm_write_gbps", ctypes.c_double),
                ("mfma_i8_tops", ctypes.c_double), ("valu_f32_tops", ctypes.c_double),
                ("mfma_i8_mhz", ctypes.c_double), ("mfma_i8_data_tops", ctypes.c_double),
                ("mfma_i8_data_mhz", ctypes.c_double)]


class EnchipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"enchip error {code}: {msg}")
        self.code = code


_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load libenchip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
    try:  # share torch's HIP runtime when torch is present (see module docstring)
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.enchip_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libenchip ABI {lib.enchip_abi_version()} != binding ABI {ABI_VERSION}")
    _lib = lib
    return lib


class F32Batch(ctypes.Structure):
    """enchip_f32_batch: one batching level of enchip_matmul_bt_f32_dev."""
    _fields_ = [("count", ctypes.c_int64), ("stride_a", ctypes.c_int64), ("stride_b", ctypes.c_int64),
                ("stride_c", ctypes.c_int64)]


def _ptr(x: Optional[np.ndarray]):
    return None if x is None else ctypes.c_void_p(x.ctypes.data)


@dataclass(frozen=True)
class Weight:
    handle: int
    N: int
    K: int


class Context:
    """One enchip context (device + stream + registered weights)."""

    def __init__(self, device: int = 0):
        self._lib = load()
        h = ctypes.c_void_p()
        rc = self._lib.enchip_open(device, ctypes.byref(h))
        if rc != OK:
            raise EnchipError(rc, self._lib.enchip_last_error(None).decode())
        self._h = h
        self.attention_products = ATT_DEFAULT

    # -- lifecycle ------------------------------------------------------------
    def close(self) -> None:
        if self._h:
            self._lib.enchip_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int) -> None:
        if rc != OK:
            raise EnchipError(rc, self._lib.enchip_last_error(self._h).decode())

    @property
    def handle(self):
        return self._h

    # -- queries / knobs --------------------------------------------------------
    def device_info(self) -> dict:
        cus, clk = ctypes.c_int(), ctypes.c_int()
        name = ctypes.create_string_buffer(64)
        self._check(self._lib.enchip_device_info(self._h, ctypes.byref(cus), ctypes.byref(clk), name, 64))
        return {"num_cus": cus.value, "clock_khz": clk.value, "arch": name.value.decode()}

    def gemm_kernel_name(self, w: Weight, M: int, act: int) -> str:
        buf = ctypes.create_string_buffer(128)
        self._check(self._lib.enchip_gemm_kernel_name(self._h, w.handle, M, act, buf, 128))
        return buf.value.decode()

    def probe_ceilings(self) -> dict:
        c = EnchipCeilings()
        self._check(self._lib.enchip_probe_ceilings(self._h, ctypes.byref(c)))
        return {"hbm_read_gbps": c.hbm_read_gbps, "hbm_write_gbps": c.hbm_write_gbps,
                "mfma_i8_tops": c.mfma_i8_tops, "valu_f32_tops": c.valu_f32_tops,
                "mfma_i8_mhz": c.mfma_i8_mhz, "mfma_i8_data_tops": c.mfma_i8_data_tops,
                "mfma_i8_data_mhz": c.mfma_i8_data_mhz}

    def set_small_m(self, max_m: int) -> None:
        self._check(self._lib.enchip_set_small_m(self._h, max_m))

    def set_scratch_limit(self, nbytes: int) -> None:
        """Cap each growable scratch buffer at nbytes (0: no cap); past it calls decline
        with ERR_OOM."""
        self._check(self._lib.enchip_set_scratch_limit(self._h, nbytes))

    def set_attention_products(self, mode: int) -> None:
        """ATT_FLASH_F16 (default), ATT_FLASH_BF16, ATT_SPLIT_BF16 or ATT_F32: how attention_f32_dev
        computes."""
        self._check(self._lib.enchip_set_attention_products(self._h, mode))
        self.attention_products = mode

    # -- host-buffer entry points ----------------------------------------------
    def quant_rows(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=np.float32)
        M, K = a.shape
        aq = np.empty((M, K), np.int8)
        s = np.empty(max(M, 1), np.float32)
        self._check(self._lib.enchip_quant_rows(self._h, _ptr(a), M, K, _ptr(aq), _ptr(s)))
        return aq, s[:M]

    def register_weight(self, wq: np.ndarray, wscale: np.ndarray) -> Weight:
        wq = np.ascontiguousarray(wq, dtype=np.int8)
        wscale = np.ascontiguousarray(wscale, dtype=np.float32)
        N, K = wq.shape
        if wscale.shape != (N,):
            raise ValueError(f"wscale shape {wscale.shape} != ({N},)")
        out = ctypes.c_uint64()
        self._check(self._lib.enchip_weight_register(self._h, _ptr(wq), _ptr(wscale), N, K, ctypes.byref(out)))
        return Weight(out.value, N, K)

    def release_weight(self, w: Weight) -> None:
        self._check(self._lib.enchip_weight_release(self._h, w.handle))

    def topk_rows_dev(self, d_scores: int, ld: int, rows: int, n: int, k: int, d_index: int, ldi: int, d_score: int,
                      lds: int, stream: int = 0) -> None:
        self._check(self._lib.enchip_topk_rows_dev(self._h, d_scores or None, ld, rows, n, k, d_index or None, ldi,
                                                   d_score or None, lds, stream or None))

    def ann_topk(self, index: Weight, queries: np.ndarray, k: int):
        """ann.I8TopKIndex.TopKBatch: (hit_index int32 [M, k], hit_score f32 [M, k]); -1 / NaN pad."""
        q = np.ascontiguousarray(queries, dtype=np.float32)
        M = q.shape[0]
        if q.shape != (M, index.K):
            raise ValueError(f"queries shape {q.shape} != (M, {index.K})")
        hi = np.empty((M, k), np.int32)
        hs = np.empty((M, k), np.float32)
        self._check(self._lib.enchip_ann_topk(self._h, index.handle, _ptr(q), M, k, _ptr(hi), _ptr(hs)))
        return hi, hs

    def ann_topk_stats(self) -> tuple:
        """(calls of ann_topk on the fused route, those of them that fell back to two passes)."""
        fused, fallbacks = _i64(), _i64()
        self._check(self._lib.enchip_ann_topk_stats(self._h, ctypes.byref(fused), ctypes.byref(fallbacks)))
        return fused.value, fallbacks.value

    def weight_image_bytes(self, N: int, K: int) -> int:
        """Bytes of the fragment-major image of an N x K weight (-1: shape refused)."""
        return int(self._lib.enchip_weight_image_bytes(N, K))

    def export_weight(self, w: Weight):
        """(image int8 [bytes], scales f32 [N]): the device's pre-swizzled copy of w."""
        image = np.empty(self.weight_image_bytes(w.N, w.K), np.int8)
        scales = np.empty(w.N, np.float32)
        self._check(self._lib.enchip_weight_export(self._h, w.handle, _ptr(image), image.size, _ptr(scales)))
        return image, scales

    def register_weight_image(self, image: np.ndarray, wscale: np.ndarray, N: int, K: int) -> Weight:
        """Registers a pre-swizzled image (export_weight / weight_cache.frag_image) as is."""
        image = np.ascontiguousarray(image, dtype=np.int8).reshape(-1)
        wscale = np.ascontiguousarray(wscale, dtype=np.float32)
        if wscale.shape != (N,):
            raise ValueError(f"wscale shape {wscale.shape} != ({N},)")
        out = ctypes.c_uint64()
        self._check(self._lib.enchip_weight_register_image(self._h, _ptr(image), image.size, _ptr(wscale), N, K,
                                                           ctypes.byref(out)))
        return Weight(out.value, N, K)

    def weight_shape(self, w: Weight):
        n, k = ctypes.c_int64(), ctypes.c_int64()
        self._check(self._lib.enchip_weight_shape(self._h, w.handle, ctypes.byref(n), ctypes.byref(k)))
        return n.value, k.value

    def linear(self, w: Weight, a: np.ndarray, bias: Optional[np.ndarray] = None, act: int = ACT_NONE,
               want_acc: bool = False):
        a = np.ascontiguousarray(a, dtype=np.float32)
        M = a.shape[0]
        if a.shape != (M, w.K):
            raise ValueError(f"a shape {a.shape} != (M, {w.K})")
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        dst = np.empty((M, w.N), np.float32)
        acc = np.empty((M, w.N), np.int32) if want_acc else None
        self._check(self._lib.enchip_w8a8_linear(self._h, w.handle, _ptr(a), M, _ptr(b), act, _ptr(dst), _ptr(acc)))
        return (dst, acc) if want_acc else dst

    def batch(self, a: np.ndarray, ops: Sequence[tuple]):
        """ops: sequence of (Weight, bias-or-None, act). Returns one dst per op."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        M, K = a.shape
        keep, arr = [], (EnchipOp * max(len(ops), 1))()
        outs = []
        for i, (w, bias, act) in enumerate(ops):
            b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
            d = np.empty((M, w.N), np.float32)
            keep.append(b)
            outs.append(d)
            arr[i] = EnchipOp(w.handle, None if b is None else b.ctypes.data, act, d.ctypes.data)
        self._check(self._lib.enchip_w8a8_batch(self._h, _ptr(a), M, K, ctypes.cast(arr, ctypes.c_void_p), len(ops)))
        return outs

    # -- device-resident entry points (raw device pointers as ints) ------------
    def quant_rows_dev(self, d_a: int, M: int, K: int, d_aq: int, d_ascale: int, stream: int = 0,
                       ldq: Optional[int] = None) -> None:
        self._check(self._lib.enchip_quant_rows_dev(self._h, d_a, M, K, d_aq, K if ldq is None else ldq,
                                                    d_ascale, stream or None))

    def pre_dev(self, w: Weight, d_aq: int, ldq: int, M: int, d_ascale: int, d_bias: int, act: int, d_dst: int,
                stream: int = 0) -> None:
        self._check(self._lib.enchip_w8a8_pre_dev(self._h, w.handle, d_aq, ldq, M, d_ascale, d_bias or None, act,
                                                  d_dst, stream or None))

    def frag_route(self, w: Weight, M: int):
        """(ok, ldq): whether a linear on w with M rows takes fragment-major codes, and the
        pitch (padded K) the frag entry points take."""
        ldq = _i64(0)
        ok = self._lib.enchip_frag_route(self._h, w.handle, M, ctypes.byref(ldq))
        return bool(ok == 1), int(ldq.value)

    def quant_rows_frag_dev(self, d_a: int, M: int, K: int, d_aq: int, ldq: int, d_ascale: int,
                            stream: int = 0) -> None:
        self._check(self._lib.enchip_quant_rows_frag_dev(self._h, d_a, M, K, d_aq, ldq, d_ascale, stream or None))

    def quant_rows_frag_gelu_dev(self, d_a: int, M: int, K: int, d_aq: int, ldq: int, d_ascale: int,
                                 stream: int = 0) -> None:
        """quant_rows_frag_dev of GELUF32(d_a), from the pre-activations d_a."""
        self._check(self._lib.enchip_quant_rows_frag_gelu_dev(self._h, d_a, M, K, d_aq, ldq, d_ascale,
                                                              stream or None))

    def matmul_bt_f32(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        """encoder.Backend.MatmulBT (encoder/backend.go:19-28): f32 a[M,K] . b[N,K]^T on the device."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[1]:
            raise ValueError(f"matmul_bt_f32: a {a.shape} and b {b.shape} must be [M,K] and [N,K]")
        M, K = a.shape
        N = b.shape[0]
        dst = np.empty((M, N), np.float32)
        self._check(self._lib.enchip_matmul_bt_f32(self._h, _ptr(a), _ptr(b), _ptr(dst), M, K, N))
        return dst

    def matmul_bt_f32_dev(self, d_a: int, lda: int, d_b: int, ldb: int, b_layout: int, d_c: int, ldc: int,
                          M: int, K: int, N: int, inner: Optional[tuple] = None, outer: Optional[tuple] = None,
                          stream: int = 0) -> None:
        """Batched device MatmulBT; inner / outer are (count, stride_a, stride_b, stride_c) in
        floats, None for one problem."""
        lv = [None if t is None else ctypes.byref(F32Batch(*t)) for t in (inner, outer)]
        self._check(self._lib.enchip_matmul_bt_f32_dev(self._h, d_a or None, lda, d_b or None, ldb, b_layout,
                                                       d_c or None, ldc, M, K, N, lv[0], lv[1], stream or None))

    def matmul_bt_q8(self, w: Weight, a: np.ndarray) -> np.ndarray:
        """encoder.Q8Backend.MatmulBTQ8 (encoder/backend_use.go:59-83): f32 a[M,K] times the
        registered weight w widened, a . (f32(wq) * wscale)^T; the activations stay f32."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        M = a.shape[0] if a.ndim == 2 else -1
        if a.shape != (M, w.K):
            raise ValueError(f"matmul_bt_q8: a shape {a.shape} != (M, {w.K})")
        dst = np.empty((M, w.N), np.float32)
        self._check(self._lib.enchip_matmul_bt_q8(self._h, w.handle, _ptr(a), M, _ptr(dst)))
        return dst

    def matmul_bt_q8_dev(self, w: Weight, d_a: int, lda: int, M: int, d_dst: int, ldd: int,
                         stream: int = 0) -> None:
        self._check(self._lib.enchip_matmul_bt_q8_dev(self._h, w.handle, d_a or None, lda, M, d_dst or None, ldd,
                                                      stream or None))

    def softmax_rows_scaled_dev(self, d_x: int, ld: int, rows: int, cols: int, scale: float, stream: int = 0) -> None:
        self._check(self._lib.enchip_softmax_rows_scaled_dev(self._h, d_x or None, ld, rows, cols, scale,
                                                             stream or None))

    def residual_layer_norm_dev(self, d_h: int, ldh: int, d_y: int, ldy: int, rows: int, D: int, d_w: int, d_b: int,
                                eps: float, stream: int = 0) -> None:
        self._check(self._lib.enchip_residual_layer_norm_dev(self._h, d_h or None, ldh, d_y or None, ldy, rows, D,
                                                             d_w or None, d_b or None, eps, stream or None))

    def residual_layer_norm_quant_dev(self, d_h: int, ldh: int, d_y: int, ldy: int, rows: int, D: int, d_w: int,
                                      d_b: int, eps: float, d_aq: int, ldq: int, d_ascale: int,
                                      stream: int = 0) -> None:
        self._check(self._lib.enchip_residual_layer_norm_quant_dev(self._h, d_h or None, ldh, d_y or None, ldy, rows, D,
                                                                   d_w or None, d_b or None, eps, d_aq or None, ldq,
                                                                   d_ascale or None, stream or None))

    def embed_rows_dev(self, d_ids: int, d_segs: int, nseq: int, L: int, d_word: int, vocab: int, d_pos: int,
                       npos: int, pos_off: int, d_type: int, type_vocab: int, D: int, d_h: int, ldh: int,
                       stream: int = 0) -> None:
        self._check(self._lib.enchip_embed_rows_dev(self._h, d_ids or None, d_segs or None, nseq, L, d_word or None,
                                                    vocab, d_pos or None, npos, pos_off, d_type or None, type_vocab,
                                                    D, d_h or None, ldh, stream or None))

    def bias_act_rows_dev(self, d_x: int, ld: int, rows: int, cols: int, d_bias: int, act: int,
                          stream: int = 0) -> None:
        self._check(self._lib.enchip_bias_act_rows_dev(self._h, d_x or None, ld, rows, cols, d_bias or None, act,
                                                       stream or None))

    def attention_f32_dev(self, d_q: int, d_k: int, d_v: int, ld: int, d_out: int, ldo: int, nseq: int, L: int,
                          heads: int, head_dim: int, scale: float, stream: int = 0) -> None:
        self._check(self._lib.enchip_attention_f32_dev(self._h, d_q or None, d_k or None, d_v or None, ld,
                                                       d_out or None, ldo, nseq, L, heads, head_dim, scale,
                                                       stream or None))

    def pool_mean_l2_dev(self, d_h: int, ldh: int, nseq: int, L: int, D: int, d_out: int, ldo: int,
                         stream: int = 0) -> None:
        self._check(self._lib.enchip_pool_mean_l2_dev(self._h, d_h or None, ldh, nseq, L, D, d_out or None, ldo,
                                                      stream or None))

    def pre_frag_dev(self, w: Weight, d_aq: int, ldq: int, M: int, d_ascale: int, d_bias: int, act: int, d_dst: int,
                     stream: int = 0) -> None:
        self._check(self._lib.enchip_w8a8_pre_frag_dev(self._h, w.handle, d_aq, ldq, M, d_ascale, d_bias or None, act,
                                                       d_dst, stream or None))

    def linear_noalloc_dev(self, w: Weight, d_a: int, M: int, d_bias: int, act: int, d_dst: int,
                           stream: int = 0) -> None:
        """linear_dev through the library's fixed per-device scratch (no allocation)."""
        self._check(self._lib.enchip_w8a8_linear_noalloc_dev(self._h, w.handle, d_a, M, d_bias or None, act, d_dst,
                                                             stream or None))

    def linear_dev(self, w: Weight, d_a: int, M: int, d_bias: int, act: int, d_dst: int, stream: int = 0) -> None:
        self._check(self._lib.enchip_w8a8_linear_dev(self._h, w.handle, d_a, M, d_bias or None, act, d_dst,
                                                     stream or None))
