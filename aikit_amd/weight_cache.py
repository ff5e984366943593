"""Pre-swizzled int8 weight files: convert a model's W8A8 weights once, then register them
straight from a memory-mapped safetensors file (enchip_weight_register_image), skipping
both load-time quantization and the per-byte host swizzle.

This is the device side of the reference's pre-quantized int8 loading path: int8 codes
wrapped without re-quantizing (linalg.WrapInt8, linalg/weightmat.go:81-88) and read from a
read-only mapping (embed.OpenSafetensorsMmap, embed/safetensors.go:290-305;
WeightMat.MappedSpan, linalg/weightmat.go:215-231).

File format: a safetensors file whose tensors are, per weight name,
  "<name>.frag"   int8 [Np*Kp]  the fragment-major image (see frag_image)
  "<name>.scales" float32 [N]   per-output-channel scales
and whose metadata holds "<name>.shape" = "N,K" and "layout" = LAYOUT.
"""
from __future__ import annotations

from typing import Dict, Tuple

import numpy as np

LAYOUT = "enchip-frag-v1: byte (n,k) at ((n/32)*(Kp/32)+k/32)*1024+((n%32)+32*((k/16)%2))*16+k%16, Np=ceil256(N), Kp=ceil64(K)"


def padded_shape(N: int, K: int) -> Tuple[int, int]:
    return (N + 255) // 256 * 256, (max(K, 1) + 63) // 64 * 64


def frag_image(wq: np.ndarray) -> np.ndarray:
    """The fragment-major image of int8 weights wq [N, K] (the layout enchip_weight_register
    builds on upload), computed on the host with numpy: for offline conversion."""
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    N, K = wq.shape
    Np, Kp = padded_shape(N, K)
    pad = np.zeros((Np, Kp), np.int8)
    pad[:N, :K] = wq
    # [Np/32, 32 rows, Kp/32, 2 halves, 16 bytes] -> [Np/32, Kp/32, 2 halves, 32 rows, 16 bytes]
    t = pad.reshape(Np // 32, 32, Kp // 32, 2, 16).transpose(0, 2, 3, 1, 4)
    return np.ascontiguousarray(t).reshape(-1)


def save(path: str, weights: Dict[str, Tuple[np.ndarray, np.ndarray]]) -> None:
    """Writes {name: (wq int8 [N, K], scales f32 [N])} as pre-swizzled images."""
    from safetensors.numpy import save_file

    tensors, meta = {}, {"layout": LAYOUT}
    for name, (wq, ws) in weights.items():
        wq = np.asarray(wq)
        N, K = wq.shape
        ws = np.ascontiguousarray(ws, dtype=np.float32)
        if ws.shape != (N,):
            raise ValueError(f"{name}: scales shape {ws.shape} != ({N},)")
        tensors[f"{name}.frag"] = frag_image(wq)
        tensors[f"{name}.scales"] = ws
        meta[f"{name}.shape"] = f"{N},{K}"
    save_file(tensors, path, metadata=meta)


def load(ctx, path: str):
    """Registers every weight of a file written by save(): {name: enchip.Weight}. The file
    is read through safetensors' memory mapping; refuses a file of another layout."""
    from safetensors import safe_open

    out = {}
    with safe_open(path, framework="numpy") as f:
        meta = f.metadata() or {}
        if meta.get("layout") != LAYOUT:
            raise ValueError(f"{path}: layout {meta.get('layout')!r} is not {LAYOUT!r}")
        for key in meta:
            if not key.endswith(".shape"):
                continue
            name = key[:-len(".shape")]
            N, K = (int(v) for v in meta[key].split(","))
            image = f.get_tensor(f"{name}.frag")
            scales = f.get_tensor(f"{name}.scales")
            try:
                out[name] = ctx.register_weight_image(image, scales, N, K)
            except Exception:
                for w in out.values():
                    ctx.release_weight(w)
                raise
    return out
