"""Pre-swizzled weight images on the host (no GPU): the numpy image builder against the
layout formula the ABI documents (include/enchip.h, enchip_weight_register_image), and the
safetensors file round trip. The device side is in tests/test_gpu_parity.py."""
import numpy as np
import pytest

from aikit_amd import weight_cache


@pytest.mark.parametrize("N,K", [(1, 1), (33, 17), (70, 100), (256, 64), (300, 768)])
def test_frag_image_follows_the_layout_formula(N, K):
    g = np.random.default_rng(N * 1000 + K)
    wq = g.integers(-127, 128, size=(N, K), dtype=np.int8)
    img = weight_cache.frag_image(wq)
    Np, Kp = weight_cache.padded_shape(N, K)
    assert img.shape == (Np * Kp,) and img.dtype == np.int8
    n, k = np.meshgrid(np.arange(N), np.arange(K), indexing="ij")
    off = ((n // 32) * (Kp // 32) + k // 32) * 1024 + ((n % 32) + 32 * ((k // 16) % 2)) * 16 + k % 16
    assert np.array_equal(img[off], wq)
    mask = np.ones(img.size, bool)
    mask[off.reshape(-1)] = False
    assert not img[mask].any(), "padding must be zero"


def test_safetensors_round_trip(tmp_path):
    from safetensors import safe_open

    g = np.random.default_rng(3)
    ws = {"l0.qkv": (g.integers(-127, 128, size=(96, 64), dtype=np.int8), g.uniform(1e-3, 1e-2, 96).astype(np.float32)),
          "l0.o": (g.integers(-127, 128, size=(64, 40), dtype=np.int8), g.uniform(1e-3, 1e-2, 64).astype(np.float32))}
    path = str(tmp_path / "w.safetensors")
    weight_cache.save(path, ws)
    with safe_open(path, framework="numpy") as f:
        meta = f.metadata()
        assert meta["layout"] == weight_cache.LAYOUT
        for name, (wq, s) in ws.items():
            assert meta[f"{name}.shape"] == f"{wq.shape[0]},{wq.shape[1]}"
            assert np.array_equal(f.get_tensor(f"{name}.frag"), weight_cache.frag_image(wq))
            assert np.array_equal(f.get_tensor(f"{name}.scales"), s)
