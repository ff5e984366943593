"""The C ABI library loads and exports exactly what include/enchip.h declares, and
declines cleanly without a device (CPU-only: no compute calls).

The reference's failure contract is "decline -> the caller's CPU path, never wrong
numbers" (encoder/backend_use.go:77-80); an init failure must reach the caller as
an error, as gpu/enccuda/backend.go:97-101 does for NewBackend.
"""
import ctypes
import os
import re

import pytest

from aikit_amd import enchip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "enchip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(enchip_[a-z0-9_]+)\s*\(", src)))


def test_header_matches_binding():
    assert declared_functions() == sorted(enchip.SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(enchip.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version():
    assert enchip.load().enchip_abi_version() == enchip.ABI_VERSION


def _has_gpu():
    lib = enchip.load()
    h = ctypes.c_void_p()
    rc = lib.enchip_open(0, ctypes.byref(h))
    if rc == enchip.OK:
        lib.enchip_close(h)
        return True
    return False


def test_open_without_device_declines_with_message():
    if _has_gpu():
        pytest.skip("a GPU is present: the no-device decline is exercised on CPU hosts")
    with pytest.raises(enchip.EnchipError) as ei:
        enchip.Context(0)
    assert ei.value.code == enchip.ERR_NO_DEVICE
    assert "no HIP device" in str(ei.value)


def test_null_handling():
    lib = enchip.load()
    assert lib.enchip_close(None) == enchip.OK  # idempotent on NULL
    assert lib.enchip_last_error(None)  # never NULL
    assert lib.enchip_open(0, None) == enchip.ERR_ARG
    assert lib.enchip_quant_rows(None, None, 0, 0, None, None) == enchip.ERR_ARG
    assert lib.enchip_w8a8_linear(None, 1, None, 0, None, 0, None, None) == enchip.ERR_ARG
    assert lib.enchip_weight_register(None, None, None, 1, 1, None) == enchip.ERR_ARG
