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


def test_go_leaf_binds_declared_symbols_at_the_abi_version():
    # gpu/enchip (the purego leaf a Go build of aikit imports) binds only symbols the
    # header declares and the library exports, checks the same ABI version the header
    # defines, and passes each bound function the header's number of arguments. (No Go
    # toolchain exists in this image, so this is the leaf's compile-free check.)
    src = "".join(open(os.path.join(ROOT, "gpu", "enchip", f)).read() for f in ("backend.go", "ann.go"))
    bound = re.findall(r'purego\.RegisterLibFunc\(&(\w+), h, "(enchip_\w+)"\)', src)
    assert bound, "no RegisterLibFunc calls found"
    declared = set(declared_functions())
    lib = ctypes.CDLL(enchip.LIB_PATH)
    hdr = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "enchip.h")).read(), flags=re.S)
    for var, name in bound:
        assert name in declared and hasattr(lib, name), name
        params = re.search(r"\b" + name + r"\s*\(([^)]*)\)", hdr).group(1).strip()
        n_c = 0 if params in ("", "void") else params.count(",") + 1
        sig = re.search(r"\b" + var + r"\s+func\(([^)]*)\)", src).group(1)
        # each comma-separated piece of a Go parameter list names one parameter
        # ("wq, wscale unsafe.Pointer" is two)
        n_go = len([p for p in sig.split(",") if p.strip()])
        assert n_go == n_c, (name, n_go, n_c)
    version = int(re.search(r"abiVersion\s*=\s*(\d+)", src).group(1))
    hdr_version = int(re.search(r"#define ENCHIP_ABI_VERSION (\d+)", hdr).group(1))
    assert version == hdr_version == enchip.ABI_VERSION
