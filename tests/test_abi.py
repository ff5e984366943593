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


def _go_param_types(sig):
    """Go parameter list -> one type per parameter, in order. A type written once covers
    the bare names before it ("wq, wscale unsafe.Pointer" is two unsafe.Pointer)."""
    pieces = [p.strip() for p in sig.replace("\n", " ").split(",") if p.strip()]
    types, pending = [], 0
    for p in pieces:
        words = p.split()
        if len(words) == 1:
            pending += 1
            continue
        types.extend([" ".join(words[1:])] * (pending + 1))
        pending = 0
    assert pending == 0, ("Go parameters without a type", sig)
    return types


def _c_param_types(params):
    """C parameter list -> one normalised type per parameter ("const float *a" ->
    "float*", "enchip_ctx **out" -> "enchip_ctx**")."""
    if params.strip() in ("", "void"):
        return []
    out = []
    for p in params.split(","):
        p = " ".join(p.replace("*", " * ").split())
        words = [w for w in p.split() if w != "const"]
        stars = words.count("*")
        base = [w for w in words if w != "*"][0]
        out.append(base + "*" * stars)
    return out


_GO_SCALAR = {"int32": {"int", "int32_t"}, "int64": {"int64_t"}, "uint64": {"uint64_t", "enchip_weight"},
              "float32": {"float"}, "float64": {"double"}}


def _go_matches_c(go, c):
    """Whether a purego parameter of Go type `go` passes the C parameter `c` with the same
    width and meaning (encoder/backend_use.go:59-83 is the seam the leaf serves)."""
    if go in _GO_SCALAR:
        return c in _GO_SCALAR[go]
    if go == "uintptr":  # the opaque context handle
        return c == "enchip_ctx*"
    if go == "unsafe.Pointer":  # a data buffer: any one-level pointer but the handle
        return c.count("*") == 1 and c != "enchip_ctx*"
    if go == "string":  # purego passes a NUL-terminated copy
        return c == "char*"
    if go.startswith("*"):  # an out-parameter: pointer to the matching scalar
        inner = go[1:]
        if inner == "uintptr":
            return c == "enchip_ctx**"
        return c.endswith("*") and c.count("*") == 1 and _go_matches_c(inner, c[:-1])
    return False


def _leaf_bindings(src):
    """(Go variable, symbol, [Go parameter types], Go result type) per bound function."""
    out = []
    for var, name in re.findall(r'purego\.RegisterLibFunc\(&(\w+), h, "(enchip_\w+)"\)', src):
        m = re.search(r"\b" + var + r"\s+func\(([^)]*)\)\s*([\w.*]*)", src)
        out.append((var, name, _go_param_types(m.group(1)), m.group(2)))
    return out


def _header_signature(hdr, name):
    m = re.search(r"\b([\w ]+?\**)\s*\b" + name + r"\s*\(([^)]*)\)", hdr)
    ret = " ".join(w for w in m.group(1).replace("*", " * ").split() if w != "const").replace(" *", "*")
    return ret, _c_param_types(m.group(2))


def _leaf_mismatches(src, hdr):
    bad = []
    for var, name, go_types, go_ret in _leaf_bindings(src):
        c_ret, c_types = _header_signature(hdr, name)
        if len(go_types) != len(c_types):
            bad.append((name, "arity", len(go_types), len(c_types)))
            continue
        for i, (g, c) in enumerate(zip(go_types, c_types)):
            if not _go_matches_c(g, c):
                bad.append((name, i, g, c))
        if not _go_matches_c(go_ret, c_ret):
            bad.append((name, "result", go_ret, c_ret))
    return bad


def _leaf_source():
    return "".join(open(os.path.join(ROOT, "gpu", "enchip", f)).read() for f in ("backend.go", "ann.go"))


def _header_source():
    return re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "enchip.h")).read(), flags=re.S)


def test_go_leaf_binds_declared_symbols_at_the_abi_version():
    # gpu/enchip (the purego leaf a Go build of aikit imports) binds only symbols the
    # header declares and the library exports, checks the same ABI version the header
    # defines, and passes each bound function the header's parameters position by
    # position at the same width (int32 <-> int, int64 <-> int64_t, uint64 <->
    # enchip_weight, uintptr <-> the context handle, unsafe.Pointer <-> a buffer pointer,
    # *T <-> an out-parameter) with the header's result type. (No Go toolchain exists in
    # this image, so this is the leaf's compile-free check.)
    src, hdr = _leaf_source(), _header_source()
    bound = _leaf_bindings(src)
    assert len(bound) >= 8, "RegisterLibFunc calls not found"
    declared = set(declared_functions())
    lib = ctypes.CDLL(enchip.LIB_PATH)
    for var, name, _, _ in bound:
        assert name in declared and hasattr(lib, name), name
    assert _leaf_mismatches(src, hdr) == []
    version = int(re.search(r"abiVersion\s*=\s*(\d+)", src).group(1))
    hdr_version = int(re.search(r"#define ENCHIP_ABI_VERSION (\d+)", hdr).group(1))
    assert version == hdr_version == enchip.ABI_VERSION


@pytest.mark.parametrize("old,new", [
    ("m int64, bias unsafe.Pointer", "m int32, bias unsafe.Pointer"),  # width: int64_t M as int32
    ("func(ctx uintptr, w uint64) int32", "func(ctx uintptr, w int32) int32"),  # handle width
    ("n, k int64, out *uint64", "n, k int64, out *int64"),  # out-parameter type
    ("cClose          func(ctx uintptr) int32", "cClose          func(ctx unsafe.Pointer) int32"),
    ("cAbiVersion     func() int32", "cAbiVersion     func() int64"),  # result width
])
def test_go_leaf_check_rejects_a_width_mismatch(old, new):
    # The position-by-position check above fails on each plausible binding mistake,
    # planted in a copy of the leaf's source (an arity-only check passes all of them).
    src, hdr = _leaf_source(), _header_source()
    assert src.count(old) == 1, old
    assert _leaf_mismatches(src.replace(old, new), hdr), new
