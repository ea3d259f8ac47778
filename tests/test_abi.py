"""The C ABI: libvnx_hip.so loads, exports every function include/vnx.h declares,
its ctypes signatures match the header, and host-side argument checks reject
bad calls before anything is launched (no GPU needed for any of this)."""
import ctypes
import os
import re

import pytest

from versenext_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vnx.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vnx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_functions():
    fns = header_functions()
    assert "vnx_spec_accept" in fns and "vnx_init" in fns and len(fns) >= 10


def test_library_exports_every_header_symbol():
    L = _lib.lib()
    for name in header_functions():
        assert hasattr(L, name), f"{name} declared in include/vnx.h but not exported"


def test_ctypes_signatures_cover_header():
    assert set(_lib.SIGNATURES) == set(header_functions())


def test_integration_guide_names_every_header_function():
    """The integration guide (INTEGRATION.md at the repository root) names
    every function the header declares, so a maintainer wiring the reference
    finds each entry point's role there."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    named = set(re.findall(r"\b(vnx_[a-z0-9_]+)\b", text))
    missing = [f for f in header_functions() if f not in named]
    assert not missing, f"not named in INTEGRATION.md: {missing}"


def header_prototypes():
    """{name: (return type, [parameter types])} of every function include/vnx.h
    declares, with qualifiers kept ('const float*', 'int64_t', ...)."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b(vnx_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        types = []
        for prm in params.split(","):
            prm = prm.strip()
            if prm and prm != "void":
                types.append(re.sub(r"\b[A-Za-z_][A-Za-z0-9_]*$", "", prm).replace(" *", "*").strip())
        out[name] = (ret.strip(), types)
    return out


def _ctype_of(c: str):
    """The ctypes type a header type binds to: every data pointer as
    c_void_p (device or host addresses), const char* as c_char_p."""
    if c == "const char*":
        return ctypes.c_char_p
    if c.endswith("*"):
        return ctypes.c_void_p
    return {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "size_t": ctypes.c_size_t, "float": ctypes.c_float,
            "double": ctypes.c_double, "int32_t": ctypes.c_int32}[c]


def test_ctypes_argtypes_match_header_parameter_types():
    """Every binding's restype and argtypes equal the header prototype's
    parameter types one by one (a pointer parameter may also bind a ctypes
    POINTER to the structure the header names)."""
    protos = header_prototypes()
    assert set(protos) == set(header_functions())
    for name, (ret, params) in protos.items():
        res, args = _lib.SIGNATURES[name]
        assert len(args) == len(params), (name, len(args), len(params))
        want_res = None if ret == "void" else _ctype_of(ret)
        assert res is want_res, (name, "return", ret, res)
        for i, (c, a) in enumerate(zip(params, args)):
            want = _ctype_of(c)
            ok = a is want or (c.endswith("*") and isinstance(a, type) and issubclass(a, ctypes._Pointer))
            assert ok, (name, i, c, a)
    # ctypes' own view of the loaded library agrees with the table
    L = _lib.lib()
    for name, (res, args) in _lib.SIGNATURES.items():
        f = getattr(L, name)
        assert list(f.argtypes) == list(args) and f.restype is res, name


def test_status_strings_and_version():
    L = _lib.lib()
    assert L.vnx_version() >= 100
    for st in (0, -1, -2, -3, -4, -5):
        assert L.vnx_status_string(st)
    assert L.vnx_status_string(-99) == b"unknown status"


def test_workspace_queries():
    L = _lib.lib()
    assert L.vnx_spec_accept_workspace(64, 8, 248320) > 64 * 17 * 12
    assert L.vnx_spec_accept_workspace(0, 8, 100) == 256
    assert L.vnx_row_lse_workspace(10, 1000) >= 256
    assert L.vnx_softmax_workspace(10, 1000) > L.vnx_row_lse_workspace(10, 1000)
    assert L.vnx_greedy_verify_workspace(4, 5, 1000) >= 256


def _p(v):
    return ctypes.c_void_p(v)


def test_host_argument_checks_reject_before_launch():
    """Bad arguments are refused on the host (these calls never touch a GPU)."""
    L = _lib.lib()
    fake = _p(1 << 20)  # never dereferenced: every call below fails its checks first
    common = dict(ws=fake, wsb=1 << 30)
    # k out of range, non-positive temperature, misaligned pointer, small ld
    assert L.vnx_spec_accept(fake, fake, 0, 4, 0, 100, 100, 100, 100, 100, fake, fake, 1.0, None, None,
                             fake, fake, None, None, None, common["ws"], common["wsb"], None) == -1
    assert L.vnx_spec_accept(fake, fake, 0, 4, 65, 100, 100, 6600, 100, 6500, fake, fake, 1.0, None, None,
                             fake, fake, None, None, None, common["ws"], common["wsb"], None) == -1
    assert L.vnx_spec_accept(fake, fake, 0, 4, 2, 100, 100, 300, 100, 200, fake, fake, 0.0, None, None,
                             fake, fake, None, None, None, common["ws"], common["wsb"], None) == -1
    assert L.vnx_spec_accept(_p((1 << 20) + 4), fake, 0, 4, 2, 100, 100, 300, 100, 200, fake, fake, 1.0,
                             None, None, fake, fake, None, None, None, common["ws"], common["wsb"], None) == -3
    assert L.vnx_spec_accept(fake, fake, 0, 4, 2, 100, 96, 300, 100, 200, fake, fake, 1.0, None, None,
                             fake, fake, None, None, None, common["ws"], common["wsb"], None) == -1
    # overlapping batch rows (sb too small), bad dtype, missing outputs, small workspace
    assert L.vnx_spec_accept(fake, fake, 0, 4, 2, 100, 100, 200, 100, 200, fake, fake, 1.0, None, None,
                             fake, fake, None, None, None, common["ws"], common["wsb"], None) == -1
    assert L.vnx_spec_accept(fake, fake, 7, 4, 2, 100, 100, 300, 100, 200, fake, fake, 1.0, None, None,
                             fake, fake, None, None, None, common["ws"], common["wsb"], None) == -3
    assert L.vnx_spec_accept(fake, fake, 0, 4, 2, 100, 100, 300, 100, 200, None, fake, 1.0, None, None,
                             fake, fake, None, None, None, common["ws"], common["wsb"], None) == -1
    assert L.vnx_spec_accept(fake, fake, 0, 4, 2, 100, 100, 300, 100, 200, fake, fake, 1.0, None, None,
                             fake, fake, None, None, None, fake, 16, None) == -2
    # greedy: rows_t must be k or k+1
    assert L.vnx_greedy_verify(fake, 0, 2, 3, 5, 100, 100, 500, fake, None, None, fake, fake,
                               fake, 1 << 30, None) == -1
    assert L.vnx_row_lse(fake, 0, 3, 100, 100, -1.0, None, fake, None, None, fake, 1 << 30, None) == -1
    assert L.vnx_row_argmax(fake, 0, 3, 100, 50, fake, fake, 1 << 30, None) == -1
    assert L.vnx_softmax(fake, 1, 3, 100, 100, 1.0, None, fake, 100, fake, 1 << 30, None) == -3  # bf16 ld%8


def test_empty_batch_is_a_no_op():
    L = _lib.lib()
    fake = _p(1 << 20)
    assert L.vnx_spec_accept(fake, fake, 0, 0, 2, 100, 100, 300, 100, 200, fake, fake, 1.0, None, None,
                             fake, fake, None, None, None, None, 0, None) == 0
    assert L.vnx_row_lse(fake, 0, 0, 100, 100, 1.0, None, fake, None, None, None, 0, None) == 0


def test_check_maps_status_to_reference_exceptions():
    with pytest.raises(ValueError):
        _lib.check(-1)
    with pytest.raises(ValueError):
        _lib.check(-2)
    with pytest.raises(RuntimeError):
        _lib.check(-5)
    _lib.check(0)
