"""The ctypes signatures the Python host binds agree with the C prototypes of include/dllm_hip.h:
same parameter count, and each parameter and return value of the same kind (pointer, 32-bit int,
64-bit int, float, string). A mismatch would pass arguments in the wrong registers without any
error, so this is checked on the host, without a GPU."""

import ctypes
import os
import re

import pytest

from dllm_qwen38_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "dllm_hip.h")


def _prototypes():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)  # preprocessor lines
    text = text.replace('extern "C" {', "").replace("}", "")
    protos = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w\s\*]*?)\s*\b(dllm_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        params = " ".join(params.split())
        plist = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        protos[name] = (" ".join(ret.split()), plist)
    return protos


def _kind_of_c(decl):
    """Kind of a C parameter declaration or return type."""
    d = decl.replace("const", " ")
    stars = d.count("*")
    base = d.replace("*", " ").split()
    # drop a trailing parameter name
    if len(base) > 1 and base[-1] not in ("int", "float", "void", "char", "int64_t", "int32_t", "long"):
        base = base[:-1]
    base = " ".join(base)
    if stars == 2:
        return "ptr-ptr"
    if stars == 1:
        return {"char": "string", "int64_t": "ptr-i64", "int": "ptr-int"}.get(base, "ptr")
    return {"int": "i32", "int64_t": "i64", "long long": "i64", "float": "f32", "size_t": "u64"}[base]


def _kind_of_ctypes(t):
    if t is ctypes.c_char_p:
        return "string"
    if t is ctypes.c_void_p:
        return "ptr"
    if t is None:
        return "void"
    if isinstance(t, type) and issubclass(t, ctypes._Pointer):
        target = t._type_
        if target is ctypes.c_void_p:
            return "ptr-ptr"
        if target in (ctypes.c_int64, ctypes.c_longlong) or (issubclass(target, ctypes._SimpleCData)
                                                              and ctypes.sizeof(target) == 8 and target._type_ in "lq"):
            return "ptr-i64"
        if target is ctypes.c_int:
            return "ptr-int"
        return "ptr"
    if t is ctypes.c_float:
        return "f32"
    if t is ctypes.c_int:
        return "i32"
    if ctypes.sizeof(t) == 8 and t._type_ in "lq":
        return "i64"
    raise AssertionError(f"unexpected ctypes type {t}")


def _compatible(c_kind, py_kind):
    # a typed pointer may be bound as void* (the host passes data_ptr() integers); not the reverse
    return c_kind == py_kind or (c_kind.startswith("ptr") and py_kind == "ptr")


def test_every_prototype_has_a_signature():
    assert sorted(_prototypes()) == sorted(_lib._SIGNATURES)


@pytest.mark.parametrize("name", sorted(_lib._SIGNATURES))
def test_signature_matches_the_header(name):
    ret_c, params_c = _prototypes()[name]
    ret_py, args_py = _lib._SIGNATURES[name]
    assert len(params_c) == len(args_py), f"{name}: {len(params_c)} parameters in C, {len(args_py)} bound"
    assert _compatible(_kind_of_c(ret_c + " r"), _kind_of_ctypes(ret_py)), f"{name}: return {ret_c} vs {ret_py}"
    for i, (pc, tp) in enumerate(zip(params_c, args_py)):
        kc, kp = _kind_of_c(pc), _kind_of_ctypes(tp)
        assert _compatible(kc, kp), f"{name} parameter {i} ({pc}): C kind {kc}, bound as {kp}"
