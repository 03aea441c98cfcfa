"""Loader for libautoresearch_amd.so.

The ctypes signatures are generated from include/ar_ops.h and
include/ar_data.h, so the Python view of the ABI cannot drift from the headers.  Loading never falls back to anything:
a missing library raises.
"""
from __future__ import annotations

import ctypes as ct
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libautoresearch_amd.so")
HEADER = os.path.join(ROOT, "include", "ar_ops.h")
HEADERS = [HEADER, os.path.join(ROOT, "include", "ar_data.h")]

_TYPES = {
    "int32_t": ct.c_int32,
    "int64_t": ct.c_int64,
    "uint64_t": ct.c_uint64,
    "float": ct.c_float,
    "double": ct.c_double,
    "size_t": ct.c_size_t,
    "void": None,
    "const char*": ct.c_char_p,
    "ar_stream_t": ct.c_void_p,
}


def _ctype(decl: str):
    decl = " ".join(decl.replace("*", " * ").split())
    # drop the parameter name (last identifier) when present
    toks = decl.split(" ")
    if len(toks) > 1 and re.match(r"^[A-Za-z_]\w*$", toks[-1]) and toks[-1] not in _TYPES and toks[-1] != "*":
        toks = toks[:-1]
    t = " ".join(toks)
    if "*" in t:
        if t.replace(" ", "") == "constchar*":
            return ct.c_char_p
        return ct.c_void_p
    t = t.replace("const ", "").strip()
    if t in _TYPES:
        return _TYPES[t]
    raise ValueError(f"unmapped C type: {decl!r}")


def parse_header(path: str = HEADER):
    """Return {name: (restype, [argtypes])} for every function in the header."""
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(ar_\w+)\s*\(([^)]*)\)\s*;", src):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        if ret.startswith("typedef"):
            continue
        argtypes = [] if args in ("", "void") else [_ctype(a) for a in args.split(",")]
        out[name] = (_ctype(ret), argtypes)
    return out


_lib = None


def load() -> ct.CDLL:
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m autoresearch_amd.build` "
            "(there is no CPU fallback)")
    lib = ct.CDLL(LIB_PATH)
    for h in HEADERS:
        for name, (res, args) in parse_header(h).items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
    _lib = lib
    return lib


class ArError(RuntimeError):
    pass


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = load().ar_last_error().decode(errors="replace")
        raise ArError(f"{what or 'ar call'} failed ({status}): {msg}")
