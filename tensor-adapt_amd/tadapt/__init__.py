"""Python handle on the gfx950 backend (libtadapt.so) through its C-ABI.

The argument types of every entry point are read from include/ta_backend.h
(and include/ta_engine.h), so the binding cannot drift from the header.
Tensors are torch tensors on the GPU (torch is only the allocator and stream
provider here); calls run on torch's current stream.  There is no CPU
fallback: if the library is missing or a call fails, an exception says so.
"""
import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(_HERE)
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libtadapt.so")
HEADERS = [os.path.join(ROOT, "include", "ta_backend.h"),
           os.path.join(ROOT, "include", "ta_engine.h")]

_CTYPES = {
    "int": ctypes.c_int, "int64_t": ctypes.c_int64, "uint64_t": ctypes.c_uint64,
    "float": ctypes.c_float, "double": ctypes.c_double, "uint32_t": ctypes.c_uint32,
}


class BackendError(RuntimeError):
    pass


def parse_header(path):
    """{name: (restype, [argtypes])} for every ta_* declaration in a header."""
    if not os.path.exists(path):
        return {}
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(ta_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        argtypes = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                if "*" in a:
                    argtypes.append(ctypes.c_void_p)
                else:
                    toks = a.replace("const ", "").split()
                    argtypes.append(_CTYPES[toks[0]])
        if "char" in ret and "*" in ret:
            restype = ctypes.c_char_p
        elif "*" in ret:
            restype = ctypes.c_void_p
        else:
            restype = _CTYPES.get(ret.replace("const", "").strip(), ctypes.c_int)
        out[name] = (restype, argtypes)
    return out


def declared():
    d = {}
    for h in HEADERS:
        d.update(parse_header(h))
    return d


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise BackendError(
                "libtadapt.so is not built (run tensor-adapt_amd/build.py or "
                "__graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in declared().items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def last_error():
    return lib().ta_last_error().decode()


def call(name, *args):
    """Call a status-returning entry point; raise BackendError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise BackendError(f"{name} failed ({rc}): {last_error()}")
    return rc


def ptr(t):
    """Device pointer of a torch tensor (None -> NULL)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
