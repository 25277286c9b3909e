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
                if "char" in a and "*" in a:
                    argtypes.append(ctypes.c_char_p)
                elif "*" in a:
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
        # torch ships its own libamdhip64 (loaded under the name
        # "libamdhip64.so"); load it first so that libtadapt.so's
        # libamdhip64.so.7 resolves to that same runtime instead of a second
        # copy from /opt/rocm (two HIP runtimes in one process lose the GPU).
        import torch  # noqa: F401
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


# ── kernel-level timer (ta_kprof_*) ─────────────────────────────────────
KPROF_KERNELS = ["gemm_big", "gemm_big_wide", "attn_fwd", "attn_bwd_dq", "attn_bwd_dkv",
                 "lora_skinny", "lora_wgrad", "gemm_chain", "gemm_swiglu"]


def kprof_select(kid):
    """Time every launch of kernel `kid` (index into KPROF_KERNELS, -1 off)."""
    call("ta_kprof_select", kid)


def kprof_pause(paused):
    """Keep the selection and what was recorded, but time no launch while paused."""
    call("ta_kprof_pause", 1 if paused else 0)


def kprof_read():
    ms, n = ctypes.c_double(), ctypes.c_int64()
    fl, by = ctypes.c_double(), ctypes.c_double()
    call("ta_kprof_read", ctypes.byref(ms), ctypes.byref(n), ctypes.byref(fl), ctypes.byref(by))
    return {"ms": ms.value, "launches": n.value, "flops": fl.value, "bytes": by.value}


def kprof_name(kid):
    return lib().ta_kprof_name(kid).decode()


# ── step engine (include/ta_engine.h) ─────────────────────────────────────
class ModelConfig(ctypes.Structure):
    _fields_ = [("vocab", ctypes.c_int), ("hidden", ctypes.c_int), ("layers", ctypes.c_int),
                ("n_q", ctypes.c_int), ("n_kv", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("inter", ctypes.c_int), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("tie", ctypes.c_int)]


class AdaptConfig(ctypes.Structure):
    _fields_ = [("rank", ctypes.c_int), ("alpha", ctypes.c_float), ("inject_mask", ctypes.c_int),
                ("lr", ctypes.c_float), ("grad_clip", ctypes.c_float),
                ("warmup", ctypes.c_int64), ("total_steps", ctypes.c_int64),
                ("b1", ctypes.c_float), ("b2", ctypes.c_float), ("eps", ctypes.c_float),
                ("wd", ctypes.c_float)]


class StepMetrics(ctypes.Structure):
    _fields_ = [("loss", ctypes.c_float), ("lr", ctypes.c_float), ("gnorm", ctypes.c_float),
                ("gnorm_raw", ctypes.c_float), ("valid_tokens", ctypes.c_int),
                ("step", ctypes.c_int), ("step_ms", ctypes.c_double),
                ("nonfinite_logits", ctypes.c_int)]


TARGETS = ("q", "k", "v", "o", "gate", "up", "down")
WHICH = {"A": 0, "B": 1, "mA": 2, "vA": 3, "mB": 4, "vB": 5, "gA": 6, "gB": 7,
         "A16": 8, "B16": 9}


class Engine:
    """Owner of one ta_engine_* handle (the MI355X LoRA step)."""

    RECOMPUTE = 1  # TA_ENGINE_RECOMPUTE
    CE_IN_DX = 2   # TA_ENGINE_CE_IN_DX

    def __init__(self, model: dict, adapt: dict, B: int, T: int, recompute: bool = False,
                 ce_in_dx: bool = False):
        self.mc = ModelConfig(**model)
        self.ac = AdaptConfig(**adapt)
        self.B, self.T = B, T
        self.recompute = bool(recompute)
        flags = (self.RECOMPUTE if recompute else 0) | (self.CE_IN_DX if ce_in_dx else 0)
        h = lib().ta_engine_create_ex(ctypes.byref(self.mc), ctypes.byref(self.ac), B, T, None,
                                      flags)
        if not h:
            raise BackendError("ta_engine_create failed: " + last_error())
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().ta_engine_destroy(self.h)
            self.h = None

    __del__ = close

    def set_weight(self, name, arr):
        import numpy as np
        a = np.ascontiguousarray(arr, np.uint16)
        call("ta_engine_set_weight", self.h, name.encode(), a.ctypes.data, a.size)

    def init_random(self, seed, std=0.02):
        call("ta_engine_init_random", self.h, seed, std)

    def step(self, inputs, targets, lr_override=0.0):
        import numpy as np
        i = np.ascontiguousarray(inputs, np.int32)
        t = np.ascontiguousarray(targets, np.int32)
        m = StepMetrics()
        call("ta_engine_step", self.h, i.ctypes.data, t.ctypes.data, lr_override,
             ctypes.byref(m))
        return {k: getattr(m, k) for k, _ in StepMetrics._fields_}

    def step_resident(self, d_inputs, d_targets, lr_override=0.0):
        """Step on device-resident int32 token tensors (torch, [B*T] each)."""
        m = StepMetrics()
        call("ta_engine_step_resident", self.h, ptr(d_inputs), ptr(d_targets), lr_override,
             ctypes.byref(m))
        return {k: getattr(m, k) for k, _ in StepMetrics._fields_}

    def profile(self, category):
        call("ta_engine_profile", self.h, category)

    def profile_read(self):
        ms, n = ctypes.c_double(), ctypes.c_int64()
        fl, by = ctypes.c_double(), ctypes.c_double()
        call("ta_engine_profile_read", self.h, ctypes.byref(ms), ctypes.byref(n),
             ctypes.byref(fl), ctypes.byref(by))
        return {"ms": ms.value, "launches": n.value, "flops": fl.value, "bytes": by.value}

    def write_adapter(self, layer, target, which, arr):
        import numpy as np
        t = TARGETS.index(target) if isinstance(target, str) else target
        w = WHICH[which]
        a = np.ascontiguousarray(arr, np.uint16 if w >= 8 else np.float32)
        call("ta_engine_write_adapter", self.h, layer, t, w, a.ctypes.data, a.size)

    def adapter(self, layer, target, which):
        import numpy as np
        t = TARGETS.index(target) if isinstance(target, str) else target
        r = self.ac.rank
        ins = {"q": self.mc.hidden, "k": self.mc.hidden, "v": self.mc.hidden,
               "o": self.mc.n_q * self.mc.head_dim, "gate": self.mc.hidden,
               "up": self.mc.hidden, "down": self.mc.inter}
        outs = {"q": self.mc.n_q * self.mc.head_dim, "k": self.mc.n_kv * self.mc.head_dim,
                "v": self.mc.n_kv * self.mc.head_dim, "o": self.mc.hidden,
                "gate": self.mc.inter, "up": self.mc.inter, "down": self.mc.hidden}
        name = TARGETS[t]
        w = WHICH[which]
        isA = w in (0, 2, 3, 6, 8)
        n = r * ins[name] if isA else outs[name] * r
        out = np.empty(n, np.uint16 if w >= 8 else np.float32)
        call("ta_engine_read_adapter", self.h, layer, t, w, out.ctypes.data, n)
        return out

    def centroid(self):
        import numpy as np
        out = np.empty(self.mc.hidden + 1, np.float64)
        call("ta_engine_centroid", self.h, out.ctypes.data)
        return out[:-1], float(out[-1])

    def buffer(self, name):
        """(device pointer, element count, is_f32) of a named engine buffer."""
        n = ctypes.c_int64(0)
        f = ctypes.c_int(0)
        p = lib().ta_engine_buffer(self.h, name.encode(), ctypes.byref(n), ctypes.byref(f))
        if not p:
            raise BackendError(last_error())
        return p, n.value, bool(f.value)

    def read_buffer(self, name):
        """Copy a named engine buffer to host as numpy (uint16 bits for BF16)."""
        import numpy as np
        _, n, is_f32 = self.buffer(name)
        out = np.empty(n, np.float32 if is_f32 else np.uint16)
        call("ta_engine_read_buffer", self.h, name.encode(), out.ctypes.data, n)
        return out

    def phase_ms(self):
        f, b, t = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        call("ta_engine_phase_ms", self.h, ctypes.byref(f), ctypes.byref(b), ctypes.byref(t))
        return f.value, b.value, t.value
