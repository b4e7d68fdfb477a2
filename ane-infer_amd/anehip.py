"""ctypes binding of libanehip.so (the C ABI declared in include/anehip.h).

This is the Python-side caller used by the tests and bench.py.  It loads the
in-tree library and raises if it is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libanehip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "anehip.h")

OK = 0
Q4_0 = 2
Q8_0 = 8

_lib = None


class AnehipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"anehip error {code}: {msg}")
        self.code = code


class ModelDesc(C.Structure):
    _fields_ = [
        ("dim", C.c_uint32), ("hidden_dim", C.c_uint32), ("n_layers", C.c_uint32),
        ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("vocab_size", C.c_uint32), ("ssm_state_size", C.c_uint32),
        ("ssm_conv_kernel", C.c_uint32), ("ssm_group_count", C.c_uint32),
        ("rope_freq_base", C.c_float), ("rms_norm_eps", C.c_float),
        ("layer_types", C.POINTER(C.c_uint8)),
    ]


def lib():
    """Loads libanehip.so (no build, no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libanehip.so not built ({LIB_PATH}); run python ane-infer_amd/build.py")
        L = C.CDLL(LIB_PATH)
        vp, sz, u32, i32, f32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_int32, C.c_float
        sig = {
            "anehip_init": (C.c_int, []),
            "anehip_last_error": (C.c_char_p, [vp]),
            "anehip_ctx_create": (C.c_int, [C.c_int, vp, C.POINTER(vp)]),
            "anehip_ctx_destroy": (None, [vp]),
            "anehip_sync": (C.c_int, [vp]),
            "anehip_dev_alloc": (C.c_int, [vp, sz, C.POINTER(vp)]),
            "anehip_dev_free": (C.c_int, [vp, vp]),
            "anehip_h2d": (C.c_int, [vp, vp, vp, sz]),
            "anehip_d2h": (C.c_int, [vp, vp, vp, sz]),
            "anehip_dev_memset": (C.c_int, [vp, vp, C.c_int, sz]),
            "anehip_timer_start": (C.c_int, [vp]),
            "anehip_timer_stop": (C.c_int, [vp, C.POINTER(f32)]),
            "anehip_quant_gemm": (C.c_int, [vp, u32, vp, u32, u32, vp, u32, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def declared_symbols() -> list[str]:
    """Function names declared in include/anehip.h."""
    import re

    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(anehip_[a-z_0-9]+)\s*\(", text, re.M)))


class DevBuf:
    """A device allocation owned by a Context."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx, self.nbytes = ctx, nbytes
        p = C.c_void_p()
        ctx._check(lib().anehip_dev_alloc(ctx.h, nbytes, C.byref(p)))
        self.ptr = p.value

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        self.ctx._check(lib().anehip_h2d(self.ctx.h, C.c_void_p(self.ptr + offset), a.ctypes.data, a.nbytes))
        return self

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        self.ctx._check(lib().anehip_d2h(self.ctx.h, out.ctypes.data, C.c_void_p(self.ptr + offset), out.nbytes))
        return out

    def free(self):
        if self.ptr:
            self.ctx._check(lib().anehip_dev_free(self.ctx.h, C.c_void_p(self.ptr)))
            self.ptr = None


class Context:
    """An anehip context on one device (bare, or with a model description)."""

    def __init__(self, device: int = 0, desc: ModelDesc | None = None):
        L = lib()
        h = C.c_void_p()
        rc = L.anehip_ctx_create(device, C.byref(desc) if desc is not None else None, C.byref(h))
        if rc != OK:
            raise AnehipError(rc, L.anehip_last_error(None).decode())
        self.h = h.value

    def _check(self, rc: int):
        if rc != OK:
            raise AnehipError(rc, lib().anehip_last_error(self.h).decode())
        return rc

    def close(self):
        if self.h:
            lib().anehip_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def alloc(self, nbytes: int) -> DevBuf:
        return DevBuf(self, nbytes)

    def to_device(self, a: np.ndarray) -> DevBuf:
        a = np.ascontiguousarray(a)
        return DevBuf(self, max(a.nbytes, 1)).upload(a)

    def sync(self):
        self._check(lib().anehip_sync(self.h))

    def timer_start(self):
        self._check(lib().anehip_timer_start(self.h))

    def timer_stop(self) -> float:
        ms = C.c_float()
        self._check(lib().anehip_timer_stop(self.h, C.byref(ms)))
        return ms.value

    def quant_gemm(self, ggml_type: int, w: DevBuf | int, m: int, n: int, x: DevBuf | int, batch: int,
                   y: DevBuf | int):
        ptr = lambda b: b.ptr if isinstance(b, DevBuf) else b
        self._check(lib().anehip_quant_gemm(self.h, ggml_type, C.c_void_p(ptr(w)), m, n, C.c_void_p(ptr(x)),
                                            batch, C.c_void_p(ptr(y))))
