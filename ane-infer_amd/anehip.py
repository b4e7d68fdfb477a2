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
            "anehip_d2d": (C.c_int, [vp, vp, vp, sz]),
            "anehip_timer_start": (C.c_int, [vp]),
            "anehip_timer_stop": (C.c_int, [vp, C.POINTER(f32)]),
            "anehip_quant_gemm": (C.c_int, [vp, u32, vp, u32, u32, vp, u32, vp]),
            "anehip_capture_begin": (C.c_int, [vp]),
            "anehip_capture_end": (C.c_int, [vp, C.POINTER(vp)]),
            "anehip_graph_launch": (C.c_int, [vp, vp]),
            "anehip_graph_destroy": (None, [vp]),
            "anehip_quant_packed_bytes": (sz, [u32, u32, u32]),
            "anehip_quant_pack": (C.c_int, [vp, u32, vp, u32, u32, vp]),
            "anehip_quant_gemv_packed": (C.c_int, [vp, u32, vp, u32, u32, vp, vp]),
            "anehip_quant_gemm_packed": (C.c_int, [vp, u32, vp, u32, u32, vp, u32, vp]),
            "anehip_rmsnorm": (C.c_int, [vp, vp, vp, vp, u32, u32, f32]),
            "anehip_silu_mul": (C.c_int, [vp, vp, vp, sz]),
            "anehip_residual_add": (C.c_int, [vp, vp, vp, sz]),
            "anehip_deltanet_step": (C.c_int, [vp, u32, u32, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "anehip_gated_rmsnorm": (C.c_int, [vp, u32, u32, vp, vp, vp, f32, vp]),
            "anehip_attention_step": (C.c_int, [vp, u32, u32, u32, u32, vp, vp, vp, f32, vp, vp, vp, vp]),
            "anehip_attention_step_noalloc": (C.c_int, [vp, u32, u32, u32, u32, vp, vp, vp, f32, vp, vp, vp, vp]),
            "anehip_argmax": (C.c_int, [vp, vp, u32, u32, vp]),
            "anehip_fill_random": (C.c_int, [vp, vp, sz, u32, u32, C.c_uint64, f32, f32]),
            "anehip_quantize": (C.c_int, [vp, u32, vp, u32, u32, vp]),
            "anehip_upload_quant": (C.c_int, [vp, i32, u32, vp, sz, u32, u32, u32]),
            "anehip_upload_f32": (C.c_int, [vp, i32, u32, vp, sz]),
            "anehip_tensor_ptr": (C.c_int, [vp, i32, u32, u32, C.POINTER(vp), C.POINTER(sz)]),
            "anehip_alloc_state": (C.c_int, [vp, u32, u32]),
            "anehip_reset_state": (C.c_int, [vp]),
            "anehip_set_pos": (C.c_int, [vp, u32, u32]),
            "anehip_get_pos": (C.c_int, [vp, u32, C.POINTER(u32)]),
            "anehip_state_ptr": (C.c_int, [vp, u32, u32, C.POINTER(vp), C.POINTER(sz)]),
            "anehip_set_graph": (C.c_int, [vp, C.c_int]),
            "anehip_decode_step": (C.c_int, [vp, vp, u32, vp]),
            "anehip_decode_step_async": (C.c_int, [vp, vp, u32]),
            "anehip_prefill": (C.c_int, [vp, u32, vp, u32, vp]),
            "anehip_logits_ptr": (C.c_int, [vp, C.POINTER(vp)]),
            "anehip_sampled_tokens": (C.c_int, [vp, vp]),
            "anehip_generate": (C.c_int, [vp, vp, u32, u32, vp]),
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

    def fill_random(self, dptr, n, dist, seed, a, b, f16=False):
        """dist 0: N(a, b^2), dist 1: U(a, b); fp32 or fp16 values."""
        dptr = dptr.ptr if isinstance(dptr, DevBuf) else dptr
        self._check(lib().anehip_fill_random(self.h, C.c_void_p(dptr), n, dist, 1 if f16 else 0, seed, a, b))

    def quantize(self, ggml_type, w_f32, m, n, out):
        ptr = lambda b: b.ptr if isinstance(b, DevBuf) else b
        self._check(lib().anehip_quantize(self.h, ggml_type, C.c_void_p(ptr(w_f32)), m, n, C.c_void_p(ptr(out))))

    def d2d(self, dst, src, nbytes):
        self._check(lib().anehip_d2d(self.h, C.c_void_p(dst), C.c_void_p(src), nbytes))

    def capture_begin(self):
        self._check(lib().anehip_capture_begin(self.h))

    def capture_end(self) -> int:
        g = C.c_void_p()
        self._check(lib().anehip_capture_end(self.h, C.byref(g)))
        return g.value

    def graph_launch(self, g: int):
        self._check(lib().anehip_graph_launch(self.h, C.c_void_p(g)))

    @staticmethod
    def graph_destroy(g: int):
        lib().anehip_graph_destroy(C.c_void_p(g))

    def call(self, name, *args):
        """Calls anehip_<name>(ctx, *args); DevBuf arguments pass their device pointer."""
        conv = [C.c_void_p(a.ptr) if isinstance(a, DevBuf) else a for a in args]
        self._check(getattr(lib(), "anehip_" + name)(self.h, *conv))

    def quant_gemm(self, ggml_type: int, w: DevBuf | int, m: int, n: int, x: DevBuf | int, batch: int,
                   y: DevBuf | int):
        ptr = lambda b: b.ptr if isinstance(b, DevBuf) else b
        self._check(lib().anehip_quant_gemm(self.h, ggml_type, C.c_void_p(ptr(w)), m, n, C.c_void_p(ptr(x)),
                                            batch, C.c_void_p(ptr(y))))


def _p(b):
    if b is None:
        return None
    return C.c_void_p(b.ptr if isinstance(b, DevBuf) else int(b))


# tensor kinds (include/anehip.h)
T = dict(ATTN_NORM=0, POST_ATTN_NORM=1, FFN_GATE=2, FFN_UP=3, FFN_DOWN=4, QKV=5, ATTN_GATE=6, SSM_A=7,
         SSM_ALPHA=8, SSM_BETA=9, SSM_CONV1D=10, SSM_DT_BIAS=11, SSM_NORM=12, SSM_OUT=13, WQ=14, WK=15, WV=16,
         WO=17, Q_NORM=18, K_NORM=19, EMBEDDING=20, FINAL_NORM=21, LM_HEAD=22)
LAYER_DELTANET, LAYER_ATTENTION = 0, 1


class Spec:
    """Model shape (the fields of anehip_model_desc)."""

    def __init__(self, dim=2048, hidden_dim=6144, n_layers=24, n_heads=8, n_kv_heads=2, head_dim=256,
                 vocab_size=151936, ssm_state_size=128, ssm_conv_kernel=4, ssm_group_count=16,
                 rope_freq_base=10000.0, rms_norm_eps=1e-6, layer_types=None, attn_interval=4):
        self.dim, self.hidden_dim, self.n_layers = dim, hidden_dim, n_layers
        self.n_heads, self.n_kv_heads, self.head_dim, self.vocab_size = n_heads, n_kv_heads, head_dim, vocab_size
        self.ssm_state_size, self.ssm_conv_kernel, self.ssm_group_count = ssm_state_size, ssm_conv_kernel, ssm_group_count
        self.rope_freq_base, self.rms_norm_eps = rope_freq_base, rms_norm_eps
        if layer_types is None:  # full attention every `attn_interval`-th layer (l % 4 == 3)
            layer_types = [LAYER_ATTENTION if l % attn_interval == attn_interval - 1 else LAYER_DELTANET
                           for l in range(n_layers)]
        self.layer_types = np.array(layer_types, np.uint8)

    def desc(self) -> ModelDesc:
        d = ModelDesc(self.dim, self.hidden_dim, self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim,
                      self.vocab_size, self.ssm_state_size, self.ssm_conv_kernel, self.ssm_group_count,
                      self.rope_freq_base, self.rms_norm_eps,
                      self.layer_types.ctypes.data_as(C.POINTER(C.c_uint8)))
        d._keep = self.layer_types
        return d

    def shapes(self, layer: int):
        """{kind: (rows, cols, is_quant)} of a layer (-1: model-level tensors)."""
        d, F, H = self.dim, self.hidden_dim, self.ssm_group_count
        qd, kvd = self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim
        if layer < 0:
            return {T["EMBEDDING"]: (self.vocab_size, d, False), T["FINAL_NORM"]: (1, d, False),
                    T["LM_HEAD"]: (self.vocab_size, d, True)}
        out = {T["ATTN_NORM"]: (1, d, False), T["POST_ATTN_NORM"]: (1, d, False), T["FFN_GATE"]: (F, d, True),
               T["FFN_UP"]: (F, d, True), T["FFN_DOWN"]: (d, F, True)}
        if self.layer_types[layer] == LAYER_DELTANET:
            out.update({T["QKV"]: (3 * d, d, True), T["ATTN_GATE"]: (d, d, True), T["SSM_A"]: (1, H, False),
                        T["SSM_ALPHA"]: (H, d, True), T["SSM_BETA"]: (H, d, True),
                        T["SSM_CONV1D"]: (3 * d, self.ssm_conv_kernel, False), T["SSM_DT_BIAS"]: (1, H, False),
                        T["SSM_NORM"]: (1, self.ssm_state_size, False), T["SSM_OUT"]: (d, d, True)})
        else:
            out.update({T["WQ"]: (2 * qd, d, True), T["WK"]: (kvd, d, True), T["WV"]: (kvd, d, True),
                        T["WO"]: (d, qd, True), T["Q_NORM"]: (1, self.head_dim, False),
                        T["K_NORM"]: (1, self.head_dim, False)})
        return out


# Synthetic random-init recipe: (distribution, a, b) per fp32 kind; quantised
# kinds are N(0, 0.02) weights quantised to the chosen type.
F32_RECIPE = {
    T["ATTN_NORM"]: (0, 1.0, 0.1), T["POST_ATTN_NORM"]: (0, 1.0, 0.1), T["FINAL_NORM"]: (0, 1.0, 0.1),
    T["SSM_NORM"]: (0, 1.0, 0.1), T["Q_NORM"]: (0, 1.0, 0.1), T["K_NORM"]: (0, 1.0, 0.1),
    T["SSM_A"]: (1, -1.0, 0.0),            # ssm_a = -a, a ~ U(0, 1)
    T["SSM_DT_BIAS"]: (0, 0.0, 1.0), T["SSM_CONV1D"]: (0, 0.0, 0.3), T["EMBEDDING"]: (0, 0.0, 0.02),
}
WEIGHT_STD = 0.02


def tensor_seed(seed: int, layer: int, kind: int) -> int:
    return (seed * 1_000_003 + (layer + 1) * 64 + kind) & 0xFFFFFFFFFFFFFFFF


class Model(Context):
    """A context with a model description: weights, state, decode step."""

    def __init__(self, spec: Spec, device: int = 0):
        self.spec = spec
        self._desc = spec.desc()
        super().__init__(device, self._desc)

    # -- weights --
    def upload_quant(self, layer, kind, blocks: np.ndarray, m, n, ggml_type=Q8_0):
        blocks = np.ascontiguousarray(blocks, np.uint8)
        self._check(lib().anehip_upload_quant(self.h, layer, kind, blocks.ctypes.data, blocks.nbytes, m, n,
                                              ggml_type))

    def upload_f32(self, layer, kind, data: np.ndarray):
        data = np.ascontiguousarray(data, np.float32)
        self._check(lib().anehip_upload_f32(self.h, layer, kind, data.ctypes.data, data.size))

    def tensor_ptr(self, layer, kind, ggml_type=Q8_0):
        p, n = C.c_void_p(), C.c_size_t()
        self._check(lib().anehip_tensor_ptr(self.h, layer, kind, ggml_type, C.byref(p), C.byref(n)))
        return p.value, n.value

    def randomize(self, seed: int = 0, ggml_type: int = Q8_0):
        """Random-init every tensor on the device (seeded; see F32_RECIPE)."""
        tmp = None
        for layer in [-1] + list(range(self.spec.n_layers)):
            for kind, (rows, cols, quant) in self.spec.shapes(layer).items():
                s = tensor_seed(seed, layer, kind)
                if quant:
                    if tmp is None or tmp.nbytes < rows * cols * 4:
                        if tmp is not None:
                            tmp.free()
                        tmp = self.alloc(rows * cols * 4)
                    self.fill_random(tmp.ptr, rows * cols, 0, s, 0.0, WEIGHT_STD)
                    dptr, _ = self.tensor_ptr(layer, kind, ggml_type)
                    self._check(lib().anehip_quantize(self.h, ggml_type, C.c_void_p(tmp.ptr), rows, cols,
                                                      C.c_void_p(dptr)))
                else:
                    dptr, _ = self.tensor_ptr(layer, kind)
                    dist, a, b = F32_RECIPE[kind]
                    self.fill_random(dptr, rows * cols, dist, s, a, b)
        self.sync()
        if tmp is not None:
            tmp.free()

    def download_tensor(self, layer, kind, ggml_type=Q8_0) -> np.ndarray:
        rows, cols, quant = self.spec.shapes(layer)[kind]
        dptr, nbytes = self.tensor_ptr(layer, kind, ggml_type)
        out = np.empty(nbytes, np.uint8)
        self._check(lib().anehip_d2h(self.h, out.ctypes.data, C.c_void_p(dptr), nbytes))
        return out if quant else out.view(np.float32)

    # -- state --
    def alloc_state(self, batch: int, max_seq: int):
        self._check(lib().anehip_alloc_state(self.h, batch, max_seq))
        self.batch, self.max_seq = batch, max_seq

    def reset_state(self):
        self._check(lib().anehip_reset_state(self.h))

    def set_pos(self, seq, pos):
        self._check(lib().anehip_set_pos(self.h, seq, pos))

    def get_pos(self, seq) -> int:
        v = C.c_uint32()
        self._check(lib().anehip_get_pos(self.h, seq, C.byref(v)))
        return v.value

    def state_ptr(self, layer, which):
        p, n = C.c_void_p(), C.c_size_t()
        self._check(lib().anehip_state_ptr(self.h, layer, which, C.byref(p), C.byref(n)))
        return p.value, n.value

    def get_state(self, layer, which, seq=None) -> np.ndarray:
        """State block `which` of a layer for the whole batch, or for sequence
        `seq` only (the state is laid out with the sequence as leading dim)."""
        p, n = self.state_ptr(layer, which)
        if seq is not None:
            n //= self.batch
            p += seq * n
        out = np.empty(n, np.uint8)
        self._check(lib().anehip_d2h(self.h, out.ctypes.data, C.c_void_p(p), n))
        return out.view(np.uint16 if which >= 2 else np.float32)

    def set_state(self, layer, which, data: np.ndarray):
        p, n = self.state_ptr(layer, which)
        data = np.ascontiguousarray(data)
        assert data.nbytes == n, (data.nbytes, n)
        self._check(lib().anehip_h2d(self.h, C.c_void_p(p), data.ctypes.data, n))

    def set_graph(self, enabled: bool):
        self._check(lib().anehip_set_graph(self.h, 1 if enabled else 0))

    # -- step --
    def step(self, tokens, want_logits=True):
        tok = np.ascontiguousarray(tokens, np.uint32)
        if want_logits:
            out = np.empty((tok.size, self.spec.vocab_size), np.float32)
            self._check(lib().anehip_decode_step(self.h, tok.ctypes.data, tok.size, out.ctypes.data))
            return out
        self._check(lib().anehip_decode_step(self.h, tok.ctypes.data, tok.size, None))
        return None

    def prefill(self, seq: int, tokens, want_logits=True):
        """Runs tokens through sequence `seq` from its position (anehip_prefill);
        returns the last token's logits [vocab]."""
        tok = np.ascontiguousarray(tokens, np.uint32)
        if want_logits:
            out = np.empty(self.spec.vocab_size, np.float32)
            self._check(lib().anehip_prefill(self.h, seq, tok.ctypes.data, tok.size, out.ctypes.data))
            return out
        self._check(lib().anehip_prefill(self.h, seq, tok.ctypes.data, tok.size, None))
        return None

    def step_async(self, tokens):
        tok = np.ascontiguousarray(tokens, np.uint32)
        self._check(lib().anehip_decode_step_async(self.h, tok.ctypes.data, tok.size))

    def sampled(self) -> np.ndarray:
        out = np.empty(self.batch, np.uint32)
        self._check(lib().anehip_sampled_tokens(self.h, out.ctypes.data))
        return out

    def generate(self, first_tokens, steps: int) -> np.ndarray:
        tok = np.ascontiguousarray(first_tokens, np.uint32)
        out = np.empty((steps, tok.size), np.uint32)
        self._check(lib().anehip_generate(self.h, tok.ctypes.data, tok.size, steps, out.ctypes.data))
        return out
