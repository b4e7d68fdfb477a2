"""ctypes binding of the CPU oracle (oracle/_build/libane_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, always as the checker / CPU baseline and never as
the measured GPU path.  The C sources restate the reference's CPU decode
arithmetic; see oracle/ane_oracle.h for citations and pinning.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libane_oracle.so")

Q4_0 = 2
Q8_0 = 8
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34}

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_sz = C.c_size_t

_lib = None


def build() -> None:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = C.CDLL(LIB_PATH)
        L.ao_f16_to_f32.restype = C.c_float
        L.ao_f16_to_f32.argtypes = [C.c_uint16]
        L.ao_f32_to_f16.restype = C.c_uint16
        L.ao_f32_to_f16.argtypes = [C.c_float]
        L.ao_f32_to_f16_array.argtypes = [_f32p, _u16p, _sz]
        L.ao_f16_to_f32_array.argtypes = [_u16p, _f32p, _sz]
        L.ao_splitmix64.restype = C.c_uint64
        L.ao_splitmix64.argtypes = [C.c_uint64]
        L.ao_fill_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_float, C.c_float, _f32p, _sz]
        L.ao_fill_uniform.argtypes = [C.c_uint64, C.c_uint64, C.c_float, C.c_float, _f32p, _sz]
        L.ao_fill_u32.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32, _u32p, _sz]
        L.ao_quantize_q8_0.argtypes = [_f32p, _sz, _sz, _u8p]
        L.ao_quantize_q4_0.argtypes = [_f32p, _sz, _sz, _u8p]
        L.ao_gen_quant.argtypes = [C.c_uint32, C.c_uint64, C.c_uint64, C.c_float, _sz, _sz, _u8p]
        L.ao_quant_bytes.restype = _sz
        L.ao_quant_bytes.argtypes = [C.c_uint32, _sz, _sz]
        L.ao_dequant_q4_0_block.argtypes = [_u8p, _f32p]
        L.ao_dequant_q8_0_block.argtypes = [_u8p, _f32p]
        L.ao_quant_gemv.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _f32p]
        L.ao_quant_gemv_mt.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _f32p, C.c_int]
        L.ao_quant_gemm.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _sz, _f32p, C.c_int]
        L.ao_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _sz, C.c_float]
        L.ao_silu_mul_inplace.argtypes = [_f32p, _f32p, _sz]
        L.ao_residual_add.argtypes = [_f32p, _f32p, _sz]
        L.ao_deltanet_core.argtypes = [_sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, _f32p,
                                       _f32p, _f32p, _f32p, _f32p]
        L.ao_gated_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, C.c_float]
        L.ao_attention_core.argtypes = [_sz, _sz, _sz, _sz, _sz, C.c_float, _f32p, _f32p, _f32p,
                                        _f32p, _f32p, C.c_int, C.c_void_p, C.c_void_p, _f32p]
        L.ao_model_create.restype = C.c_void_p
        L.ao_model_create.argtypes = [C.c_uint32] * 10 + [C.c_float, C.c_float, _u8p]
        L.ao_model_destroy.argtypes = [C.c_void_p]
        L.ao_model_set_quant.restype = C.c_int
        L.ao_model_set_quant.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_uint32,
                                         C.c_uint32, C.c_uint32]
        L.ao_model_set_f32.restype = C.c_int
        L.ao_model_set_f32.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, _sz]
        L.ao_seq_create.restype = C.c_void_p
        L.ao_seq_create.argtypes = [C.c_void_p, C.c_uint32, C.c_int]
        L.ao_seq_destroy.argtypes = [C.c_void_p]
        L.ao_seq_set_pos.argtypes = [C.c_void_p, C.c_uint32]
        L.ao_seq_get_pos.restype = C.c_uint32
        L.ao_seq_get_pos.argtypes = [C.c_void_p]
        for fn in ("ao_seq_conv_state", "ao_seq_recurrent_state", "ao_seq_k_cache",
                   "ao_seq_v_cache"):
            getattr(L, fn).restype = C.c_void_p
            getattr(L, fn).argtypes = [C.c_void_p, C.c_uint32]
        L.ao_forward_token.restype = C.c_int
        L.ao_forward_token.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, _f32p, C.c_int]
        L.ao_argmax.restype = C.c_uint32
        L.ao_argmax.argtypes = [_f32p, _sz]
        L.ao_max_threads.restype = C.c_int
        _lib = L
    return _lib


# ---- thin numpy wrappers --------------------------------------------------

def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().ao_f32_to_f16_array(a.reshape(-1), out.reshape(-1), a.size)
    return out


def f16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().ao_f16_to_f32_array(a.reshape(-1), out.reshape(-1), a.size)
    return out


def normal(seed: int, stream: int, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().ao_fill_normal(seed, stream, mean, std, out, n)
    return out


def uniform(seed: int, stream: int, n: int, lo=0.0, hi=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().ao_fill_uniform(seed, stream, lo, hi, out, n)
    return out


def randint(seed: int, stream: int, n: int, bound: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().ao_fill_u32(seed, stream, bound, out, n)
    return out


def quant_bytes(t: int, m: int, n: int) -> int:
    return m * (n // 32) * BLOCK_BYTES[t]


def quantize(t: int, w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    m, n = w.shape
    out = np.empty(quant_bytes(t, m, n), np.uint8)
    (lib().ao_quantize_q8_0 if t == Q8_0 else lib().ao_quantize_q4_0)(w, m, n, out)
    return out


def gen_quant(t: int, seed: int, stream: int, m: int, n: int, std=0.02) -> np.ndarray:
    out = np.empty(quant_bytes(t, m, n), np.uint8)
    lib().ao_gen_quant(t, seed, stream, std, m, n, out)
    return out


def dequant(t: int, w: np.ndarray, m: int, n: int) -> np.ndarray:
    """Full dequantised matrix (float32) via the per-block restatements."""
    bb = BLOCK_BYTES[t]
    blocks = np.ascontiguousarray(w).reshape(m * (n // 32), bb)
    out = np.empty((m * (n // 32), 32), np.float32)
    fn = lib().ao_dequant_q8_0_block if t == Q8_0 else lib().ao_dequant_q4_0_block
    o = np.empty(32, np.float32)
    for i in range(blocks.shape[0]):
        fn(np.ascontiguousarray(blocks[i]), o)
        out[i] = o
    return out.reshape(m, n)


def gemv(t: int, w: np.ndarray, m: int, n: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(m, np.float32)
    if threads == 1:
        lib().ao_quant_gemv(t, w, m, n, x, y)
    else:
        lib().ao_quant_gemv_mt(t, w, m, n, x, y, threads)
    return y


def gemm(t: int, w: np.ndarray, m: int, n: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    batch = x.shape[0]
    y = np.empty((batch, m), np.float32)
    lib().ao_quant_gemm(t, w, m, n, x.reshape(-1), batch, y.reshape(-1), threads)
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().ao_rmsnorm(out, x, np.ascontiguousarray(w, np.float32), x.size, eps)
    return out


def deltanet_core(qkv, beta_raw, alpha_raw, conv_w, ssm_a, dt_bias, conv_state, S, n_heads, dk):
    """One DeltaNet core step; conv_state and S (float32, C-contiguous) update in place."""
    chunk = n_heads * dk
    ksize = conv_w.size // (3 * chunk)
    out = np.empty(chunk, np.float32)
    f = lambda a: np.ascontiguousarray(a, np.float32).reshape(-1)
    assert conv_state.dtype == np.float32 and conv_state.flags.c_contiguous
    assert S.dtype == np.float32 and S.flags.c_contiguous
    lib().ao_deltanet_core(chunk, n_heads, dk, ksize, f(qkv), f(beta_raw), f(alpha_raw),
                           f(conv_w), f(ssm_a), f(dt_bias), conv_state.reshape(-1), S.reshape(-1),
                           out)
    return out


def gated_rmsnorm(heads, gate, norm_w, n_heads, eps):
    heads = np.ascontiguousarray(heads, np.float32)
    out = np.empty_like(heads)
    lib().ao_gated_rmsnorm(out, heads, np.ascontiguousarray(gate, np.float32),
                           np.ascontiguousarray(norm_w, np.float32), n_heads,
                           heads.size // n_heads, eps)
    return out


def attention_core(q_full, k_in, v_in, q_norm, k_norm, k_cache, v_cache, pos, n_heads, n_kv_heads,
                   hd, rope_base=10000.0):
    """One attention core step; k_cache/v_cache ([kvh][max_seq][hd], float32 or uint16 fp16 bits)
    are written at pos in place."""
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    kv_f16 = 1 if k_cache.dtype == np.uint16 else 0
    max_seq = k_cache.shape[1]
    out = np.empty(n_heads * hd, np.float32)
    f = lambda a: np.ascontiguousarray(a, np.float32).reshape(-1)
    lib().ao_attention_core(n_heads, n_kv_heads, hd, max_seq, pos, rope_base, f(q_full), f(k_in),
                            f(v_in), f(q_norm), f(k_norm), kv_f16,
                            k_cache.ctypes.data_as(C.c_void_p), v_cache.ctypes.data_as(C.c_void_p),
                            out)
    return out


def argmax(logits: np.ndarray) -> int:
    return int(lib().ao_argmax(np.ascontiguousarray(logits, np.float32), logits.size))


def max_threads() -> int:
    return int(lib().ao_max_threads())


class OracleModel:
    """The oracle's qwen35_forward_token over host tensors registered by kind
    (same kinds and shapes as include/anehip.h).  Arrays passed to set_* are
    kept alive here because the C side borrows them."""

    def __init__(self, dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size, ssm_state_size,
                 ssm_conv_kernel, ssm_group_count, rope_freq_base, rms_norm_eps, layer_types):
        self.layer_types = np.ascontiguousarray(layer_types, np.uint8)
        self.vocab = vocab_size
        self.n_layers = n_layers
        self.h = lib().ao_model_create(dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size,
                                       ssm_state_size, ssm_conv_kernel, ssm_group_count, rope_freq_base,
                                       rms_norm_eps, self.layer_types)
        self._keep = []

    def set_quant(self, layer, kind, data, rows, cols, ggml_type):
        data = np.ascontiguousarray(data, np.uint8)
        self._keep.append(data)
        assert lib().ao_model_set_quant(self.h, layer, kind, data.ctypes.data, rows, cols, ggml_type) == 0

    def set_f32(self, layer, kind, data):
        data = np.ascontiguousarray(data, np.float32)
        self._keep.append(data)
        assert lib().ao_model_set_f32(self.h, layer, kind, data.ctypes.data, data.size) == 0

    def close(self):
        if self.h:
            lib().ao_model_destroy(self.h)
            self.h = None


class OracleSeq:
    """One sequence's state (conv windows, recurrent states, KV cache, pos)."""

    def __init__(self, model: OracleModel, max_seq: int, kv_f16: bool = True):
        self.m, self.max_seq = model, max_seq
        self.h = lib().ao_seq_create(model.h, max_seq, 1 if kv_f16 else 0)

    def view(self, layer, which, count, dtype):
        fn = {0: lib().ao_seq_conv_state, 1: lib().ao_seq_recurrent_state, 2: lib().ao_seq_k_cache,
              3: lib().ao_seq_v_cache}[which]
        ptr = fn(self.h, layer)
        buf = (C.c_char * (count * np.dtype(dtype).itemsize)).from_address(ptr)
        return np.frombuffer(buf, dtype=dtype, count=count)

    @property
    def pos(self):
        return int(lib().ao_seq_get_pos(self.h))

    @pos.setter
    def pos(self, p):
        lib().ao_seq_set_pos(self.h, p)

    def forward(self, token: int, threads: int = 0) -> np.ndarray:
        logits = np.empty(self.m.vocab, np.float32)
        rc = lib().ao_forward_token(self.m.h, self.h, token, logits, threads)
        if rc != 0:
            raise RuntimeError("oracle forward failed (missing tensor or pos >= max_seq)")
        return logits

    def close(self):
        if self.h:
            lib().ao_seq_destroy(self.h)
            self.h = None
