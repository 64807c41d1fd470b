"""ctypes bindings for the CPU oracle (oracle/talos_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the HIP backend and the CPU
baseline timed beside it.  Only tests/, the smoke check and bench.py's
cpu_baseline leg load it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libtalos_oracle.so")
# the same source at -O3 -mavx2 (bit-identical results): the CPU baseline
SIMD_LIB_PATH = os.path.join(HERE, "build", "libtalos_oracle_simd.so")

F32, Q4_0, Q8_0, Q6_K = 0, 2, 8, 14
_F = C.POINTER(C.c_float)
_U8 = C.POINTER(C.c_uint8)


class Config(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("n_embd", C.c_uint32), ("n_ff", C.c_uint32), ("context_length", C.c_uint32),
                ("vocab_size", C.c_uint32), ("rope_dim", C.c_uint32), ("rms_eps", C.c_float),
                ("rope_freq_base", C.c_float)]


_libs = {}


def build() -> str:
    """Compile the oracle with its Makefile (gcc): the parity build and the
    AVX2 build."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def host_has_avx2() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            return any(line.startswith("flags") and " avx2" in line for line in f)
    except OSError:
        return False


def lib(simd: bool = False) -> C.CDLL:
    """The parity build, or (simd) the -O3 -mavx2 build of the same source."""
    if simd not in _libs:
        path = SIMD_LIB_PATH if simd else LIB_PATH
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        sig = {
            "tor_f16_to_f32": (C.c_float, [C.c_uint16]),
            "tor_f32_to_f16": (C.c_uint16, [C.c_float]),
            "tor_dequantize": (None, [C.c_int, _U8, _F, C.c_size_t]),
            "tor_quantize_q8_0": (None, [_F, _U8, C.c_size_t]),
            "tor_quantize_q4_0": (None, [_F, _U8, C.c_size_t]),
            "tor_quantize_q6_k": (None, [_F, _U8, C.c_size_t]),
            "tor_dot": (C.c_float, [_F, _F, C.c_size_t]),
            "tor_matvec_f32": (None, [_F, _F, _F, C.c_size_t, C.c_size_t, C.c_int]),
            "tor_matvec_quant": (None, [_U8, C.c_int, _F, _F, C.c_size_t, C.c_size_t, C.c_int]),
            "tor_rmsnorm": (None, [_F, _F, C.c_float, _F, C.c_size_t]),
            "tor_softmax": (None, [_F, C.c_size_t]),
            "tor_silu": (C.c_float, [C.c_float]),
            "tor_swiglu": (None, [_F, _F, _F, C.c_size_t]),
            "tor_rope": (None, [_F, C.c_size_t, C.c_size_t, C.c_size_t, C.c_float]),
            "tor_argmax": (C.c_uint32, [_F, C.c_size_t]),
            "tor_sample": (C.c_uint32, [_F, C.c_size_t, C.c_float, C.c_size_t, C.c_int, C.c_float, C.c_float]),
            "tor_token_nll": (C.c_float, [_F, C.c_size_t, C.c_uint32]),
            "tor_model_load": (C.c_void_p, [C.c_void_p, C.c_size_t, C.c_int, C.c_char_p, C.c_size_t]),
            "tor_model_free": (None, [C.c_void_p]),
            "tor_model_config": (None, [C.c_void_p, C.POINTER(Config)]),
            "tor_model_cap_context": (None, [C.c_void_p, C.c_size_t]),
            "tor_model_set_threads": (None, [C.c_void_p, C.c_int]),
            "tor_model_forward": (C.c_int, [C.c_void_p, C.c_uint32, C.c_size_t, _F]),
            "tor_model_forward_hidden": (C.c_int, [C.c_void_p, C.c_uint32, C.c_size_t, _F]),
            "tor_model_reset": (None, [C.c_void_p]),
            "tor_model_kv_len": (C.c_size_t, [C.c_void_p]),
            "tor_model_set_kv": (C.c_int, [C.c_void_p, _F, _F, C.c_size_t]),
            "tor_model_get_kv": (C.c_int, [C.c_void_p, _F, _F, C.c_size_t]),
            "tor_gguf_parse": (C.c_void_p, [C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]),
            "tor_gguf_free": (None, [C.c_void_p]),
            "tor_gguf_get_u32": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint32)]),
            "tor_gguf_get_f32": (C.c_int, [C.c_void_p, C.c_char_p, _F]),
            "tor_gguf_get_str": (C.c_char_p, [C.c_void_p, C.c_char_p]),
            "tor_gguf_arr_str_len": (C.c_long, [C.c_void_p, C.c_char_p]),
            "tor_gguf_tensor_count": (C.c_size_t, [C.c_void_p]),
            "tor_gguf_tensor_info": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_char_p),
                                               C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                               C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)]),
            "tor_gguf_tensor_raw": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p),
                                              C.POINTER(C.c_size_t), C.POINTER(C.c_int), C.c_char_p,
                                              C.c_size_t]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _libs[simd] = L
    return _libs[simd]


def _f(a):
    return a.ctypes.data_as(_F)


def _u8(a):
    return a.ctypes.data_as(_U8)


def f16_to_f32(h: int) -> float:
    return lib().tor_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().tor_f32_to_f16(f)


def block(t):
    return {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q6_K: (256, 210)}[t]


def dequantize(t: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, np.float32)
    lib().tor_dequantize(t, _u8(raw), _f(out), n)
    return out


def quantize(t: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    be, bb = block(t)
    out = np.zeros(x.size // be * bb, np.uint8)
    fn = {Q8_0: lib().tor_quantize_q8_0, Q4_0: lib().tor_quantize_q4_0, Q6_K: lib().tor_quantize_q6_k}[t]
    fn(_f(x), _u8(out), x.size)
    return out


def matvec(t: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int, nthreads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(rows, np.float32)
    if t == F32:
        ww = np.ascontiguousarray(w, dtype=np.float32)
        lib().tor_matvec_f32(_f(ww), _f(x), _f(out), rows, cols, nthreads)
    else:
        ww = np.ascontiguousarray(w, dtype=np.uint8)
        lib().tor_matvec_quant(_u8(ww), t, _f(x), _f(out), rows, cols, nthreads)
    return out


def dot(a, b) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().tor_dot(_f(a), _f(b), a.size)


def rmsnorm(x, w, eps) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().tor_rmsnorm(_f(x), _f(w), eps, _f(out), x.size)
    return out


def softmax(x) -> np.ndarray:
    x = np.array(x, np.float32)
    lib().tor_softmax(_f(x), x.size)
    return x


def silu(x: float) -> float:
    return lib().tor_silu(x)


def swiglu(g, u) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().tor_swiglu(_f(g), _f(u), _f(out), g.size)
    return out


def rope(v, pos, n_head, head_dim, freq_base) -> np.ndarray:
    v = np.array(v, np.float32)
    lib().tor_rope(_f(v), pos, n_head, head_dim, freq_base)
    return v


def argmax(logits) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().tor_argmax(_f(logits), logits.size)


def sample(logits, temperature: float, top_k=None, top_p=None, u: float = 0.5) -> int:
    """src/sample.rs:19-76 with the rng draw passed in as u in [0, 1)."""
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().tor_sample(_f(logits), logits.size, temperature, 0 if top_k is None else int(top_k),
                            0 if top_p is None else 1, 0.0 if top_p is None else float(top_p), u)


def token_nll(logits, target: int) -> float:
    """src/eval.rs:17-22."""
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().tor_token_nll(_f(logits), logits.size, target)


def perplexity(model, tokens) -> tuple:
    """src/eval.rs:35-52 on an OracleModel: chunks of context_length, each
    from a reset cache, the NLL of every next token summed in f64.
    Returns (perplexity, per-position NLLs)."""
    assert len(tokens) >= 2
    ctx = model.cfg.context_length
    nll, nlls = 0.0, []
    for c0 in range(0, len(tokens), ctx):
        chunk = tokens[c0:c0 + ctx]
        if len(chunk) < 2:
            break
        model.reset()
        for pos in range(len(chunk) - 1):
            lg = model.forward(chunk[pos], pos)
            v = token_nll(lg, chunk[pos + 1])
            nlls.append(v)
            nll += float(v)
    return float(np.float32(np.exp(nll / len(nlls)))), nlls


class OracleModel:
    """Model::forward on the CPU (src/model/llama.rs:85-183).  The GGUF bytes
    must outlive this object; pass (address, length) of memory the caller
    keeps alive, or a bytes object (kept referenced here)."""

    def __init__(self, data, nthreads: int = 1, simd: bool = False):
        self._L = lib(simd)
        if isinstance(data, (bytes, bytearray, np.ndarray)):
            self._keep = np.ascontiguousarray(np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray)
                                              else data, np.uint8)
            addr, n = self._keep.ctypes.data, self._keep.size
        else:
            addr, n = data
            self._keep = None
        err = C.create_string_buffer(512)
        h = self._L.tor_model_load(C.c_void_p(addr), n, nthreads, err, 512)
        if not h:
            raise RuntimeError(err.value.decode())
        self._h = h
        cfg = Config()
        self._L.tor_model_config(self._h, C.byref(cfg))
        self.cfg = cfg

    def close(self):
        if getattr(self, "_h", None):
            self._L.tor_model_free(self._h)
            self._h = None

    __del__ = close

    def set_threads(self, n):
        self._L.tor_model_set_threads(self._h, n)

    def forward(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.cfg.vocab_size, np.float32)
        if self._L.tor_model_forward(self._h, token, pos, _f(out)):
            raise RuntimeError("oracle forward failed")
        return out

    def forward_hidden(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.cfg.n_embd, np.float32)
        if self._L.tor_model_forward_hidden(self._h, token, pos, _f(out)):
            raise RuntimeError("oracle forward failed")
        return out

    def reset(self):
        self._L.tor_model_reset(self._h)

    def cap_context(self, n):
        self._L.tor_model_cap_context(self._h, n)
        cfg = Config()
        self._L.tor_model_config(self._h, C.byref(cfg))
        self.cfg = cfg

    def kv_len(self) -> int:
        return self._L.tor_model_kv_len(self._h)

    def set_kv(self, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self._L.tor_model_set_kv(self._h, _f(k), _f(v), k.shape[1])

    def get_kv(self, n_pos: int):
        """K and V of the first n_pos cached positions, [layer, pos, kv_dim]."""
        c = self.cfg
        kvd = c.n_head_kv * (c.n_embd // c.n_head)
        k = np.empty((c.n_layer, n_pos, kvd), np.float32)
        v = np.empty_like(k)
        if self._L.tor_model_get_kv(self._h, _f(k), _f(v), n_pos) != 0:
            raise ValueError(f"only {self.kv_len()} positions cached")
        return k, v


class OracleGguf:
    """GGUF v3 parse (src/gguf/reader.rs:193-351) over bytes kept alive here."""

    def __init__(self, data: bytes):
        self._keep = np.frombuffer(bytes(data), np.uint8).copy()
        err = C.create_string_buffer(512)
        h = lib().tor_gguf_parse(C.c_void_p(self._keep.ctypes.data), self._keep.size, err, 512)
        if not h:
            raise ValueError(err.value.decode())
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib().tor_gguf_free(self._h)
            self._h = None

    __del__ = close

    def u32(self, key: str):
        v = C.c_uint32()
        return v.value if lib().tor_gguf_get_u32(self._h, key.encode(), C.byref(v)) else None

    def f32(self, key: str):
        v = C.c_float()
        return v.value if lib().tor_gguf_get_f32(self._h, key.encode(), C.byref(v)) else None

    def str(self, key: str):
        v = lib().tor_gguf_get_str(self._h, key.encode())
        return v.decode() if v is not None else None

    def arr_str_len(self, key: str) -> int:
        return lib().tor_gguf_arr_str_len(self._h, key.encode())

    def tensors(self):
        out = []
        for i in range(lib().tor_gguf_tensor_count(self._h)):
            name = C.c_char_p()
            nd = C.c_uint32()
            dims = (C.c_uint64 * 4)()
            ty = C.c_uint32()
            off = C.c_uint64()
            lib().tor_gguf_tensor_info(self._h, i, C.byref(name), C.byref(nd), dims, C.byref(ty), C.byref(off))
            out.append((name.value.decode(), [dims[k] for k in range(nd.value)], ty.value, off.value))
        return out

    def tensor_raw(self, name: str):
        p = C.c_void_p()
        n = C.c_size_t()
        ty = C.c_int()
        err = C.create_string_buffer(256)
        if lib().tor_gguf_tensor_raw(self._h, name.encode(), C.byref(p), C.byref(n), C.byref(ty), err, 256):
            raise KeyError(err.value.decode())
        return ty.value, bytes((C.c_uint8 * n.value).from_address(p.value))
