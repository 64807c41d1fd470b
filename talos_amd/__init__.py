"""talos_amd -- MI355X (gfx950) batch-1 decode backend for Talos GGUF/Llama models.

Python bindings over the C ABI in include/talos_hip.h (the backend that replaces
Tsuskov/talos src/math/metal/mod.rs) and include/talos_host.h (the host Model,
mirroring src/model/llama.rs).  Everything runs in libtalos_hip.so; importing
this package never falls back to a CPU path -- if the library is missing the
import of `lib()` raises.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libtalos_hip.so")

GGML_F32, GGML_Q4_0, GGML_Q8_0, GGML_Q6_K = 0, 2, 8, 14
TYPE_NAMES = {GGML_F32: "F32", GGML_Q4_0: "Q4_0", GGML_Q8_0: "Q8_0", GGML_Q6_K: "Q6_K"}
BLOCK = {GGML_F32: (1, 4), GGML_Q4_0: (32, 18), GGML_Q8_0: (32, 34), GGML_Q6_K: (256, 210)}

STATUS = {0: "OK", 1: "ERR_ARG", 2: "ERR_HIP", 3: "ERR_DTYPE", 4: "ERR_SHAPE",
          5: "ERR_MISSING_WEIGHT", 6: "ERR_POS", 7: "ERR_TOKEN"}


PATHS = {0: "none", 1: "persistent", 2: "graph", 3: "graph_generic"}


class TalosError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code
        self.status = STATUS.get(code, str(code))


class HipCfg(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("n_embd", C.c_uint32), ("n_ff", C.c_uint32), ("vocab_size", C.c_uint32),
                ("context_length", C.c_uint32), ("rms_eps", C.c_float),
                ("rope_freq_base", C.c_float), ("device", C.c_int32)]


class SynthSpecC(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("n_embd", C.c_uint32), ("n_ff", C.c_uint32), ("vocab_size", C.c_uint32),
                ("context_length", C.c_uint32), ("rope_freq_base", C.c_float),
                ("rms_eps", C.c_float), ("layer_type", C.c_uint32), ("output_type", C.c_uint32),
                ("embd_type", C.c_uint32), ("seed", C.c_uint64), ("stdev", C.c_float)]


_lib = None

_P = C.c_void_p
_F = C.POINTER(C.c_float)
_U32 = C.POINTER(C.c_uint32)

_SIGS = {
    # include/talos_hip.h
    "talos_hip_create": (C.c_int, [C.POINTER(HipCfg), C.POINTER(_P)]),
    "talos_hip_destroy": (None, [_P]),
    "talos_hip_last_error": (C.c_char_p, [_P]),
    "talos_hip_upload_weight": (C.c_int, [_P, C.c_char_p, _P, C.c_size_t, C.c_uint32, C.c_size_t, C.c_size_t]),
    "talos_hip_forward": (C.c_int, [_P, _F, C.c_uint32, _F]),
    "talos_hip_forward_hidden": (C.c_int, [_P, _F, C.c_uint32, _F]),
    "talos_hip_forward_token": (C.c_int, [_P, C.c_uint32, C.c_uint32, _F, _U32]),
    "talos_hip_decode_greedy": (C.c_int, [_P, C.c_uint32, C.c_uint32, C.c_uint32, _U32]),
    "talos_hip_kv_reset": (C.c_int, [_P]),
    "talos_hip_sample": (C.c_int, [_P, C.c_float, C.c_uint32, C.c_float, C.c_float, _U32]),
    "talos_hip_sample_dev": (C.c_int, [_P, _P, C.c_uint32, C.c_float, C.c_uint32, C.c_float, C.c_float, _P]),
    "talos_hip_sample_noalloc": (C.c_int, [_P, _P, C.c_uint32, C.c_float, C.c_uint32, C.c_float, C.c_float, _P]),
    "talos_hip_decode_sample": (C.c_int, [_P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32, C.c_float,
                                          _F, _U32]),
    "talos_hip_perplexity": (C.c_int, [_P, _U32, C.c_uint32, _F, _F]),
    "talos_hip_kv_read": (C.c_int, [_P, C.c_uint32, _F, _F]),
    "talos_hip_kv_write": (C.c_int, [_P, C.c_uint32, _F, _F]),
    "talos_hip_prefill": (C.c_int, [_P, _U32, C.c_uint32, C.c_uint32, _F, _U32]),
    "talos_hip_matvec": (C.c_int, [_P, C.c_char_p, _P, C.c_size_t, C.c_uint32, C.c_size_t, C.c_size_t, _F, _F]),
    "talos_hip_matvec_dev": (C.c_int, [_P, C.c_char_p, _P, _P]),
    "talos_hip_bench_kernel": (C.c_int, [_P, C.c_char_p, C.c_uint32, _F, C.POINTER(C.c_double)]),
    "talos_hip_bench_token": (C.c_int, [_P, C.c_uint32, C.c_uint32, C.c_uint32, _F, C.POINTER(C.c_double)]),
    "talos_hip_bench_matvec": (C.c_int, [_P, C.POINTER(C.c_char_p), C.c_uint32, C.c_uint32, _F,
                                         C.POINTER(C.c_double)]),
    "talos_hip_bench_copy": (C.c_int, [_P, C.c_size_t, C.c_uint32, _F]),
    "talos_hip_phase_timeline": (C.c_int, [_P, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64), C.c_size_t,
                                            _U32, _U32, C.POINTER(C.c_double)]),
    "talos_hip_path": (C.c_int, [_P, C.POINTER(C.c_int)]),
    "talos_hip_set_spin_limit": (C.c_int, [_P, C.c_uint32]),
    "talos_hip_stream": (_P, [_P]),
    "talos_hip_sync": (C.c_int, [_P]),
    # include/talos_host.h
    "talos_model_load": (C.c_int, [C.c_char_p, C.c_int32, C.POINTER(_P)]),
    "talos_model_load_bytes": (C.c_int, [_P, C.c_size_t, C.c_int32, C.POINTER(_P)]),
    "talos_model_free": (None, [_P]),
    "talos_model_last_error": (C.c_char_p, [_P]),
    "talos_model_config": (C.c_int, [_P, C.POINTER(HipCfg)]),
    "talos_model_gguf_bytes": (C.c_int, [_P, C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(C.c_size_t)]),
    "talos_model_cap_context": (C.c_int, [_P, C.c_size_t]),
    "talos_model_forward_gpu": (C.c_int, [_P, C.c_uint32, C.c_size_t, _F]),
    "talos_model_forward_hidden_gpu": (C.c_int, [_P, C.c_uint32, C.c_size_t, _F]),
    "talos_model_reset": (C.c_int, [_P]),
    "talos_model_dequant_row": (C.c_int, [_P, C.c_uint32, _F]),
    "talos_model_forward_token": (C.c_int, [_P, C.c_uint32, C.c_size_t, _F, _U32]),
    "talos_model_decode_greedy": (C.c_int, [_P, C.c_uint32, C.c_size_t, C.c_uint32, _U32]),
    "talos_model_prefill": (C.c_int, [_P, _U32, C.c_uint32, C.c_size_t, _F, _U32]),
    "talos_model_backend": (_P, [_P]),
    "talos_synth_model_load": (C.c_int, [C.POINTER(SynthSpecC), C.c_int32, C.c_int32, C.POINTER(_P)]),
    "talos_synth_model_bytes": (C.c_int, [C.POINTER(SynthSpecC), C.c_int32,
                                          C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(C.c_size_t)]),
    "talos_synth_model_write": (C.c_int, [C.POINTER(SynthSpecC), C.c_int32, C.c_char_p]),
    "talos_synth_free": (None, [C.POINTER(C.c_uint8)]),
    "talos_synth_normal": (C.c_int, [C.c_uint64, C.c_char_p, C.c_uint64, C.c_size_t, C.c_float, _F]),
    "talos_quantize": (C.c_int, [C.c_uint32, _F, C.c_size_t, C.POINTER(C.c_uint8)]),
    "talos_synth_last_error": (C.c_char_p, []),
}


def lib() -> C.CDLL:
    """The loaded backend library.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m talos_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _u32ptr(a: np.ndarray):
    return a.ctypes.data_as(_U32)


# ----------------------------------------------------------------- backend --
class HipBackend:
    """Direct use of the C ABI (include/talos_hip.h): the drop-in boundary."""

    def __init__(self, n_layer, n_head, n_head_kv, n_embd, n_ff, vocab_size, context_length,
                 rms_eps=1e-5, rope_freq_base=10000.0, device=0):
        L = lib()
        cfg = HipCfg(n_layer, n_head, n_head_kv, n_embd, n_ff, vocab_size, context_length,
                     rms_eps, rope_freq_base, device)
        h = _P()
        rc = L.talos_hip_create(C.byref(cfg), C.byref(h))
        if rc:
            raise TalosError(rc, L.talos_hip_last_error(None).decode())
        self._h = h
        self.cfg = cfg

    def _check(self, rc):
        if rc:
            raise TalosError(rc, lib().talos_hip_last_error(self._h).decode())

    def close(self):
        if getattr(self, "_h", None):
            lib().talos_hip_destroy(self._h)
            self._h = None

    __del__ = close

    def upload(self, name: str, data: np.ndarray, ggml_type: int, rows: int, cols: int):
        b = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        self._check(lib().talos_hip_upload_weight(self._h, name.encode(), b.ctypes.data_as(_P), b.size,
                                                  ggml_type, rows, cols))

    def forward(self, x_embed: np.ndarray, pos: int) -> np.ndarray:
        x = np.ascontiguousarray(x_embed, dtype=np.float32)
        out = np.empty(self.cfg.vocab_size, np.float32)
        self._check(lib().talos_hip_forward(self._h, _fptr(x), pos, _fptr(out)))
        return out

    def forward_hidden(self, x_embed: np.ndarray, pos: int) -> np.ndarray:
        x = np.ascontiguousarray(x_embed, dtype=np.float32)
        out = np.empty(self.cfg.n_embd, np.float32)
        self._check(lib().talos_hip_forward_hidden(self._h, _fptr(x), pos, _fptr(out)))
        return out

    def forward_token(self, token: int, pos: int, want_logits=True):
        out = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        am = C.c_uint32()
        self._check(lib().talos_hip_forward_token(self._h, token, pos,
                                                  _fptr(out) if out is not None else None, C.byref(am)))
        return out, am.value

    def decode_greedy(self, token: int, pos: int, n_steps: int) -> np.ndarray:
        out = np.empty(max(n_steps, 1), np.uint32)
        self._check(lib().talos_hip_decode_greedy(self._h, token, pos, n_steps, _u32ptr(out)))
        return out[:n_steps]

    def prefill(self, tokens, pos: int, want_logits=True):
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        am = C.c_uint32()
        self._check(lib().talos_hip_prefill(self._h, _u32ptr(t), t.size, pos,
                                            _fptr(out) if out is not None else None, C.byref(am)))
        return out, am.value

    def kv_reset(self):
        self._check(lib().talos_hip_kv_reset(self._h))

    def kv_write(self, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        assert k.shape == v.shape and k.ndim == 3
        self._check(lib().talos_hip_kv_write(self._h, k.shape[1], _fptr(k), _fptr(v)))

    def kv_read(self, n_pos: int):
        kvd = self.cfg.n_head_kv * (self.cfg.n_embd // self.cfg.n_head)
        k = np.empty((self.cfg.n_layer, n_pos, kvd), np.float32)
        v = np.empty_like(k)
        self._check(lib().talos_hip_kv_read(self._h, n_pos, _fptr(k), _fptr(v)))
        return k, v

    def matvec(self, name: str, data: np.ndarray, ggml_type: int, rows: int, cols: int,
               x: np.ndarray) -> np.ndarray:
        b = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        xx = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(rows, np.float32)
        self._check(lib().talos_hip_matvec(self._h, name.encode(), b.ctypes.data_as(_P), b.size, ggml_type,
                                           rows, cols, _fptr(xx), _fptr(out)))
        return out

    def matvec_dev(self, name: str, d_x: int, d_out: int):
        self._check(lib().talos_hip_matvec_dev(self._h, name.encode(), C.c_void_p(d_x), C.c_void_p(d_out)))

    def bench_kernel(self, kind: str, reps: int):
        """(mean launch microseconds, algorithmic bytes per launch)."""
        us = C.c_float()
        b = C.c_double()
        self._check(lib().talos_hip_bench_kernel(self._h, kind.encode(), reps, C.byref(us), C.byref(b)))
        return us.value, b.value

    def bench_matvec(self, names, reps: int):
        """(mean launch microseconds, algorithmic bytes per launch) of the
        standalone matvec rotating over the resident weights `names`."""
        arr = (C.c_char_p * len(names))(*[n.encode() for n in names])
        us = C.c_float()
        b = C.c_double()
        self._check(lib().talos_hip_bench_matvec(self._h, arr, len(names), reps, C.byref(us), C.byref(b)))
        return us.value, b.value

    def bench_copy(self, nbytes: int, reps: int) -> float:
        """Mean microseconds of a plain device copy of nbytes (read + write),
        back to back on this context's stream: the launch floor beside
        bench_matvec."""
        us = C.c_float()
        self._check(lib().talos_hip_bench_copy(self._h, nbytes, reps, C.byref(us)))
        return us.value

    def sample_dev(self, d_logits: int, n: int, d_token: int, temperature: float, top_k=None, top_p=None,
                   u: float = 0.5):
        """talos_hip_sample_dev on device pointers (enqueued, not waited for)."""
        self._check(lib().talos_hip_sample_dev(self._h, C.c_void_p(d_logits), n, temperature,
                                               0 if top_k is None else int(top_k),
                                               float("inf") if top_p is None else float(top_p), u,
                                               C.c_void_p(d_token)))

    def sample_noalloc(self, d_logits: int, n: int, d_token: int, temperature: float, top_k=None, top_p=None,
                       u: float = 0.5):
        """talos_hip_sample_noalloc: the same draw with the library's fixed
        scratch (no allocation; n <= 131072)."""
        self._check(lib().talos_hip_sample_noalloc(self._h, C.c_void_p(d_logits), n, temperature,
                                                   0 if top_k is None else int(top_k),
                                                   float("inf") if top_p is None else float(top_p), u,
                                                   C.c_void_p(d_token)))

    def path(self) -> str:
        """The token step's implementation for the resident weights."""
        p = C.c_int()
        self._check(lib().talos_hip_path(self._h, C.byref(p)))
        return PATHS[p.value]

    def stream(self) -> int:
        return lib().talos_hip_stream(self._h) or 0

    def sync(self):
        self._check(lib().talos_hip_sync(self._h))


# ------------------------------------------------------------------- model --
@dataclass
class SynthSpec:
    """A seeded synthetic Llama model (weights N(0, stdev), norms 1.0)."""
    n_layer: int
    n_head: int
    n_head_kv: int
    n_embd: int
    n_ff: int
    vocab_size: int
    context_length: int
    rope_freq_base: float = 10000.0
    rms_eps: float = 1e-5
    layer_type: int = GGML_F32
    output_type: int = GGML_F32
    embd_type: int = GGML_F32
    seed: int = 42
    stdev: float = 0.02
    name: str = field(default="", compare=False)

    def c(self) -> SynthSpecC:
        return SynthSpecC(self.n_layer, self.n_head, self.n_head_kv, self.n_embd, self.n_ff,
                          self.vocab_size, self.context_length, self.rope_freq_base, self.rms_eps,
                          self.layer_type, self.output_type, self.embd_type, self.seed, self.stdev)

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head

    @property
    def kv_dim(self) -> int:
        return self.n_head_kv * self.head_dim


def _synth_err():
    return lib().talos_synth_last_error().decode()


def synth_bytes(spec: SynthSpec, nthreads: int = 8) -> np.ndarray:
    """The model as GGUF bytes (a uint8 array)."""
    L = lib()
    p = C.POINTER(C.c_uint8)()
    n = C.c_size_t()
    s = spec.c()
    rc = L.talos_synth_model_bytes(C.byref(s), nthreads, C.byref(p), C.byref(n))
    if rc:
        raise TalosError(rc, _synth_err())
    try:
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy()
    finally:
        L.talos_synth_free(p)


def synth_write(spec: SynthSpec, path: str, nthreads: int = 8) -> None:
    s = spec.c()
    rc = lib().talos_synth_model_write(C.byref(s), nthreads, path.encode())
    if rc:
        raise TalosError(rc, _synth_err())


def synth_normal(seed: int, name: str, i0: int, n: int, stdev: float = 0.02) -> np.ndarray:
    out = np.empty(n, np.float32)
    rc = lib().talos_synth_normal(seed, name.encode(), i0, n, stdev, _fptr(out))
    if rc:
        raise TalosError(rc, "synth_normal")
    return out


def quantize(ggml_type: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    be, bb = BLOCK[ggml_type]
    out = np.empty(x.size // be * bb, np.uint8)
    rc = lib().talos_quantize(ggml_type, _fptr(x), x.size, out.ctypes.data_as(C.POINTER(C.c_uint8)))
    if rc:
        raise TalosError(rc, _synth_err())
    return out


class Model:
    """The host Model (src/model/llama.rs) whose forward runs on the GPU."""

    def __init__(self, handle):
        self._h = handle
        cfg = HipCfg()
        self._check(lib().talos_model_config(self._h, C.byref(cfg)))
        self.cfg = cfg

    @classmethod
    def load(cls, path: str, device: int = 0) -> "Model":
        h = _P()
        rc = lib().talos_model_load(path.encode(), device, C.byref(h))
        if rc:
            raise TalosError(rc, lib().talos_model_last_error(None).decode())
        return cls(h)

    @classmethod
    def load_bytes(cls, data, device: int = 0) -> "Model":
        h = _P()
        arr = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data
        arr = np.ascontiguousarray(arr, np.uint8)
        rc = lib().talos_model_load_bytes(arr.ctypes.data_as(_P), arr.size, device, C.byref(h))
        if rc:
            raise TalosError(rc, lib().talos_model_last_error(None).decode())
        return cls(h)

    @classmethod
    def synth(cls, spec: SynthSpec, nthreads: int = 8, device: int = 0) -> "Model":
        h = _P()
        s = spec.c()
        rc = lib().talos_synth_model_load(C.byref(s), nthreads, device, C.byref(h))
        if rc:
            raise TalosError(rc, _synth_err())
        return cls(h)

    def _check(self, rc):
        if rc:
            raise TalosError(rc, lib().talos_model_last_error(self._h).decode())

    def close(self):
        if getattr(self, "_h", None):
            lib().talos_model_free(self._h)
            self._h = None

    __del__ = close

    def gguf_view(self):
        """(address, length) of the GGUF bytes the model reads."""
        p = C.POINTER(C.c_uint8)()
        n = C.c_size_t()
        self._check(lib().talos_model_gguf_bytes(self._h, C.byref(p), C.byref(n)))
        return C.cast(p, C.c_void_p).value, n.value

    def cap_context(self, max_ctx: int):
        self._check(lib().talos_model_cap_context(self._h, max_ctx))
        cfg = HipCfg()
        self._check(lib().talos_model_config(self._h, C.byref(cfg)))
        self.cfg = cfg

    def forward_gpu(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.cfg.vocab_size, np.float32)
        self._check(lib().talos_model_forward_gpu(self._h, token, pos, _fptr(out)))
        return out

    def forward_hidden_gpu(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.cfg.n_embd, np.float32)
        self._check(lib().talos_model_forward_hidden_gpu(self._h, token, pos, _fptr(out)))
        return out

    step = forward_gpu
    step_hidden = forward_hidden_gpu

    def reset(self):
        self._check(lib().talos_model_reset(self._h))

    def dequant_row(self, token: int) -> np.ndarray:
        out = np.empty(self.cfg.n_embd, np.float32)
        self._check(lib().talos_model_dequant_row(self._h, token, _fptr(out)))
        return out

    def forward_token(self, token: int, pos: int, want_logits: bool = True):
        out = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        am = C.c_uint32()
        self._check(lib().talos_model_forward_token(self._h, token, pos,
                                                    _fptr(out) if out is not None else None, C.byref(am)))
        return out, am.value

    def decode_greedy(self, token: int, pos: int, n_steps: int) -> np.ndarray:
        out = np.empty(max(n_steps, 1), np.uint32)
        self._check(lib().talos_model_decode_greedy(self._h, token, pos, n_steps, _u32ptr(out)))
        return out[:n_steps]

    def prefill(self, tokens, pos: int = 0, want_logits: bool = True):
        """Feed `tokens` at pos.. on the device (main.rs:88-94); returns
        (last logits or None, last argmax)."""
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        am = C.c_uint32()
        self._check(lib().talos_model_prefill(self._h, _u32ptr(t), t.size, pos,
                                              _fptr(out) if out is not None else None, C.byref(am)))
        return out, am.value

    @staticmethod
    def _topp(top_p):
        return float("inf") if top_p is None else float(top_p)

    def sample(self, temperature: float, top_k=None, top_p=None, u: float = 0.5) -> int:
        """Draw from the latest step's logits on the device (src/sample.rs:19-76;
        u is the uniform draw)."""
        t = C.c_uint32()
        self._hip(lib().talos_hip_sample, temperature, 0 if top_k is None else int(top_k), self._topp(top_p), u,
                  C.byref(t))
        return t.value

    def decode_sample(self, token: int, pos: int, u, temperature: float, top_k=None, top_p=None) -> np.ndarray:
        """Sampled decode on the device: len(u) steps, draw s with u[s]."""
        uu = np.ascontiguousarray(u, np.float32)
        out = np.empty(max(uu.size, 1), np.uint32)
        self._hip(lib().talos_hip_decode_sample, token, pos, uu.size, temperature,
                  0 if top_k is None else int(top_k), self._topp(top_p), _fptr(uu), _u32ptr(out))
        return out[: uu.size]

    def perplexity(self, tokens):
        """(perplexity, per-position NLLs) of teacher-forced tokens
        (src/eval.rs:35-52) on the device."""
        t = np.ascontiguousarray(tokens, np.uint32)
        nll = np.empty(max(t.size - 1, 1), np.float32)
        p = C.c_float()
        self._hip(lib().talos_hip_perplexity, _u32ptr(t), t.size, C.byref(p), _fptr(nll))
        ctx = self.cfg.context_length
        scored = sum(min(ctx, t.size - c0) - 1 for c0 in range(0, t.size, ctx) if min(ctx, t.size - c0) >= 2)
        return p.value, nll[:scored]

    def sample_dev(self, d_logits: int, n: int, d_token: int, temperature: float, top_k=None, top_p=None,
                   u: float = 0.5):
        """talos_hip_sample_dev on device pointers (enqueued, not waited for)."""
        self._hip(lib().talos_hip_sample_dev, C.c_void_p(d_logits), n, temperature,
                  0 if top_k is None else int(top_k), self._topp(top_p), u, C.c_void_p(d_token))

    def sync(self):
        self._hip(lib().talos_hip_sync)

    def _hip(self, fn, *args):
        h = self.backend_handle()
        rc = fn(h, *args)
        if rc:
            raise TalosError(rc, lib().talos_hip_last_error(h).decode())

    def kv_read(self, n_pos: int):
        """K and V caches [layer, pos, kv_dim] of the first n_pos positions."""
        kvd = self.cfg.n_head_kv * (self.cfg.n_embd // self.cfg.n_head)
        k = np.empty((self.cfg.n_layer, n_pos, kvd), np.float32)
        v = np.empty_like(k)
        self._hip(lib().talos_hip_kv_read, n_pos, _fptr(k), _fptr(v))
        return k, v

    def kv_write(self, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        assert k.shape == v.shape and k.ndim == 3 and k.shape[0] == self.cfg.n_layer
        self._hip(lib().talos_hip_kv_write, k.shape[1], _fptr(k), _fptr(v))

    def bench_kernel(self, kind: str, reps: int):
        """(mean launch microseconds, algorithmic bytes per launch) of one
        decode kernel kind on this model's resident weights."""
        h = self.backend_handle()
        us = C.c_float()
        b = C.c_double()
        rc = lib().talos_hip_bench_kernel(h, kind.encode(), reps, C.byref(us), C.byref(b))
        if rc:
            raise TalosError(rc, lib().talos_hip_last_error(h).decode())
        return us.value, b.value

    def bench_token(self, token: int, pos: int, reps: int):
        """(mean step microseconds, algorithmic bytes per step) of the
        device-token decode step at `pos`, timed with HIP events."""
        h = self.backend_handle()
        us = C.c_float()
        b = C.c_double()
        rc = lib().talos_hip_bench_token(h, token, pos, reps, C.byref(us), C.byref(b))
        if rc:
            raise TalosError(rc, lib().talos_hip_last_error(h).decode())
        return us.value, b.value

    def bench_copy(self, nbytes: int, reps: int) -> float:
        """Mean microseconds of a plain device copy of nbytes."""
        h = self.backend_handle()
        us = C.c_float()
        rc = lib().talos_hip_bench_copy(h, nbytes, reps, C.byref(us))
        if rc:
            raise TalosError(rc, lib().talos_hip_last_error(h).decode())
        return us.value

    def phase_timeline(self, token: int, pos: int):
        """Per-workgroup wall-clock marks (ns) of one persistent-kernel step:
        an array [nblocks, slots]."""
        h = self.backend_handle()
        cap = 1 << 22
        marks = np.zeros(cap, np.uint64)
        nb, sl = C.c_uint32(), C.c_uint32()
        tick = C.c_double()
        rc = lib().talos_hip_phase_timeline(h, token, pos, marks.ctypes.data_as(C.POINTER(C.c_uint64)), cap,
                                            C.byref(nb), C.byref(sl), C.byref(tick))
        if rc:
            raise TalosError(rc, lib().talos_hip_last_error(h).decode())
        t = marks[: nb.value * sl.value].reshape(nb.value, sl.value).astype(np.float64) * tick.value
        return t

    def path(self) -> str:
        """The token step's implementation: "persistent", "graph" or
        "graph_generic" (talos_hip_path)."""
        h = self.backend_handle()
        p = C.c_int()
        rc = lib().talos_hip_path(h, C.byref(p))
        if rc:
            raise TalosError(rc, lib().talos_hip_last_error(h).decode())
        return PATHS[p.value]

    def set_spin_limit(self, polls: int):
        """Poll limit of the persistent kernel's bounded waits (0: default)."""
        h = self.backend_handle()
        rc = lib().talos_hip_set_spin_limit(h, polls)
        if rc:
            raise TalosError(rc, lib().talos_hip_last_error(h).decode())

    def backend_handle(self) -> int:
        h = lib().talos_model_backend(self._h)
        if not h:
            raise TalosError(1, lib().talos_model_last_error(self._h).decode())
        return h
