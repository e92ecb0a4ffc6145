"""ctypes bindings for the CPU oracle (oracle/vdx_oracle.c).

TEST INFRASTRUCTURE ONLY: the oracle is a plain-C restatement of the
reference sampler ``TVdxSampler`` (src/VindexLLM.Sampler.pas).  Only tests/,
``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this
module, always as the reference the GPU results are compared with or as the
timed CPU baseline, never as the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libvdx_oracle.so")
_lib = None

KMAX = 1024
PATH_GREEDY, PATH_TOPK, PATH_FULL = 0, 1, 2


class Config(C.Structure):
    """TVdxSamplerConfig (src/VindexLLM.Sampler.pas:26-34), 32 bytes."""

    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_int32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("repeat_penalty", C.c_float),
        ("repeat_window", C.c_int32),
        ("seed", C.c_int64),
    ]


class Trace(C.Structure):
    _fields_ = [
        ("path", C.c_int32),
        ("k", C.c_int32),
        ("max_logit", C.c_float),
        ("inv_temp", C.c_float),
        ("slot_idx", C.c_int32 * KMAX),
        ("slot_val", C.c_float * KMAX),
        ("order_idx", C.c_int32 * KMAX),
        ("order_q", C.c_float * KMAX),
        ("n_replacements", C.c_int32),
        ("sum_initial", C.c_double),
        ("sum_final", C.c_double),
        ("target", C.c_double),
        ("cdf_lo", C.c_double),
        ("cdf_hi", C.c_double),
        ("fallback", C.c_int32),
        ("token", C.c_int32),
    ]


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        P = C.POINTER
        L.vdxo_splitmix64.argtypes = [P(C.c_uint64)]
        L.vdxo_splitmix64.restype = C.c_uint64
        L.vdxo_seed.argtypes = [P(C.c_uint64), C.c_uint64]
        L.vdxo_next_u64.argtypes = [P(C.c_uint64)]
        L.vdxo_next_u64.restype = C.c_uint64
        L.vdxo_next_float.argtypes = [P(C.c_uint64)]
        L.vdxo_next_float.restype = C.c_float
        L.vdxo_wrap_mul.argtypes = [C.c_uint64, C.c_uint64]
        L.vdxo_wrap_mul.restype = C.c_uint64
        L.vdxo_wrap_add.argtypes = [C.c_uint64, C.c_uint64]
        L.vdxo_wrap_add.restype = C.c_uint64
        L.vdxo_philox4x64_10.argtypes = [P(C.c_uint64), P(C.c_uint64), P(C.c_uint64)]
        L.vdxo_philox_uniform.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.vdxo_philox_uniform.restype = C.c_float
        L.vdxo_u24.argtypes = [C.c_uint64]
        L.vdxo_u24.restype = C.c_float
        L.vdxo_apply_penalty.argtypes = [P(C.c_float), C.c_int32, P(C.c_int32), C.c_int32, C.c_float]
        L.vdxo_process_row.argtypes = [P(C.c_float), C.c_int32, P(Config), P(C.c_int32),
                                       C.c_int32, C.c_float, P(Trace)]
        L.vdxo_process_row.restype = C.c_int32
        L.vdxo_process_batch.argtypes = [P(C.c_float), C.c_int32, C.c_int32, C.c_int64, P(Config),
                                         P(C.c_int32), C.c_int32, P(C.c_int32), P(C.c_float),
                                         P(C.c_int32)]
        L.vdxo_process_batch_mt.argtypes = L.vdxo_process_batch.argtypes + [C.c_int32]
        L.vdxo_sampler_create.restype = C.c_void_p
        L.vdxo_sampler_destroy.argtypes = [C.c_void_p]
        L.vdxo_default_config.argtypes = [P(Config)]
        L.vdxo_sampler_set_config.argtypes = [C.c_void_p, P(Config), C.c_uint64]
        L.vdxo_sampler_get_config.argtypes = [C.c_void_p, P(Config)]
        L.vdxo_sampler_process.argtypes = [C.c_void_p, P(C.c_float), C.c_int32, P(Trace)]
        L.vdxo_sampler_process.restype = C.c_int32
        L.vdxo_sampler_add_to_history.argtypes = [C.c_void_p, C.c_int32]
        L.vdxo_sampler_reset_history.argtypes = [C.c_void_p]
        L.vdxo_sampler_history.argtypes = [C.c_void_p, P(C.c_int32), C.c_int32, P(C.c_int32)]
        L.vdxo_sampler_history.restype = C.c_int32
        L.vdxo_sampler_rng_state.argtypes = [C.c_void_p, P(C.c_uint64)]
        L.vdxo_matvec_q4_0.argtypes = [P(C.c_uint8), P(C.c_float), C.c_int32, C.c_int32, P(C.c_float)]
        L.vdxo_matvec_q4_0_blocked.argtypes = [P(C.c_uint8), P(C.c_float), C.c_int32, C.c_int32,
                                               P(C.c_float)]
        L.vdxo_matvec_q4_0_mt.argtypes = [P(C.c_uint8), P(C.c_float), C.c_int32, C.c_int32,
                                          P(C.c_float), C.c_int32, C.c_int32]
        for fn in ("vdxo_matvec_q8_0", "vdxo_matvec_q8_0_blocked", "vdxo_matvec_f16",
                   "vdxo_matvec_f16_blocked"):
            getattr(L, fn).argtypes = [P(C.c_uint8), P(C.c_float), C.c_int32, C.c_int32, P(C.c_float)]
        L.vdxo_matvec_mt.argtypes = [P(C.c_uint8), C.c_int32, P(C.c_float), C.c_int32, C.c_int32,
                                     P(C.c_float), C.c_int32, C.c_int32]
        L.vdxo_rmsnorm.argtypes = [P(C.c_float), P(C.c_float), C.c_float, C.c_int32, P(C.c_float)]
        L.vdxo_half_to_float.argtypes = [C.c_uint16]
        L.vdxo_half_to_float.restype = C.c_float
        _lib = L
    return _lib


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _ip(a):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def make_config(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0,
                repeat_window=64, seed=0) -> Config:
    return Config(temperature, top_k, top_p, min_p, repeat_penalty, repeat_window, seed)


def default_config() -> Config:
    c = Config()
    lib().vdxo_default_config(C.byref(c))
    return c


def process_row(logits: np.ndarray, cfg: Config, u: float, hist=None, trace: bool = False):
    """One Process() call with the draw replaced by ``u``.  ``logits`` (float32,
    contiguous) is mutated in place by the penalty, as in the reference."""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
    if hist is not None and len(hist):
        h = np.ascontiguousarray(hist, dtype=np.int32)
        hp, hc = _ip(h), len(h)
    else:
        hp, hc = None, 0
    tr = Trace() if trace else None
    tok = lib().vdxo_process_row(_fp(logits), int(logits.shape[-1]), C.byref(cfg), hp, hc,
                                 float(u), C.byref(tr) if tr is not None else None)
    return (tok, tr) if trace else tok


def process_batch(logits: np.ndarray, cfg: Config, u: np.ndarray, hist=None, hcount=None,
                  threads: int = 1) -> np.ndarray:
    """Rows of ``logits`` (B x V float32) processed serially (threads=1) or
    split over ``threads`` POSIX threads; mutates logits like the reference."""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"] and logits.ndim == 2
    B, V = logits.shape
    u = np.ascontiguousarray(u, dtype=np.float32)
    tok = np.zeros(B, dtype=np.int32)
    if hist is not None:
        hist = np.ascontiguousarray(hist, dtype=np.int32)
        hcount = np.ascontiguousarray(hcount if hcount is not None
                                      else np.full(B, hist.shape[1]), dtype=np.int32)
        hp, hs, hcp = _ip(hist), hist.shape[1], _ip(hcount)
    else:
        hp, hs, hcp = None, 0, None
    if threads <= 1:
        lib().vdxo_process_batch(_fp(logits), B, V, V, C.byref(cfg), hp, hs, hcp, _fp(u), _ip(tok))
    else:
        lib().vdxo_process_batch_mt(_fp(logits), B, V, V, C.byref(cfg), hp, hs, hcp, _fp(u),
                                    _ip(tok), int(threads))
    return tok


def splitmix64_stream(seed: int, n: int):
    L = lib()
    s = C.c_uint64(seed)
    return [L.vdxo_splitmix64(C.byref(s)) for _ in range(n)]


def xoshiro_stream(state, n: int):
    L = lib()
    st = (C.c_uint64 * 4)(*state)
    return [L.vdxo_next_u64(st) for _ in range(n)]


def seed_state(seed: int):
    st = (C.c_uint64 * 4)()
    lib().vdxo_seed(st, C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF))
    return list(st)


def philox4x64_10(ctr, key):
    c = (C.c_uint64 * 4)(*ctr)
    k = (C.c_uint64 * 2)(*key)
    o = (C.c_uint64 * 4)()
    lib().vdxo_philox4x64_10(c, k, o)
    return list(o)


def philox_uniform(seed: int, row: int, step: int) -> float:
    return lib().vdxo_philox_uniform(seed & 0xFFFFFFFFFFFFFFFF, row, step)


def matvec_q4_0(w: np.ndarray, x: np.ndarray, in_dim: int, rows: int) -> np.ndarray:
    out = np.zeros(rows, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().vdxo_matvec_q4_0(w.ctypes.data_as(C.POINTER(C.c_uint8)), _fp(x), in_dim, rows, _fp(out))
    return out


def matvec_q4_0_blocked(w: np.ndarray, x: np.ndarray, in_dim: int, rows: int) -> np.ndarray:
    out = np.zeros(rows, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().vdxo_matvec_q4_0_blocked(w.ctypes.data_as(C.POINTER(C.c_uint8)), _fp(x), in_dim, rows,
                                   _fp(out))
    return out


def matvec_q4_0_mt(w: np.ndarray, x: np.ndarray, in_dim: int, rows: int, blocked: bool,
                   threads: int = 8) -> np.ndarray:
    """Either summation order over `threads` host threads (x is one hidden vector)."""
    out = np.zeros(rows, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().vdxo_matvec_q4_0_mt(w.ctypes.data_as(C.POINTER(C.c_uint8)), _fp(x), in_dim, rows,
                              _fp(out), 1 if blocked else 0, int(threads))
    return out


TENSOR_F16, TENSOR_Q4_0, TENSOR_Q8_0 = 1, 2, 8  # GGML type ids (GGUFReader.pas:34-42)
_MV = {(TENSOR_Q4_0, False): "vdxo_matvec_q4_0", (TENSOR_Q4_0, True): "vdxo_matvec_q4_0_blocked",
       (TENSOR_Q8_0, False): "vdxo_matvec_q8_0", (TENSOR_Q8_0, True): "vdxo_matvec_q8_0_blocked",
       (TENSOR_F16, False): "vdxo_matvec_f16", (TENSOR_F16, True): "vdxo_matvec_f16_blocked"}


def matvec(w: np.ndarray, wtype: int, x: np.ndarray, in_dim: int, rows: int, blocked: bool,
           threads: int = 1) -> np.ndarray:
    """The lm_head of one hidden vector in the shader's order (blocked=False)
    or the library kernel's (blocked=True), for wtype TENSOR_Q4_0 / _Q8_0 / _F16."""
    out = np.zeros(rows, dtype=np.float32)
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if threads > 1:
        lib().vdxo_matvec_mt(w.ctypes.data_as(C.POINTER(C.c_uint8)), int(wtype), _fp(x), in_dim, rows,
                             _fp(out), 1 if blocked else 0, int(threads))
    else:
        getattr(lib(), _MV[(int(wtype), bool(blocked))])(w.ctypes.data_as(C.POINTER(C.c_uint8)), _fp(x),
                                                        in_dim, rows, _fp(out))
    return out


def rmsnorm(h: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """shaders/rmsnorm_copy.comp on one vector."""
    h = np.ascontiguousarray(h, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(h)
    lib().vdxo_rmsnorm(_fp(h), _fp(w), float(eps), int(h.size), _fp(out))
    return out


class Sampler:
    """The stateful TVdxSampler object restated (Sampler.pas:37-91)."""

    def __init__(self):
        self._h = lib().vdxo_sampler_create()

    def __del__(self):
        if getattr(self, "_h", None):
            lib().vdxo_sampler_destroy(self._h)
            self._h = None

    def set_config(self, cfg: Config, timer_seed: int = 0x1234):
        lib().vdxo_sampler_set_config(self._h, C.byref(cfg), timer_seed)

    def get_config(self) -> Config:
        c = Config()
        lib().vdxo_sampler_get_config(self._h, C.byref(c))
        return c

    def process(self, logits: np.ndarray, trace: bool = False):
        tr = Trace() if trace else None
        tok = lib().vdxo_sampler_process(self._h, _fp(logits), int(logits.shape[-1]),
                                         C.byref(tr) if tr is not None else None)
        return (tok, tr) if trace else tok

    def add_to_history(self, tok: int):
        lib().vdxo_sampler_add_to_history(self._h, int(tok))

    def reset_history(self):
        lib().vdxo_sampler_reset_history(self._h)

    def history(self):
        buf = (C.c_int32 * 65536)()
        pos = C.c_int32()
        n = lib().vdxo_sampler_history(self._h, buf, 65536, C.byref(pos))
        return list(buf[:n]), pos.value

    def rng_state(self):
        st = (C.c_uint64 * 4)()
        lib().vdxo_sampler_rng_state(self._h, st)
        return list(st)
