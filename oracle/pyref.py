"""ctypes driver of the compiled reference (oracle/_ref/libpickle_ref.so).

TEST INFRASTRUCTURE ONLY.  The library is the reference's own C sources
compiled in place by oracle/Makefile plus oracle/ref_probe.c; this module
runs pickle_fast_forward on a GGUF file and reads back the fast state's
work buffers, RoPE tables and KV cache.  It is used to produce the golden
fixtures under tests/golden/ and, where the library is present, by the CPU
tests to check the oracle against the reference directly.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_LIB_PATH = os.path.join(HERE, "_ref", "libpickle_ref.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_Z = ctypes.c_size_t
_lib = None

XN, Q, K, V, AO = 0, 1, 2, 3, 4


def available() -> bool:
    return os.path.exists(REF_LIB_PATH)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        L = ctypes.CDLL(REF_LIB_PATH)
        sig = {
            "ref_open": (_I, [ctypes.c_char_p, _I, ctypes.POINTER(_P)]),
            "ref_close": (None, [_P]),
            "ref_shape": (None, [_P, ctypes.POINTER(_I)]),
            "ref_rope_theta": (ctypes.c_float, [_P]),
            "ref_get_pos": (_Z, [_P]),
            "ref_set_pos": (None, [_P, _Z]),
            "ref_forward1": (_I, [_P, ctypes.c_int32, _P]),
            "ref_forward_n": (_I, [_P, _P, _Z, _P]),
            "ref_forward_stateless": (_I, [_P, ctypes.c_int32, _P]),
            "ref_read_state": (_I, [_P, _I, _P, _Z]),
            "ref_kv_rows": (_I, [_P, _I, _I, _Z, _Z, _P, _I]),
            "ref_rope": (_I, [_P, _I, _Z, _Z, _P]),
            "ref_argmax": (ctypes.c_int32, [_P, _Z]),
            "ref_selftest": (_I, [ctypes.POINTER(ctypes.c_int32)]),
            "ref_set_threads": (None, [_I]),
            "ref_state_ptr": (_P, [_P]),
            "ref_arch_ptr": (_P, [_P]),
            "ref_write_state": (_I, [_P, _I, _P, _Z]),
            "ref_get_threads": (_I, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class RefModel:
    """One loaded GGUF model with its pickle_fast_state_t and pickle_fast_kv_t."""

    def __init__(self, path: str, n_layers_override: int = 0):
        h = _P()
        rc = lib().ref_open(path.encode(), n_layers_override, ctypes.byref(h))
        if rc != 0:
            raise RuntimeError(f"ref_open({path}) rc={rc}")
        self.h = h
        s = (_I * 10)()
        lib().ref_shape(h, s)
        (self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim, self.hidden_dim,
         self.intermediate_dim, self.vocab_size, self.max_seq, self.half, _) = list(s)

    def close(self):
        if self.h:
            lib().ref_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def pos(self) -> int:
        return lib().ref_get_pos(self.h)

    @pos.setter
    def pos(self, p: int):
        lib().ref_set_pos(self.h, p)

    def forward1(self, token: int) -> np.ndarray:
        logits = np.zeros(self.vocab_size, np.float32)
        rc = lib().ref_forward1(self.h, token, logits.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"pickle_fast_forward rc={rc}")
        return logits

    def forward1_rc(self, token: int) -> int:
        logits = np.zeros(self.vocab_size, np.float32)
        return lib().ref_forward1(self.h, token, logits.ctypes.data)

    def forward_stateless(self, token: int) -> np.ndarray:
        logits = np.zeros(self.vocab_size, np.float32)
        rc = lib().ref_forward_stateless(self.h, token, logits.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"pickle_fast_forward(kv=NULL) rc={rc}")
        return logits

    def state(self, which: int) -> np.ndarray:
        n = {XN: self.hidden_dim, Q: self.n_heads * self.head_dim,
             K: self.n_kv_heads * self.head_dim, V: self.n_kv_heads * self.head_dim,
             AO: self.n_heads * self.head_dim}[which]
        out = np.zeros(n, np.float32)
        lib().ref_read_state(self.h, which, out.ctypes.data, n)
        return out

    def kv_read(self, which_v: int, layer: int, p0: int, n: int) -> np.ndarray:
        out = np.zeros((n, self.n_kv_heads, self.head_dim), np.float32)
        rc = lib().ref_kv_rows(self.h, which_v, layer, p0, n, out.ctypes.data, 0)
        if rc != 0:
            raise RuntimeError(f"ref_kv_rows rc={rc}")
        return out

    def kv_write(self, which_v: int, layer: int, p0: int, rows: np.ndarray):
        rows = np.ascontiguousarray(rows, np.float32)
        n = rows.shape[0]
        rc = lib().ref_kv_rows(self.h, which_v, layer, p0, n, rows.ctypes.data, 1)
        if rc != 0:
            raise RuntimeError(f"ref_kv_rows rc={rc}")

    def rope_inv_freq(self) -> np.ndarray:
        out = np.zeros(self.half, np.float32)
        lib().ref_rope(self.h, 0, 0, 0, out.ctypes.data)
        return out

    def rope_rows(self, which: str, p0: int, n: int) -> np.ndarray:
        out = np.zeros((n, self.half), np.float32)
        rc = lib().ref_rope(self.h, 1 if which == "sin" else 2, p0, n, out.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"ref_rope rc={rc}")
        return out


def argmax(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return int(lib().ref_argmax(logits.ctypes.data, logits.size))


def selftest() -> tuple[int, int]:
    tok = ctypes.c_int32(-1)
    rc = lib().ref_selftest(ctypes.byref(tok))
    return rc, tok.value
