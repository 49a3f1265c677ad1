"""numpy front end of the C oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by the CPU-baseline leg of bench.py, to check the GPU path and to time
the CPU baseline.  The product never imports it.

Each wrapper takes and returns float32 numpy arrays in the reference's
layouts (see pk_oracle.h for the file:line each function restates).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
# The same source at -O3 with 512-bit vectors: bit-identical results (checked
# in tests/test_oracle.py), used to time the CPU baseline.
LIB_AVX512_PATH = os.path.join(HERE, "liboracle_avx512.so")
BUILDS = {"plain": LIB_PATH, "avx512": LIB_AVX512_PATH}
REF_LIB_PATH = os.path.join(HERE, "_ref", "libpickle_ref.so")

_libs: dict = {}
_build = "plain"
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t


def use_build(name: str) -> str:
    """Select the oracle build the wrappers below call ("plain", the -O2
    build, or "avx512"); returns the previous selection."""
    global _build
    if name not in BUILDS:
        raise ValueError(name)
    prev, _build = _build, name
    return prev


def lib() -> ctypes.CDLL:
    if _build not in _libs:
        path = BUILDS[_build]
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = ctypes.CDLL(path)
        sig = {
            "pko_rope_half": (_I, [_I]),
            "pko_rope_inv_freq": (None, [_P, _I, _F]),
            "pko_rope_fill": (None, [_P, _P, _P, _I, _I, _I]),
            "pko_rope_apply": (None, [_P, _I, _I, _I, _P, _P]),
            "pko_kv_append_f32": (None, [_P, _P, _I, _I, _I, _P, _P]),
            "pko_attend_f32": (_I, [_P, _P, _I, _I, _I, _Z, _P, _P, _I]),
            "pko_attend_stateless": (None, [_P, _I, _I, _I, _P]),
            "pko_decode_step_f32": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P,
                                         _P, _P, _I]),
            "pko_prefill_f32": (_I, [_P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P,
                                     _I]),
            "pko_f32_to_f16": (ctypes.c_uint16, [_F]),
            "pko_f16_to_f32": (_F, [ctypes.c_uint16]),
            "pko_f32_to_f16_n": (None, [_P, _P, _Z]),
            "pko_f16_to_f32_n": (None, [_P, _P, _Z]),
            "pko_decode_step_f16": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P,
                                         _I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _libs[_build] = L
    return _libs[_build]


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the oracle must be C-contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rope_half(head_dim: int) -> int:
    return lib().pko_rope_half(head_dim)


def rope_tables(head_dim: int, theta: float, n_pos: int):
    """(inv_freq[half], sin[n_pos][half], cos[n_pos][half]) with rows 0..n_pos-1."""
    half = rope_half(head_dim)
    inv = np.zeros(max(half, 1), np.float32)
    sin = np.zeros((n_pos, max(half, 1)), np.float32)
    cos = np.zeros((n_pos, max(half, 1)), np.float32)
    lib().pko_rope_inv_freq(_ptr(inv), head_dim, theta)
    if n_pos > 0:
        lib().pko_rope_fill(_ptr(sin), _ptr(cos), _ptr(inv), half, 0, n_pos - 1)
    return inv[:half], sin[:, :half].copy(), cos[:, :half].copy()


def rope_apply(x: np.ndarray, head_dim: int, sin_row: np.ndarray, cos_row: np.ndarray):
    """Rotated copy of x [n_heads][head_dim]."""
    y = _f32(x).copy()
    n_heads = y.size // head_dim
    half = rope_half(head_dim)
    lib().pko_rope_apply(_ptr(y), n_heads, head_dim, half, _ptr(_f32(sin_row)),
                         _ptr(_f32(cos_row)))
    return y


def attend(k_cache: np.ndarray, v_cache: np.ndarray, q_rot: np.ndarray, n_heads: int,
           attend_n: int, n_threads: int = 1) -> np.ndarray:
    """Attention of rotated q [H][D] over cache rows [0, attend_n) ([pos][HK][D])."""
    k_cache = _f32(k_cache)
    v_cache = _f32(v_cache)
    _, HK, D = k_cache.shape
    ao = np.zeros((n_heads, D), np.float32)
    rc = lib().pko_attend_f32(_ptr(k_cache), _ptr(v_cache), HK, D, n_heads, attend_n,
                              _ptr(_f32(q_rot)), _ptr(ao), n_threads)
    if rc != 0:
        raise RuntimeError(f"pko_attend_f32 rc={rc}")
    return ao


def decode_step(k_cache: np.ndarray, v_cache: np.ndarray, pos: int, q: np.ndarray,
                k: np.ndarray, v: np.ndarray, sin: np.ndarray, cos: np.ndarray,
                n_threads: int = 1):
    """One decode step; k_cache/v_cache [max_seq][HK][D] float32 are updated in
    place.  Returns (ao [H][D], q_rot [H][D], k_rot [HK][D])."""
    assert k_cache.dtype == np.float32 and k_cache.flags["C_CONTIGUOUS"]
    _, HK, D = k_cache.shape
    q = _f32(q)
    H = q.size // D
    half = rope_half(D)
    ao = np.zeros((H, D), np.float32)
    qr = np.zeros((H, D), np.float32)
    kr = np.zeros((HK, D), np.float32)
    rc = lib().pko_decode_step_f32(_ptr(k_cache), _ptr(v_cache), HK, D, H, pos,
                                   _ptr(_f32(sin)), _ptr(_f32(cos)), half, _ptr(q),
                                   _ptr(_f32(k)), _ptr(_f32(v)), _ptr(ao), _ptr(qr), _ptr(kr),
                                   n_threads)
    if rc != 0:
        raise RuntimeError(f"pko_decode_step_f32 rc={rc}")
    return ao, qr, kr


def prefill(k_cache: np.ndarray, v_cache: np.ndarray, pos0: int, q: np.ndarray,
            k: np.ndarray, v: np.ndarray, sin: np.ndarray, cos: np.ndarray,
            n_threads: int = 1) -> np.ndarray:
    """Token-loop prefill; q [n][H][D], k/v [n][HK][D]; returns ao [n][H][D]."""
    assert k_cache.dtype == np.float32 and k_cache.flags["C_CONTIGUOUS"]
    _, HK, D = k_cache.shape
    q = _f32(q)
    n = q.shape[0]
    H = q.shape[1]
    ao = np.zeros((n, H, D), np.float32)
    rc = lib().pko_prefill_f32(_ptr(k_cache), _ptr(v_cache), HK, D, H, pos0, n,
                               _ptr(_f32(sin)), _ptr(_f32(cos)), rope_half(D), _ptr(q),
                               _ptr(_f32(k)), _ptr(_f32(v)), _ptr(ao), n_threads)
    if rc != 0:
        raise RuntimeError(f"pko_prefill_f32 rc={rc}")
    return ao


def decode_step_f16(k_cache: np.ndarray, v_cache: np.ndarray, pos: int, q, k, v, sin, cos,
                    n_threads: int = 1) -> np.ndarray:
    """fp16-KV decode step; k_cache/v_cache are uint16 [max_seq][HK][D], updated
    in place (row pos gets the fp16-rounded k_rot and v)."""
    assert k_cache.dtype == np.uint16 and k_cache.flags["C_CONTIGUOUS"]
    _, HK, D = k_cache.shape
    q = _f32(q)
    H = q.size // D
    ao = np.zeros((H, D), np.float32)
    rc = lib().pko_decode_step_f16(_ptr(k_cache), _ptr(v_cache), HK, D, H, pos,
                                   _ptr(_f32(sin)), _ptr(_f32(cos)), rope_half(D), _ptr(q),
                                   _ptr(_f32(k)), _ptr(_f32(v)), _ptr(ao), n_threads)
    if rc != 0:
        raise RuntimeError(f"pko_decode_step_f16 rc={rc}")
    return ao


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    h = np.zeros(x.shape, np.uint16)
    lib().pko_f32_to_f16_n(_ptr(x), _ptr(h), x.size)
    return h


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    x = np.zeros(h.shape, np.float32)
    lib().pko_f16_to_f32_n(_ptr(h), _ptr(x), h.size)
    return x


def attend_stateless(v: np.ndarray, n_heads: int) -> np.ndarray:
    v = _f32(v)
    HK, D = v.shape
    ao = np.zeros((n_heads, D), np.float32)
    lib().pko_attend_stateless(_ptr(v), HK, D, n_heads, _ptr(ao))
    return ao
