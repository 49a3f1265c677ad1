"""lestramanika_amd -- MI355X (gfx950) attention block for pickle's fast path.

Python bindings (ctypes) to ``libpkh.so``, the C ABI declared in
``include/pkh_attn.h``.  The product path is the HIP library; this module
only loads it and marshals pointers.  There is no fallback: if the library
is missing, ``load()`` raises.

Device memory for the ``*_async`` entry points comes from the caller (for
example ``torch.empty(..., device="cuda").data_ptr()``), as do streams
(``torch.cuda.current_stream().cuda_stream``).
"""
from __future__ import annotations

import ctypes
import os

__all__ = [
    "LIB_PATH", "PkhError", "KV", "Rope", "KVBatch", "load",
    "PKH_OK", "PKH_ERR_MEMORY", "PKH_ERR_IO", "PKH_ERR_ARG", "PKH_ERR_RANGE",
    "PKH_KV_F32", "PKH_KV_F16",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpkh.so")

PKH_OK = 0
PKH_ERR_MEMORY = -3
PKH_ERR_IO = -5
PKH_ERR_ARG = -6
PKH_ERR_RANGE = -7
PKH_KV_F32 = 0
PKH_KV_F16 = 1

_NAMES = {0: "PKH_OK", -3: "PKH_ERR_MEMORY", -5: "PKH_ERR_IO",
          -6: "PKH_ERR_ARG", -7: "PKH_ERR_RANGE"}


class PkhError(RuntimeError):
    """A non-zero status from libpkh.so."""

    def __init__(self, code: int, what: str):
        super().__init__(f"{what} returned {_NAMES.get(code, code)}")
        self.code = code


class KV(ctypes.Structure):
    """pkh_kv_t: device mirror of pickle_fast_kv_t."""
    _fields_ = [
        ("n_layers", ctypes.c_int),
        ("n_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("max_seq", ctypes.c_int),
        ("k_stride_layer", ctypes.c_size_t),
        ("v_stride_layer", ctypes.c_size_t),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("dtype", ctypes.c_int),
        ("device", ctypes.c_int),
        ("stride_pos", ctypes.c_size_t),
        ("stride_head", ctypes.c_size_t),
    ]


class Rope(ctypes.Structure):
    """pkh_rope_t: device copy of the sin/cos tables."""
    _fields_ = [
        ("max_seq", ctypes.c_int),
        ("half", ctypes.c_int),
        ("filled_upto", ctypes.c_int),
        ("sin", ctypes.c_void_p),
        ("cos", ctypes.c_void_p),
        ("device", ctypes.c_int),
    ]


class KVBatch(ctypes.Structure):
    """pkh_kv_batch_t: several sequences' caches in one allocation."""
    _fields_ = [
        ("n_layers", ctypes.c_int),
        ("n_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("n_seqs", ctypes.c_int),
        ("dtype", ctypes.c_int),
        ("device", ctypes.c_int),
        ("layer_stride", ctypes.c_size_t),
        ("slot0", ctypes.POINTER(ctypes.c_int64)),
        ("max_seq", ctypes.POINTER(ctypes.c_int)),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("d_slot0", ctypes.c_void_p),
        ("stride_pos", ctypes.c_size_t),
        ("stride_head", ctypes.c_size_t),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_FP = ctypes.POINTER(ctypes.c_float)

# name -> (restype, argtypes)
_SIGS = {
    "pkh_init": (_I, [_I]),
    "pkh_version": (ctypes.c_char_p, []),
    "pkh_kv_alloc": (_I, [_I, _I, _I, _I, _I, ctypes.POINTER(KV)]),
    "pkh_kv_free": (None, [ctypes.POINTER(KV)]),
    "pkh_kv_copy_rows": (_I, [ctypes.POINTER(KV), _I, _I, _I, _I, _P, _I]),
    "pkh_rope_alloc": (_I, [_I, _I, ctypes.POINTER(Rope)]),
    "pkh_rope_free": (None, [ctypes.POINTER(Rope)]),
    "pkh_rope_upload": (_I, [ctypes.POINTER(Rope), _P, _P, _I]),
    "pkh_rope_host_tables": (None, [_I, _F, _I, _I, _P, _P, _P]),
    "pkh_attn_decode": (_I, [ctypes.POINTER(KV), ctypes.POINTER(Rope), _I, _I, _I,
                             _P, _P, _P, _P]),
    "pkh_attn_decode_async": (_I, [ctypes.POINTER(KV), ctypes.POINTER(Rope), _I, _I, _I,
                                   _P, _P, _P, _P, _P]),
    "pkh_attn_prefill": (_I, [ctypes.POINTER(KV), ctypes.POINTER(Rope), _I, _I, _I, _I,
                              _P, _P, _P, _P]),
    "pkh_attn_prefill_async": (_I, [ctypes.POINTER(KV), ctypes.POINTER(Rope), _I, _I, _I,
                                    _I, _P, _P, _P, _P, _P]),
    "pkh_kv_batch_alloc": (_I, [_I, _I, _I, _I, ctypes.POINTER(_I), _I,
                                ctypes.POINTER(KVBatch)]),
    "pkh_kv_batch_free": (None, [ctypes.POINTER(KVBatch)]),
    "pkh_plan_create": (_I, [ctypes.POINTER(KVBatch), ctypes.POINTER(_I), _I,
                             ctypes.POINTER(_P)]),
    "pkh_plan_free": (None, [_P]),
    "pkh_attn_decode_batch_async": (_I, [ctypes.POINTER(KVBatch), ctypes.POINTER(Rope),
                                         _P, _I, _P, _P, _P, _P, _P]),
    "pkh_kv_batch_copy_rows": (_I, [ctypes.POINTER(KVBatch), _I, _I, _I, _I, _I, _P, _I]),
    "pkh_plan_update": (_I, [_P, ctypes.POINTER(_I), _P]),
    "pkh_attn_prefill_batch_async": (_I, [ctypes.POINTER(KVBatch), ctypes.POINTER(Rope), _I, _I,
                                          _I, _I, _I, _P, _P, _P, _P, _P]),
    "pkh_attn_decode_noalloc_async": (_I, [ctypes.POINTER(KV), ctypes.POINTER(Rope), _I, _I, _I,
                                           _P, _P, _P, _P, _P]),
    "pkh_tune_decode_chunk": (_I, [_I]),
    "pkh_tune_decode_wait": (_I, [_I]),
}

_lib = None


def load(path: str | None = None) -> ctypes.CDLL:
    """Load libpkh.so (built in-tree by ``__graft_entry__.build()``).

    Raises FileNotFoundError when the library has not been built: the
    attention path has no CPU fallback.
    """
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    # PyTorch-ROCm ships its own HIP runtime under the same soname
    # (libamdhip64.so.7).  Importing torch first makes libpkh.so bind to that
    # copy, so a process that also uses torch for device memory and streams
    # runs one HIP runtime, not two.  Importing torch does not touch the GPU.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(p):
        raise FileNotFoundError(
            f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(p)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(code: int, what: str) -> None:
    """Raise PkhError for a non-zero status."""
    if code != PKH_OK:
        raise PkhError(code, what)
