"""Helpers shared by the GPU tests: device caches and tables through the C ABI,
oracle runs on the same seeded inputs, and error reporting."""
from __future__ import annotations

import ctypes
import sys

import numpy as np

import lestramanika_amd as pk
from oracle import pyoracle as po


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def normal(seed: int, shape) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


class DeviceKV:
    """A pkh_kv_t owned by a test."""

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq, dtype=pk.PKH_KV_F32):
        self.lib = pk.load()
        self.kv = pk.KV()
        pk.check(self.lib.pkh_kv_alloc(n_layers, n_kv_heads, head_dim, max_seq, dtype,
                                       ctypes.byref(self.kv)), "pkh_kv_alloc")

    @property
    def ref(self):
        return ctypes.byref(self.kv)

    def write(self, which_v, layer, pos0, rows: np.ndarray):
        rows = np.ascontiguousarray(rows)
        pk.check(self.lib.pkh_kv_copy_rows(self.ref, which_v, layer, pos0, rows.shape[0],
                                           rows.ctypes.data, 1), "pkh_kv_copy_rows")

    def read(self, which_v, layer, pos0, n) -> np.ndarray:
        dt = np.uint16 if self.kv.dtype == pk.PKH_KV_F16 else np.float32
        out = np.zeros((n, self.kv.n_kv_heads, self.kv.head_dim), dt)
        pk.check(self.lib.pkh_kv_copy_rows(self.ref, which_v, layer, pos0, n,
                                           out.ctypes.data, 0), "pkh_kv_copy_rows")
        return out

    def free(self):
        self.lib.pkh_kv_free(self.ref)


class DeviceRope:
    """A pkh_rope_t filled from the oracle's tables (bit-equal to the
    reference's state tables, see test_oracle)."""

    def __init__(self, head_dim, theta, n_pos, max_seq=None):
        self.lib = pk.load()
        self.rope = pk.Rope()
        _, self.sin, self.cos = po.rope_tables(head_dim, theta, n_pos)
        half = self.sin.shape[1]
        pk.check(self.lib.pkh_rope_alloc(max_seq or n_pos, half, ctypes.byref(self.rope)),
                 "pkh_rope_alloc")
        pk.check(self.lib.pkh_rope_upload(ctypes.byref(self.rope), self.sin.ctypes.data,
                                          self.cos.ctypes.data, n_pos), "pkh_rope_upload")

    @property
    def ref(self):
        return ctypes.byref(self.rope)

    def free(self):
        self.lib.pkh_rope_free(self.ref)


def decode_host(kv: DeviceKV, rope: DeviceRope, layer, pos, q, k, v) -> np.ndarray:
    lib = pk.load()
    H = q.shape[0]
    ao = np.zeros_like(q, dtype=np.float32)
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
    pk.check(lib.pkh_attn_decode(kv.ref, rope.ref, layer, pos, H, q.ctypes.data, k.ctypes.data,
                                 v.ctypes.data, ao.ctypes.data), "pkh_attn_decode")
    return ao


def maxerr(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def prefill_host(kv: DeviceKV, rope: DeviceRope, layer, pos0, q, k, v) -> np.ndarray:
    lib = pk.load()
    n, H = q.shape[0], q.shape[1]
    ao = np.zeros_like(q, dtype=np.float32)
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
    pk.check(lib.pkh_attn_prefill(kv.ref, rope.ref, layer, pos0, n, H, q.ctypes.data,
                                  k.ctypes.data, v.ctypes.data, ao.ctypes.data),
             "pkh_attn_prefill")
    return ao


class DeviceKVBatch:
    """A pkh_kv_batch_t owned by a test: several sequences' caches."""

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq, dtype=pk.PKH_KV_F32):
        import ctypes as ct
        self.lib = pk.load()
        self.kvb = pk.KVBatch()
        ms = (ct.c_int * len(max_seq))(*max_seq)
        pk.check(self.lib.pkh_kv_batch_alloc(n_layers, n_kv_heads, head_dim, len(max_seq), ms,
                                             dtype, ct.byref(self.kvb)), "pkh_kv_batch_alloc")

    @property
    def ref(self):
        return ctypes.byref(self.kvb)

    def write(self, which_v, layer, seq, pos0, rows: np.ndarray):
        rows = np.ascontiguousarray(rows)
        pk.check(self.lib.pkh_kv_batch_copy_rows(self.ref, which_v, layer, seq, pos0,
                                                 rows.shape[0], rows.ctypes.data, 1),
                 "pkh_kv_batch_copy_rows")

    def read(self, which_v, layer, seq, pos0, n) -> np.ndarray:
        dt = np.uint16 if self.kvb.dtype == pk.PKH_KV_F16 else np.float32
        out = np.zeros((n, self.kvb.n_kv_heads, self.kvb.head_dim), dt)
        pk.check(self.lib.pkh_kv_batch_copy_rows(self.ref, which_v, layer, seq, pos0, n,
                                                 out.ctypes.data, 0), "pkh_kv_batch_copy_rows")
        return out

    def free(self):
        self.lib.pkh_kv_batch_free(self.ref)


class Plan:
    """A pkh_plan_t for one decode step of every sequence."""

    def __init__(self, kvb: DeviceKVBatch, pos, n_heads):
        self.lib = pk.load()
        self.ptr = ctypes.c_void_p()
        arr = (ctypes.c_int * len(pos))(*pos)
        pk.check(self.lib.pkh_plan_create(kvb.ref, arr, n_heads, ctypes.byref(self.ptr)),
                 "pkh_plan_create")

    def free(self):
        self.lib.pkh_plan_free(self.ptr)
