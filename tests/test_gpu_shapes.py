"""GPU parity over the reference's whole shape domain, through the C ABI.

The reference attends for any head_dim (its scalar score loop takes head_dim
% 16 != 0, src/pickle_fast.c:2023-2032) and any (H, HK): query head h reads
KV head h*HK/H (src/pickle_fast.c:1963), so group sizes need not be powers of
two, H need not be a multiple of HK, and some KV heads serve no query head
when H < HK (their rows are still appended, src/pickle_fast.c:1938-1944).
These cases run every entry point against the oracle, which follows the
reference on all of them: decode (fp32 and fp16 caches, one and many split-K
chunks), prefill, ragged decode, and the reference's own cache layout.

Tolerances as elsewhere: max-abs 1e-4 for fp32 decode, 2e-3 for fp16 caches
and prefill's fp16 operands; appended rows bit for bit.
"""
import ctypes

import numpy as np
import pytest

import lestramanika_amd as pk
from oracle import pyoracle as po
from pkh_util import DeviceRope, log, maxerr, normal

from test_gpu_decode import _check as decode_check
from test_gpu_prefill import _check_free as prefill_check
from test_gpu_ragged import Case

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_F16 = 2e-3

# (H, HK, D): groups of 3, 5, 6, 7 (Llama-3.2-3B, Qwen2.5-32B, Qwen2-1.5B,
# Qwen2-7B shapes), uneven groups (H % HK != 0), H < HK, groups past the
# kernels' slot size (16 and 32 heads per KV head: several slots re-read the
# KV head), and head dims off the 16/32/64/128/256 set (24, 80, 96, 112, 160,
# 192, and widths whose rotation half is not a multiple of 4 or 16).
DECODE_SHAPES = [
    (24, 8, 128), (40, 8, 128), (12, 2, 64), (28, 4, 128),
    (6, 4, 16), (10, 4, 32), (7, 3, 64), (2, 4, 64),
    (32, 2, 64), (32, 1, 128), (16, 2, 256), (12, 1, 256),
    (8, 2, 24), (8, 2, 80), (16, 4, 96), (4, 4, 112), (4, 1, 160), (4, 2, 192),
    (6, 3, 6), (4, 2, 20), (3, 3, 13), (5, 2, 200), (1, 1, 1),
]


def _id(s):
    return f"H{s[0]}-HK{s[1]}-D{s[2]}"


@pytest.mark.parametrize("shape", DECODE_SHAPES, ids=_id)
def test_decode_any_shape(shape):
    H, HK, D = shape
    for pos in (0, 37, 3000):      # 3000 rows: several split-K chunks per head slot
        decode_check(H, HK, D, pos, 1e4, 500 + H + 3 * HK + 7 * D + pos)


@pytest.mark.parametrize("shape", [(24, 8, 80), (28, 4, 96), (6, 4, 24), (32, 1, 160)], ids=_id)
def test_decode_any_shape_fp16(shape):
    H, HK, D = shape
    for pos in (5, 2500):
        decode_check(H, HK, D, pos, 5e5, 600 + H + D + pos, dtype=pk.PKH_KV_F16)


def test_decode_any_shape_graph_with_no_alloc_entry():
    """A non-uniform shape through the no-alloc entry point equals the
    allocating one bit for bit."""
    import torch
    lib = pk.load()
    from pkh_util import DeviceKV
    H, HK, D, pos = 10, 4, 80, 2200
    kv = DeviceKV(1, HK, D, pos + 1)
    rope = DeviceRope(D, 1e4, pos + 1)
    try:
        kv.write(0, 0, 0, normal(801, (pos, HK, D)))
        kv.write(1, 0, 0, normal(802, (pos, HK, D)))
        dev = torch.device("cuda")
        q, k, v = (torch.from_numpy(normal(803 + i, s)).to(dev)
                   for i, s in enumerate(((H, D), (HK, D), (HK, D))))
        a = torch.zeros((H, D), device=dev)
        b = torch.zeros((H, D), device=dev)
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert lib.pkh_attn_decode_async(kv.ref, rope.ref, 0, pos, H, q.data_ptr(), k.data_ptr(),
                                         v.data_ptr(), a.data_ptr(), s) == 0
        assert lib.pkh_attn_decode_noalloc_async(kv.ref, rope.ref, 0, pos, H, q.data_ptr(),
                                                 k.data_ptr(), v.data_ptr(), b.data_ptr(), s) == 0
        torch.cuda.synchronize()
        assert torch.equal(a, b)
    finally:
        kv.free()
        rope.free()


PREFILL_SHAPES = [
    (24, 8, 128, 0, 300), (28, 4, 128, 40, 200), (12, 2, 64, 0, 129), (6, 4, 16, 0, 100),
    (10, 4, 32, 70, 90), (2, 4, 64, 10, 70), (32, 1, 64, 0, 150), (16, 1, 256, 0, 70),
    (8, 2, 24, 50, 130), (16, 4, 80, 0, 257), (12, 2, 96, 100, 100), (4, 2, 20, 0, 40),
    (3, 3, 13, 5, 33), (6, 3, 6, 0, 20), (4, 1, 160, 0, 65), (1, 1, 1, 0, 9),
]


@pytest.mark.parametrize("case", PREFILL_SHAPES, ids=lambda c: f"H{c[0]}-HK{c[1]}-D{c[2]}-p{c[3]}-n{c[4]}")
def test_prefill_any_shape(case):
    H, HK, D, pos0, n = case
    prefill_check(H, HK, D, pos0, n, 1e4, 700 + H + 3 * HK + D + pos0 + n)


@pytest.mark.parametrize("case", [(24, 8, 96, 30, 100), (6, 4, 24, 0, 77)],
                         ids=lambda c: f"H{c[0]}-HK{c[1]}-D{c[2]}")
def test_prefill_any_shape_fp16(case):
    H, HK, D, pos0, n = case
    prefill_check(H, HK, D, pos0, n, 5e5, 750 + D + n, dtype=pk.PKH_KV_F16)


@pytest.mark.parametrize("shape,dtype", [((24, 8, 80), pk.PKH_KV_F32), ((6, 4, 24), pk.PKH_KV_F32),
                                         ((28, 4, 96), pk.PKH_KV_F16), ((2, 4, 64), pk.PKH_KV_F32)],
                         ids=["H24-HK8-D80", "H6-HK4-D24", "H28-HK4-D96-f16", "H2-HK4-D64"])
def test_ragged_any_shape(shape, dtype):
    H, HK, D = shape
    log(f"ragged H{H} HK{HK} D{D} dtype {dtype}")
    c = Case(H, HK, D, [100, 3000, 5, 1200], 1e4, 900 + D, dtype)
    try:
        worst = c.step(c.ctx)
        log(f"  max-abs err {worst:.3e}")
        assert worst <= (TOL_F16 if dtype == pk.PKH_KV_F16 else TOL_F32)
    finally:
        c.free()


def _ref_layout_kv(K, V, dtype):
    L, max_seq, HK, D = K.shape
    kv = pk.KV()
    kv.n_layers, kv.n_kv_heads, kv.head_dim, kv.max_seq = L, HK, D, max_seq
    kv.k_stride_layer = kv.v_stride_layer = max_seq * HK * D
    kv.k, kv.v = K.data_ptr(), V.data_ptr()
    kv.dtype, kv.device = dtype, 0
    kv.stride_pos, kv.stride_head = HK * D, D
    return kv


def test_reference_layout_any_shape():
    """Decode, then prefill, of an uneven-group, head_dim-24 shape in the
    reference's own [pos][kv_head][head_dim] layout (stride_pos 48,
    stride_head 24): key elements past a row's 24 belong to the next KV
    head and must not leak into its scores."""
    import torch
    lib = pk.load()
    dev = torch.device("cuda")
    H, HK, D, pos = 6, 2, 24, 1500
    max_seq = pos + 101
    kc, vc = normal(911, (max_seq, HK, D)), normal(912, (max_seq, HK, D))
    kc[pos:], vc[pos:] = 0.0, 0.0
    K = torch.from_numpy(kc).to(dev)[None].contiguous()
    V = torch.from_numpy(vc).to(dev)[None].contiguous()
    rope = DeviceRope(D, 1e4, max_seq)
    try:
        kv = _ref_layout_kv(K, V, pk.PKH_KV_F32)
        q, k, v = normal(913, (H, D)), normal(914, (HK, D)), normal(915, (HK, D))
        ao = np.zeros_like(q)
        pk.check(lib.pkh_attn_decode(ctypes.byref(kv), rope.ref, 0, pos, H, q.ctypes.data,
                                     k.ctypes.data, v.ctypes.data, ao.ctypes.data),
                 "pkh_attn_decode")
        ref, _, k_rot = po.decode_step(kc, vc, pos, q, k, v, rope.sin, rope.cos, 16)
        torch.cuda.synchronize()
        assert np.array_equal(K[0, pos].cpu().numpy(), k_rot)
        err = maxerr(ao, ref)
        log(f"decode, reference layout H{H} HK{HK} D{D}: max-abs err {err:.3e}")
        assert err <= TOL_F32
        n = 100
        qn, kn, vn = normal(916, (n, H, D)), normal(917, (n, HK, D)), normal(918, (n, HK, D))
        aon = np.zeros_like(qn)
        pk.check(lib.pkh_attn_prefill(ctypes.byref(kv), rope.ref, 0, pos + 1, n, H,
                                      qn.ctypes.data, kn.ctypes.data, vn.ctypes.data,
                                      aon.ctypes.data), "pkh_attn_prefill")
        refn = po.prefill(kc, vc, pos + 1, qn, kn, vn, rope.sin, rope.cos, 16)
        torch.cuda.synchronize()
        assert np.array_equal(K[0].cpu().numpy(), kc), "cache k rows"
        assert np.array_equal(V[0].cpu().numpy(), vc), "cache v rows"
        err = maxerr(aon, refn)
        log(f"prefill, reference layout: max-abs err {err:.3e}")
        assert err <= TOL_F16
    finally:
        rope.free()
