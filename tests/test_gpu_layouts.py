"""GPU parity with the KV cache in the reference's own layout, described
through pkh_kv_t's strides: separate K and V buffers, each layer
[pos][kv_head][head_dim] (src/pickle_fast.c:1940-1942), so stride_pos =
n_kv_heads * head_dim and stride_head = head_dim.  The caches are torch
tensors; the library only sees their device pointers.

Tolerances as for the default layout: max-abs 1e-4 (fp32 decode), 2e-3 (fp16
KV, and prefill's fp16 operands); appended rows bit for bit.
"""
import ctypes

import numpy as np
import pytest

import lestramanika_amd as pk
from oracle import pyoracle as po
from pkh_util import DeviceRope, log, maxerr, normal

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_F16 = 2e-3


def _ref_layout_kv(K, V, dtype):
    """A pkh_kv_t over torch tensors K, V of shape [layers][max_seq][HK][D]."""
    L, max_seq, HK, D = K.shape
    kv = pk.KV()
    kv.n_layers, kv.n_kv_heads, kv.head_dim, kv.max_seq = L, HK, D, max_seq
    kv.k_stride_layer = kv.v_stride_layer = max_seq * HK * D
    kv.k, kv.v = K.data_ptr(), V.data_ptr()
    kv.dtype, kv.device = dtype, 0
    kv.stride_pos, kv.stride_head = HK * D, D
    return kv


def _decode(kv, rope, layer, pos, q, k, v):
    lib = pk.load()
    ao = np.zeros_like(q)
    pk.check(lib.pkh_attn_decode(ctypes.byref(kv), rope.ref, layer, pos, q.shape[0],
                                 q.ctypes.data, k.ctypes.data, v.ctypes.data, ao.ctypes.data),
             "pkh_attn_decode")
    return ao


def test_decode_reference_layout_f32():
    import torch
    dev = torch.device("cuda")
    H, HK, D, pos, layer = 32, 8, 128, 2500, 1
    max_seq = pos + 1
    log(f"decode, reference layout, fp32: H{H} HK{HK} D{D} pos {pos} layer {layer}/2")
    kc, vc = normal(71, (max_seq, HK, D)), normal(72, (max_seq, HK, D))
    q, k, v = normal(73, (H, D)), normal(74, (HK, D)), normal(75, (HK, D))
    K = torch.zeros((2, max_seq, HK, D), dtype=torch.float32, device=dev)
    V = torch.zeros_like(K)
    K[layer, :pos] = torch.from_numpy(kc[:pos]).to(dev)
    V[layer, :pos] = torch.from_numpy(vc[:pos]).to(dev)
    rope = DeviceRope(D, 5e5, pos + 1)
    try:
        ao = _decode(_ref_layout_kv(K, V, pk.PKH_KV_F32), rope, layer, pos, q, k, v)
        kr, vr = kc.copy(), vc.copy()
        ref, _, k_rot = po.decode_step(kr, vr, pos, q, k, v, rope.sin, rope.cos, 16)
        torch.cuda.synchronize()
        assert np.array_equal(K[layer, pos].cpu().numpy(), k_rot), "appended k row"
        assert np.array_equal(V[layer, pos].cpu().numpy(), v), "appended v row"
        assert not K[0].any() and not V[0].any(), "other layer written"
        err = maxerr(ao, ref)
        log(f"  max-abs err {err:.3e}")
        assert err <= TOL_F32
    finally:
        rope.free()


def test_decode_reference_layout_f16():
    import torch
    dev = torch.device("cuda")
    H, HK, D, pos, layer = 16, 4, 64, 3100, 1
    max_seq = pos + 1
    log(f"decode, reference layout, fp16: H{H} HK{HK} D{D} pos {pos} layer {layer}/2")
    kc16 = po.f32_to_f16_bits(normal(81, (max_seq, HK, D)))
    vc16 = po.f32_to_f16_bits(normal(82, (max_seq, HK, D)))
    q, k, v = normal(83, (H, D)), normal(84, (HK, D)), normal(85, (HK, D))
    K = torch.zeros((2, max_seq, HK, D), dtype=torch.int16, device=dev)
    V = torch.zeros_like(K)
    K[layer, :pos] = torch.from_numpy(kc16[:pos].view(np.int16)).to(dev)
    V[layer, :pos] = torch.from_numpy(vc16[:pos].view(np.int16)).to(dev)
    rope = DeviceRope(D, 1e4, pos + 1)
    try:
        ao = _decode(_ref_layout_kv(K, V, pk.PKH_KV_F16), rope, layer, pos, q, k, v)
        k16, v16 = kc16.copy(), vc16.copy()
        ref = po.decode_step_f16(k16, v16, pos, q, k, v, rope.sin, rope.cos, 16)
        torch.cuda.synchronize()
        assert np.array_equal(K[layer, pos].cpu().numpy().view(np.uint16), k16[pos]), \
            "appended k row"
        assert np.array_equal(V[layer, pos].cpu().numpy().view(np.uint16), v16[pos]), \
            "appended v row"
        assert not K[0].any() and not V[0].any(), "other layer written"
        err = maxerr(ao, ref)
        log(f"  max-abs err {err:.3e}")
        assert err <= TOL_F16
    finally:
        rope.free()


def test_prefill_reference_layout_f32():
    import torch
    lib = pk.load()
    dev = torch.device("cuda")
    H, HK, D, pos0, n, layer = 32, 8, 128, 150, 333, 1
    max_seq = pos0 + n
    log(f"prefill, reference layout, fp32: H{H} HK{HK} D{D} pos0 {pos0} n {n} layer {layer}/2")
    ctx_k, ctx_v = normal(91, (pos0, HK, D)), normal(92, (pos0, HK, D))
    q, k, v = normal(93, (n, H, D)), normal(94, (n, HK, D)), normal(95, (n, HK, D))
    K = torch.zeros((2, max_seq, HK, D), dtype=torch.float32, device=dev)
    V = torch.zeros_like(K)
    K[layer, :pos0] = torch.from_numpy(ctx_k).to(dev)
    V[layer, :pos0] = torch.from_numpy(ctx_v).to(dev)
    rope = DeviceRope(D, 5e5, max_seq)
    try:
        kv = _ref_layout_kv(K, V, pk.PKH_KV_F32)
        ao = np.zeros_like(q)
        pk.check(lib.pkh_attn_prefill(ctypes.byref(kv), rope.ref, layer, pos0, n, H,
                                      q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                      ao.ctypes.data), "pkh_attn_prefill")
        kc = np.zeros((max_seq, HK, D), np.float32)
        vc = np.zeros_like(kc)
        kc[:pos0], vc[:pos0] = ctx_k, ctx_v
        ref = po.prefill(kc, vc, pos0, q, k, v, rope.sin, rope.cos, 16)
        torch.cuda.synchronize()
        assert np.array_equal(K[layer].cpu().numpy(), kc), "cache k rows"
        assert np.array_equal(V[layer].cpu().numpy(), vc), "cache v rows"
        assert not K[0].any() and not V[0].any(), "other layer written"
        err = maxerr(ao, ref)
        log(f"  max-abs err {err:.3e}")
        assert err <= TOL_F16
    finally:
        rope.free()
