"""GPU check of pkh_attn_decode_noalloc_async, the decode entry point that
allocates nothing, through the C ABI.

Its kernels and split are those of pkh_attn_decode_async, so on the same
inputs its output must equal that entry point's bit for bit (and both must
match the oracle within the fp32 tolerance, 1e-4).  Two calls in a row, the
second with a smaller context, show that the fixed scratch's leftover
contents from the first call do not leak into the second.  A graph captured
around the entry point (no warm-up call is needed to size anything) replays
to the eager result, and a split larger than the fixed scratch is refused
with PKH_ERR_ARG before any launch.
"""
import ctypes

import numpy as np
import pytest

import lestramanika_amd as pk
from oracle import pyoracle as po
from pkh_util import DeviceKV, DeviceRope, log, maxerr, normal

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4


def _inputs(torch, H, HK, D, pos, seed):
    dev = torch.device("cuda")
    kv = DeviceKV(1, HK, D, pos + 1)
    rope = DeviceRope(D, 5e5, pos + 1)
    kc = normal(seed, (pos + 1, HK, D))
    vc = normal(seed + 1, (pos + 1, HK, D))
    kv.write(0, 0, 0, kc[:pos])
    kv.write(1, 0, 0, vc[:pos])
    q, k, v = normal(seed + 2, (H, D)), normal(seed + 3, (HK, D)), normal(seed + 4, (HK, D))
    ref, _, _ = po.decode_step(kc, vc, pos, q, k, v, rope.sin, rope.cos, 16)
    dq, dk, dv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
    return kv, rope, dq, dk, dv, ref


def test_noalloc_decode_matches_allocating_entry_on_two_calls():
    import torch
    lib = pk.load()
    H, HK, D = 32, 8, 128
    for pos, seed in ((8192, 701), (3000, 711)):      # second call: smaller context
        log(f"no-alloc decode H{H} HK{HK} D{D} pos{pos} seed{seed}")
        kv, rope, q, k, v, ref = _inputs(torch, H, HK, D, pos, seed)
        try:
            a = torch.full((H, D), float("nan"), device="cuda")
            b = torch.full((H, D), float("nan"), device="cuda")
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            rc = lib.pkh_attn_decode_noalloc_async(kv.ref, rope.ref, 0, pos, H, q.data_ptr(),
                                                   k.data_ptr(), v.data_ptr(), b.data_ptr(), s)
            assert rc == pk.PKH_OK, rc
            rc = lib.pkh_attn_decode_async(kv.ref, rope.ref, 0, pos, H, q.data_ptr(),
                                           k.data_ptr(), v.data_ptr(), a.data_ptr(), s)
            assert rc == pk.PKH_OK, rc
            torch.cuda.synchronize()
            assert torch.equal(a, b), "no-alloc and allocating entry points differ"
            err = maxerr(b.cpu().numpy(), ref)
            log(f"  identical to pkh_attn_decode_async; max-abs err vs oracle {err:.3e}")
            assert err <= TOL_F32
        finally:
            kv.free()
            rope.free()


def test_noalloc_decode_in_captured_graph():
    import torch
    lib = pk.load()
    H, HK, D, pos = 32, 8, 128, 5000
    kv, rope, q, k, v, ref = _inputs(torch, H, HK, D, pos, 721)
    try:
        out = torch.zeros((H, D), device="cuda")

        def call():
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            rc = lib.pkh_attn_decode_noalloc_async(kv.ref, rope.ref, 0, pos, H, q.data_ptr(),
                                                   k.data_ptr(), v.data_ptr(), out.data_ptr(), s)
            assert rc == pk.PKH_OK, rc

        call()
        torch.cuda.synchronize()
        eager = out.clone()
        assert maxerr(eager.cpu().numpy(), ref) <= TOL_F32
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                call()
        torch.cuda.synchronize()
        for it in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {it}"
            out.zero_()
            call()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"eager call {it}"
        log("3 graph replays of the no-alloc entry match its eager result")
    finally:
        kv.free()
        rope.free()


def test_noalloc_decode_refuses_a_split_beyond_its_scratch():
    import torch
    lib = pk.load()
    H, HK, D, pos = 32, 8, 128, 20000
    kv = DeviceKV(1, HK, D, pos + 1)
    rope = DeviceRope(D, 5e5, pos + 1)
    prev = lib.pkh_tune_decode_chunk(32)      # 626 chunks: 10.4 MB of partials
    try:
        buf = torch.zeros((H, D), device="cuda")
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        p = buf.data_ptr()
        rc = lib.pkh_attn_decode_noalloc_async(kv.ref, rope.ref, 0, pos, H, p, p, p, p, s)
        assert rc == pk.PKH_ERR_ARG
        torch.cuda.synchronize()
        assert not buf.any(), "nothing was launched"
    finally:
        lib.pkh_tune_decode_chunk(prev)
        kv.free()
        rope.free()
