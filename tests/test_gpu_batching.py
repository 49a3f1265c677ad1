"""Continuous batching on the GPU, through the C ABI: sequences prefilled into
their slots of one batch cache, then decode steps of all of them in one
launch per layer, replayed from a single captured HIP graph whose positions
advance through pkh_plan_update -- against separate oracle runs of each
sequence (the reference keeps one sequence per cache; docs/ROADMAP.md:56-62
plans batching, "done when interleaved sequences equal separate runs").

Tolerances: 2e-3 for prefill (fp16 MFMA operands), 1e-4 for fp32 decode.
"""
import ctypes

import numpy as np
import pytest

import lestramanika_amd as pk
from oracle import pyoracle as po
from pkh_util import DeviceKVBatch, DeviceRope, Plan, log, maxerr

pytestmark = pytest.mark.gpu

TOL_PREFILL = 2e-3
TOL_DECODE = 1e-4


def _pos_arg(t):
    return ctypes.cast(ctypes.c_void_p(t.data_ptr()), ctypes.POINTER(ctypes.c_int))


def test_two_sequences_interleaved_in_one_captured_graph():
    import torch
    lib = pk.load()
    dev = torch.device("cuda")
    H, HK, D, L, theta = 8, 2, 64, 2, 1e4
    caps, prompts = [300, 500], [60, 125]
    kvb = DeviceKVBatch(L, HK, D, caps)
    rope = DeviceRope(D, theta, max(caps))
    sin, cos = rope.sin, rope.cos
    rng = np.random.default_rng(2024)
    normal = lambda *shape: rng.standard_normal(shape, dtype=np.float32)
    kc = [[np.zeros((caps[s], HK, D), np.float32) for _ in range(L)] for s in range(2)]
    vc = [[np.zeros((caps[s], HK, D), np.float32) for _ in range(L)] for s in range(2)]
    plan = None
    try:
        # Prefill each sequence into its slots, every layer.
        s_ = torch.cuda.current_stream()
        for s, n in enumerate(prompts):
            for layer in range(L):
                q, k, v = normal(n, H, D), normal(n, HK, D), normal(n, HK, D)
                tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
                out = torch.empty((n, H, D), device=dev)
                rc = lib.pkh_attn_prefill_batch_async(kvb.ref, rope.ref, s, layer, 0, n, H, tq.data_ptr(),
                                                      tk.data_ptr(), tv.data_ptr(), out.data_ptr(),
                                                      ctypes.c_void_p(s_.cuda_stream))
                assert rc == pk.PKH_OK, rc
                torch.cuda.synchronize()
                ref = po.prefill(kc[s][layer], vc[s][layer], 0, q, k, v, sin, cos, 16)
                err = maxerr(out.cpu().numpy(), ref)
                assert err <= TOL_PREFILL, (s, layer, err)
                assert np.array_equal(kvb.read(0, layer, s, 0, n), kc[s][layer][:n])
                assert np.array_equal(kvb.read(1, layer, s, 0, n), vc[s][layer][:n])
        log(f"prefilled sequences of {prompts[0]} and {prompts[1]} tokens into one batch cache")

        plan = Plan(kvb, prompts, H)
        dq = torch.empty((L, 2, H, D), device=dev)
        dk = torch.empty((L, 2, HK, D), device=dev)
        dv = torch.empty((L, 2, HK, D), device=dev)
        dout = torch.empty((L, 2, H, D), device=dev)
        pos = torch.tensor(prompts, dtype=torch.int32).pin_memory()

        def step(stream):
            sp = ctypes.c_void_p(stream.cuda_stream)
            assert lib.pkh_plan_update(plan.ptr, _pos_arg(pos), sp) == pk.PKH_OK
            for layer in range(L):
                rc = lib.pkh_attn_decode_batch_async(kvb.ref, rope.ref, plan.ptr, layer,
                                                     dq[layer].data_ptr(), dk[layer].data_ptr(),
                                                     dv[layer].data_ptr(), dout[layer].data_ptr(), sp)
                assert rc == pk.PKH_OK, rc

        def check(i, p):
            worst = 0.0
            for layer in range(L):
                for s in range(2):
                    ref, _, _ = po.decode_step(kc[s][layer], vc[s][layer], p[s], hq[layer][s],
                                               hk[layer][s], hv[layer][s], sin, cos, 16)
                    worst = max(worst, maxerr(dout[layer, s].cpu().numpy(), ref))
                    assert np.array_equal(kvb.read(0, layer, s, p[s], 1)[0], kc[s][layer][p[s]])
            log(f"step {i}: positions {p}, max-abs err vs separate oracle runs {worst:.3e}")
            assert worst <= TOL_DECODE

        graph = None
        for i in range(10):
            p = [prompts[0] + i, prompts[1] + i]
            hq, hk, hv = normal(L, 2, H, D), normal(L, 2, HK, D), normal(L, 2, HK, D)
            dq.copy_(torch.from_numpy(hq))
            dk.copy_(torch.from_numpy(hk))
            dv.copy_(torch.from_numpy(hv))
            pos.copy_(torch.tensor(p, dtype=torch.int32))
            torch.cuda.synchronize()
            if i == 0:
                step(torch.cuda.current_stream())       # eager: sizes the library's scratch
                torch.cuda.synchronize()
                check(i, p)
                graph = torch.cuda.CUDAGraph()
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    with torch.cuda.graph(graph, stream=side):
                        step(side)
                torch.cuda.synchronize()
                continue
            graph.replay()                               # positions come from the pinned array
            torch.cuda.synchronize()
            check(i, p)

        # A replayed position past sequence 0's capacity: NaN for it, no row
        # written anywhere in its slots; sequence 1 steps on as usual.
        p = [caps[0], prompts[1] + 10]
        before = kvb.read(0, 0, 0, 0, caps[0]).copy()
        hq, hk, hv = normal(L, 2, H, D), normal(L, 2, HK, D), normal(L, 2, HK, D)
        dq.copy_(torch.from_numpy(hq))
        dk.copy_(torch.from_numpy(hk))
        dv.copy_(torch.from_numpy(hv))
        pos.copy_(torch.tensor(p, dtype=torch.int32))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isnan(dout[:, 0]).all()
        assert np.array_equal(kvb.read(0, 0, 0, 0, caps[0]), before)
        for layer in range(L):
            ref, _, _ = po.decode_step(kc[1][layer], vc[1][layer], p[1], hq[layer][1], hk[layer][1],
                                       hv[layer][1], sin, cos, 16)
            assert maxerr(dout[layer, 1].cpu().numpy(), ref) <= TOL_DECODE
        # The host-side check refuses the same positions before enqueuing anything.
        bad = (ctypes.c_int * 2)(*p)
        assert lib.pkh_plan_update(plan.ptr, bad, None) == pk.PKH_ERR_RANGE
    finally:
        if plan is not None:
            plan.free()
        kvb.free()
        rope.free()


def test_prefill_into_a_slot_leaves_other_sequences_alone():
    """Prefill of sequence 1 of three writes only its own slots."""
    import torch
    lib = pk.load()
    dev = torch.device("cuda")
    H, HK, D, caps, n = 4, 2, 32, [40, 70, 50], 64
    kvb = DeviceKVBatch(1, HK, D, caps)
    rope = DeviceRope(D, 1e4, max(caps))
    try:
        rng = np.random.default_rng(7)
        q = rng.standard_normal((n, H, D), dtype=np.float32)
        k = rng.standard_normal((n, HK, D), dtype=np.float32)
        v = rng.standard_normal((n, HK, D), dtype=np.float32)
        tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
        out = torch.empty((n, H, D), device=dev)
        rc = lib.pkh_attn_prefill_batch_async(kvb.ref, rope.ref, 1, 0, 0, n, H, tq.data_ptr(), tk.data_ptr(),
                                              tv.data_ptr(), out.data_ptr(), None)
        assert rc == pk.PKH_OK
        torch.cuda.synchronize()
        kc = np.zeros((caps[1], HK, D), np.float32)
        vc = np.zeros_like(kc)
        ref = po.prefill(kc, vc, 0, q, k, v, rope.sin, rope.cos, 16)
        assert maxerr(out.cpu().numpy(), ref) <= TOL_PREFILL
        for s in (0, 2):
            assert not kvb.read(0, 0, s, 0, caps[s]).any() and not kvb.read(1, 0, s, 0, caps[s]).any()
        assert np.array_equal(kvb.read(0, 0, 1, 0, n), kc[:n])
        # a prompt past the sequence's capacity is refused before any launch
        assert lib.pkh_attn_prefill_batch_async(kvb.ref, rope.ref, 1, 0, 10, n, H, tq.data_ptr(),
                                                tk.data_ptr(), tv.data_ptr(), out.data_ptr(),
                                                None) == pk.PKH_ERR_RANGE
        assert lib.pkh_attn_prefill_batch_async(kvb.ref, rope.ref, 3, 0, 0, 8, H, tq.data_ptr(),
                                                tk.data_ptr(), tv.data_ptr(), out.data_ptr(),
                                                None) == pk.PKH_ERR_RANGE
    finally:
        kvb.free()
        rope.free()
