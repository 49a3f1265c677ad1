"""GPU parity of the decode path (pkh_attn_decode*) against the oracle and the
reference's own outputs, through the C ABI.

Tolerances (written here, as stated for the path): max-abs 1e-4 for an fp32
KV cache, 2e-3 for fp16.  The appended cache row is compared bit for bit.
"""
import ctypes
import glob
import os

import numpy as np
import pytest

import lestramanika_amd as pk
from oracle import pyoracle as po
from pkh_util import DeviceKV, DeviceRope, decode_host, log, maxerr, normal

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_F16 = 2e-3
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _run_case(H, HK, D, pos, theta, seed, dtype=pk.PKH_KV_F32, layer=0, n_layers=1,
              max_seq=None, threads=16):
    max_seq = max_seq or pos + 1
    kc = normal(seed, (max_seq, HK, D))
    vc = normal(seed + 1, (max_seq, HK, D))
    q = normal(seed + 2, (H, D))
    k = normal(seed + 3, (HK, D))
    v = normal(seed + 4, (HK, D))
    kv = DeviceKV(n_layers, HK, D, max_seq, dtype)
    rope = DeviceRope(D, theta, pos + 1, max_seq=max_seq)
    try:
        if dtype == pk.PKH_KV_F16:
            kc16, vc16 = po.f32_to_f16_bits(kc), po.f32_to_f16_bits(vc)
            kv.write(0, layer, 0, kc16[:pos])
            kv.write(1, layer, 0, vc16[:pos])
            ao = decode_host(kv, rope, layer, pos, q, k, v)
            k16, v16 = kc16[:pos + 1].copy(), vc16[:pos + 1].copy()
            ref = po.decode_step_f16(k16, v16, pos, q, k, v, rope.sin, rope.cos, threads)
            row_k, row_v = kv.read(0, layer, pos, 1)[0], kv.read(1, layer, pos, 1)[0]
            assert np.array_equal(row_k, k16[pos]) and np.array_equal(row_v, v16[pos])
        else:
            kv.write(0, layer, 0, kc[:pos])
            kv.write(1, layer, 0, vc[:pos])
            ao = decode_host(kv, rope, layer, pos, q, k, v)
            kr_c, vr_c = kc[:pos + 1].copy(), vc[:pos + 1].copy()
            ref, _, k_rot = po.decode_step(kr_c, vr_c, pos, q, k, v, rope.sin, rope.cos, threads)
            row_k, row_v = kv.read(0, layer, pos, 1)[0], kv.read(1, layer, pos, 1)[0]
            assert np.array_equal(row_k, k_rot), "appended k row differs from the oracle"
            assert np.array_equal(row_v, v), "appended v row differs"
        return ao, ref, kv, rope
    except BaseException:
        kv.free()
        rope.free()
        raise


def _check(H, HK, D, pos, theta, seed, dtype=pk.PKH_KV_F32, **kw):
    log(f"decode H{H} HK{HK} D{D} pos{pos} theta{theta:g} dtype{dtype} seed{seed} {kw}")
    ao, ref, kv, rope = _run_case(H, HK, D, pos, theta, seed, dtype, **kw)
    kv.free()
    rope.free()
    err = maxerr(ao, ref)
    log(f"  max-abs err {err:.3e}")
    assert err <= (TOL_F16 if dtype == pk.PKH_KV_F16 else TOL_F32)
    return err


PROBES = [p for p in sorted(glob.glob(os.path.join(GOLDEN, "attn_probe_*.npz")))]


@pytest.mark.parametrize("path", PROBES, ids=[os.path.basename(p)[11:-4] for p in PROBES])
def test_decode_matches_reference_outputs(path):
    """GPU decode against the compiled reference's own ao on the probe inputs."""
    z = np.load(path)
    H, HK, D, pos = (int(x) for x in z["shape"])
    log(f"probe {os.path.basename(path)}")
    kv = DeviceKV(1, HK, D, pos + 1)
    rope = DeviceRope(D, float(z["theta"]), pos + 1)
    try:
        if pos:
            kv.write(0, 0, 0, z["cache_k"])
            kv.write(1, 0, 0, z["cache_v"])
        ao = decode_host(kv, rope, 0, pos, z["q"], z["k"], z["v"])
        assert np.array_equal(kv.read(0, 0, pos, 1)[0], z["row_k"])
        assert np.array_equal(kv.read(1, 0, pos, 1)[0], z["row_v"])
        err = maxerr(ao, z["ao"])
        log(f"  max-abs err vs reference {err:.3e}")
        assert err <= TOL_F32
    finally:
        kv.free()
        rope.free()


def test_decode_bad_arguments_are_rejected():
    lib = pk.load()
    kv = DeviceKV(1, 4, 16, 8)
    rope = DeviceRope(16, 1e4, 8)
    try:
        q = np.zeros((6, 16), np.float32)
        k = np.zeros((4, 16), np.float32)
        ao = np.zeros_like(q)
        rc = lib.pkh_attn_decode(kv.ref, rope.ref, 0, 3, 0, q.ctypes.data, k.ctypes.data,
                                 k.ctypes.data, ao.ctypes.data)
        assert rc == pk.PKH_ERR_ARG          # no query heads
        rc = lib.pkh_attn_decode(kv.ref, rope.ref, 0, 8, 8, q.ctypes.data, k.ctypes.data,
                                 k.ctypes.data, ao.ctypes.data)
        assert rc == pk.PKH_ERR_RANGE
    finally:
        kv.free()
        rope.free()


def test_decode_tinyllama_shape_ctx2048():
    """TinyLlama-1.1B shape: H32 HK4 D64, 2048 cached rows, theta 1e4, seed 2."""
    _check(32, 4, 64, 2048, 1e4, 2)


def test_decode_llama3_8b_shape_ctx8192():
    """Llama-3-8B shape: H32 HK8 D128, 8192 cached rows, theta 5e5, seed 3,
    on layer 1 of a two-layer cache."""
    _check(32, 8, 128, 8192, 5e5, 3, layer=1, n_layers=2)


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_decode_shape_sweep(D, G):
    HK = 2
    for pos in (0, 1, 63, 130, 1031):
        _check(G * HK, HK, D, pos, 1e4, 100 + D + G + pos)


@pytest.mark.parametrize("D,G", [(16, 2), (64, 8), (128, 4), (128, 8), (256, 1)])
def test_decode_fp16_kv(D, G):
    for pos in (0, 5, 700, 4100):
        _check(G * 2, 2, D, pos, 5e5, 200 + D + pos, dtype=pk.PKH_KV_F16)


def test_decode_chunking_is_invisible():
    """Different split-K chunk sizes (one chunk, many chunks) agree within
    tolerance, and a repeated call is bit-identical."""
    lib = pk.load()
    H, HK, D, pos = 32, 8, 128, 3000
    outs = []
    try:
        for chunk in (0, 32, 96, 512, 4096):
            lib.pkh_tune_decode_chunk(chunk)
            ao, ref, kv, rope = _run_case(H, HK, D, pos, 5e5, 9)
            ao2 = decode_host(kv, rope, 0, pos, normal(11, (H, D)), normal(12, (HK, D)),
                              normal(13, (HK, D)))
            ao3 = decode_host(kv, rope, 0, pos, normal(11, (H, D)), normal(12, (HK, D)),
                              normal(13, (HK, D)))
            kv.free()
            rope.free()
            assert np.array_equal(ao2, ao3)
            err = maxerr(ao, ref)
            log(f"chunk {chunk}: max-abs err {err:.3e}")
            assert err <= TOL_F32
            outs.append(ao)
    finally:
        lib.pkh_tune_decode_chunk(0)
    for o in outs[1:]:
        assert maxerr(o, outs[0]) <= 2 * TOL_F32


def test_decode_more_chunks_than_threads():
    """More than 256 chunks per KV head: the merging work item polls and
    clears the ready flags in several passes per thread and merges the
    partials in several batches; two calls in a row must both match the
    oracle (a flag left set would hand the second call a stale partial)."""
    lib = pk.load()
    H, HK, D, pos = 32, 8, 128, 12000
    try:
        lib.pkh_tune_decode_chunk(32)     # 376 chunks per KV head
        for seed in (51, 52):
            ao, ref, kv, rope = _run_case(H, HK, D, pos, 5e5, seed)
            kv.free()
            rope.free()
            err = maxerr(ao, ref)
            log(f"seed {seed}: max-abs err {err:.3e}")
            assert err <= TOL_F32
    finally:
        lib.pkh_tune_decode_chunk(0)


def test_decode_other_layers_untouched():
    H, HK, D, pos = 8, 2, 64, 100
    ao, ref, kv, rope = _run_case(H, HK, D, pos, 1e4, 21, layer=1, n_layers=3, max_seq=128)
    try:
        assert maxerr(ao, ref) <= TOL_F32
        for L in (0, 2):
            assert not kv.read(0, L, 0, 128).any() and not kv.read(1, L, 0, 128).any()
        # rows past pos in the written layer are still zero
        assert not kv.read(0, 1, pos + 1, 128 - pos - 1).any()
    finally:
        kv.free()
        rope.free()


def test_decode_async_on_torch_stream_matches_host_entry():
    import torch
    lib = pk.load()
    H, HK, D, pos = 32, 8, 128, 5000
    ao, ref, kv, rope = _run_case(H, HK, D, pos, 5e5, 31)
    try:
        dev = torch.device("cuda")
        q = torch.from_numpy(normal(33, (H, D))).to(dev)
        k = torch.from_numpy(normal(34, (HK, D))).to(dev)
        v = torch.from_numpy(normal(35, (HK, D))).to(dev)
        out = torch.empty((H, D), dtype=torch.float32, device=dev)
        s = torch.cuda.current_stream()
        rc = lib.pkh_attn_decode_async(kv.ref, rope.ref, 0, pos, H, q.data_ptr(), k.data_ptr(),
                                       v.data_ptr(), out.data_ptr(), ctypes.c_void_p(s.cuda_stream))
        assert rc == 0
        torch.cuda.synchronize()
        host = decode_host(kv, rope, 0, pos, q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy())
        assert np.array_equal(out.cpu().numpy(), host)
    finally:
        kv.free()
        rope.free()


def test_decode_split_combine_alternating_inputs():
    """Back-to-back decodes of one layer with alternating inputs and several
    chunk sizes: every result must match the oracle, so a stale split-K
    partial or a missed last-work-item hand-off would show."""
    lib = pk.load()
    H, HK, D, pos = 32, 8, 128, 6000
    kv = DeviceKV(1, HK, D, pos + 1)
    rope = DeviceRope(D, 5e5, pos + 1)
    try:
        kc = normal(41, (pos + 1, HK, D))
        vc = normal(42, (pos + 1, HK, D))
        kv.write(0, 0, 0, kc[:pos])
        kv.write(1, 0, 0, vc[:pos])
        sets = [(normal(43 + 3 * i, (H, D)), normal(44 + 3 * i, (HK, D)),
                 normal(45 + 3 * i, (HK, D))) for i in range(2)]
        refs = []
        for q, k, v in sets:
            kr, vr = kc[:pos + 1].copy(), vc[:pos + 1].copy()
            refs.append(po.decode_step(kr, vr, pos, q, k, v, rope.sin, rope.cos, 16)[0])
        for chunk in (0, 64, 256, 1024):
            lib.pkh_tune_decode_chunk(chunk)
            for it in range(6):
                q, k, v = sets[it % 2]
                ao = decode_host(kv, rope, 0, pos, q, k, v)
                err = maxerr(ao, refs[it % 2])
                assert err <= TOL_F32, (chunk, it, err)
            log(f"chunk {chunk}: 6 alternating calls within tolerance")
    finally:
        lib.pkh_tune_decode_chunk(0)
        kv.free()
        rope.free()


def test_decode_interleaved_shapes():
    """Multi-chunk decodes of five shapes, cycled twice on one device: the
    shapes share the split-K partial buffer and ready flags under different
    layouts and chunk counts, and every call must match the oracle -- a
    partial written under another shape's layout, or left by an earlier
    call, must never be merged."""
    shapes = [(32, 8, 128, 3000), (32, 4, 64, 2500), (8, 2, 256, 1800), (8, 8, 32, 4000),
              (32, 8, 64, 3300)]
    for rnd in range(2):
        for i, (H, HK, D, pos) in enumerate(shapes):
            _check(H, HK, D, pos + rnd, 5e5, 300 + 10 * i + rnd)


def test_decode_graph_replay_after_scratch_growth():
    """A HIP graph captured around a decode stays valid after a later call
    outgrows the library's split-K scratch: the outgrown partial and flag
    buffers stay allocated, so the graph's kernels still address live memory.
    Every replay, with eager work and synchronizations between replays,
    matches the eager result of the same call bit for bit."""
    import torch
    lib = pk.load()
    dev = torch.device("cuda")
    H, HK, D, pos = 32, 8, 128, 3000
    kv = DeviceKV(1, HK, D, pos + 1)
    rope = DeviceRope(D, 5e5, pos + 1)
    big_kv = big_rope = None
    try:
        kv.write(0, 0, 0, normal(61, (pos, HK, D)))
        kv.write(1, 0, 0, normal(62, (pos, HK, D)))
        q = torch.from_numpy(normal(63, (H, D))).to(dev)
        k = torch.from_numpy(normal(64, (HK, D))).to(dev)
        v = torch.from_numpy(normal(65, (HK, D))).to(dev)
        out = torch.zeros((H, D), dtype=torch.float32, device=dev)

        def call():
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            rc = lib.pkh_attn_decode_async(kv.ref, rope.ref, 0, pos, H, q.data_ptr(), k.data_ptr(),
                                           v.data_ptr(), out.data_ptr(), s)
            assert rc == 0, rc

        call()
        torch.cuda.synchronize()
        eager = out.clone()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                call()
        torch.cuda.synchronize()
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), "first replay"
        # A much larger split (1875 chunks per KV head) outgrows every buffer
        # the earlier calls of this process sized.
        big_pos = 60000
        big_kv = DeviceKV(1, HK, D, big_pos + 1)
        big_rope = DeviceRope(D, 5e5, big_pos + 1)
        prev = lib.pkh_tune_decode_chunk(32)
        try:
            big = decode_host(big_kv, big_rope, 0, big_pos, normal(66, (H, D)),
                              normal(67, (HK, D)), normal(68, (HK, D)))
        finally:
            lib.pkh_tune_decode_chunk(prev)
        assert np.isfinite(big).all()
        log("scratch grown by a 60001-row decode split into 32-row chunks")
        for it in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {it} after growth"
            out.zero_()
            call()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"eager call {it} after growth"
        log("3 replays after growth match the eager result")
    finally:
        kv.free()
        rope.free()
        if big_kv is not None:
            big_kv.free()
        if big_rope is not None:
            big_rope.free()


def test_init_selects_only_existing_devices():
    """pkh_init accepts the devices the runtime reports and rejects others
    with PKH_ERR_ARG, leaving the current device in place."""
    import torch
    lib = pk.load()
    n = torch.cuda.device_count()
    assert lib.pkh_init(0) == pk.PKH_OK
    assert lib.pkh_init(-1) == pk.PKH_ERR_ARG
    assert lib.pkh_init(n) == pk.PKH_ERR_ARG
    assert lib.pkh_init(0) == pk.PKH_OK
    _check(8, 2, 64, 300, 1e4, 91)   # the library still decodes on device 0


def test_decode_wait_bound_gives_nan_and_leaves_no_state():
    """The split-K merger's bounded wait, forced to give up from the host
    (a bound of 0 polling rounds): every head it merges comes out NaN, never
    a merge of missing partials, and the kernel still ends normally.  The
    next calls with the default bound match the oracle, so the timed-out
    launch left no ready flag behind for a later launch to mistake for its
    own partial."""
    lib = pk.load()
    H, HK, D, pos = 32, 8, 128, 3000
    prev_chunk = lib.pkh_tune_decode_chunk(256)      # 12 chunks per KV head
    prev_wait = lib.pkh_tune_decode_wait(0)
    try:
        ao, ref, kv, rope = _run_case(H, HK, D, pos, 5e5, 81)
        try:
            assert np.isnan(ao).all(), "a wait that ran out must yield NaN"
            log("wait bound 0: all heads NaN")
            lib.pkh_tune_decode_wait(-1)
            q, k, v = normal(83, (H, D)), normal(84, (HK, D)), normal(85, (HK, D))
            for it in range(2):
                ao = decode_host(kv, rope, 0, pos, q, k, v)
                kc = kv.read(0, 0, 0, pos + 1)
                vc = kv.read(1, 0, 0, pos + 1)
                kc[pos] = 0.0
                vc[pos] = 0.0
                ref, _, _ = po.decode_step(kc, vc, pos, q, k, v, rope.sin, rope.cos, 16)
                err = maxerr(ao, ref)
                log(f"  default bound, call {it}: max-abs err {err:.3e}")
                assert err <= TOL_F32
        finally:
            kv.free()
            rope.free()
    finally:
        lib.pkh_tune_decode_wait(prev_wait)
        lib.pkh_tune_decode_chunk(prev_chunk)
