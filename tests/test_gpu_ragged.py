"""GPU parity of ragged multi-sequence decode (pkh_attn_decode_batch_async)
against the oracle run one sequence at a time, through the C ABI.

The reference has no batch API (it keeps one sequence per pickle_fast_kv_t),
so the oracle for sequence s is its single-sequence decode step on that
sequence's rows.  Tolerances: max-abs 1e-4 for an fp32 cache, 2e-3 for fp16
(the oracle then runs in fp32 on the fp16-widened rows); appended rows are
compared bit for bit.
"""
import ctypes

import numpy as np
import pytest

import lestramanika_amd as pk
from oracle import pyoracle as po
from pkh_util import DeviceKVBatch, DeviceRope, Plan, log, maxerr

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_F16 = 2e-3


def _rng_normal(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32)


class Case:
    """Ragged caches of n sequences (context ctx[s], new token at ctx[s])
    filled on the device, plus the host copy the oracle reads."""

    def __init__(self, H, HK, D, ctx, theta, seed, dtype, n_layers=1, layer=0, spare=0):
        self.H, self.HK, self.D, self.dtype, self.layer = H, HK, D, dtype, layer
        self.ctx = list(ctx)
        self.max_seq = [c + 1 + spare for c in self.ctx]
        self.kvb = DeviceKVBatch(n_layers, HK, D, self.max_seq, dtype)
        self.rope = DeviceRope(D, theta, max(self.max_seq), max_seq=max(self.max_seq))
        rng = np.random.default_rng(seed)
        self.k_rows, self.v_rows = [], []
        for s, c in enumerate(self.ctx):
            kc = np.zeros((self.max_seq[s], HK, D), np.float32)
            vc = np.zeros_like(kc)
            kc[:c] = _rng_normal(rng, (c, HK, D))
            vc[:c] = _rng_normal(rng, (c, HK, D))
            if dtype == pk.PKH_KV_F16:
                kc, vc = po.f32_to_f16_bits(kc), po.f32_to_f16_bits(vc)
            if c:
                self.kvb.write(0, layer, s, 0, kc[:c])
                self.kvb.write(1, layer, s, 0, vc[:c])
            self.k_rows.append(kc)
            self.v_rows.append(vc)
        self.rng = rng

    def step(self, pos):
        """One decode step at positions pos[s] (device), then the oracle for
        every sequence; returns the largest max-abs error."""
        import torch
        lib = pk.load()
        n, H, HK, D = len(pos), self.H, self.HK, self.D
        q = _rng_normal(self.rng, (n, H, D))
        k = _rng_normal(self.rng, (n, HK, D))
        v = _rng_normal(self.rng, (n, HK, D))
        plan = Plan(self.kvb, pos, H)
        try:
            dev = torch.device("cuda")
            tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
            out = torch.empty((n, H, D), dtype=torch.float32, device=dev)
            s_ = torch.cuda.current_stream()
            rc = lib.pkh_attn_decode_batch_async(self.kvb.ref, self.rope.ref, plan.ptr, self.layer,
                                                 tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                                                 out.data_ptr(), ctypes.c_void_p(s_.cuda_stream))
            assert rc == 0, rc
            torch.cuda.synchronize()
            ao = out.cpu().numpy()
        finally:
            plan.free()
        worst = 0.0
        for s, p in enumerate(pos):
            kc, vc = self.k_rows[s], self.v_rows[s]
            if self.dtype == pk.PKH_KV_F16:
                ref = po.decode_step_f16(kc, vc, p, q[s], k[s], v[s], self.rope.sin,
                                         self.rope.cos, 16)
            else:
                ref, _, _ = po.decode_step(kc, vc, p, q[s], k[s], v[s], self.rope.sin,
                                           self.rope.cos, 16)
            assert np.array_equal(self.kvb.read(0, self.layer, s, p, 1)[0], kc[p]), \
                f"appended k row of sequence {s} differs"
            assert np.array_equal(self.kvb.read(1, self.layer, s, p, 1)[0], vc[p]), \
                f"appended v row of sequence {s} differs"
            worst = max(worst, maxerr(ao[s], ref))
        return worst

    def free(self):
        self.kvb.free()
        self.rope.free()


def _check(H, HK, D, ctx, theta, seed, dtype=pk.PKH_KV_F32, **kw):
    log(f"ragged H{H} HK{HK} D{D} dtype {dtype} seed {seed} ctx {list(ctx)[:8]}"
        f"{'...' if len(ctx) > 8 else ''} ({len(ctx)} seqs) {kw}")
    case = Case(H, HK, D, ctx, theta, seed, dtype, **kw)
    try:
        err = case.step(list(case.ctx))
    finally:
        case.free()
    log(f"  max-abs err {err:.3e}")
    assert err <= (TOL_F16 if dtype == pk.PKH_KV_F16 else TOL_F32)


def test_ragged_16_sequences_llama3_fp16():
    """16 sequences with contexts drawn from U[4096, 32768] (numpy
    default_rng(5)), Llama-3-8B shape H32 HK8 D128, fp16 cache, theta 5e5,
    on layer 1 of a two-layer cache."""
    ctx = np.random.default_rng(5).integers(4096, 32768, size=16, endpoint=True).tolist()
    _check(32, 8, 128, ctx, 5e5, 5, pk.PKH_KV_F16, n_layers=2, layer=1)


def test_ragged_mixed_lengths_fp32():
    """One-row, short, tile-straddling and multi-chunk contexts in one batch."""
    _check(8, 2, 64, [0, 1, 63, 64, 700, 2100, 5], 1e4, 11)


@pytest.mark.parametrize("D,G", [(16, 2), (32, 8), (64, 1), (128, 4), (256, 2)])
def test_ragged_shapes(D, G):
    for dtype in (pk.PKH_KV_F32, pk.PKH_KV_F16):
        _check(2 * G, 2, D, [3, 130, 1500, 40], 5e5, 20 + D + G, dtype)


def test_ragged_single_sequence_matches_single_entry():
    """A batch of one sequence equals the single-sequence path's oracle."""
    _check(32, 8, 128, [3000], 5e5, 31)


def test_ragged_consecutive_steps_and_chunk_sizes():
    """Three decode steps in a row (each appends a row the next one reads),
    under several split sizes, so one-chunk and many-chunk sequences mix."""
    lib = pk.load()
    try:
        for chunk in (0, 64, 512):
            lib.pkh_tune_decode_chunk(chunk)
            ctx = [10, 900, 300, 2500]
            case = Case(16, 4, 128, ctx, 5e5, 41 + chunk, pk.PKH_KV_F32, spare=3)
            try:
                for t in range(3):
                    err = case.step([c + t for c in ctx])
                    log(f"chunk {chunk} step {t}: max-abs err {err:.3e}")
                    assert err <= TOL_F32
            finally:
                case.free()
    finally:
        lib.pkh_tune_decode_chunk(0)


def test_ragged_rejects_bad_plans():
    lib = pk.load()
    kvb = DeviceKVBatch(1, 2, 64, [8, 16])
    try:
        ptr = ctypes.c_void_p()
        assert lib.pkh_plan_create(kvb.ref, (ctypes.c_int * 2)(8, 3), 4,
                                   ctypes.byref(ptr)) == pk.PKH_ERR_RANGE   # pos >= max_seq
        assert lib.pkh_plan_create(kvb.ref, (ctypes.c_int * 2)(1, 3), 0,
                                   ctypes.byref(ptr)) == pk.PKH_ERR_ARG     # no query heads
        assert lib.pkh_kv_batch_copy_rows(kvb.ref, 0, 0, 2, 0, 1, ctypes.c_void_p(1),
                                          0) == pk.PKH_ERR_RANGE              # no sequence 2
    finally:
        kvb.free()


def test_ragged_after_split_decode_with_fewer_counters():
    """A single-sequence decode split into many chunks (its partials fill the
    scratch), then a ragged step that needs more (sequence, KV head)
    counters than that decode did: the ragged step must still match the
    oracle, i.e. partials of one launch never land where another counts."""
    from pkh_util import DeviceKV, decode_host, normal
    lib = pk.load()
    try:
        lib.pkh_tune_decode_chunk(64)
        H, HK, D, pos = 4, 1, 128, 4000
        kv = DeviceKV(1, HK, D, pos + 1)
        rope = DeviceRope(D, 5e5, pos + 1)
        try:
            kc, vc = normal(61, (pos + 1, HK, D)), normal(62, (pos + 1, HK, D))
            kv.write(0, 0, 0, kc[:pos])
            kv.write(1, 0, 0, vc[:pos])
            q, k, v = normal(63, (H, D)), normal(64, (HK, D)), normal(65, (HK, D))
            ao = decode_host(kv, rope, 0, pos, q, k, v)
            ref, _, _ = po.decode_step(kc, vc, pos, q, k, v, rope.sin, rope.cos, 16)
            assert maxerr(ao, ref) <= TOL_F32
        finally:
            kv.free()
            rope.free()
        _check(32, 8, 128, [900, 3000, 1500, 64, 2200, 700, 4000, 10] * 2, 5e5, 66)
    finally:
        lib.pkh_tune_decode_chunk(0)


def test_ragged_graph_replay_after_scratch_growth():
    """A HIP graph of one ragged step over two layers, captured after a warm-up
    step, stays valid after a later call outgrows the split-K scratch and
    flags; every replay, with eager calls between, matches the eager step
    bit for bit, and the eager step matches the oracle."""
    import torch
    from pkh_util import DeviceKV, decode_host, normal
    lib = pk.load()
    dev = torch.device("cuda")
    H, HK, D = 32, 8, 128
    ctx = [700, 2600, 40, 1500]
    case = Case(H, HK, D, ctx, 5e5, 71, pk.PKH_KV_F32, n_layers=2, layer=1)
    plan = Plan(case.kvb, ctx, H)
    big_kv = big_rope = None
    try:
        n = len(ctx)
        q = [torch.from_numpy(normal(72 + l, (n, H, D))).to(dev) for l in range(2)]
        k = [torch.from_numpy(normal(74 + l, (n, HK, D))).to(dev) for l in range(2)]
        v = [torch.from_numpy(normal(76 + l, (n, HK, D))).to(dev) for l in range(2)]
        out = [torch.zeros((n, H, D), dtype=torch.float32, device=dev) for _ in range(2)]

        def step():
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for l in range(2):
                rc = lib.pkh_attn_decode_batch_async(case.kvb.ref, case.rope.ref, plan.ptr, l,
                                                     q[l].data_ptr(), k[l].data_ptr(),
                                                     v[l].data_ptr(), out[l].data_ptr(), s)
                assert rc == 0, rc

        step()
        torch.cuda.synchronize()
        eager = [o.clone() for o in out]
        for s_, p in enumerate(ctx):
            kc, vc = case.k_rows[s_].copy(), case.v_rows[s_].copy()
            ref, _, _ = po.decode_step(kc, vc, p, q[1][s_].cpu().numpy(), k[1][s_].cpu().numpy(),
                                       v[1][s_].cpu().numpy(), case.rope.sin, case.rope.cos, 16)
            assert maxerr(eager[1][s_].cpu().numpy(), ref) <= TOL_F32, s_
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                step()
        torch.cuda.synchronize()
        # A decode split into 5001 chunks per KV head (82 MB of partials)
        # outgrows every buffer the earlier calls of this process sized.
        big_pos = 80000
        big_kv = DeviceKV(1, HK, D, big_pos + 1)
        big_rope = DeviceRope(D, 5e5, big_pos + 1)
        prev = lib.pkh_tune_decode_chunk(16)
        try:
            big = decode_host(big_kv, big_rope, 0, big_pos, normal(78, (H, D)),
                              normal(79, (HK, D)), normal(80, (HK, D)))
        finally:
            lib.pkh_tune_decode_chunk(prev)
        assert np.isfinite(big).all()
        for it in range(3):
            for o in out:
                o.zero_()
            graph.replay()
            torch.cuda.synchronize()
            for l in range(2):
                assert torch.equal(out[l], eager[l]), f"replay {it} layer {l}"
            for o in out:
                o.zero_()
            step()
            torch.cuda.synchronize()
            for l in range(2):
                assert torch.equal(out[l], eager[l]), f"eager step {it} layer {l}"
        log("3 graph replays of a 2-layer ragged step after growth match the eager step")
    finally:
        plan.free()
        case.free()
        if big_kv is not None:
            big_kv.free()
        if big_rope is not None:
            big_rope.free()


def test_ragged_300_short_sequences():
    """300 sequences with contexts drawn from U[0, 2000] (numpy
    default_rng(12)), fp16 cache: thousands of work items whose sequence the
    kernel finds by binary search over the plan's chunk starts, one-row
    sequences among them."""
    ctx = np.random.default_rng(12).integers(0, 2000, size=300, endpoint=True).tolist()
    ctx[:3] = [0, 1, 2000]
    _check(8, 2, 64, ctx, 1e4, 12, pk.PKH_KV_F16)
