"""GPU runs of the reference-side binding (lestramanika_amd/host/pickle_seam.c)
driven through the reference's own structs.

The compiled reference (oracle/_ref/libpickle_ref.so) loads a one-layer
probe model and builds its real pickle_fast_state_t and pickle_arch_t; the
binding (oracle/_ref/libpickle_seam.so, the seam file compiled against the
reference's headers) allocates the device cache from them, extends nothing
itself but uploads the state's own RoPE rows, and runs the attention block
on the state's q/k/v work buffers, writing state->ao.  The results must
equal the reference's own outputs on its golden probes (max-abs 1e-4 for
ao, appended rows bit for bit), and a prefill through the binding must match
the oracle's token loop (2e-3, fp16 operands).
"""
import ctypes
import glob
import os

import numpy as np
import pytest

import lestramanika_amd as pk
from oracle import gguf, pyoracle as po, pyref
from pkh_util import log, maxerr

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
SEAM = os.path.join(ROOT, "oracle", "_ref", "libpickle_seam.so")
PROBES = sorted(glob.glob(os.path.join(GOLDEN, "attn_probe_*.npz")))


class PicklePkh(ctypes.Structure):
    """pickle_pkh_t: the device cache and RoPE table of the binding."""
    _fields_ = [("kv", pk.KV), ("rope", pk.Rope)]


def _seam():
    if not (os.path.exists(SEAM) and pyref.available()):
        pytest.skip("the binding and the compiled reference are built only where the reference tree is")
    pk.load()                       # libpkh.so in this process first
    s = ctypes.CDLL(SEAM)
    P = ctypes.c_void_p
    for name, res, args in [("pickle_pkh_alloc", ctypes.c_int, [P, P, P]),
                            ("pickle_pkh_free", None, [P]),
                            ("pickle_pkh_attention", ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_size_t]),
                            ("pickle_pkh_prefill", ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_size_t,
                                                                  ctypes.c_size_t, P, P, P, P])]:
        fn = getattr(s, name)
        fn.restype, fn.argtypes = res, args
    return s


@pytest.mark.parametrize("path", PROBES, ids=[os.path.basename(p)[11:-4] for p in PROBES])
def test_binding_decode_through_reference_state(path, tmp_path):
    seam = _seam()
    lib = pk.load()
    z = np.load(path)
    H, HK, D, pos = (int(x) for x in z["shape"])
    theta = float(z["theta"])
    log(f"binding decode, probe {os.path.basename(path)}")
    model = str(tmp_path / "probe.gguf")
    gguf.write_probe(model, n_heads=H, n_kv_heads=HK, head_dim=D, theta=theta, ctx=pos + 4, seed=0)
    R = pyref.lib()
    with pyref.RefModel(model) as m:
        state, arch = R.ref_state_ptr(m.h), R.ref_arch_ptr(m.h)
        p = PicklePkh()
        assert seam.pickle_pkh_alloc(arch, state, ctypes.byref(p)) == pk.PKH_OK
        try:
            m.rope_rows("sin", 0, pos + 1)           # the reference extends its own tables
            if pos:
                for which, rows in ((0, z["cache_k"]), (1, z["cache_v"])):
                    rows = np.ascontiguousarray(rows, np.float32)
                    pk.check(lib.pkh_kv_copy_rows(ctypes.byref(p.kv), which, 0, 0, pos,
                                                  rows.ctypes.data, 1), "pkh_kv_copy_rows")
            for which, a in ((pyref.Q, z["q"]), (pyref.K, z["k"]), (pyref.V, z["v"])):
                a = np.ascontiguousarray(a, np.float32)
                assert R.ref_write_state(m.h, which, a.ctypes.data, a.size) == 0
            assert seam.pickle_pkh_attention(state, ctypes.byref(p), 0, pos) == pk.PKH_OK
            err = maxerr(m.state(pyref.AO).reshape(H, D), z["ao"])
            log(f"  state->ao max-abs err vs the reference {err:.3e}")
            assert err <= 1e-4
            for which, want in ((0, z["row_k"]), (1, z["row_v"])):
                row = np.zeros((1, HK, D), np.float32)
                pk.check(lib.pkh_kv_copy_rows(ctypes.byref(p.kv), which, 0, pos, 1,
                                              row.ctypes.data, 0), "pkh_kv_copy_rows")
                assert np.array_equal(row[0], want)
            # pos past the cache: PICKLE_ERR_RANGE before any device work
            assert seam.pickle_pkh_attention(state, ctypes.byref(p), 0, pos + 4) == pk.PKH_ERR_RANGE
        finally:
            seam.pickle_pkh_free(ctypes.byref(p))


def test_binding_prefill_through_reference_state(tmp_path):
    seam = _seam()
    H, HK, D, pos0, n, theta = 8, 2, 64, 30, 97, 1e4
    model = str(tmp_path / "probe.gguf")
    gguf.write_probe(model, n_heads=H, n_kv_heads=HK, head_dim=D, theta=theta, ctx=pos0 + n, seed=0)
    rng = np.random.default_rng(17)
    ctx_k = rng.standard_normal((pos0, HK, D), dtype=np.float32)
    ctx_v = rng.standard_normal((pos0, HK, D), dtype=np.float32)
    q = rng.standard_normal((n, H, D), dtype=np.float32)
    k = rng.standard_normal((n, HK, D), dtype=np.float32)
    v = rng.standard_normal((n, HK, D), dtype=np.float32)
    lib = pk.load()
    R = pyref.lib()
    with pyref.RefModel(model) as m:
        state, arch = R.ref_state_ptr(m.h), R.ref_arch_ptr(m.h)
        p = PicklePkh()
        assert seam.pickle_pkh_alloc(arch, state, ctypes.byref(p)) == pk.PKH_OK
        try:
            for which, rows in ((0, ctx_k), (1, ctx_v)):
                pk.check(lib.pkh_kv_copy_rows(ctypes.byref(p.kv), which, 0, 0, pos0,
                                              rows.ctypes.data, 1), "pkh_kv_copy_rows")
            ao = np.zeros_like(q)
            assert seam.pickle_pkh_prefill(state, ctypes.byref(p), 0, pos0, n, q.ctypes.data,
                                           k.ctypes.data, v.ctypes.data, ao.ctypes.data) == pk.PKH_OK
            sin = m.rope_rows("sin", 0, pos0 + n)
            cos = m.rope_rows("cos", 0, pos0 + n)
        finally:
            seam.pickle_pkh_free(ctypes.byref(p))
    kc = np.zeros((pos0 + n, HK, D), np.float32)
    vc = np.zeros_like(kc)
    kc[:pos0], vc[:pos0] = ctx_k, ctx_v
    ref = po.prefill(kc, vc, pos0, q, k, v, sin, cos, 16)
    err = maxerr(ao, ref)
    log(f"binding prefill H{H} HK{HK} D{D} pos0 {pos0} n {n}: max-abs err {err:.3e}")
    assert err <= 2e-3
