"""CPU checks of the oracle (oracle/pk_oracle.c), against which the GPU path is checked.

What pins it:
  * the reference's own outputs (tests/golden/, written by make_golden.py from
    the compiled reference): bit-exact for RoPE, the cache append and, for
    head_dim % 16 == 0, the attention output;
  * the compiled reference itself when oracle/_ref is built (this container);
  * a float64 textbook attention on small random shapes;
  * closed forms and invariants that a dropped term, a wrong sign or index or
    a transposed operand would break;
  * numpy's IEEE binary16 conversion for the fp16 helpers.
"""
import glob
import hashlib
import json
import os
import re

import numpy as np
import pytest

from oracle import pyoracle as po
from oracle import pyref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PROBES = sorted(glob.glob(os.path.join(GOLDEN, "attn_probe_*.npz")))


def _probe_inputs(z):
    H, HK, D, pos = (int(x) for x in z["shape"])
    theta = float(z["theta"])
    _, sin, cos = po.rope_tables(D, theta, pos + 1)
    kc = np.zeros((pos + 1, HK, D), np.float32)
    vc = np.zeros_like(kc)
    kc[:pos] = z["cache_k"]
    vc[:pos] = z["cache_v"]
    return H, HK, D, pos, theta, sin, cos, kc, vc


@pytest.mark.parametrize("path", PROBES, ids=[os.path.basename(p)[11:-4] for p in PROBES])
def test_oracle_matches_reference_probe(path):
    z = np.load(path)
    H, HK, D, pos, theta, sin, cos, kc, vc = _probe_inputs(z)
    ao, qr, kr = po.decode_step(kc, vc, pos, z["q"], z["k"], z["v"], sin, cos)
    assert np.array_equal(qr, z["q_rot"])
    assert np.array_equal(kr, z["k_rot"])
    assert np.array_equal(kc[pos], z["row_k"])
    assert np.array_equal(vc[pos], z["row_v"])
    if D % 16 == 0:
        # the reference's AVX-512 score/PV loops, restated in the same order
        assert np.array_equal(ao, z["ao"])
    else:
        # the reference's scalar loop reduces in a compiler-chosen order
        np.testing.assert_allclose(ao, z["ao"], rtol=0, atol=1e-6)


def test_golden_probes_are_sensitive():
    """Mistakes planted in the oracle's inputs are caught by the goldens."""
    z = np.load(os.path.join(GOLDEN, "attn_probe_h4k1d128_p200.npz"))
    H, HK, D, pos, theta, sin, cos, kc, vc = _probe_inputs(z)
    ref = z["ao"]

    def run(q=None, sn=sin, cs=cos, k_cache=kc):
        kk, vv = k_cache.copy(), vc.copy()
        ao, _, _ = po.decode_step(kk, vv, pos, z["q"] if q is None else q, z["k"], z["v"], sn, cs)
        return float(np.max(np.abs(ao - ref)))

    assert run() == 0.0
    assert run(sn=-sin) > 1e-3                       # rotation sign
    assert run(q=z["q"][::-1].copy()) > 1e-3         # query/head order
    assert run(q=z["q"] * 2.0) > 1e-3                # softmax scale
    shifted = np.roll(kc, 1, axis=0)
    assert run(k_cache=shifted) > 1e-3               # position index


def test_rope_tables_match_reference_digests():
    tabs = json.load(open(os.path.join(GOLDEN, "rope_tables.json")))
    for key, t in tabs.items():
        inv, sin, cos = po.rope_tables(t["head_dim"], t["theta"], t["n_pos"])
        assert hashlib.sha256(inv.tobytes()).hexdigest() == t["inv_freq"], key
        assert hashlib.sha256(sin.tobytes()).hexdigest() == t["sin"], key
        assert hashlib.sha256(cos.tobytes()).hexdigest() == t["cos"], key


def test_rope_inv_freq_closed_form():
    for D, theta in [(16, 1e4), (64, 1e4), (128, 5e5), (256, 1e4)]:
        inv, _, _ = po.rope_tables(D, theta, 1)
        half = min(D // 2, 64)
        exact = theta ** (-(2.0 * np.arange(half)) / D)
        np.testing.assert_allclose(inv, exact, rtol=2e-6)


def test_rope_invariants():
    rng = np.random.default_rng(7)
    D, theta = 64, 1e4
    _, sin, cos = po.rope_tables(D, theta, 300)
    x = rng.standard_normal((3, D)).astype(np.float32)
    # position 0 is the identity
    assert np.array_equal(po.rope_apply(x, D, sin[0], cos[0]), x)
    # pair norms are preserved
    y = po.rope_apply(x, D, sin[257], cos[257])
    h = D // 2
    np.testing.assert_allclose(x[:, :h] ** 2 + x[:, h:] ** 2, y[:, :h] ** 2 + y[:, h:] ** 2,
                               rtol=1e-5, atol=1e-6)
    # <R_m q, R_n k> depends only on m - n
    q, k = x[0], x[1]
    d1 = float(np.dot(po.rope_apply(q, D, sin[100], cos[100]).astype(np.float64),
                      po.rope_apply(k, D, sin[90], cos[90]).astype(np.float64)))
    d2 = float(np.dot(po.rope_apply(q, D, sin[210], cos[210]).astype(np.float64),
                      po.rope_apply(k, D, sin[200], cos[200]).astype(np.float64)))
    assert abs(d1 - d2) < 1e-4
    # head_dim 256 rotates only the first 128 elements (half capped at 64)
    D2 = 256
    _, s2, c2 = po.rope_tables(D2, theta, 10)
    z = rng.standard_normal((1, D2)).astype(np.float32)
    r = po.rope_apply(z, D2, s2[9], c2[9])
    assert np.array_equal(r[:, 128:], z[:, 128:])
    assert not np.array_equal(r[:, :128], z[:, :128])


def _attend_f64(kc, vc, q_rot, H, n):
    _, HK, D = kc.shape
    out = np.zeros((H, D))
    for h in range(H):
        g = h * HK // H
        s = kc[:n, g].astype(np.float64) @ q_rot[h].astype(np.float64) / np.sqrt(D)
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h] = w @ vc[:n, g].astype(np.float64)
    return out


@pytest.mark.parametrize("H,HK,D,n", [(4, 2, 16, 1), (4, 2, 16, 37), (8, 1, 64, 300),
                                      (4, 4, 32, 129), (6, 4, 16, 50), (2, 1, 256, 70),
                                      (4, 2, 24, 33), (32, 8, 128, 520)])
def test_attend_vs_float64(H, HK, D, n):
    rng = np.random.default_rng(H * 1000 + D + n)
    kc = rng.standard_normal((n, HK, D)).astype(np.float32)
    vc = rng.standard_normal((n, HK, D)).astype(np.float32)
    q = rng.standard_normal((H, D)).astype(np.float32)
    ao = po.attend(kc, vc, q, H, n, n_threads=4)
    np.testing.assert_allclose(ao, _attend_f64(kc, vc, q, H, n), rtol=0, atol=2e-6)


def test_attend_special_cases():
    rng = np.random.default_rng(3)
    H, HK, D = 8, 2, 64
    v = rng.standard_normal((40, HK, D)).astype(np.float32)
    k = rng.standard_normal((40, HK, D)).astype(np.float32)
    q = rng.standard_normal((H, D)).astype(np.float32)
    # one row: o = v0 exactly
    ao = po.attend(k, v, q, H, 1)
    for h in range(H):
        assert np.array_equal(ao[h], v[0, h * HK // H])
    # identical keys: uniform weights -> mean of V
    kk = np.repeat(k[:1], 40, axis=0)
    ao = po.attend(kk, v, q, H, 40)
    for h in range(H):
        np.testing.assert_allclose(ao[h], v[:, h * HK // H].astype(np.float64).mean(0), atol=1e-6)
    # q = 0: uniform weights as well
    ao = po.attend(k, v, np.zeros_like(q), H, 40)
    for h in range(H):
        np.testing.assert_allclose(ao[h], v[:, h * HK // H].astype(np.float64).mean(0), atol=1e-6)
    # heads of one group with equal queries give equal outputs
    q2 = q.copy()
    q2[1] = q2[0]
    ao = po.attend(k, v, q2, H, 40)
    assert np.array_equal(ao[0], ao[1])
    # the thread count does not change the result
    assert np.array_equal(po.attend(k, v, q, H, 40, 1), po.attend(k, v, q, H, 40, 7))
    # the kv == NULL path returns v of the head's group
    st = po.attend_stateless(v[0], H)
    for h in range(H):
        assert np.array_equal(st[h], v[0, h * HK // H])


def test_prefill_is_the_token_loop():
    rng = np.random.default_rng(4)
    H, HK, D, n, pos0 = 4, 2, 32, 20, 5
    _, sin, cos = po.rope_tables(D, 1e4, pos0 + n)
    kc = np.zeros((pos0 + n, HK, D), np.float32)
    vc = np.zeros_like(kc)
    kc[:pos0] = rng.standard_normal((pos0, HK, D))
    vc[:pos0] = rng.standard_normal((pos0, HK, D))
    q = rng.standard_normal((n, H, D)).astype(np.float32)
    k = rng.standard_normal((n, HK, D)).astype(np.float32)
    v = rng.standard_normal((n, HK, D)).astype(np.float32)
    k1, v1 = kc.copy(), vc.copy()
    ao = po.prefill(k1, v1, pos0, q, k, v, sin, cos)
    k2, v2 = kc.copy(), vc.copy()
    for i in range(n):
        a, _, _ = po.decode_step(k2, v2, pos0 + i, q[i], k[i], v[i], sin, cos)
        assert np.array_equal(a, ao[i])
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


def test_f16_conversion_matches_ieee():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = po.f16_bits_to_f32(bits)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    rng = np.random.default_rng(5)
    xs = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),      # subnormal range
        (rng.standard_normal(50000) * 7e4).astype(np.float32),       # overflow range
        ref[fin],                                                   # exact values
        (ref[fin][:-1] + np.diff(ref[fin]) / 2).astype(np.float32),  # ties
        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 65519.996, 5.96e-8,
                  2.98e-8, 2.9802322e-08, 1e-9], np.float32),
    ])
    xs = xs[np.isfinite(xs.astype(np.float64))]
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(po.f32_to_f16_bits(xs), want)


def test_decode_f16_is_f32_on_widened_cache():
    rng = np.random.default_rng(6)
    H, HK, D, pos = 8, 2, 128, 77
    _, sin, cos = po.rope_tables(D, 5e5, pos + 1)
    kh = po.f32_to_f16_bits(rng.standard_normal((pos + 1, HK, D)))
    vh = po.f32_to_f16_bits(rng.standard_normal((pos + 1, HK, D)))
    q = rng.standard_normal((H, D)).astype(np.float32)
    k = rng.standard_normal((HK, D)).astype(np.float32)
    v = rng.standard_normal((HK, D)).astype(np.float32)
    kf, vf = po.f16_bits_to_f32(kh), po.f16_bits_to_f32(vh)
    ao16 = po.decode_step_f16(kh, vh, pos, q, k, v, sin, cos)
    _, qr, kr = po.decode_step(kf, vf, pos, q, k, v, sin, cos)
    assert np.array_equal(kh[pos], po.f32_to_f16_bits(kr))
    assert np.array_equal(vh[pos], po.f32_to_f16_bits(v))
    kf[pos] = po.f16_bits_to_f32(kh[pos])
    vf[pos] = po.f16_bits_to_f32(vh[pos])
    assert np.array_equal(ao16, po.attend(kf, vf, qr, H, pos + 1))


# ---- against the compiled reference (this container only) -----------------

needs_ref = pytest.mark.skipif(not pyref.available(), reason="oracle/_ref not built")


@needs_ref
def test_reference_selftest_still_passes():
    assert pyref.selftest() == (0, 5)


@needs_ref
@pytest.mark.parametrize("H,HK,D,theta,pos", [(8, 2, 64, 1e4, 700), (4, 2, 128, 5e5, 1500),
                                               (4, 4, 16, 1e4, 3)])
def test_oracle_matches_live_reference(tmp_path, H, HK, D, theta, pos):
    from oracle import gguf
    path = str(tmp_path / "probe.gguf")
    gguf.write_probe(path, n_heads=H, n_kv_heads=HK, head_dim=D, theta=theta, ctx=pos + 4,
                     seed=pos)
    rng = np.random.default_rng(pos)
    kc = np.zeros((pos + 1, HK, D), np.float32)
    vc = np.zeros_like(kc)
    kc[:pos] = rng.standard_normal((pos, HK, D))
    vc[:pos] = rng.standard_normal((pos, HK, D))
    with pyref.RefModel(path) as m:
        m.kv_write(0, 0, 0, kc[:pos])
        m.kv_write(1, 0, 0, vc[:pos])
        m.pos = pos
        m.forward1(1)
        xn = m.state(pyref.XN)
        ref_ao = m.state(pyref.AO).reshape(H, D)
        inv_ref = m.rope_inv_freq()
        sin_ref = m.rope_rows("sin", 0, pos + 1)
        cos_ref = m.rope_rows("cos", 0, pos + 1)
    inv, sin, cos = po.rope_tables(D, theta, pos + 1)
    assert np.array_equal(inv, inv_ref)
    assert np.array_equal(sin, sin_ref) and np.array_equal(cos, cos_ref)
    q = xn[:H * D].reshape(H, D)
    k = xn[H * D:H * D + HK * D].reshape(HK, D)
    v = xn[H * D + HK * D:].reshape(HK, D)
    ao, _, _ = po.decode_step(kc, vc, pos, q, k, v, sin, cos, n_threads=4)
    assert np.array_equal(ao, ref_ao)


@needs_ref
def test_reference_range_errors(tmp_path):
    """pos >= max_seq and token >= vocab are PICKLE_ERR_RANGE in the reference
    (src/pickle_fast.c:1883-1885); the GPU entry points keep the pos check."""
    from oracle import gguf
    path = str(tmp_path / "probe.gguf")
    gguf.write_probe(path, n_heads=2, n_kv_heads=1, head_dim=16, theta=1e4, ctx=4, seed=0)
    with pyref.RefModel(path) as m:
        m.pos = 4
        assert m.forward1_rc(1) == -7
        m.pos = 0
        assert m.forward1_rc(8) == -7


def _run_all_builds(fn):
    """fn() under each oracle build; returns the results by build."""
    out = {}
    for build in ("plain", "avx512"):
        prev = po.use_build(build)
        try:
            out[build] = fn()
        finally:
            po.use_build(prev)
    return out


@pytest.mark.parametrize("path", PROBES, ids=[os.path.basename(p)[11:-4] for p in PROBES])
def test_avx512_build_is_bit_identical_on_probes(path):
    """The CPU baseline's build of the oracle (-O3, 512-bit vectors) gives the
    -O2 build's results bit for bit on the reference's golden probes."""
    z = np.load(path)
    H, HK, D, pos, theta, sin, cos, kc, vc = _probe_inputs(z)

    def run():
        return po.decode_step(kc.copy(), vc.copy(), pos, z["q"], z["k"], z["v"], sin, cos, 4)[0]

    r = _run_all_builds(run)
    assert np.array_equal(r["plain"], r["avx512"])
    assert np.abs(r["avx512"] - z["ao"]).max() <= 1e-6


@pytest.mark.parametrize("H,HK,D,pos", [(32, 8, 128, 3000), (8, 2, 24, 500), (6, 4, 16, 300),
                                        (4, 2, 80, 900), (7, 3, 96, 257)])
def test_avx512_build_is_bit_identical_on_random_steps(H, HK, D, pos):
    """Decode (fp32 and fp16 caches) and a short prefill, on random inputs
    with the scalar (head_dim % 16 != 0) and 16-lane score loops."""
    rng = np.random.default_rng(H * 1000 + D + pos)
    kc0 = rng.standard_normal((pos + 1, HK, D), dtype=np.float32)
    vc0 = rng.standard_normal((pos + 1, HK, D), dtype=np.float32)
    q = rng.standard_normal((H, D), dtype=np.float32)
    k = rng.standard_normal((HK, D), dtype=np.float32)
    v = rng.standard_normal((HK, D), dtype=np.float32)
    qn = rng.standard_normal((9, H, D), dtype=np.float32)
    kn = rng.standard_normal((9, HK, D), dtype=np.float32)
    vn = rng.standard_normal((9, HK, D), dtype=np.float32)
    _, sin, cos = po.rope_tables(D, 5e5, pos + 10)

    def run():
        a = po.decode_step(kc0.copy(), vc0.copy(), pos, q, k, v, sin, cos, 4)[0]
        b = po.decode_step_f16(po.f32_to_f16_bits(kc0), po.f32_to_f16_bits(vc0), pos, q, k, v,
                               sin, cos, 4)
        kc = np.zeros((pos + 10, HK, D), np.float32)
        vc = np.zeros_like(kc)
        kc[:pos + 1], vc[:pos + 1] = kc0, vc0
        c = po.prefill(kc, vc, pos + 1, qn, kn, vn, sin, cos, 4)
        return a, b, c

    r = _run_all_builds(run)
    for x, y in zip(r["plain"], r["avx512"]):
        assert np.array_equal(x, y)


def test_avx512_build_uses_512_bit_fma():
    """The CPU baseline's build really is vectorised: its code holds 512-bit
    fused multiply-adds, the -O2 build's none."""
    import shutil
    import subprocess
    objdump = shutil.which("objdump")
    if not objdump:
        pytest.skip("no objdump")

    def zmm_fmas(path):
        text = subprocess.run([objdump, "-d", path], capture_output=True, text=True, check=True).stdout
        return len(re.findall(r"vfmadd\w+ps\s+%zmm", text))

    assert zmm_fmas(po.LIB_AVX512_PATH) > 0
    assert zmm_fmas(po.LIB_PATH) == 0
