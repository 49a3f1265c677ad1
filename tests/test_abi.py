"""CPU checks of the C ABI library (lestramanika_amd/libpkh.so).

No kernel runs here: the library is loaded, its exports are checked against
include/pkh_attn.h, its host-only helpers are compared with the oracle, and
every argument check that returns before touching the device is exercised.
"""
import ctypes
import hashlib
import json
import os
import re

import numpy as np
import pytest

import lestramanika_amd as pk
from oracle import pyoracle as po

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pkh_attn.h")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pkh_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = pk.load()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(pk._SIGS), "bindings and header disagree"
    assert b"gfx950" in lib.pkh_version()


def test_oracle_library_exports():
    lib = po.lib()
    for name in ["pko_rope_inv_freq", "pko_rope_fill", "pko_rope_apply", "pko_attend_f32",
                 "pko_decode_step_f32", "pko_decode_step_f16", "pko_prefill_f32"]:
        assert hasattr(lib, name)


def test_host_rope_tables_match_oracle_and_reference():
    lib = pk.load()
    tabs = json.load(open(os.path.join(GOLDEN, "rope_tables.json")))
    for key, t in tabs.items():
        D, theta, n = t["head_dim"], t["theta"], t["n_pos"]
        half = min(D // 2, 64)
        inv = np.zeros(half, np.float32)
        sin = np.zeros((n, half), np.float32)
        cos = np.zeros((n, half), np.float32)
        lib.pkh_rope_host_tables(D, theta, 0, n - 1, inv.ctypes.data, sin.ctypes.data,
                                 cos.ctypes.data)
        assert hashlib.sha256(inv.tobytes()).hexdigest() == t["inv_freq"], key
        assert hashlib.sha256(sin.tobytes()).hexdigest() == t["sin"], key
        assert hashlib.sha256(cos.tobytes()).hexdigest() == t["cos"], key
        oi, os_, oc = po.rope_tables(D, theta, min(n, 64))
        assert np.array_equal(inv, oi) and np.array_equal(sin[:64], os_)


def _fake_kv(n_layers=2, HK=2, D=64, max_seq=16, dtype=pk.PKH_KV_F32):
    kv = pk.KV()
    kv.n_layers, kv.n_kv_heads, kv.head_dim, kv.max_seq = n_layers, HK, D, max_seq
    kv.k_stride_layer = kv.v_stride_layer = max_seq * HK * D
    kv.k = kv.v = 0x1000      # never dereferenced: every call below fails its checks first
    kv.dtype = dtype
    kv.stride_pos, kv.stride_head = HK * D, D
    return kv


def _fake_rope(max_seq=16, half=32, filled=16):
    r = pk.Rope()
    r.max_seq, r.half, r.filled_upto = max_seq, half, filled
    r.sin = r.cos = 0x2000
    return r


def test_argument_checks_return_before_device_work():
    lib = pk.load()
    kv, rope = _fake_kv(), _fake_rope()
    dummy = ctypes.c_void_p(0x3000)
    dec = lambda kv_, rope_, layer, pos, H: lib.pkh_attn_decode(
        ctypes.byref(kv_) if kv_ is not None else None,
        ctypes.byref(rope_) if rope_ is not None else None, layer, pos, H,
        dummy, dummy, dummy, dummy)
    assert dec(None, rope, 0, 0, 4) == pk.PKH_ERR_ARG
    assert dec(kv, None, 0, 0, 4) == pk.PKH_ERR_ARG
    assert dec(kv, rope, 2, 0, 4) == pk.PKH_ERR_RANGE        # layer
    assert dec(kv, rope, -1, 0, 4) == pk.PKH_ERR_RANGE
    assert dec(kv, rope, 0, 16, 4) == pk.PKH_ERR_RANGE       # pos >= max_seq
    assert dec(kv, rope, 0, -1, 4) == pk.PKH_ERR_RANGE
    assert dec(kv, _fake_rope(filled=5), 0, 5, 4) == pk.PKH_ERR_RANGE   # table not uploaded
    assert dec(kv, rope, 0, 0, 0) == pk.PKH_ERR_ARG          # no query heads
    assert dec(kv, rope, 0, 0, -4) == pk.PKH_ERR_ARG
    assert dec(kv, _fake_rope(half=16), 0, 0, 4) == pk.PKH_ERR_ARG      # table of another D
    assert dec(_fake_kv(D=24), _fake_rope(half=16), 0, 0, 4) == pk.PKH_ERR_ARG
    assert dec(_fake_kv(D=264), _fake_rope(half=64), 0, 0, 4) == pk.PKH_ERR_ARG  # head_dim > 256
    assert dec(_fake_kv(HK=0), rope, 0, 0, 4) == pk.PKH_ERR_ARG
    bad = _fake_kv()
    bad.stride_pos = 3                                        # strides that cannot hold a row
    assert dec(bad, rope, 0, 0, 4) == pk.PKH_ERR_ARG
    assert lib.pkh_attn_decode_async(ctypes.byref(kv), ctypes.byref(rope), 0, 0, 4,
                                     None, dummy, dummy, dummy, None) == pk.PKH_ERR_ARG
    pf = lambda pos0, n: lib.pkh_attn_prefill(ctypes.byref(kv), ctypes.byref(rope), 0, pos0, n,
                                              4, dummy, dummy, dummy, dummy)
    assert pf(0, 0) in (pk.PKH_ERR_ARG,)
    assert pf(10, 7) in (pk.PKH_ERR_RANGE, pk.PKH_ERR_ARG)
    # row copies: a range whose end overflows int is still out of range
    cp = lambda pos0, n: lib.pkh_kv_copy_rows(ctypes.byref(kv), 0, 0, pos0, n, dummy, 0)
    assert cp(2**31 - 8, 16) == pk.PKH_ERR_RANGE
    assert cp(10, 7) == pk.PKH_ERR_RANGE
    assert cp(0, -1) == pk.PKH_ERR_ARG
    k = pk.KV()
    assert lib.pkh_kv_alloc(0, 2, 64, 16, 0, ctypes.byref(k)) == pk.PKH_ERR_ARG
    assert lib.pkh_kv_alloc(1, 2, 64, 16, 7, ctypes.byref(k)) == pk.PKH_ERR_ARG
    assert lib.pkh_kv_alloc(1, 2, 64, 16, 0, None) == pk.PKH_ERR_ARG
    r = pk.Rope()
    assert lib.pkh_rope_alloc(16, 65, ctypes.byref(r)) == pk.PKH_ERR_ARG
    assert lib.pkh_rope_alloc(16, -1, ctypes.byref(r)) == pk.PKH_ERR_ARG
    assert lib.pkh_rope_alloc(0, 8, ctypes.byref(r)) == pk.PKH_ERR_ARG
    b = pk.KVBatch()
    ms = (ctypes.c_int * 2)(16, 0)
    assert lib.pkh_kv_batch_alloc(1, 2, 64, 2, ms, 0, ctypes.byref(b)) == pk.PKH_ERR_ARG
    plan = ctypes.c_void_p()
    assert lib.pkh_plan_create(None, None, 4, ctypes.byref(plan)) == pk.PKH_ERR_ARG
    # freeing zeroed structs is a no-op, as for the reference's *_free
    lib.pkh_kv_free(ctypes.byref(pk.KV()))
    lib.pkh_rope_free(ctypes.byref(pk.Rope()))
    lib.pkh_kv_batch_free(ctypes.byref(pk.KVBatch()))
    lib.pkh_plan_free(None)


def test_tuning_hook_round_trips():
    lib = pk.load()
    prev = lib.pkh_tune_decode_chunk(512)
    assert lib.pkh_tune_decode_chunk(prev) == 512


def test_size_limits_return_before_device_work():
    """Calls past the 32-bit addressing limits return PKH_ERR_ARG before any
    allocation or launch (the fake pointers are never dereferenced)."""
    lib = pk.load()
    dummy = ctypes.c_void_p(0x3000)
    # Decode: (attended rows + 1) * stride_pos * 4 bytes must stay below
    # 2 GiB -- 2,097,150 positions of an fp32 head_dim 128 cache.
    big = 2_200_000
    kv = _fake_kv(n_layers=1, HK=8, D=128, max_seq=big + 1)
    kv.stride_pos, kv.stride_head = 2 * 128, (big + 1) * 2 * 128
    rope = _fake_rope(max_seq=big + 1, half=64, filled=big + 1)
    dec = lambda pos: lib.pkh_attn_decode_async(ctypes.byref(kv), ctypes.byref(rope), 0, pos, 32,
                                                dummy, dummy, dummy, dummy, None)
    assert dec(2_097_151) == pk.PKH_ERR_ARG
    assert dec(big) == pk.PKH_ERR_ARG
    # Prefill: 2,097,088 positions at most for head_dim 128 (launch grid),
    # 1,945,184 for head_dim 256 (32-bit tile offsets).
    pf = lambda kv_, rope_, H, n: lib.pkh_attn_prefill_async(
        ctypes.byref(kv_), ctypes.byref(rope_), 0, 0, n, H, dummy, dummy, dummy, dummy, None)
    assert pf(kv, rope, 32, 2_097_089) == pk.PKH_ERR_ARG
    kv256 = _fake_kv(n_layers=1, HK=2, D=256, max_seq=big + 1)
    kv256.stride_pos, kv256.stride_head = 2 * 256, (big + 1) * 2 * 256
    assert pf(kv256, rope, 8, 1_945_185) == pk.PKH_ERR_ARG


def test_header_builds_and_links_from_c99(tmp_path):
    """pkh_attn.h is plain C: a C99 host compiles against it with warnings as
    errors, links -lpkh and runs the entry points that need no GPU."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lib_dir = os.path.dirname(pk.LIB_PATH)
    exe = str(tmp_path / "c_abi_host")
    subprocess.run([cc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "c_abi_host.c"), "-o", exe, "-L", lib_dir,
                    f"-Wl,-rpath,{lib_dir}", "-lpkh", "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert "c host ok" in r.stdout


def test_seam_binding_compiles_against_the_reference_headers(tmp_path):
    """lestramanika_amd/host/pickle_seam.c -- the binding a pickle maintainer
    adds -- compiles as C11 with warnings as errors against the reference's
    own src/pickle.h and src/pickle_fast.h (its static asserts check that
    pkh_kv_t mirrors pickle_fast_kv_t field by field and that the status
    codes agree), and links against libpkh.so and the compiled reference
    with no undefined symbol.  Needs the reference tree, which only this
    build container has."""
    import shutil
    import subprocess
    from oracle import pyref
    src = "/root/reference/src"
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc or not os.path.isdir(src) or not pyref.available():
        pytest.skip("reference tree or compiled reference not present")
    out = tmp_path / "libseam.so"
    cmd = [cc, "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-fPIC", "-shared",
           "-Wl,--no-undefined", f"-I{src}", f"-I{os.path.join(ROOT, 'include')}",
           "-o", str(out), os.path.join(ROOT, "lestramanika_amd", "host", "pickle_seam.c"),
           f"-L{os.path.join(ROOT, 'lestramanika_amd')}", "-lpkh",
           f"-L{os.path.dirname(pyref.REF_LIB_PATH)}", "-lpickle_ref"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
