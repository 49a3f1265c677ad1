"""Write the golden fixtures of tests/golden/ by running the compiled reference.

Run from the repository root after `make -C oracle` (which compiles the
reference's sources in place into oracle/_ref/libpickle_ref.so):

    python tests/golden/make_golden.py

Outputs (all produced by the reference's own pickle_fast_forward and
pickle_fast_state_extend_rope; nothing here is computed by this repository's
code except the synthetic inputs):

  attn_probe_<name>.npz   one decode step of the reference's attention block
                          on a one-layer probe model (q/k/v = slices of the
                          normed input, see gguf.write_probe): the cache rows
                          it attended, pre-RoPE q/k/v, rotated q/k, the
                          appended cache row and the attention output ao.
  tiny_e2e[_unitnorm].npz the tiny Llama (dim 64, 2 layers, H4/HK2/D16, FFN
                          172, vocab 256, theta 1e4, F32 weights N(0, 0.02)
                          seed 0): prompt of 8 ids from default_rng(1), 24
                          greedy tokens, logits and the attention output of
                          every layer for every forward call.
  rope_tables.json        sha256 of the reference's inv_freq and sin/cos
                          rows for the shapes the tests and bench use.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

from oracle import gguf  # noqa: E402
from oracle import pyref  # noqa: E402

# name: (H, HK, D, theta, pos, seed)
PROBES = {
    "h4k2d16_p31": (4, 2, 16, 1e4, 31, 11),
    "h4k2d16_p0": (4, 2, 16, 1e4, 0, 12),
    "h8k1d64_p300": (8, 1, 64, 1e4, 300, 13),
    "h4k1d128_p200": (4, 1, 128, 5e5, 200, 14),
    "h2k2d32_p50": (2, 2, 32, 1e4, 50, 15),
    "h6k4d16_p20": (6, 4, 16, 1e4, 20, 16),       # H % HK != 0: uneven groups
    "h4k2d24_p20": (4, 2, 24, 1e4, 20, 17),       # D % 16 != 0: scalar path
    "h2k1d256_p40": (2, 1, 256, 1e4, 40, 18),     # half capped at 64
}

TABLES = [(16, 1e4, 64), (64, 1e4, 2049), (128, 5e5, 8193), (128, 5e5, 32769),
          (32, 1e4, 512), (256, 1e4, 128), (24, 1e4, 64)]

PROBE_TOKEN = 3


def probe(name, H, HK, D, theta, pos, seed, tmp):
    path = os.path.join(tmp, f"{name}.gguf")
    gguf.write_probe(path, n_heads=H, n_kv_heads=HK, head_dim=D, theta=theta,
                     ctx=pos + 8, seed=seed)
    rng = np.random.default_rng(seed + 1000)
    kc = rng.standard_normal((pos, HK, D)).astype(np.float32)
    vc = rng.standard_normal((pos, HK, D)).astype(np.float32)
    with pyref.RefModel(path) as m:
        assert (m.n_heads, m.n_kv_heads, m.head_dim) == (H, HK, D)
        if pos:
            m.kv_write(0, 0, 0, kc)
            m.kv_write(1, 0, 0, vc)
        m.pos = pos
        m.forward1(PROBE_TOKEN)
        xn = m.state(pyref.XN)
        q = xn[:H * D].reshape(H, D)
        k = xn[H * D:H * D + HK * D].reshape(HK, D)
        v = xn[H * D + HK * D:].reshape(HK, D)
        # The selection projections reproduce slices of xn exactly.
        assert np.array_equal(m.state(pyref.V).reshape(HK, D), v)
        out = dict(
            shape=np.array([H, HK, D, pos], np.int64), theta=np.float32(theta),
            cache_k=kc, cache_v=vc, q=q, k=k, v=v,
            q_rot=m.state(pyref.Q).reshape(H, D), k_rot=m.state(pyref.K).reshape(HK, D),
            row_k=m.kv_read(0, 0, pos, 1)[0], row_v=m.kv_read(1, 0, pos, 1)[0],
            ao=m.state(pyref.AO).reshape(H, D),
        )
    np.savez_compressed(os.path.join(HERE, f"attn_probe_{name}.npz"), **out)


def tiny(tmp, norm_offset, suffix):
    path = os.path.join(tmp, f"tiny{suffix}.gguf")
    w = gguf.write_tiny(path, seed=0, norm_offset=norm_offset)
    c = gguf.TINY
    prompt = np.random.default_rng(1).integers(0, c["vocab"], 8).astype(np.int32)
    n_gen = 24
    feed, gen, logits_all, ao_last = [], [], [], []
    with pyref.RefModel(path) as m:
        logits = None
        for t in prompt:
            logits = m.forward1(int(t))
            feed.append(int(t))
            logits_all.append(logits)
            ao_last.append(m.state(pyref.AO))
        for i in range(n_gen):
            nxt = pyref.argmax(logits)
            gen.append(nxt)
            if i < n_gen - 1:
                logits = m.forward1(nxt)
                feed.append(nxt)
                logits_all.append(logits)
                ao_last.append(m.state(pyref.AO))
    # Layer 0's attention output: the same model truncated to one layer
    # (pickle_arch_t.n_layers), fed the same tokens.
    ao_first = []
    with pyref.RefModel(path, n_layers_override=1) as m1:
        for t in feed:
            m1.forward1(int(t))
            ao_first.append(m1.state(pyref.AO))
    # The same prompt in one pickle_fast_forward call (the reference's prefill)
    # gives the same logits as the token-by-token feed.
    with pyref.RefModel(path) as m2:
        lg = np.zeros(c["vocab"], np.float32)
        rc = pyref.lib().ref_forward_n(m2.h, prompt.ctypes.data, len(prompt), lg.ctypes.data)
        assert rc == 0 and np.array_equal(lg, logits_all[len(prompt) - 1])
    np.savez_compressed(
        os.path.join(HERE, f"tiny_e2e{suffix}.npz"),
        prompt=prompt, generated=np.array(gen, np.int32), fed=np.array(feed, np.int32),
        logits=np.array(logits_all, np.float32),
        ao=np.stack([np.array(ao_first), np.array(ao_last)]).astype(np.float32),
        norm_offset=np.float32(norm_offset), weights_sha256=np.array(gguf.weights_digest(w)))


def tables(tmp):
    out = {}
    for D, theta, n in TABLES:
        path = os.path.join(tmp, f"tab_{D}_{n}.gguf")
        gguf.write_probe(path, n_heads=1, n_kv_heads=1, head_dim=D, theta=theta, ctx=n, seed=0)
        with pyref.RefModel(path) as m:
            inv = m.rope_inv_freq()
            s = m.rope_rows("sin", 0, n)
            c = m.rope_rows("cos", 0, n)
        out[f"{D}_{theta:g}_{n}"] = dict(
            head_dim=D, theta=theta, n_pos=n,
            inv_freq=hashlib.sha256(inv.tobytes()).hexdigest(),
            sin=hashlib.sha256(s.tobytes()).hexdigest(),
            cos=hashlib.sha256(c.tobytes()).hexdigest(),
            sample_rows={str(p): [s[p].tolist(), c[p].tolist()] for p in (0, 1, n // 2, n - 1)},
        )
    with open(os.path.join(HERE, "rope_tables.json"), "w") as f:
        json.dump(out, f, indent=1)


def main():
    if not pyref.available():
        sys.exit("oracle/_ref/libpickle_ref.so not built (make -C oracle)")
    rc, tok = pyref.selftest()
    assert rc == 0 and tok == 5, (rc, tok)     # the reference's own regression gate
    with tempfile.TemporaryDirectory() as tmp:
        for name, args in PROBES.items():
            probe(name, *args, tmp)
        tiny(tmp, 0.0, "")
        tiny(tmp, 1.0, "_unitnorm")
        tables(tmp)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
