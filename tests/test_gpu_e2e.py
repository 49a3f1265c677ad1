"""End-to-end check of the drop-in on the tiny Llama (dim 64, 2 layers,
H4/HK2/D16, FFN 172, vocab 256, theta 1e4, F32 weights N(0, 0.02) from
default_rng(0)): the model's forward pass with its attention block replaced
by the C ABI must reproduce the compiled reference's greedy tokens and
per-layer attention outputs (tests/golden/tiny_e2e*.npz).

Everything outside the attention block -- embedding lookup, RMSNorm, the
Q/K/V/O and FFN projections, SwiGLU, logits -- is a numpy restatement of
pickle_fast_forward (src/pickle_fast.c:1881-2150, pickle_fast_rmsnorm
:114-120) used here as the harness; it calls the library the way a patched
pickle_fast_forward would: one pkh_attn_decode per layer and token in place
of :1910-2094.

Tolerances: per-layer ao max-abs 1e-4 on the decode path; the MFMA prefill
of the prompt (fp16 operands) is held to 2e-3; the greedy tokens must be
identical on both paths.
"""
import os
import sys

import numpy as np
import pytest

import lestramanika_amd as pk
from pkh_util import DeviceKV, DeviceRope, decode_host, log, maxerr, prefill_host

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from oracle import gguf  # noqa: E402

pytestmark = pytest.mark.gpu

EPS = np.float32(1e-5)
FIXTURES = [("tiny_e2e.npz", 0.0), ("tiny_e2e_unitnorm.npz", 1.0)]


def rmsnorm(x, w):
    """src/pickle_fast.c:114-120: x * w * 1/sqrt(mean(x^2) + eps), fp32."""
    x = x.astype(np.float32)
    mean = np.float32(np.sum(x * x, axis=-1, dtype=np.float32, keepdims=True) / np.float32(x.shape[-1]))
    rsq = np.float32(1.0) / np.sqrt(mean + EPS, dtype=np.float32)
    return (x * w * rsq).astype(np.float32)


class TinyModel:
    def __init__(self, norm_offset):
        self.c = gguf.TINY
        self.w = gguf.tiny_weights(0, norm_offset)
        c = self.c
        self.H, self.HK, self.D = c["n_heads"], c["n_kv_heads"], c["head_dim"]
        self.kv = DeviceKV(c["n_layers"], self.HK, self.D, c["ctx"])
        self.rope = DeviceRope(self.D, c["theta"], c["ctx"])

    def free(self):
        self.kv.free()
        self.rope.free()

    def _ffn(self, x, L):
        w = self.w
        xn2 = rmsnorm(x, w[f"blk.{L}.ffn_norm.weight"])
        gate = xn2 @ w[f"blk.{L}.ffn_gate.weight"].T
        up = xn2 @ w[f"blk.{L}.ffn_up.weight"].T
        act = gate * (np.float32(1.0) / (np.float32(1.0) + np.exp(-gate))) * up
        return x + act.astype(np.float32) @ w[f"blk.{L}.ffn_down.weight"].T

    def _qkv(self, x, L):
        w = self.w
        xn = rmsnorm(x, w[f"blk.{L}.attn_norm.weight"])
        return (xn @ w[f"blk.{L}.attn_q.weight"].T, xn @ w[f"blk.{L}.attn_k.weight"].T,
                xn @ w[f"blk.{L}.attn_v.weight"].T)

    def _logits(self, x):
        xf = rmsnorm(x, self.w["output_norm.weight"])
        return xf @ self.w["output.weight"].T

    def forward1(self, tok, pos):
        """One token through every layer (the reference's token loop);
        returns logits and each layer's ao."""
        H, HK, D = self.H, self.HK, self.D
        x = self.w["token_embd.weight"][tok].astype(np.float32)
        aos = []
        for L in range(self.c["n_layers"]):
            q, k, v = self._qkv(x, L)
            ao = decode_host(self.kv, self.rope, L, pos, q.reshape(H, D), k.reshape(HK, D),
                             v.reshape(HK, D)).reshape(-1)
            aos.append(ao)
            x = x + ao @ self.w[f"blk.{L}.attn_output.weight"].T
            x = self._ffn(x, L)
        return self._logits(x), aos

    def prefill(self, toks):
        """The whole prompt layer by layer, attention through the MFMA
        prefill; returns the last token's logits and each layer's ao rows."""
        H, HK, D, n = self.H, self.HK, self.D, len(toks)
        X = self.w["token_embd.weight"][np.asarray(toks)].astype(np.float32)
        aos = []
        for L in range(self.c["n_layers"]):
            Q, K, V = self._qkv(X, L)
            AO = prefill_host(self.kv, self.rope, L, 0, Q.reshape(n, H, D), K.reshape(n, HK, D),
                              V.reshape(n, HK, D)).reshape(n, -1)
            aos.append(AO)
            X = X + AO @ self.w[f"blk.{L}.attn_output.weight"].T
            X = self._ffn(X, L)
        return self._logits(X[-1]), aos


def _golden(name, norm_offset):
    z = np.load(os.path.join(HERE, "golden", name))
    w = gguf.tiny_weights(0, norm_offset)
    assert gguf.weights_digest(w) == str(z["weights_sha256"]), "weights differ from the fixture's"
    return z


@pytest.mark.parametrize("name,norm_offset", FIXTURES, ids=[f[0][:-4] for f in FIXTURES])
def test_tiny_llama_greedy_decode_matches_reference(name, norm_offset):
    z = _golden(name, norm_offset)
    log(f"e2e decode {name}: prompt {z['prompt'].tolist()}")
    m = TinyModel(norm_offset)
    try:
        fed, gen, err_ao, err_lg = [], [], 0.0, 0.0
        logits, pos = None, 0
        for t in z["prompt"]:
            logits, aos = m.forward1(int(t), pos)
            err_ao = max(err_ao, maxerr(aos[0], z["ao"][0][pos]), maxerr(aos[-1], z["ao"][1][pos]))
            err_lg = max(err_lg, maxerr(logits, z["logits"][pos]))
            pos += 1
        n_gen = len(z["generated"])
        for i in range(n_gen):
            nxt = int(np.argmax(logits))     # first maximum, as pickle_fast_argmax
            gen.append(nxt)
            if i < n_gen - 1:
                logits, aos = m.forward1(nxt, pos)
                err_ao = max(err_ao, maxerr(aos[0], z["ao"][0][pos]),
                             maxerr(aos[-1], z["ao"][1][pos]))
                err_lg = max(err_lg, maxerr(logits, z["logits"][pos]))
                pos += 1
        log(f"  generated {gen}")
        log(f"  ao max-abs err {err_ao:.3e}, logits max-abs err {err_lg:.3e}")
        assert gen == z["generated"].tolist()
        assert err_ao <= 1e-4
    finally:
        m.free()


@pytest.mark.parametrize("name,norm_offset", FIXTURES, ids=[f[0][:-4] for f in FIXTURES])
def test_tiny_llama_prefill_then_decode_matches_reference(name, norm_offset):
    """The prompt prefilled layer-major on MFMA, then greedy decode: same
    tokens as the reference's token loop."""
    z = _golden(name, norm_offset)
    m = TinyModel(norm_offset)
    try:
        prompt = z["prompt"].tolist()
        logits, aos = m.prefill(prompt)
        n = len(prompt)
        err_ao = max(maxerr(aos[0], z["ao"][0][:n]), maxerr(aos[-1], z["ao"][1][:n]))
        log(f"e2e prefill {name}: prompt ao max-abs err {err_ao:.3e}")
        assert err_ao <= 2e-3
        gen, pos = [], n
        n_gen = len(z["generated"])
        for i in range(n_gen):
            nxt = int(np.argmax(logits))
            gen.append(nxt)
            if i < n_gen - 1:
                logits, _ = m.forward1(nxt, pos)
                pos += 1
        log(f"  generated {gen}")
        assert gen == z["generated"].tolist()
    finally:
        m.free()
