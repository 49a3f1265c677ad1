"""Minimal GGUF v3 writer for the synthetic Llama models used by the tests.

Writes what the reference's loader reads (src/pickle.c:293-375: header,
metadata table, tensor table, 32-byte aligned F32 data) and the Llama
metadata keys of pickle_arch_detect (src/pickle.c:988-1036).  Tensor dims
are written [rows, cols] like the reference's own generator
(tools/make_tiny_gguf.py:57); weights are row-major W[out][in].
"""
from __future__ import annotations

import hashlib
import struct

import numpy as np

ALIGN = 32
GGUF_U32, GGUF_F32, GGUF_BOOL, GGUF_STRING = 4, 6, 7, 8


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path: str, meta: list[tuple[str, int, object]],
               tensors: list[tuple[str, np.ndarray]]) -> None:
    out = bytearray()
    out += struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(meta))
    for key, typ, val in meta:
        out += _str(key) + struct.pack("<I", typ)
        if typ == GGUF_U32:
            out += struct.pack("<I", int(val))
        elif typ == GGUF_F32:
            out += struct.pack("<f", float(val))
        elif typ == GGUF_BOOL:
            out += struct.pack("<B", 1 if val else 0)
        elif typ == GGUF_STRING:
            out += _str(str(val))
        else:
            raise ValueError(typ)
    offsets, cur = [], 0
    for _, arr in tensors:
        offsets.append(cur)
        cur += arr.size * 4
        cur += (-cur) % ALIGN
    for (name, arr), off in zip(tensors, offsets):
        dims = arr.shape
        out += _str(name) + struct.pack("<I", len(dims))
        for d in dims:
            out += struct.pack("<Q", d)
        out += struct.pack("<IQ", 0, off)          # GGML_F32
    out += b"\0" * ((-len(out)) % ALIGN)
    for name, arr in tensors:
        out += np.ascontiguousarray(arr, np.float32).tobytes()
        out += b"\0" * ((-len(out)) % ALIGN)
    with open(path, "wb") as f:
        f.write(out)


def llama_meta(*, n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, ctx, vocab,
               theta, eps=1e-5, name="synthetic"):
    return [
        ("general.architecture", GGUF_STRING, "llama"),
        ("general.name", GGUF_STRING, name),
        ("llama.block_count", GGUF_U32, n_layers),
        ("llama.embedding_length", GGUF_U32, hidden),
        ("llama.feed_forward_length", GGUF_U32, ffn),
        ("llama.attention.head_count", GGUF_U32, n_heads),
        ("llama.attention.head_count_kv", GGUF_U32, n_kv_heads),
        ("llama.context_length", GGUF_U32, ctx),
        ("llama.rope.dimension_count", GGUF_U32, head_dim),
        ("llama.attention.layer_norm_rms_epsilon", GGUF_F32, eps),
        ("llama.rope.freq_base", GGUF_F32, theta),
        ("llama.vocab_size", GGUF_U32, vocab),
        ("llama.tie_word_embeddings", GGUF_BOOL, False),
    ]


# ---- the tiny end-to-end model --------------------------------------------

TINY = dict(n_layers=2, hidden=64, ffn=172, n_heads=4, n_kv_heads=2, head_dim=16,
            ctx=64, vocab=256, theta=10000.0)


def tiny_weights(seed: int = 0, norm_offset: float = 0.0) -> dict[str, np.ndarray]:
    """F32 weights drawn from N(0, 0.02), in the tensor order below, from
    numpy's default_rng(seed).  norm_offset is added to the RMSNorm weights
    (0 gives the all-N(0, 0.02) model; 1 keeps activations O(1))."""
    c = TINY
    rng = np.random.default_rng(seed)
    hd, ff, H, HK, D, V = c["hidden"], c["ffn"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["vocab"]
    shapes = [("token_embd.weight", (V, hd))]
    for L in range(c["n_layers"]):
        shapes += [
            (f"blk.{L}.attn_norm.weight", (hd,)),
            (f"blk.{L}.attn_q.weight", (H * D, hd)),
            (f"blk.{L}.attn_k.weight", (HK * D, hd)),
            (f"blk.{L}.attn_v.weight", (HK * D, hd)),
            (f"blk.{L}.attn_output.weight", (hd, H * D)),
            (f"blk.{L}.ffn_norm.weight", (hd,)),
            (f"blk.{L}.ffn_gate.weight", (ff, hd)),
            (f"blk.{L}.ffn_up.weight", (ff, hd)),
            (f"blk.{L}.ffn_down.weight", (hd, ff)),
        ]
    shapes += [("output_norm.weight", (hd,)), ("output.weight", (V, hd))]
    w = {}
    for name, shp in shapes:
        a = (rng.standard_normal(shp) * 0.02).astype(np.float32)
        if name.endswith("norm.weight") and norm_offset:
            a = (norm_offset + a).astype(np.float32)
        w[name] = a
    return w


def weights_digest(w: dict[str, np.ndarray]) -> str:
    h = hashlib.sha256()
    for name in sorted(w):
        h.update(name.encode())
        h.update(np.ascontiguousarray(w[name], np.float32).tobytes())
    return h.hexdigest()


def write_tiny(path: str, seed: int = 0, norm_offset: float = 0.0) -> dict[str, np.ndarray]:
    w = tiny_weights(seed, norm_offset)
    c = TINY
    meta = llama_meta(n_layers=c["n_layers"], hidden=c["hidden"], ffn=c["ffn"],
                      n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"], head_dim=c["head_dim"],
                      ctx=c["ctx"], vocab=c["vocab"], theta=c["theta"], name="tiny-llama")
    write_gguf(path, meta, list(w.items()))
    return w


# ---- attention probe model ------------------------------------------------

def write_probe(path: str, *, n_heads, n_kv_heads, head_dim, theta, ctx, seed, vocab=8):
    """A one-layer model whose Q/K/V projections select disjoint slices of the
    normed input (0/1 rows), so the reference's q, k, v equal slices of its
    own state->xn exactly; everything after attention is zero."""
    H, HK, D = n_heads, n_kv_heads, head_dim
    hd = H * D + 2 * HK * D
    ff = 16
    rng = np.random.default_rng(seed)
    emb = rng.standard_normal((vocab, hd)).astype(np.float32)
    sel = np.eye(hd, dtype=np.float32)
    t = [
        ("token_embd.weight", emb),
        ("blk.0.attn_norm.weight", np.ones(hd, np.float32)),
        ("blk.0.attn_q.weight", sel[0:H * D].copy()),
        ("blk.0.attn_k.weight", sel[H * D:H * D + HK * D].copy()),
        ("blk.0.attn_v.weight", sel[H * D + HK * D:].copy()),
        ("blk.0.attn_output.weight", np.zeros((hd, H * D), np.float32)),
        ("blk.0.ffn_norm.weight", np.ones(hd, np.float32)),
        ("blk.0.ffn_gate.weight", np.zeros((ff, hd), np.float32)),
        ("blk.0.ffn_up.weight", np.zeros((ff, hd), np.float32)),
        ("blk.0.ffn_down.weight", np.zeros((hd, ff), np.float32)),
        ("output_norm.weight", np.ones(hd, np.float32)),
        ("output.weight", np.zeros((vocab, hd), np.float32)),
    ]
    meta = llama_meta(n_layers=1, hidden=hd, ffn=ff, n_heads=H, n_kv_heads=HK, head_dim=D,
                      ctx=ctx, vocab=vocab, theta=theta, name="attention-probe")
    write_gguf(path, meta, t)


# ---- timing model for the CPU baseline --------------------------------------

def write_timing_model(path: str, *, n_layers, n_heads, n_kv_heads, head_dim, ctx, theta,
                       hidden=64, ffn=64, vocab=256, seed=0):
    """A Llama model with the attention shape (H, HK, head_dim) of a real
    model and a small hidden size, so that the reference's forward pass at a
    long context is almost all attention (src/pickle_fast.c:1946-2094): its
    Q/K/V/O projections are H*head_dim x hidden (src/pickle_fast.c:1903-1908,
    2112), and head_dim comes from llama.rope.dimension_count
    (src/pickle.c:1006-1007).  Weights N(0, 0.02), F32."""
    H, HK, D = n_heads, n_kv_heads, head_dim
    rng = np.random.default_rng(seed)
    w = lambda *shape: (rng.standard_normal(shape) * 0.02).astype(np.float32)
    t = [("token_embd.weight", w(vocab, hidden))]
    for L in range(n_layers):
        t += [
            (f"blk.{L}.attn_norm.weight", np.ones(hidden, np.float32)),
            (f"blk.{L}.attn_q.weight", w(H * D, hidden)),
            (f"blk.{L}.attn_k.weight", w(HK * D, hidden)),
            (f"blk.{L}.attn_v.weight", w(HK * D, hidden)),
            (f"blk.{L}.attn_output.weight", w(hidden, H * D)),
            (f"blk.{L}.ffn_norm.weight", np.ones(hidden, np.float32)),
            (f"blk.{L}.ffn_gate.weight", w(ffn, hidden)),
            (f"blk.{L}.ffn_up.weight", w(ffn, hidden)),
            (f"blk.{L}.ffn_down.weight", w(hidden, ffn)),
        ]
    t += [("output_norm.weight", np.ones(hidden, np.float32)), ("output.weight", w(vocab, hidden))]
    meta = llama_meta(n_layers=n_layers, hidden=hidden, ffn=ffn, n_heads=H, n_kv_heads=HK,
                      head_dim=D, ctx=ctx, vocab=vocab, theta=theta, name="attention-timing")
    write_gguf(path, meta, t)
