"""Small Llama models built in numpy for the shape-domain tests: random
weights in GGUF v3 bytes (tests/gguf_writer.py), each tensor in the ggml
type a test asks for.  Test infrastructure only."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O
from tests.gguf_writer import GgufWriter, llama_meta


def layer_names(n_layer: int):
    for l in range(n_layer):
        p = f"blk.{l}."
        yield from (p + s for s in ("attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
                                    "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight",
                                    "ffn_up.weight", "ffn_down.weight"))


def shapes(*, embd, n_head, n_head_kv, ff, vocab, n_layer):
    """Tensor name -> [rows, cols] (norms: [cols]) as src/model/weights.rs
    binds them: head_dim = embd // n_head, kv_dim = n_head_kv * head_dim."""
    kv = n_head_kv * (embd // n_head)
    S = {"token_embd.weight": (vocab, embd), "output_norm.weight": (embd,), "output.weight": (vocab, embd)}
    for l in range(n_layer):
        p = f"blk.{l}."
        S.update({p + "attn_norm.weight": (embd,), p + "attn_q.weight": (embd, embd),
                  p + "attn_k.weight": (kv, embd), p + "attn_v.weight": (kv, embd),
                  p + "attn_output.weight": (embd, embd), p + "ffn_norm.weight": (embd,),
                  p + "ffn_gate.weight": (ff, embd), p + "ffn_up.weight": (ff, embd),
                  p + "ffn_down.weight": (embd, ff)})
    return S


def uniform_model(seed, *, scale=0.5, norm_offset=0.0, **shape):
    """Every tensor uniform in (-scale, scale) (tests/forward_gpu.rs:62-92
    draws every tensor, norms included, from -0.5..0.5); norm_offset is
    added to the norms."""
    rng = np.random.default_rng(seed)
    W = {}
    for name, s in shapes(**shape).items():
        a = rng.uniform(-scale, scale, s).astype(np.float32)
        if len(s) == 1:
            a = (a + np.float32(norm_offset)).astype(np.float32)
        W[name] = a
    return W


def normal_model(seed, *, stdev=0.02, **shape):
    """Matrices N(0, stdev), norms 1.0 (the synthetic benchmark models)."""
    rng = np.random.default_rng(seed)
    W = {}
    for name, s in shapes(**shape).items():
        W[name] = (np.ones(s, np.float32) if len(s) == 1
                   else (rng.standard_normal(s, dtype=np.float32) * np.float32(stdev)))
    return W


def gguf_bytes(W, *, embd, n_head, n_head_kv, ff, vocab, n_layer, ctx, types=None, default_type=0,
               theta=10000.0, eps=1e-5) -> bytes:
    """GGUF bytes of W; matrices in types.get(name, default_type) (quantized
    with the oracle's quantizers, the reference's test quantizers), norms
    F32."""
    types = types or {}
    g = GgufWriter()
    llama_meta(g, ctx=ctx, embd=embd, n_layer=n_layer, ff=ff, n_head=n_head, n_head_kv=n_head_kv, vocab=vocab,
               eps=eps, theta=theta)
    for name, a in W.items():
        t = 0 if a.ndim == 1 else types.get(name, default_type)
        if t == 0:
            g.tensor(name, list(a.shape[::-1]), a)
        else:
            g.tensor(name, [a.shape[1], a.shape[0]], O.quantize(t, a), t)
    return g.finish()
