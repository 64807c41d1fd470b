"""Model-level pins of the oracle: the GGUF reader known-answer file of
src/gguf/reader.rs tests, the GQA == replicated-MHA invariant of
tests/gqa.rs, and an independent float64 restatement of the forward
(src/model/llama.rs:96-183) on tiny models, in F32 and in the quantized
formats.  A dropped residual, a wrong head -> KV-head map, a misplaced
rmsnorm or RoPE convention each fails one of these.
"""
import math
import struct

import numpy as np
import pytest

from oracle import oracle as O
from tests.gguf_writer import GgufWriter, llama_meta


# ---- src/gguf/reader.rs tests: round_trips_metadata_and_tensors ----------

def reader_test_file() -> bytes:
    g = GgufWriter()
    g.u32("answer.u32", 42)
    g.f32("scale.f32", 2.5)
    g.boolean("flag.bool", True)
    g.arr_str("names.arr", ["alpha", "beta", "gamma"])
    g.arr_i32("types.arr", [-7, 0, 9])
    g.tensor("tensor.one", [3, 2], np.array([1, 2, 3, 4, 5, 6], np.float32))
    g.tensor("tensor.two", [3], np.array([-1.5, 0.0, 42.25], np.float32))
    return g.finish()


def test_gguf_reader_known_file():
    g = O.OracleGguf(reader_test_file())
    assert g.u32("answer.u32") == 42
    assert g.f32("scale.f32") == 2.5
    assert g.arr_str_len("names.arr") == 3
    assert g.u32("scale.f32") is None       # wrong-type access
    assert g.str("missing") is None
    t = g.tensors()
    assert [(n, d, ty) for n, d, ty, _ in t] == [("tensor.one", [3, 2], 0), ("tensor.two", [3], 0)]
    assert [off for *_, off in t] == [0, 32]  # 32-byte aligned data offsets
    ty, raw = g.tensor_raw("tensor.one")
    assert ty == 0 and np.frombuffer(raw, np.float32).tolist() == [1, 2, 3, 4, 5, 6]
    ty, raw = g.tensor_raw("tensor.two")
    assert np.frombuffer(raw, np.float32).tolist() == [-1.5, 0.0, 42.25]
    with pytest.raises(KeyError):
        g.tensor_raw("missing")
    g.close()


@pytest.mark.parametrize("mutate,what", [
    (lambda b: b"GGUX" + b[4:], "magic"),
    (lambda b: b[:4] + struct.pack("<I", 2) + b[8:], "version"),
    (lambda b: b[:20], "truncated header"),
    (lambda b: b[:60], "truncated metadata"),
])
def test_gguf_reader_rejects(mutate, what):
    with pytest.raises(ValueError):
        O.OracleGguf(mutate(reader_test_file()))


def test_gguf_reader_bounds_checks_tensor_data_on_access():
    # src/gguf/reader.rs:320,347: the index parses; reading a tensor that
    # runs past the end of the file is an error.
    g = O.OracleGguf(reader_test_file()[:-8])
    g.tensor_raw("tensor.one")
    with pytest.raises(KeyError):
        g.tensor_raw("tensor.two")
    g.close()


# ---- tiny models ----------------------------------------------------------

def rand_model(rng, *, embd, n_head, n_head_kv, ff, vocab, n_layer, scale=0.5):
    rv = lambda *shape: rng.uniform(-scale, scale, shape).astype(np.float32)
    hd = embd // n_head
    W = {"token_embd.weight": rv(vocab, embd), "output_norm.weight": rv(embd) + 1.0,
         "output.weight": rv(vocab, embd)}
    for l in range(n_layer):
        p = f"blk.{l}."
        W[p + "attn_norm.weight"] = rv(embd) + 1.0
        W[p + "attn_q.weight"] = rv(embd, embd)
        W[p + "attn_k.weight"] = rv(n_head_kv * hd, embd)
        W[p + "attn_v.weight"] = rv(n_head_kv * hd, embd)
        W[p + "attn_output.weight"] = rv(embd, embd)
        W[p + "ffn_norm.weight"] = rv(embd) + 1.0
        W[p + "ffn_gate.weight"] = rv(ff, embd)
        W[p + "ffn_up.weight"] = rv(ff, embd)
        W[p + "ffn_down.weight"] = rv(embd, ff)
    return W


def gguf_of(W, *, embd, n_head, n_head_kv, ff, vocab, n_layer, ctx=32, theta=10000.0, qtype=0, eps=1e-5):
    g = GgufWriter()
    llama_meta(g, ctx=ctx, embd=embd, n_layer=n_layer, ff=ff, n_head=n_head, n_head_kv=n_head_kv, vocab=vocab,
               eps=eps, theta=theta)
    for name, a in W.items():
        if a.ndim == 2 and qtype != 0 and name != "token_embd.weight":
            g.tensor(name, [a.shape[1], a.shape[0]], O.quantize(qtype, a), qtype)
        else:
            g.tensor(name, list(a.shape[::-1]), a)
    return g.finish()


def np_dequant(qtype, a):
    """Round trip through the format (the weights the model really holds)."""
    if qtype == 0 or a.ndim == 1:
        return a.astype(np.float64)
    return O.dequantize(qtype, O.quantize(qtype, a), a.size).reshape(a.shape).astype(np.float64)


def np_forward(W, tokens, *, embd, n_head, n_head_kv, n_layer, theta=10000.0, eps=1e-5, qtype=0):
    """float64 forward of src/model/llama.rs:96-183, written independently of
    the oracle: returns the logits after each token."""
    D = {k: np_dequant(qtype if k != "token_embd.weight" else 0, v) for k, v in W.items()}
    hd = embd // n_head
    group = n_head // n_head_kv

    def rms(x, w):
        return x / math.sqrt(np.mean(x * x) + eps) * w

    def rope(v, pos, nh):
        # adjacent pairs (2i, 2i+1), i < hd // 2, of the first nh heads; an
        # odd hd leaves each head's last element, and elements past the
        # heads stay as they are
        v = v.copy()
        i = np.arange(hd // 2)
        ang = pos * theta ** (-2.0 * i / hd)
        c, s = np.cos(ang), np.sin(ang)
        for h in range(nh):
            x0, x1 = v[h * hd + 2 * i].copy(), v[h * hd + 2 * i + 1].copy()
            v[h * hd + 2 * i] = x0 * c - x1 * s
            v[h * hd + 2 * i + 1] = x0 * s + x1 * c
        return v

    K = [[] for _ in range(n_layer)]
    V = [[] for _ in range(n_layer)]
    out = []
    for pos, tok in enumerate(tokens):
        x = D["token_embd.weight"][tok].copy()
        for l in range(n_layer):
            p = f"blk.{l}."
            h = rms(x, D[p + "attn_norm.weight"])
            q = rope(D[p + "attn_q.weight"] @ h, pos, n_head)
            K[l].append(rope(D[p + "attn_k.weight"] @ h, pos, n_head_kv))
            V[l].append(D[p + "attn_v.weight"] @ h)
            Ks, Vs = np.array(K[l]), np.array(V[l])
            att = np.zeros(embd)
            for hh in range(n_head):
                kv = hh // group
                sc = Ks[:, kv * hd:(kv + 1) * hd] @ q[hh * hd:(hh + 1) * hd] / math.sqrt(hd)
                pr = np.exp(sc - sc.max())
                pr /= pr.sum()
                att[hh * hd:(hh + 1) * hd] = pr @ Vs[:, kv * hd:(kv + 1) * hd]
            x = x + D[p + "attn_output.weight"] @ att
            h = rms(x, D[p + "ffn_norm.weight"])
            gt, up = D[p + "ffn_gate.weight"] @ h, D[p + "ffn_up.weight"] @ h
            x = x + D[p + "ffn_down.weight"] @ (gt / (1.0 + np.exp(-gt)) * up)
        out.append(D["output.weight"] @ rms(x, D["output_norm.weight"]))
    return out


SHAPE = dict(embd=64, n_head=4, n_head_kv=2, ff=96, vocab=40, n_layer=2)


@pytest.mark.parametrize("qtype,tol", [(O.F32, 1e-4), (O.Q8_0, 1e-4), (O.Q4_0, 1e-4)])
def test_forward_matches_float64_restatement(qtype, tol):
    rng = np.random.default_rng(17 + qtype)
    W = rand_model(rng, **SHAPE, scale=0.3)
    data = gguf_of(W, **SHAPE, qtype=qtype)
    m = O.OracleModel(data)
    toks = [3, 1, 4, 1, 5, 9]
    ref = np_forward(W, toks, embd=64, n_head=4, n_head_kv=2, n_layer=2, qtype=qtype)
    for pos, t in enumerate(toks):
        got = m.forward(t, pos)
        d = float(np.abs(got - ref[pos]).max())
        assert d <= tol * max(1.0, float(np.abs(ref[pos]).max())), f"pos {pos}: {d}"
    m.close()


# Shapes the reference accepts beyond the benchmark ones (src/model/
# llama.rs:45-51 asks only that n_head_kv divide n_head): its own GPU
# contract model (tests/forward_gpu.rs:62: head_dim 4), an odd head_dim with
# n_embd not a multiple of n_head (30 = 4 * 7 + 2), and a GQA group of 12.
GENERIC_SHAPES = [
    dict(embd=16, n_head=4, n_head_kv=2, ff=32, vocab=16, n_layer=2),
    dict(embd=30, n_head=4, n_head_kv=2, ff=40, vocab=24, n_layer=2),
    dict(embd=96, n_head=12, n_head_kv=1, ff=64, vocab=20, n_layer=2),
]


@pytest.mark.parametrize("shape", GENERIC_SHAPES, ids=["contract_hd4", "odd_hd7", "group12"])
def test_forward_matches_float64_generic_shapes(shape):
    rng = np.random.default_rng(29)
    W = rand_model(rng, **shape, scale=0.5)
    data = gguf_of(W, **shape)
    m = O.OracleModel(data)
    toks = [1, 3, 5, 7, 2, 4]
    ref = np_forward(W, [t % shape["vocab"] for t in toks], embd=shape["embd"], n_head=shape["n_head"],
                     n_head_kv=shape["n_head_kv"], n_layer=shape["n_layer"])
    for pos, t in enumerate(toks):
        got = m.forward(t % shape["vocab"], pos)
        d = float(np.abs(got - ref[pos]).max())
        assert d <= 1e-4 * max(1.0, float(np.abs(ref[pos]).max())), f"pos {pos}: {d}"
    m.close()


def test_forward_hidden_is_prelogit_state():
    rng = np.random.default_rng(3)
    W = rand_model(rng, **SHAPE, scale=0.3)
    data = gguf_of(W, **SHAPE)
    a, b = O.OracleModel(data), O.OracleModel(data)
    for pos, t in enumerate([2, 7, 1]):
        lg = a.forward(t, pos)
        hid = b.forward_hidden(t, pos)
        np.testing.assert_allclose(lg, W["output.weight"].astype(np.float64) @ hid, atol=1e-5)
    a.close()
    b.close()


def test_gqa_matches_replicated_mha():
    # tests/gqa.rs: EMBD 16, 4 heads, 2 KV heads, FF 32, vocab 16, 2 layers;
    # K/V of a GQA model keep the group leaders' heads, the MHA twin repeats
    # each leader over its group.  Tokens 1..5 -> last logits within 1e-5.
    E, NH, NKV, HD, FF, VOC, NL = 16, 4, 2, 4, 32, 16, 2
    G = NH // NKV
    rng = np.random.default_rng(7)
    rv = lambda *s: rng.uniform(-0.5, 0.5, s).astype(np.float32)
    embd, onorm, out = rv(VOC, E), rv(E), rv(VOC, E)
    layers = [dict(an=rv(E), q=rv(E, E), k=rv(E, E), v=rv(E, E), o=rv(E, E), fn=rv(E), g=rv(FF, E), u=rv(FF, E),
                   d=rv(E, FF)) for _ in range(NL)]

    def build(gqa):
        W = {"token_embd.weight": embd, "output_norm.weight": onorm, "output.weight": out}
        rows = NKV if gqa else NH
        for l, ly in enumerate(layers):
            lead = [(r * G if gqa else (r // G) * G) for r in range(rows)]
            k = np.concatenate([ly["k"][h * HD:(h + 1) * HD] for h in lead])
            v = np.concatenate([ly["v"][h * HD:(h + 1) * HD] for h in lead])
            p = f"blk.{l}."
            W.update({p + "attn_norm.weight": ly["an"], p + "attn_q.weight": ly["q"], p + "attn_k.weight": k,
                      p + "attn_v.weight": v, p + "attn_output.weight": ly["o"], p + "ffn_norm.weight": ly["fn"],
                      p + "ffn_gate.weight": ly["g"], p + "ffn_up.weight": ly["u"], p + "ffn_down.weight": ly["d"]})
        return gguf_of(W, embd=E, n_head=NH, n_head_kv=NKV if gqa else NH, ff=FF, vocab=VOC, n_layer=NL)

    res = []
    for gqa in (True, False):
        m = O.OracleModel(build(gqa))
        for pos, t in enumerate([1, 2, 3, 4, 5]):
            lg = m.forward(t, pos)
        res.append(lg)
        m.close()
    assert float(np.abs(res[0] - res[1]).max()) <= 1e-5


def test_reset_and_cap_context():
    rng = np.random.default_rng(9)
    W = rand_model(rng, **SHAPE, scale=0.3)
    m = O.OracleModel(gguf_of(W, **SHAPE, ctx=32))
    a = [m.forward(t, p) for p, t in enumerate([5, 6, 7])]
    assert m.kv_len() == 3
    m.reset()
    assert m.kv_len() == 0
    b = [m.forward(t, p) for p, t in enumerate([5, 6, 7])]
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    m.cap_context(8)
    assert m.cfg.context_length == 8
    m.close()


def test_kv_injection_resumes_the_forward():
    """set_kv / get_kv use the forward's own cache layout [layer][pos][kv_dim]:
    a second model started from the first one's cache continues bit for bit,
    and position 0's K row of layer 0 is Wk . rmsnorm(embedding) (RoPE at
    position 0 is the identity)."""
    rng = np.random.default_rng(21)
    W = rand_model(rng, **SHAPE, scale=0.3)
    data = gguf_of(W, **SHAPE)
    a, b = O.OracleModel(data), O.OracleModel(data)
    toks = [3, 1, 4, 1, 5]
    for p, t in enumerate(toks):
        a.forward(t, p)
    k, v = a.get_kv(len(toks))
    assert k.shape == (SHAPE["n_layer"], len(toks), SHAPE["n_head_kv"] * SHAPE["embd"] // SHAPE["n_head"])
    x = W["token_embd.weight"][toks[0]].astype(np.float64)
    xn = x / np.sqrt(np.mean(x * x) + 1e-5) * W["blk.0.attn_norm.weight"]
    np.testing.assert_allclose(k[0, 0], W["blk.0.attn_k.weight"].astype(np.float64) @ xn, atol=1e-5)
    np.testing.assert_allclose(v[0, 0], W["blk.0.attn_v.weight"].astype(np.float64) @ xn, atol=1e-5)
    b.set_kv(k, v)
    assert b.kv_len() == len(toks)
    la, lb = a.forward(9, len(toks)), b.forward(9, len(toks))
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    with pytest.raises(ValueError):
        a.get_kv(99)
    a.close()
    b.close()


@pytest.mark.parametrize("qtype", [O.F32, O.Q8_0, O.Q4_0])
def test_simd_build_is_bit_identical(qtype):
    """The CPU baseline's -O3 -mavx2 build of the oracle gives the parity
    build's logits bit for bit (no FMA contraction, no reassociation)."""
    if not O.host_has_avx2():
        pytest.skip("host has no AVX2")
    rng = np.random.default_rng(41 + qtype)
    W = rand_model(rng, **SHAPE, scale=0.3)
    data = gguf_of(W, **SHAPE, qtype=qtype)
    a = O.OracleModel(data, nthreads=4)
    b = O.OracleModel(data, nthreads=4, simd=True)
    for pos, t in enumerate([3, 1, 4, 1, 5, 9, 2, 6]):
        la, lb = a.forward(t, pos), b.forward(t, pos)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), f"pos {pos}"
    a.close()
    b.close()


def test_simd_build_is_bit_identical_q6k_output():
    from tests import models as MB
    shape = dict(embd=256, n_head=4, n_head_kv=2, ff=512, vocab=300, n_layer=1)
    W = MB.normal_model(8, **shape)
    types = {n: 2 for n in MB.layer_names(1)}
    types["output.weight"] = 14
    data = MB.gguf_bytes(W, ctx=16, types=types, **shape)
    if not O.host_has_avx2():
        pytest.skip("host has no AVX2")
    a = O.OracleModel(data, nthreads=4)
    b = O.OracleModel(data, nthreads=4, simd=True)
    for pos, t in enumerate([3, 1, 4, 1]):
        assert np.array_equal(a.forward(t, pos).view(np.uint32), b.forward(t, pos).view(np.uint32))
    a.close()
    b.close()
