"""CPU-side checks of the product library: the C ABI it exports, the host
model's GGUF handling (src/gguf/reader.rs, src/model/config.rs and
weights.rs error behaviour), the seeded synthesizer and the quantizer.  No
call here touches a GPU: the backend context is created lazily by the
first forward."""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

import talos_amd as T
from oracle import oracle as O
from talos_amd import configs
from tests.gguf_writer import GgufWriter, llama_meta

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in ("talos_hip.h", "talos_host.h"):
        txt = open(os.path.join(ROOT, "include", h)).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(talos_\w+)\s*\(", txt, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol(talos):
    L = T.lib()
    decl = declared_functions()
    assert len(decl) >= 30
    missing = [n for n in decl if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"
    # and the Python binding covers exactly the declared ABI
    assert sorted(T.exported_symbols()) == decl


# ---- host GGUF / config error behaviour ------------------------------------

def tiny_gguf(**over):
    d = dict(ctx=16, embd=32, n_layer=1, ff=48, n_head=4, n_head_kv=2, vocab=20)
    d.update({k: v for k, v in over.items() if k in d})
    g = GgufWriter(version=over.get("version", 3), magic=over.get("magic", b"GGUF"))
    if over.get("arch", "llama") != "llama":
        g.str("general.architecture", over["arch"])
    else:
        llama_meta(g, **d)
    rng = np.random.default_rng(0)
    E, FF, V, hd = d["embd"], d["ff"], d["vocab"], d["embd"] // d["n_head"]
    kv = d["n_head_kv"] * hd
    skip = over.get("skip", "")
    t = {"token_embd.weight": (V, E), "output_norm.weight": (E,), "output.weight": (V, E),
         "blk.0.attn_norm.weight": (E,), "blk.0.attn_q.weight": (E, E), "blk.0.attn_k.weight": (kv, E),
         "blk.0.attn_v.weight": (kv, E), "blk.0.attn_output.weight": (E, E), "blk.0.ffn_norm.weight": (E,),
         "blk.0.ffn_gate.weight": (FF, E), "blk.0.ffn_up.weight": (FF, E), "blk.0.ffn_down.weight": (E, FF)}
    for name, shape in t.items():
        if name == skip:
            continue
        if name == over.get("bad_shape"):
            shape = (shape[0] + 1,) + shape[1:]
        g.tensor(name, list(shape[::-1]), rng.normal(0, 0.02, shape).astype(np.float32))
    return g.finish()


def test_host_loads_tiny_and_reports_config(talos):
    m = T.Model.load_bytes(tiny_gguf())
    c = m.cfg
    assert (c.n_layer, c.n_head, c.n_head_kv, c.n_embd, c.n_ff, c.vocab_size, c.context_length) == \
        (1, 4, 2, 32, 48, 20, 16)
    assert abs(c.rms_eps - 1e-5) < 1e-12 and c.rope_freq_base == 10000.0
    m.cap_context(8)
    assert m.cfg.context_length == 8
    m.cap_context(1000)  # never grows past the model's own context
    assert m.cfg.context_length == 8
    m.close()


@pytest.mark.parametrize("over,frag", [
    (dict(magic=b"GGUX"), "magic"),
    (dict(version=2), "version"),
    (dict(arch="gpt2"), "architecture"),
    (dict(n_head=4, n_head_kv=3), "head_count"),
    (dict(skip="blk.0.ffn_up.weight"), "blk.0.ffn_up.weight"),
    (dict(bad_shape="blk.0.attn_k.weight"), "blk.0.attn_k.weight"),
])
def test_host_rejects_bad_models(talos, over, frag):
    with pytest.raises(T.TalosError) as e:
        T.Model.load_bytes(tiny_gguf(**over))
    assert frag in str(e.value)


def test_host_rejects_truncated_file(talos):
    data = tiny_gguf()
    for cut in (3, 24, 200, len(data) - 16):
        with pytest.raises(T.TalosError):
            T.Model.load_bytes(data[:cut])


def test_host_dequant_row_matches_oracle(talos):
    # the embedding lookup (dtype.rs dequantize of one row) for each format
    for t in (O.F32, O.Q8_0, O.Q4_0, O.Q6_K):
        spec = T.SynthSpec(n_layer=1, n_head=2, n_head_kv=1, n_embd=256, n_ff=256, vocab_size=8,
                           context_length=8, layer_type=T.GGML_F32, output_type=T.GGML_F32, embd_type=t, seed=5,
                           name=f"emb{t}")
        data = T.synth_bytes(spec, nthreads=2)
        m = T.Model.load_bytes(data)
        g = O.OracleGguf(bytes(data))
        ty, raw = g.tensor_raw("token_embd.weight")
        assert ty == t
        full = O.dequantize(t, np.frombuffer(raw, np.uint8), 8 * 256).reshape(8, 256)
        for tok in (0, 3, 7):
            np.testing.assert_array_equal(m.dequant_row(tok), full[tok])
        m.close()
        g.close()


# ---- synthesizer and quantizer ------------------------------------------------

def test_synth_is_deterministic_and_seeded(talos):
    spec = configs.tiny_f32().spec
    a = T.synth_bytes(spec, nthreads=1)
    b = T.synth_bytes(spec, nthreads=4)
    assert a.size == b.size and np.array_equal(a, b)
    spec2 = T.SynthSpec(**{**spec.__dict__, "seed": spec.seed + 1})
    c = T.synth_bytes(spec2, nthreads=2)
    assert a.size == c.size and not np.array_equal(a, c)


def test_synth_normal_statistics(talos):
    x = T.synth_normal(42, "blk.0.attn_q.weight", 0, 200000, 0.02)
    assert abs(float(x.mean())) < 2e-4 and abs(float(x.std()) - 0.02) < 2e-4
    # windows of one stream agree (counter-based generator)
    y = T.synth_normal(42, "blk.0.attn_q.weight", 1000, 500, 0.02)
    np.testing.assert_array_equal(x[1000:1500], y)
    z = T.synth_normal(42, "blk.0.attn_k.weight", 0, 1000, 0.02)
    assert not np.array_equal(x[:1000], z)


def test_synth_model_parses_in_oracle(talos):
    wl = configs.gqa_q8()
    data = T.synth_bytes(wl.spec, nthreads=4)
    m = O.OracleModel(data)
    assert (m.cfg.n_layer, m.cfg.n_head, m.cfg.n_head_kv, m.cfg.n_embd) == (8, 8, 2, 512)
    lg = m.forward(1, 0)
    assert lg.shape == (4096,) and np.isfinite(lg).all()
    m.close()


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.Q6_K])
def test_product_quantizer_matches_oracle(talos, t):
    rng = np.random.default_rng(t)
    x = rng.normal(0, 0.02, 256 * 40).astype(np.float32)
    x[:256] = 0.0
    assert np.array_equal(T.quantize(t, x), O.quantize(t, x))


def test_workload_byte_counts(talos):
    s = configs.mistral7b_q4().spec
    # Q4_0: 18 bytes / 32; Q6_K: 210 / 256; norms f32
    n, ff, kv, V = 4096, 14336, 1024, 32000
    layer = (n * n * 2 + n * kv * 2 + n * ff * 3) * 18 // 32 + 2 * n * 4
    exp = 32 * layer + V * n * 210 // 256 + n * 4 + n * 18 // 32
    assert configs.bytes_per_token_weights(s) == exp
    assert configs.kv_bytes_per_position(s) == 32 * 2 * kv * 4
