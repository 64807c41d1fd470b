"""Batched prompt processing (talos_hip_prefill on the matrix cores)
against the reference's token-by-token prompt loop (src/main.rs:88-94,
Model::step per token) as the oracle runs it: the last step's logits within
the format's tolerance with the same argmax, and the K/V cache rows of every
prompt position within the same bar; a prompt longer than one chunk (1024
tokens) against the device's own token-by-token feed; and greedy decoding
that continues from either kind of prefill identically."""
import numpy as np
import pytest

from tests import models as MB
from tests.conftest import record_parity

pytestmark = pytest.mark.gpu


def _step(msg):
    print(f"\n[prefill] {msg}", flush=True)


@pytest.mark.parametrize("which,n,tol", [("tiny_f32", 8, 1e-4), ("gqa_q8", 16, 1e-3), ("mistral7b_q4", 32, 1e-3),
                                         ("tiny_f32", 200, 1e-4), ("gqa_q8", 300, 1e-3), ("mistral7b_q4", 136, 1e-3)])
def test_batched_prefill_matches_oracle(talos, oracle, which, n, tol):
    """Prompts of one to a few 64-token GEMM tiles, the last one partial."""
    from talos_amd import configs
    wl = getattr(configs, which)() if which != "mistral7b_q4" else configs.mistral7b_q4(ctx=256)
    _step(f"{which}: {n}-token prompt")
    m = talos.Model.synth(wl.spec, nthreads=16)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    prompt = [int(t) for t in np.random.default_rng(wl.spec.seed + 1).integers(0, wl.spec.vocab_size, n)]
    lg, am = m.prefill(prompt, 0)
    for p, t in enumerate(prompt):
        c = ref.forward(t, p)
    d = float(np.abs(lg - c).max())
    print(f"  last logits max abs {d:.3e}; argmax gpu {am} cpu {oracle.argmax(c)}", flush=True)
    assert d <= tol
    assert am == oracle.argmax(c)
    kg, vg = m.kv_read(n)
    kc, vc = ref.get_kv(n)
    dk = float(max(np.abs(kg - kc).max(), np.abs(vg - vc).max()))
    print(f"  K/V cache max abs {dk:.3e}", flush=True)
    assert dk <= tol
    record_parity(f"{which}_batched_prefill_{n}", max(d, dk), tol, path="batched_prefill")
    ref.close()
    m.close()


def test_multi_chunk_prefill_and_continuation(talos, oracle, monkeypatch):
    """2100 tokens (two full chunks and a partial one) on a GQA Q8_0 model
    with a 2304-position context: the batched prefill's last logits and
    cache against the oracle's token loop, then 16 greedy steps continue as
    after the device's token-by-token feed."""
    from talos_amd import SynthSpec, GGML_F32, GGML_Q8_0
    spec = SynthSpec(n_layer=4, n_head=8, n_head_kv=2, n_embd=512, n_ff=1376, vocab_size=4096,
                     context_length=2304, layer_type=GGML_Q8_0, output_type=GGML_Q8_0, embd_type=GGML_F32,
                     seed=48, name="gqa_q8_ctx2304")
    n = 2100
    prompt = [int(t) for t in np.random.default_rng(49).integers(0, spec.vocab_size, n)]
    _step("2100-token prompt, batched")
    m = talos.Model.synth(spec)
    lg, am = m.prefill(prompt, 0)
    kg, vg = m.kv_read(n)
    cont = m.decode_greedy(am, n, 16)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    for p, t in enumerate(prompt):
        c = ref.forward(t, p)
    d = float(np.abs(lg - c).max())
    kc, vc = ref.get_kv(n)
    dk = float(max(np.abs(kg - kc).max(), np.abs(vg - vc).max()))
    print(f"  last logits max abs {d:.3e}, K/V max abs {dk:.3e}", flush=True)
    assert d <= 1e-3 and dk <= 1e-3 and am == oracle.argmax(c)
    record_parity("gqa_q8_batched_prefill_2100", max(d, dk), 1e-3, path="batched_prefill")
    ref.close()
    m.close()
    _step("the same prompt one step per token")
    monkeypatch.setenv("TALOS_HIP_BATCH", "0")
    m2 = talos.Model.synth(spec)
    lg2, am2 = m2.prefill(prompt, 0)
    assert am2 == am and float(np.abs(lg2 - lg).max()) <= 1e-3
    assert list(m2.decode_greedy(am2, n, 16)) == list(cont)
    m2.close()


@pytest.mark.parametrize("pfa16", [None, "0"], ids=["attn_f16", "attn_f32"])
def test_prefill_after_decode_wide_group(talos, oracle, monkeypatch, pfa16):
    """A prompt, greedy decode steps, then a second prompt at the next
    position, on a Q8_0 model with 8 q heads per KV head (head_dim 64: the
    attention's 8-wave blocks): the second prefill attends over rows the
    decode steps wrote, which the split-f16 attention reads through its
    shadow of the cache.  Last logits and every cache row against the
    oracle's token loop over the same sequence; TALOS_HIP_PFA16=0 runs the
    f32-MFMA attention on the same case."""
    from talos_amd import SynthSpec, GGML_F32, GGML_Q8_0
    if pfa16 is not None:
        monkeypatch.setenv("TALOS_HIP_PFA16", pfa16)
    spec = SynthSpec(n_layer=2, n_head=16, n_head_kv=2, n_embd=1024, n_ff=1024, vocab_size=512,
                     context_length=256, layer_type=GGML_Q8_0, output_type=GGML_Q8_0, embd_type=GGML_F32,
                     seed=61, name="group8_q8")
    rng = np.random.default_rng(62)
    p1 = [int(t) for t in rng.integers(0, spec.vocab_size, 40)]
    p2 = [int(t) for t in rng.integers(0, spec.vocab_size, 70)]
    _step(f"group-8 Q8_0: 40-token prompt, 12 greedy steps, 70-token prompt at 52 (PFA16={pfa16})")
    m = talos.Model.synth(spec)
    _, am = m.prefill(p1, 0)
    toks = [int(t) for t in m.decode_greedy(am, len(p1), 12)]
    fed = p1 + [int(am)] + toks[:11]
    lg, am2 = m.prefill(p2, len(fed))
    seq = fed + p2
    kg, vg = m.kv_read(len(seq))
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    for p, t in enumerate(seq):
        c = ref.forward(t, p)
    kc, vc = ref.get_kv(len(seq))
    d = float(np.abs(lg - c).max())
    dk = float(max(np.abs(kg - kc).max(), np.abs(vg - vc).max()))
    print(f"  last logits max abs {d:.3e}, K/V max abs {dk:.3e}; argmax gpu {am2} cpu {oracle.argmax(c)}",
          flush=True)
    assert d <= 1e-3 and dk <= 1e-3 and am2 == oracle.argmax(c)
    record_parity(f"group8_q8_prefill_after_decode_{'f32attn' if pfa16 else 'f16attn'}", max(d, dk), 1e-3,
                  path="batched_prefill")
    ref.close()
    m.close()


@pytest.mark.parametrize("case", ["q6k_layers", "mixed_formats"])
def test_prefill_q6k_and_mixed_formats(talos, oracle, case):
    """Layer matrices in Q6_K (the f32-MFMA GEMM dequantizing Q6_K), and a
    model whose layer tensors mix F32, Q8_0, Q4_0 and Q6_K (q/k/v and
    gate/up then go out as one GEMM launch per format): a 100-token batched
    prefill's last logits and every cache row against the oracle's token
    loop."""
    from talos_amd import SynthSpec, GGML_F32, GGML_Q6_K
    if case == "q6k_layers":
        spec = SynthSpec(n_layer=2, n_head=8, n_head_kv=2, n_embd=512, n_ff=1024, vocab_size=1024,
                         context_length=256, layer_type=GGML_Q6_K, output_type=GGML_Q6_K, embd_type=GGML_F32,
                         seed=71, name="q6k_layers")
        m = talos.Model.synth(spec)
        vocab = spec.vocab_size
    else:
        shape = dict(embd=256, n_head=4, n_head_kv=2, ff=512, vocab=300, n_layer=2)
        W = MB.normal_model(63, **shape)
        types = {"output.weight": 14, "token_embd.weight": 8}
        for l in range(shape["n_layer"]):
            p = f"blk.{l}."
            types.update({p + "attn_q.weight": 8, p + "attn_k.weight": 2, p + "attn_v.weight": 0,
                          p + "attn_output.weight": 2, p + "ffn_gate.weight": 8, p + "ffn_up.weight": 0,
                          p + "ffn_down.weight": 14})
        m = talos.Model.load_bytes(MB.gguf_bytes(W, ctx=128, types=types, **shape))
        vocab = shape["vocab"]
    n = 100
    prompt = [int(t) for t in np.random.default_rng(72).integers(0, vocab, n)]
    _step(f"{case}: {n}-token prompt")
    lg, am = m.prefill(prompt, 0)
    kg, vg = m.kv_read(n)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    for p, t in enumerate(prompt):
        c = ref.forward(t, p)
    kc, vc = ref.get_kv(n)
    d = float(np.abs(lg - c).max())
    dk = float(max(np.abs(kg - kc).max(), np.abs(vg - vc).max()))
    print(f"  last logits max abs {d:.3e}, K/V max abs {dk:.3e}; argmax gpu {am} cpu {oracle.argmax(c)}", flush=True)
    assert d <= 1e-3 and dk <= 1e-3 and am == oracle.argmax(c)
    record_parity(f"{case}_batched_prefill_{n}", max(d, dk), 1e-3, path="batched_prefill")
    ref.close()
    m.close()


@pytest.mark.parametrize("which,n", [("gqa_q8", 300), ("mistral7b_q4", 40)])
def test_prefill_f32_matrix_cores(talos, oracle, monkeypatch, which, n):
    """TALOS_HIP_PF16=0: the Q4_0 / Q8_0 GEMMs and the attention on the f32
    matrix cores (k_pf_gemm, a separate SwiGLU pass, k_pf_attn) -- the
    fallback of the split-f16 kernels -- against the oracle's token loop."""
    from talos_amd import configs
    monkeypatch.setenv("TALOS_HIP_PF16", "0")
    wl = getattr(configs, which)() if which != "mistral7b_q4" else configs.mistral7b_q4(ctx=128)
    _step(f"{which}: {n}-token prompt on f32 matrix cores")
    m = talos.Model.synth(wl.spec, nthreads=16)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    prompt = [int(t) for t in np.random.default_rng(wl.spec.seed + 5).integers(0, wl.spec.vocab_size, n)]
    lg, am = m.prefill(prompt, 0)
    for p, t in enumerate(prompt):
        c = ref.forward(t, p)
    kg, vg = m.kv_read(n)
    kc, vc = ref.get_kv(n)
    d = float(np.abs(lg - c).max())
    dk = float(max(np.abs(kg - kc).max(), np.abs(vg - vc).max()))
    print(f"  last logits max abs {d:.3e}, K/V max abs {dk:.3e}; argmax gpu {am} cpu {oracle.argmax(c)}", flush=True)
    assert d <= 1e-3 and dk <= 1e-3 and am == oracle.argmax(c)
    record_parity(f"{which}_f32mfma_prefill_{n}", max(d, dk), 1e-3, path="batched_prefill")
    ref.close()
    m.close()


@pytest.mark.parametrize("which,n", [("gqa_q8", 300), ("mistral7b_q4", 40)])
def test_prefill_tiled_weights_bit_identical(talos, oracle, monkeypatch, which, n):
    """The split-f16 GEMMs reading the tiled weight copies (the default) give
    the same bits as reading the row-major matrices (TALOS_HIP_PF_TILED=0):
    each lane loads the same bytes either way.  Both against the oracle's
    token loop as well.  (gqa_q8's down-projection, 1376 columns, has no
    tiled copy: that launch reads the matrix itself in both runs.)"""
    from talos_amd import configs
    wl = getattr(configs, which)() if which != "mistral7b_q4" else configs.mistral7b_q4(ctx=128)
    prompt = [int(t) for t in np.random.default_rng(wl.spec.seed + 7).integers(0, wl.spec.vocab_size, n)]
    monkeypatch.setenv("TALOS_HIP_PF_TILED", "1")
    _step(f"{which}: {n}-token prompt, tiled weight copies")
    m = talos.Model.synth(wl.spec, nthreads=16)
    lt, at = m.prefill(prompt, 0)
    kt, vt = m.kv_read(n)
    lt, kt, vt = lt.copy(), kt.copy(), vt.copy()
    m.close()
    monkeypatch.setenv("TALOS_HIP_PF_TILED", "0")
    _step(f"{which}: {n}-token prompt, row-major weights")
    m = talos.Model.synth(wl.spec, nthreads=16)
    lr, ar = m.prefill(prompt, 0)
    kr, vr = m.kv_read(n)
    assert at == ar
    assert np.array_equal(lt, lr) and np.array_equal(kt, kr) and np.array_equal(vt, vr)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    for p, t in enumerate(prompt):
        c = ref.forward(t, p)
    kc, vc = ref.get_kv(n)
    d = float(np.abs(lt - c).max())
    dk = float(max(np.abs(kt - kc).max(), np.abs(vt - vc).max()))
    print(f"  tiled == row-major bit for bit; last logits max abs {d:.3e}, K/V max abs {dk:.3e}", flush=True)
    assert d <= 1e-3 and dk <= 1e-3 and at == oracle.argmax(c)
    record_parity(f"{which}_tiled_weights_prefill_{n}", max(d, dk), 1e-3, path="batched_prefill")
    ref.close()
    m.close()
