"""Whole-token GPU forward vs the oracle's CPU forward.

The reference's contract for this path is tests/forward_gpu.rs: the GPU
forward matches the CPU forward over a multi-token GQA sequence and two GPU
runs are bit-identical.  Here, on seeded synthetic models of the benchmark
shapes:
  * logits max-abs <= 1e-4 (F32 model) / 1e-3 (quantized models) at every
    step, hidden state likewise for forward_hidden;
  * greedy tokens identical to the CPU's (argmax, ties to the last index);
  * reruns bit-identical; the device-side embedding/argmax path gives the
    same logits as the host-embedding path.
"""
import numpy as np
import pytest

from tests import models as MB
from tests.conftest import record_parity

pytestmark = pytest.mark.gpu


def _step(msg):
    print(f"\n[forward] {msg}", flush=True)


def _prompt(seed, n, vocab):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


def _parity(model, ref, prompt, steps, tol):
    """Feed the prompt, then `steps` greedy tokens, through both the GPU model
    and the CPU oracle.  Returns the GPU logits of every forward and the
    generated tokens (the feed sequence is prompt + generated)."""
    from oracle import oracle as O
    model.reset()
    ref.reset()
    gen, all_logits, worst = [], [], 0.0
    n = len(prompt) + steps
    for i in range(n):
        tok = prompt[i] if i < len(prompt) else gen[i - len(prompt)]
        g = model.forward_gpu(tok, i)
        c = ref.forward(tok, i)
        d = float(np.abs(g - c).max())
        worst = max(worst, d)
        assert d <= tol, f"step {i}: max abs logit diff {d:.3e} > {tol:.0e}"
        if i >= len(prompt) - 1:
            ga, ca = O.argmax(g), O.argmax(c)
            assert ga == ca, f"greedy token differs after step {i}: gpu {ga} cpu {ca}"
            if len(gen) < steps:
                gen.append(ga)
        all_logits.append(g)
    print(f"  worst max-abs logit diff {worst:.3e}", flush=True)
    _parity.worst = worst
    return all_logits, gen


@pytest.fixture(scope="module")
def tiny(talos, oracle):
    from talos_amd import configs
    wl = configs.tiny_f32()
    m = talos.Model.synth(wl.spec)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=8)
    yield wl, m, ref
    ref.close()
    m.close()


def test_tiny_f32_parity_and_greedy(tiny):
    wl, m, ref = tiny
    _step("tiny_f32 8-token prompt + 64 greedy steps")
    prompt = _prompt(wl.spec.seed + 1, wl.prompt_len, wl.spec.vocab_size)
    logits, gen = _parity(m, ref, prompt, wl.decode_steps, 1e-4)
    assert len(gen) == wl.decode_steps
    record_parity("tiny_f32_8+64", _parity.worst, 1e-4, steps=wl.prompt_len + wl.decode_steps, path=m.path())
    # Determinism (tests/forward_gpu.rs:183-190): rerun, bit-identical logits.
    _step("tiny_f32 rerun determinism")
    m.reset()
    pos = 0
    for i, tok in enumerate(prompt + gen):
        again = m.forward_gpu(tok, pos)
        assert np.array_equal(again.view(np.uint32), logits[i].view(np.uint32)), f"step {i} not bit-identical"
        pos += 1


def test_tiny_f32_hidden(tiny):
    wl, m, ref = tiny
    _step("tiny_f32 forward_hidden")
    m.reset()
    ref.reset()
    for pos, tok in enumerate([1, 3, 5, 7, 2, 4]):
        g = m.forward_hidden_gpu(tok, pos)
        c = ref.forward_hidden(tok, pos)
        assert float(np.abs(g - c).max()) <= 1e-4


def test_tiny_device_token_path(tiny, oracle):
    wl, m, ref = tiny
    _step("tiny_f32 device embedding + argmax vs host path")
    prompt = [5, 9, 2, 6]
    m.reset()
    host = [m.forward_gpu(t, p) for p, t in enumerate(prompt)]
    m.reset()
    for p, t in enumerate(prompt):
        dev, am = m.forward_token(t, p)
        assert np.array_equal(dev.view(np.uint32), host[p].view(np.uint32))
        assert am == oracle.argmax(host[p])
    # greedy loop on the device == host-driven greedy loop
    _step("tiny_f32 decode_greedy vs host greedy")
    start = oracle.argmax(host[-1])
    toks = m.decode_greedy(start, len(prompt), 16)
    m.reset()
    for p, t in enumerate(prompt):
        m.forward_gpu(t, p)
    tok, pos, want = start, len(prompt), []
    for _ in range(16):
        lg = m.forward_gpu(tok, pos)
        tok = oracle.argmax(lg)
        want.append(tok)
        pos += 1
    assert list(toks) == want


def test_tiny_errors(tiny, talos):
    wl, m, ref = tiny
    with pytest.raises(talos.TalosError) as e:
        m.forward_gpu(1, wl.spec.context_length)
    assert e.value.status == "ERR_POS"
    with pytest.raises(talos.TalosError) as e:
        m.forward_gpu(wl.spec.vocab_size, 0)
    assert e.value.status == "ERR_TOKEN"
    with pytest.raises(talos.TalosError) as e:
        m.decode_greedy(1, wl.spec.context_length - 2, 4)
    assert e.value.status == "ERR_POS"


def test_backend_missing_weight(talos):
    b = talos.HipBackend(n_layer=1, n_head=2, n_head_kv=1, n_embd=64, n_ff=128, vocab_size=32,
                         context_length=8)
    with pytest.raises(talos.TalosError) as e:
        b.forward(np.zeros(64, np.float32), 0)
    assert e.value.status == "ERR_MISSING_WEIGHT"
    b.close()


def test_gqa_q8_parity(talos, oracle):
    from talos_amd import configs
    wl = configs.gqa_q8()
    _step("gqa_q8 16-token prompt + 256 greedy steps")
    m = talos.Model.synth(wl.spec)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=8)
    prompt = _prompt(wl.spec.seed + 1, wl.prompt_len, wl.spec.vocab_size)
    _parity(m, ref, prompt, wl.decode_steps, 1e-3)
    record_parity("gqa_q8_16+256", _parity.worst, 1e-3, steps=wl.prompt_len + wl.decode_steps, path=m.path())
    ref.close()
    m.close()


@pytest.mark.parametrize("mega", ["1", "0"], ids=["persistent", "graph"])
def test_argmax_tie_goes_to_last_index(talos, oracle, monkeypatch, mega):
    """src/sample.rs:7-14: ties return the last index.  output.weight rows 100
    and 300 are the same bytes, 4 x the step's hidden state, so their logits
    tie exactly and are the largest; the device argmax (and the greedy loop
    it feeds) must pick 300, as the oracle does."""
    monkeypatch.setenv("TALOS_HIP_MEGA", mega)
    shape = dict(embd=512, n_head=8, n_head_kv=2, ff=1376, vocab=512, n_layer=2)
    W = MB.normal_model(71, **shape)
    base = MB.gguf_bytes(W, ctx=64, default_type=8, **shape)
    ref = oracle.OracleModel(base, nthreads=8)
    h = ref.forward_hidden(17, 0)
    ref.close()
    W["output.weight"][100] = 4.0 * h
    W["output.weight"][300] = 4.0 * h
    data = MB.gguf_bytes(W, ctx=64, default_type=8, **shape)
    ref = oracle.OracleModel(data, nthreads=8)
    m = talos.Model.load_bytes(data)
    lg, am = m.forward_token(17, 0)
    assert m.path() == ("persistent" if mega == "1" else "graph")
    assert lg[100] == lg[300] and lg[300] == lg.max(), "the two rows must tie at the maximum"
    c = ref.forward(17, 0)
    assert oracle.argmax(c) == 300
    assert am == 300, f"device argmax {am}, ties go to the last index (300)"
    # the greedy loop's first token comes from the same device argmax
    m.reset()
    toks = m.decode_greedy(17, 0, 1)
    assert int(toks[0]) == 300
    ref.close()
    m.close()


@pytest.mark.timeout(900)
def test_mistral7b_q4_headline_workload(talos, oracle):
    """The headline workload itself: the 7B-shape Q4_0 model (output Q6_K),
    KV sized to ctx 4096, a random 32-token prompt and 128 greedy steps,
    every step's logits within 1e-3 of the oracle's and the greedy tokens
    identical (the oracle's 160 forwards take about a minute on 16 threads).
    At a divergence the top-2 gap of the oracle's logits is printed."""
    from talos_amd import configs
    from oracle import oracle as O
    wl = configs.mistral7b_q4(ctx=4096)
    _step("mistral7b_q4 (ctx 4096) synth for the 32 + 128 headline run")
    m = talos.Model.synth(wl.spec, nthreads=16)
    ref = O.OracleModel(m.gguf_view(), nthreads=16)
    prompt = _prompt(wl.spec.seed + 1, wl.prompt_len, wl.spec.vocab_size)
    gen, worst = [], 0.0
    for i in range(wl.prompt_len + wl.decode_steps):
        tok = prompt[i] if i < wl.prompt_len else gen[-1]
        g, am = m.forward_token(tok, i)
        c = ref.forward(tok, i)
        d = float(np.abs(g - c).max())
        worst = max(worst, d)
        if i % 16 == 0:
            print(f"  step {i}: max abs {d:.3e} (worst {worst:.3e})", flush=True)
        top2 = np.sort(c)[-2:]
        assert d <= 1e-3, f"step {i}: max abs logit diff {d:.3e} > 1e-3 (oracle top-2 gap {top2[1] - top2[0]:.3e})"
        if i >= wl.prompt_len - 1:
            ca = O.argmax(c)
            assert am == ca, f"step {i}: greedy gpu {am} cpu {ca}, oracle top-2 gap {top2[1] - top2[0]:.3e}"
            gen.append(am)
    assert len(gen) == wl.decode_steps + 1
    print(f"  headline 32 + 128: worst max-abs {worst:.3e}", flush=True)
    record_parity("mistral7b_q4_32+128_ctx4096", worst, 1e-3, steps=wl.prompt_len + wl.decode_steps,
                  path=m.path())
    ref.close()
    m.close()


def test_mistral7b_q4_short_parity(talos, oracle):
    """The 7B-shape Q4_0 model (output Q6_K): 4-token prompt + 4 greedy steps
    against the CPU forward (the full 32+128 run is compared by token
    sequence in the benchmark's own check)."""
    from talos_amd import configs
    wl = configs.mistral7b_q4(ctx=256)
    _step("mistral7b_q4 synth (4 GB)")
    m = talos.Model.synth(wl.spec, nthreads=16)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    prompt = _prompt(wl.spec.seed + 1, 4, wl.spec.vocab_size)
    _step("mistral7b_q4 parity 4 + 4")
    _parity(m, ref, prompt, 4, 1e-3)
    record_parity("mistral7b_q4_4+4_ctx256", _parity.worst, 1e-3, steps=8, path=m.path())
    ref.close()
    m.close()


def test_mistral7b_q4_matrix_core_parity(talos, oracle, monkeypatch):
    """The same 7B-shape parity with the layer matvecs of the persistent
    kernel on the matrix cores (TALOS_HIP_MFMA=1, read when the backend
    context is created)."""
    from talos_amd import configs
    monkeypatch.setenv("TALOS_HIP_MFMA", "1")
    wl = configs.mistral7b_q4(ctx=256)
    _step("mistral7b_q4 synth for the matrix-core path")
    m = talos.Model.synth(wl.spec, nthreads=16)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    prompt = _prompt(wl.spec.seed + 2, 4, wl.spec.vocab_size)
    _step("mistral7b_q4 matrix-core parity 4 + 4")
    _parity(m, ref, prompt, 4, 1e-3)
    record_parity("mistral7b_q4_4+4_matrix_cores", _parity.worst, 1e-3, steps=8, path=m.path())
    ref.close()
    m.close()


def test_gqa_q8_f32_x_parity(talos, oracle, monkeypatch):
    """The vector-ALU layer matvecs with f32 x (TALOS_HIP_DOT4=0, read when
    the backend context is created) instead of the default int8-plane x, and
    split-sequence attention at every length (TALOS_HIP_ATTN_DIRECT=0)."""
    from talos_amd import configs
    monkeypatch.setenv("TALOS_HIP_DOT4", "0")
    monkeypatch.setenv("TALOS_HIP_ATTN_DIRECT", "0")
    wl = configs.gqa_q8()
    _step("gqa_q8 with f32 x: 16-token prompt + 32 greedy steps")
    m = talos.Model.synth(wl.spec)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=8)
    prompt = _prompt(wl.spec.seed + 3, wl.prompt_len, wl.spec.vocab_size)
    _parity(m, ref, prompt, 32, 1e-3)
    record_parity("gqa_q8_16+32_f32_x_split_attention", _parity.worst, 1e-3, steps=wl.prompt_len + 32,
                  path=m.path())
    ref.close()
    m.close()
