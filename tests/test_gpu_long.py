"""Prompt feed on the device and long-context decode.

The reference fills its cache with one Model::step per prompt token
(src/main.rs:88-94).  talos_hip_prefill runs that loop with the tokens fed
on the device (TALOS_HIP_BATCH=0, and any shape the batched kernels do not
take), which must equal a host loop of forward_token bit for bit (logits and
cache); by default it processes the prompt in batches on the matrix cores,
which must agree with that loop and with the oracle within the quantized
tolerance.

Long context (7B shape, every matrix Q8_0, cache 16384 + 64 positions): the
oracle cannot fill 16384 positions in test time, because its attention is a
serial loop (src/model/llama.rs:139-155).  So a seeded 16384-position K/V
state is written into both the GPU cache (talos_hip_kv_write) and the
oracle's (tor_model_set_kv).  Decode steps from position 16384 are then
compared: logits max-abs <= 1e-3 and greedy tokens identical.  At full size
the device greedy loop must also be bit-identical across reruns, and the
cache must read back exactly what was written.
"""
import numpy as np
import pytest

from tests.conftest import record_parity

pytestmark = pytest.mark.gpu

TOL_Q = 1e-3  # quantized formats: max-abs on logits


def _step(msg):
    print(f"\n[long] {msg}", flush=True)


def _prompt(seed, n, vocab):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.uint32)


@pytest.fixture(scope="module")
def gqa(talos, oracle):
    from talos_amd import configs
    wl = configs.gqa_q8()
    m = talos.Model.synth(wl.spec)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=8)
    yield wl, m, ref
    ref.close()
    m.close()


def test_prefill_equals_token_loop(gqa, talos, oracle, monkeypatch):
    """Device-fed prompt (one step per token) == host loop of forward_token,
    bit for bit; the batched prefill and the oracle's prompt loop within
    1e-3 of it; the first greedy token agrees."""
    wl, m, ref = gqa
    prompt = _prompt(wl.spec.seed + 7, wl.prompt_len, wl.spec.vocab_size)
    n = len(prompt)
    _step(f"gqa_q8 host forward_token loop over a {n}-token prompt")
    m.reset()
    host = None
    for p, t in enumerate(prompt):
        host, am_host = m.forward_token(int(t), p)
    k_host, v_host = m.kv_read(n)
    _step("gqa_q8 device token-by-token prefill of the same prompt")
    monkeypatch.setenv("TALOS_HIP_BATCH", "0")
    m1 = talos.Model.synth(wl.spec)
    dev, am_dev = m1.prefill(prompt, 0)
    k_dev, v_dev = m1.kv_read(n)
    m1.close()
    assert np.array_equal(dev.view(np.uint32), host.view(np.uint32))
    assert am_dev == am_host == oracle.argmax(dev)
    assert np.array_equal(k_dev.view(np.uint32), k_host.view(np.uint32))
    assert np.array_equal(v_dev.view(np.uint32), v_host.view(np.uint32))
    _step("gqa_q8 batched prefill of the same prompt")
    m.reset()
    bat, am_bat = m.prefill(prompt, 0)
    k_bat, v_bat = m.kv_read(n)
    db = float(max(np.abs(bat - host).max(), np.abs(k_bat - k_host).max(), np.abs(v_bat - v_host).max()))
    print(f"  batched vs token loop max-abs {db:.3e}", flush=True)
    assert db <= TOL_Q and am_bat == am_host
    _step("gqa_q8 prefill vs the oracle's prompt loop")
    ref.reset()
    for p, t in enumerate(prompt):
        c = ref.forward(int(t), p)
    d = float(np.abs(dev - c).max())
    print(f"  max-abs logit diff {d:.3e}", flush=True)
    assert d <= TOL_Q
    assert oracle.argmax(c) == am_dev


def test_prefill_then_greedy_continues(gqa, oracle):
    """prefill(prompt[:k]) then prefill(prompt[k:], pos=k) == one prefill,
    and decode_greedy from the result matches the host-driven greedy loop."""
    wl, m, ref = gqa
    prompt = _prompt(wl.spec.seed + 8, 12, wl.spec.vocab_size)
    m.reset()
    whole, am = m.prefill(prompt, 0)
    m.reset()
    m.prefill(prompt[:5], 0, want_logits=False)
    split, am2 = m.prefill(prompt[5:], 5)
    assert np.array_equal(whole.view(np.uint32), split.view(np.uint32)) and am == am2
    toks = m.decode_greedy(am, len(prompt), 8)
    m.reset()
    m.prefill(prompt, 0, want_logits=False)
    tok, want = am, []
    for p in range(len(prompt), len(prompt) + 8):
        _, tok = m.forward_token(tok, p, want_logits=False)
        want.append(tok)
    assert list(toks) == want


def test_prefill_errors(gqa, talos):
    wl, m, ref = gqa
    V, ctx = wl.spec.vocab_size, wl.spec.context_length
    with pytest.raises(talos.TalosError) as e:
        m.prefill(np.array([1, V, 2], np.uint32), 0)
    assert e.value.status == "ERR_TOKEN"
    with pytest.raises(talos.TalosError) as e:
        m.prefill(np.array([1, 2, 3], np.uint32), ctx - 2)
    assert e.value.status == "ERR_POS"
    # a full-context feed is in bounds (the last fed token sits at ctx - 1)
    out, am = m.prefill(np.ones(4, np.uint32), ctx - 4)
    assert np.isfinite(out).all() and 0 <= am < V
    empty, am0 = m.prefill(np.zeros(0, np.uint32), 0, want_logits=False)
    assert am0 == 0


@pytest.fixture(scope="module")
def long_q8(talos, oracle):
    from talos_amd import configs
    wl = configs.mistral7b_q8_long()
    _step(f"mistral7b_q8_long synth (7.6 GB), cache {wl.spec.context_length} positions")
    m = talos.Model.synth(wl.spec, nthreads=16)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=16)
    yield wl, m, ref
    ref.close()
    m.close()


def test_long_q8_short_prompt_parity(long_q8, oracle):
    """The 7B-shape Q8_0 model from position 0: a 4-token prompt fed on the
    device, then 4 greedy steps, against the oracle step by step."""
    wl, m, ref = long_q8
    prompt = _prompt(wl.spec.seed + 5, 4, wl.spec.vocab_size)
    _step("mistral7b_q8 4-token prompt + 4 greedy steps vs the oracle")
    m.reset()
    ref.reset()
    g, tok = m.prefill(prompt, 0)
    for p, t in enumerate(prompt):
        c = ref.forward(int(t), p)
    worst = 0.0
    for s in range(5):
        d = float(np.abs(g - c).max())
        worst = max(worst, d)
        print(f"  pos {len(prompt) - 1 + s}: max-abs logit diff {d:.3e}", flush=True)
        assert d <= TOL_Q
        assert tok == oracle.argmax(c)
        if s == 4:
            record_parity("mistral7b_q8_4+4_batched_prefill", worst, TOL_Q, steps=8, path=m.path())
            break
        pos = len(prompt) + s
        g, nxt = m.forward_token(tok, pos)
        c = ref.forward(tok, pos)
        tok = nxt


def _seeded_kv(spec, n_pos, seed):
    """K and V of n_pos positions, [layer, pos, kv_dim].  The scale 1.28 is
    the standard deviation of a k/v projection of a unit-RMS input through
    N(0, 0.02) weights of 4096 columns (0.02 * sqrt(4096))."""
    rng = np.random.default_rng(seed)
    shape = (spec.n_layer, n_pos, spec.kv_dim)
    k = rng.standard_normal(shape, dtype=np.float32)
    k *= np.float32(1.28)
    v = rng.standard_normal(shape, dtype=np.float32)
    v *= np.float32(1.28)
    return k, v


def test_long_context_decode_parity(long_q8, oracle):
    wl, m, ref = long_q8
    P = wl.prompt_len  # 16384 cached positions
    _step(f"seeded K/V state of {P} positions into the GPU cache and the oracle")
    k, v = _seeded_kv(wl.spec, P, wl.spec.seed + 3)
    m.kv_write(k, v)
    ref.set_kv(k, v)
    _step("cache read-back (every layer, every position)")
    k2, v2 = m.kv_read(P)
    assert np.array_equal(k2.view(np.uint32), k.view(np.uint32))
    assert np.array_equal(v2.view(np.uint32), v.view(np.uint32))
    del k2, v2, k, v
    tok, worst, greedy = int(_prompt(wl.spec.seed + 4, 1, wl.spec.vocab_size)[0]), 0.0, []
    for s in range(3):
        pos = P + s
        _step(f"decode step at pos {pos}: GPU vs oracle")
        g, ga = m.forward_token(tok, pos)
        c = ref.forward(tok, pos)
        d = float(np.abs(g - c).max())
        worst = max(worst, d)
        ca = oracle.argmax(c)
        print(f"  max-abs logit diff {d:.3e}; argmax gpu {ga} cpu {ca}", flush=True)
        assert d <= TOL_Q, f"pos {pos}: max abs logit diff {d:.3e}"
        assert ga == ca
        greedy.append(ga)
        tok = ga
    print(f"  worst {worst:.3e}", flush=True)
    record_parity("mistral7b_q8_16k_seeded_kv_3_steps", worst, TOL_Q, steps=3, path=m.path())
    # The device greedy loop over the 64 steps of the workload, twice:
    # bit-identical reruns, and its first steps are the oracle's greedy tokens.
    _step(f"decode_greedy {wl.decode_steps} steps from pos {P}, twice")
    first = int(_prompt(wl.spec.seed + 4, 1, wl.spec.vocab_size)[0])
    a = m.decode_greedy(first, P, wl.decode_steps)
    b = m.decode_greedy(first, P, wl.decode_steps)
    assert list(a) == list(b)
    assert list(a[:3]) == greedy
