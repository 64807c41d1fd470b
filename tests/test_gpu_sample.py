"""Sampling and perplexity on the device against the oracle's restatements
of src/sample.rs:19-76 and src/eval.rs:17-52.

The draws are compared token for token with the oracle on the same logits
and the same uniform draw u.  The device sums in a different (fixed) order
than the reference's sequential f32 sums, so a case whose u * mass or top_p
falls within 1e-5 of a cumulative-probability boundary (float64) is not
compared; such cases are counted and must stay rare.
"""
import numpy as np
import pytest

from tests.conftest import record_parity

pytestmark = pytest.mark.gpu


def _margins(lg, temperature, top_k, top_p, u):
    """float64 distances of top_p and u * mass from the cumulative sums."""
    lg = np.asarray(lg, np.float64)
    order = np.lexsort((-np.arange(lg.size), -lg))  # descending logit, then descending index
    k = lg.size if top_k is None else min(max(top_k, 1), lg.size)
    kept = np.array(order[:k])
    p = np.exp((lg[kept] - lg[kept[0]]) / temperature)
    p /= p.sum()
    cum = np.cumsum(p)
    m = k
    mp = np.inf
    if top_p is not None:
        mp = float(np.min(np.abs(cum - top_p)))
        hit = np.nonzero(cum >= top_p)[0]
        if hit.size:
            m = int(hit[0]) + 1
    r = u * cum[m - 1]
    mu = float(np.min(np.abs(cum[:m] - r)))
    return min(mp, mu)


@pytest.fixture(scope="module")
def backend(talos):
    b = talos.HipBackend(n_layer=1, n_head=2, n_head_kv=1, n_embd=64, n_ff=128, vocab_size=32, context_length=8)
    yield b
    b.close()


def test_device_draws_match_oracle(backend, oracle):
    from tests.hipmem import DeviceBuffer
    rng = np.random.default_rng(31)
    cases = compared = 0
    out = DeviceBuffer(16)
    d = DeviceBuffer(100003 * 4)
    for n in (4, 37, 512, 32000, 100003):
        for sigma in (1.0, 4.0):
            lg = (rng.standard_normal(n) * sigma).astype(np.float32)
            if n == 512:
                lg = (np.round(lg * 2) / 2 + 0.0).astype(np.float32)  # many equal logits (no -0)
            d.upload(lg)
            for temperature in (0.0, 0.7, 1.0, 1.5):
                for top_k in (None, 1, 2, 40, 1000):
                    for top_p in (None, 0.5, 0.9, 1e-6):
                        u = float(rng.random())
                        cases += 1
                        want = oracle.sample(lg, temperature, top_k, top_p, u)
                        if temperature > 0 and _margins(lg, temperature, top_k, top_p, u) < 1e-5:
                            continue
                        backend.sample_dev(d.ptr, n, out.ptr, temperature, top_k, top_p, u)
                        backend.sync()
                        got = int(out.download(np.uint32, 1)[0])
                        compared += 1
                        assert got == want, (f"n {n} sigma {sigma} T {temperature} top_k {top_k} top_p {top_p} "
                                             f"u {u}: device {got} oracle {want}")
    d.free()
    out.free()
    print(f"\n[sample] {compared} of {cases} draws compared (the rest within 1e-5 of a boundary)", flush=True)
    assert compared >= 0.95 * cases


def test_decode_sample_matches_step_by_step(talos, oracle):
    """The device sampled-decode loop equals forward_token + a draw per step
    (the same draws), and each draw equals the oracle's on those logits."""
    from talos_amd import configs
    wl = configs.gqa_q8()
    m = talos.Model.synth(wl.spec)
    u = np.random.default_rng(7).random(24).astype(np.float32)
    T, K, Pp = 0.8, 50, 0.95
    toks = m.decode_sample(11, 0, u, T, K, Pp)
    m.reset()
    tok, checked = 11, 0
    for s in range(24):
        lg, _ = m.forward_token(tok, s)
        nxt = m.sample(T, K, Pp, float(u[s]))
        assert nxt == toks[s], f"step {s}: loop {toks[s]} step-by-step {nxt}"
        if _margins(lg, T, K, Pp, float(u[s])) >= 1e-5:
            assert nxt == oracle.sample(lg, T, K, Pp, float(u[s]))
            checked += 1
        tok = nxt
    assert checked >= 20
    m.close()


@pytest.mark.parametrize("which,n,tol", [("tiny_f32", 300, 1e-4), ("gqa_q8", 80, 1e-3)])
def test_perplexity_matches_oracle(talos, oracle, which, n, tol):
    """Per-position NLLs within the logit tolerance of the model's format,
    perplexity within that relative; tiny_f32's 300 tokens span two chunks
    of its 256-token context."""
    from talos_amd import configs
    wl = getattr(configs, which)()
    m = talos.Model.synth(wl.spec)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=8)
    toks = [int(t) for t in np.random.default_rng(wl.spec.seed + 5).integers(0, wl.spec.vocab_size, n)]
    ppl, nll = m.perplexity(toks)
    rppl, rnll = oracle.perplexity(ref, toks)
    assert len(nll) == len(rnll)
    worst = float(np.abs(nll - np.asarray(rnll, np.float32)).max())
    print(f"\n[ppl] {which}: device {ppl:.5f} oracle {rppl:.5f}, worst NLL diff {worst:.2e}", flush=True)
    assert worst <= tol
    assert abs(ppl - rppl) <= tol * rppl
    record_parity(f"{which}_perplexity_{n}", worst, tol, path=m.path())
    ref.close()
    m.close()


def test_perplexity_of_a_uniform_model_is_the_vocab(talos):
    from tests import models as MB
    shape = dict(embd=64, n_head=4, n_head_kv=2, ff=96, vocab=40, n_layer=1)
    W = MB.uniform_model(3, scale=0.3, norm_offset=1.0, **shape)
    W["output.weight"][:] = 0.0
    m = talos.Model.load_bytes(MB.gguf_bytes(W, ctx=8, **shape))
    toks = [int(t) for t in np.random.default_rng(2).integers(0, 40, 21)]
    ppl, nll = m.perplexity(toks)
    assert nll.size == 18
    assert abs(ppl - 40.0) < 1e-3
    m.close()


def test_sample_errors(talos):
    from talos_amd import configs
    m = talos.Model.synth(configs.tiny_f32().spec)
    m.forward_token(1, 0)
    with pytest.raises(talos.TalosError):
        m.sample(1.0, None, None, 1.5)  # u outside [0, 1)
    with pytest.raises(talos.TalosError):
        m.perplexity([3])
    m.close()
