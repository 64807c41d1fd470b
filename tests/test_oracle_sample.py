"""Pins of the oracle's sampling and perplexity restatements
(src/sample.rs:19-76, src/eval.rs:17-52): the reference's own tests for
these functions, closed forms, and a brute-force check that sweeping the
uniform draw reproduces the softmax distribution of the kept set."""
import math

import numpy as np
import pytest

from oracle import oracle as O

L4 = np.array([0.1, 9.0, -3.0, 2.0], np.float32)


# ---- src/sample.rs tests (the rng draw replaced by swept values of u) ----

def test_argmax_picks_max():
    assert O.argmax(L4) == 1


def test_temp_zero_is_greedy():
    for u in (0.0, 0.3, 0.999):
        assert O.sample(L4, 0.0, None, None, u) == 1


def test_top_k_one_is_greedy():
    for u in np.linspace(0, 0.999, 50):
        assert O.sample(L4, 1.0, 1, None, float(u)) == 1


def test_tiny_top_p_is_greedy():
    for u in np.linspace(0, 0.999, 50):
        assert O.sample(L4, 1.0, None, 1e-6, float(u)) == 1


def test_sampled_token_stays_in_top_k():
    seen = {O.sample(L4, 1.0, 2, None, float(u)) for u in np.linspace(0, 0.9999, 200)}
    assert seen <= {1, 3} and seen == {1, 3}


# ---- closed forms and brute force -----------------------------------------

@pytest.mark.parametrize("temp", [0.5, 1.0, 2.0])
def test_sweeping_u_reproduces_softmax(temp):
    """Over a fine grid of u, token i is drawn for a fraction of the grid
    equal to softmax(l / T)_i (float64 closed form): a wrong temperature
    placement, a dropped normalisation or a reversed order fails it."""
    rng = np.random.default_rng(5)
    lg = rng.normal(0, 1.5, 7).astype(np.float32)
    p = np.exp((lg.astype(np.float64) - lg.max()) / temp)
    p /= p.sum()
    grid = (np.arange(20000) + 0.5) / 20000
    counts = np.bincount([O.sample(lg, temp, None, None, float(u)) for u in grid], minlength=7)
    assert np.abs(counts / grid.size - p).max() < 2e-4


def test_top_p_keeps_the_shortest_prefix():
    """top_p: the kept tokens are exactly the shortest prefix of the sorted
    logits whose probability reaches p (float64 reference, thresholds away
    from the cumulative sums)."""
    rng = np.random.default_rng(9)
    lg = rng.normal(0, 2.0, 50).astype(np.float32)
    order = np.argsort(-lg.astype(np.float64), kind="stable")
    p = np.exp(lg[order].astype(np.float64) - lg.max())
    p /= p.sum()
    cum = np.cumsum(p)
    for top_p in (0.3, 0.6, 0.9):
        m = int(np.searchsorted(cum, top_p) + 1)
        assert min(abs(cum - top_p)) > 1e-4
        seen = {O.sample(lg, 1.0, None, top_p, float(u)) for u in np.linspace(0, 0.99999, 4000)}
        assert seen == set(order[:m].tolist())


def test_ties_order_by_descending_index():
    lg = np.array([1.0, 3.0, 3.0, 0.0], np.float32)
    assert O.sample(lg, 1.0, 1, None, 0.5) == 2  # top-1 of a tie is the last index, as argmax
    assert O.argmax(lg) == 2


# ---- src/eval.rs tests -----------------------------------------------------

def test_uniform_logits_score_ln_vocab():
    lg = np.zeros(50, np.float32)
    for t in (0, 7, 49):
        assert abs(O.token_nll(lg, t) - math.log(50)) < 1e-4


def test_confident_correct_prediction_scores_near_zero():
    lg = np.zeros(16, np.float32)
    lg[5] = 100.0
    assert O.token_nll(lg, 5) < 1e-3


def test_nll_matches_hand_computed_softmax():
    lg = np.array([1.0, 2.0, 3.0], np.float32)
    want = -math.log(math.exp(3) / (math.exp(1) + math.exp(2) + math.exp(3)))
    assert abs(O.token_nll(lg, 2) - want) < 1e-5


def test_perplexity_of_a_uniform_model_is_the_vocab():
    """A model whose output projection is all zero predicts uniformly:
    every NLL is ln V, so the perplexity is V, whatever the tokens and the
    chunking (context 8, 21 tokens: chunks of 8, 8, 5)."""
    from tests import models as MB
    shape = dict(embd=32, n_head=4, n_head_kv=2, ff=48, vocab=40, n_layer=1)
    W = MB.uniform_model(3, scale=0.3, norm_offset=1.0, **shape)
    W["output.weight"][:] = 0.0
    m = O.OracleModel(MB.gguf_bytes(W, ctx=8, **shape))
    toks = [int(t) for t in np.random.default_rng(2).integers(0, 40, 21)]
    ppl, nlls = O.perplexity(m, toks)
    assert len(nlls) == 7 + 7 + 4
    assert abs(ppl - 40.0) < 1e-3
    m.close()
