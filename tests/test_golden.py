"""The stored fixtures of tests/golden (written by make_fixtures.py with the
oracle): the oracle must reproduce them bit for bit (CPU), and the HIP path
must meet them within the logit tolerance with identical greedy tokens
(GPU)."""
import json
import os

import numpy as np
import pytest

import talos_amd as T
from oracle import oracle as O
from talos_amd import configs

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(HERE, name)) as f:
        return json.load(f)


def oracle_greedy(m, prompt, n):
    for p, t in enumerate(prompt):
        lg = m.forward(t, p)
    last = lg.copy()
    toks, tok = [], O.argmax(lg)
    for i in range(n):
        toks.append(int(tok))
        lg = m.forward(tok, len(prompt) + i)
        tok = O.argmax(lg)
    return last, toks


def test_oracle_reproduces_tiny_f32_fixture(talos):
    fx = load("tiny_f32.json")
    m = O.OracleModel(T.synth_bytes(configs.tiny_f32().spec, nthreads=4), nthreads=2)
    last, toks = oracle_greedy(m, fx["prompt"], len(fx["greedy"]))
    m.close()
    np.testing.assert_array_equal(last, np.array(fx["last_logits"], np.float32))
    assert toks == fx["greedy"]


def test_oracle_reproduces_gqa_q8_fixture(talos):
    fx = load("gqa_q8.json")
    m = O.OracleModel(T.synth_bytes(configs.gqa_q8().spec, nthreads=4), nthreads=4)
    last, toks = oracle_greedy(m, fx["prompt"], len(fx["greedy"]))
    m.close()
    np.testing.assert_array_equal(last[:64], np.array(fx["last_logits_head"], np.float32))
    assert O.argmax(last) == fx["last_argmax"]
    assert toks == fx["greedy"]


@pytest.mark.gpu
def test_gpu_meets_tiny_f32_fixture(talos):
    fx = load("tiny_f32.json")
    m = T.Model.synth(configs.tiny_f32().spec)
    for p, t in enumerate(fx["prompt"]):
        lg = m.forward_gpu(t, p)
    d = float(np.abs(lg - np.array(fx["last_logits"], np.float32)).max())
    assert d <= 1e-4, f"max abs logit diff {d} (F32 tolerance 1e-4)"
    toks = m.decode_greedy(O.argmax(lg), len(fx["prompt"]), len(fx["greedy"]) - 1)
    assert [O.argmax(lg)] + [int(x) for x in toks] == fx["greedy"]
    m.close()


@pytest.mark.gpu
def test_gpu_meets_gqa_q8_fixture(talos):
    fx = load("gqa_q8.json")
    m = T.Model.synth(configs.gqa_q8().spec)
    am = None
    for p, t in enumerate(fx["prompt"]):
        lg, am = m.forward_token(t, p)
    d = float(np.abs(lg[:64] - np.array(fx["last_logits_head"], np.float32)).max())
    assert d <= 1e-3, f"max abs logit diff {d} (quantized tolerance 1e-3)"
    assert am == fx["last_argmax"]
    toks = m.decode_greedy(am, len(fx["prompt"]), len(fx["greedy"]) - 1)
    assert [int(am)] + [int(x) for x in toks] == fx["greedy"]
    m.close()
