"""The reference's shape domain at the C-ABI boundary.

src/model/llama.rs:45-51 accepts any Llama config whose head_count_kv
divides head_count, and its GPU kernels take any head_dim
(src/math/metal/kernels.metal:165-237).  Every such model must run here,
each through the path the backend picks for it (talos_hip_path):
  * the reference's own GPU contract model (tests/forward_gpu.rs:62-65: c16,
    4 heads, 2 KV heads, head_dim 4, ff 32, vocab 16, 2 layers, ctx 8, every
    tensor uniform in -0.5..0.5, prompt [1, 3, 5, 7, 2, 4]): forward and
    forward_hidden against the oracle at 1e-4, reruns bit-identical
    (tests/forward_gpu.rs:183-190);
  * an odd head_dim with n_embd not a multiple of n_head, and a GQA group of
    12 (generic-shape kernels);
  * a group-8 model (32 q heads over 4 KV heads, head_dim 64) and a model
    whose tensors mix F32, Q8_0, Q4_0 and Q6_K, at 1e-3 with identical greedy
    tokens;
  * the graph path forced (TALOS_HIP_MEGA=0) on the tiny F32 and GQA Q8_0
    benchmark models.
"""
import os

import numpy as np
import pytest

from tests import models as MB
from tests.conftest import record_parity

pytestmark = pytest.mark.gpu


def _step(msg):
    print(f"\n[shapes] {msg}", flush=True)


def _run(talos, oracle, data, prompt, steps, tol, case, hidden=False):
    """Feed prompt then `steps` greedy tokens through the GPU model and the
    oracle; max-abs logits (and hidden state) within tol at every step,
    greedy tokens identical.  Returns (model, the GPU logits per step)."""
    m = talos.Model.load_bytes(data)
    ref = oracle.OracleModel(data, nthreads=8)
    gen, out, worst = [], [], 0.0
    for i in range(len(prompt) + steps):
        tok = prompt[i] if i < len(prompt) else gen[-1]
        g = m.forward_gpu(tok, i)
        c = ref.forward(tok, i)
        d = float(np.abs(g - c).max())
        worst = max(worst, d)
        assert d <= tol, f"{case} step {i}: max abs logit diff {d:.3e} > {tol:.0e}"
        out.append(g)
        if i >= len(prompt) - 1:
            ga, ca = oracle.argmax(g), oracle.argmax(c)
            assert ga == ca, f"{case} step {i}: greedy token gpu {ga} cpu {ca}"
            gen.append(ga)
    if hidden:
        m.reset()
        ref.reset()
        for i, tok in enumerate(prompt):
            gh, ch = m.forward_hidden_gpu(tok, i), ref.forward_hidden(tok, i)
            d = float(np.abs(gh - ch).max())
            worst = max(worst, d)
            assert d <= tol, f"{case} hidden step {i}: {d:.3e}"
    ref.close()
    print(f"  {case}: worst max-abs {worst:.3e} (bar {tol:.0e}), path {m.path()}", flush=True)
    record_parity(case, worst, tol, steps=len(prompt) + steps, path=m.path())
    return m, out


def test_reference_contract_model(talos, oracle):
    shape = dict(embd=16, n_head=4, n_head_kv=2, ff=32, vocab=16, n_layer=2)
    data = MB.gguf_bytes(MB.uniform_model(82, **shape), ctx=8, **shape)
    prompt = [1, 3, 5, 7, 2, 4]
    _step("reference GPU contract model (head_dim 4): forward + forward_hidden, 6 positions")
    m, run1 = _run(talos, oracle, data, prompt, 0, 1e-4, "contract_hd4", hidden=True)
    assert m.path() == "graph_generic"
    m.reset()
    for pos, tok in enumerate(prompt):
        again = m.forward_gpu(tok, pos)
        assert np.array_equal(again.view(np.uint32), run1[pos].view(np.uint32)), f"pos {pos} not bit-identical"
    m.close()


@pytest.mark.parametrize("shape,ctx,steps", [
    (dict(embd=30, n_head=4, n_head_kv=2, ff=40, vocab=24, n_layer=2), 16, 10),
    (dict(embd=96, n_head=12, n_head_kv=1, ff=64, vocab=20, n_layer=2), 96, 80),
], ids=["odd_hd7", "group12"])
def test_generic_shapes(talos, oracle, shape, ctx, steps):
    data = MB.gguf_bytes(MB.uniform_model(7, scale=0.3, norm_offset=1.0, **shape), ctx=ctx, **shape)
    _step(f"generic shape {shape}: 6 + {steps} positions")
    m, _ = _run(talos, oracle, data, [1, 3, 5, 7, 2, 4], steps, 1e-4, f"generic_{shape['embd']}", hidden=True)
    assert m.path() == "graph_generic"
    m.close()


def test_group8_model(talos, oracle):
    """32 q heads over 4 KV heads (head_dim 64), Q4_0 layers, Q8_0 output:
    the graph path with the one-kernel attention at group 8, over 88
    positions (past one attention slice of 64)."""
    shape = dict(embd=2048, n_head=32, n_head_kv=4, ff=2048, vocab=512, n_layer=2)
    W = MB.normal_model(61, **shape)
    types = {n: 2 for n in MB.layer_names(shape["n_layer"])}
    types["output.weight"] = 8
    data = MB.gguf_bytes(W, ctx=128, types=types, **shape)
    _step("group-8 model: 8 + 80 positions")
    m, _ = _run(talos, oracle, data, [11, 3, 400, 7, 99, 4, 250, 17], 80, 1e-3, "group8_q4")
    assert m.path() == "graph"
    m.close()


def test_mixed_format_model(talos, oracle):
    """q Q8_0, k Q4_0, v F32, o Q4_0, gate Q8_0, up F32, down Q6_K, output
    Q6_K, embedding Q8_0: split q/k/v and gate/up on the generic path."""
    shape = dict(embd=256, n_head=4, n_head_kv=2, ff=512, vocab=300, n_layer=2)
    W = MB.normal_model(62, **shape)
    types = {"output.weight": 14, "token_embd.weight": 8}
    for l in range(shape["n_layer"]):
        p = f"blk.{l}."
        types.update({p + "attn_q.weight": 8, p + "attn_k.weight": 2, p + "attn_v.weight": 0,
                      p + "attn_output.weight": 2, p + "ffn_gate.weight": 8, p + "ffn_up.weight": 0,
                      p + "ffn_down.weight": 14})
    data = MB.gguf_bytes(W, ctx=64, types=types, **shape)
    _step("mixed-format model: 8 + 40 positions")
    m, _ = _run(talos, oracle, data, [1, 2, 3, 250, 5, 6, 7, 8], 40, 1e-3, "mixed_formats")
    assert m.path() == "graph_generic"
    m.close()


@pytest.mark.parametrize("which,tol,steps", [("tiny_f32", 1e-4, 64), ("gqa_q8", 1e-3, 256)])
def test_graph_path_forced(talos, oracle, monkeypatch, which, tol, steps):
    """The benchmark models with the persistent kernel off (TALOS_HIP_MEGA=0,
    read when the backend context is created): the ~5-kernel graph."""
    from talos_amd import configs
    monkeypatch.setenv("TALOS_HIP_MEGA", "0")
    wl = getattr(configs, which)()
    _step(f"{which} on the graph path: {wl.prompt_len} + {steps}")
    m = talos.Model.synth(wl.spec)
    ref = oracle.OracleModel(m.gguf_view(), nthreads=8)
    prompt = [int(t) for t in np.random.default_rng(wl.spec.seed + 1).integers(0, wl.spec.vocab_size,
                                                                                  wl.prompt_len)]
    gen, worst = [], 0.0
    for i in range(wl.prompt_len + steps):
        tok = prompt[i] if i < wl.prompt_len else gen[-1]
        g = m.forward_gpu(tok, i)
        c = ref.forward(tok, i)
        d = float(np.abs(g - c).max())
        worst = max(worst, d)
        assert d <= tol, f"{which} step {i}: {d:.3e}"
        if i >= wl.prompt_len - 1:
            assert oracle.argmax(g) == oracle.argmax(c), f"{which} step {i}: greedy token differs"
            gen.append(oracle.argmax(g))
    assert m.path() == "graph"
    print(f"  {which} graph path: worst max-abs {worst:.3e}", flush=True)
    record_parity(f"{which}_graph_path", worst, tol, steps=wl.prompt_len + steps, path="graph")
    ref.close()
    m.close()


def test_path_reported_for_benchmark_models(talos):
    from talos_amd import configs
    m = talos.Model.synth(configs.tiny_f32().spec)
    m.forward_token(1, 0)
    assert m.path() == "persistent"
    m.close()
