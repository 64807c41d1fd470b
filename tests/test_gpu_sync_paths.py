"""The persistent kernel's synchronisation variants compute the same bits.

At the 7B shape (Q4_0 layers, Q6_K output) the default decode step
  * lets the attention items wait only for the blocks that produced their
    q, k and v rows, the o-projection staging (short sequences) only for
    the attention item blocks, and each down-projection column quarter only
    for the blocks whose gate/up waves (contiguous runs of row pairs) wrote
    its inputs, and
  * runs the down-projection's column quarters on different workgroups, the
    quarter sums added in quarter order by the next staging.
TALOS_HIP_ATTN_WAIT=0 puts full grid barriers back (and the gate/up pairs
strided over the waves); TALOS_HIP_BAR1=0 makes every grid barrier wait for
block 0's release word instead of reading all arrivals itself;
TALOS_HIP_DSPLIT=1
splits the quarters over the waves of one workgroup, summed in the same
order in LDS.  Neither changes an arithmetic operation or its order, so the
logits and the cache must match the default bit for bit (the default path
itself is checked against the oracle by the parity tests).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(talos, spec, prompt):
    m = talos.Model.synth(spec, nthreads=16)
    try:
        m.reset()
        out = []
        for p, t in enumerate(prompt):
            logits, am = m.forward_token(int(t), p)
            out.append((logits.copy(), am))
        k, v = m.kv_read(len(prompt))
        return out, k, v
    finally:
        m.close()


@pytest.mark.parametrize("direct", [None, "0"], ids=["attn_default", "attn_split"])
def test_sync_variants_bit_identical(talos, monkeypatch, direct):
    """With TALOS_HIP_ATTN_DIRECT=0 in both runs the attention takes its
    split-sequence items at every length, so the producer-only waits of the
    attention slices run together with the gate/up runs and the quarter
    down waits and are compared against full barriers too."""
    from talos_amd import configs
    wl = configs.mistral7b_q4(ctx=256)
    prompt = np.random.default_rng(wl.spec.seed + 11).integers(0, wl.spec.vocab_size, 6).astype(np.uint32)
    if direct is not None:
        monkeypatch.setenv("TALOS_HIP_ATTN_DIRECT", direct)
    print(f"\n[sync] default synchronisation (attention direct={direct})", flush=True)
    base, kb, vb = _run(talos, wl.spec, prompt)
    monkeypatch.setenv("TALOS_HIP_ATTN_WAIT", "0")
    monkeypatch.setenv("TALOS_HIP_DSPLIT", "1")
    monkeypatch.setenv("TALOS_HIP_BAR1", "0")
    print("[sync] two-hop grid barriers, in-workgroup quarter split", flush=True)
    alt, ka, va = _run(talos, wl.spec, prompt)
    for i, ((a, am_a), (b, am_b)) in enumerate(zip(base, alt)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"pos {i}: logits differ"
        assert am_a == am_b
    assert np.array_equal(kb.view(np.uint32), ka.view(np.uint32))
    assert np.array_equal(vb.view(np.uint32), va.view(np.uint32))


def test_whole_down_rows_close(talos, monkeypatch):
    """TALOS_HIP_DSPLIT=0 keeps the down-projection rows whole: the same
    products summed in another order, so the logits agree with the default
    (itself pinned to the oracle) within the quantized tolerance, with the
    same greedy tokens."""
    from talos_amd import configs
    wl = configs.mistral7b_q4(ctx=256)
    prompt = np.random.default_rng(wl.spec.seed + 12).integers(0, wl.spec.vocab_size, 4).astype(np.uint32)
    print("\n[sync] default down-projection", flush=True)
    base, _, _ = _run(talos, wl.spec, prompt)
    monkeypatch.setenv("TALOS_HIP_DSPLIT", "0")
    print("[sync] whole down rows", flush=True)
    alt, _, _ = _run(talos, wl.spec, prompt)
    for i, ((a, am_a), (b, am_b)) in enumerate(zip(base, alt)):
        d = float(np.abs(a - b).max())
        print(f"  pos {i}: max-abs logit diff {d:.3e}", flush=True)
        assert d <= 1e-3
        assert am_a == am_b


def test_cooperative_launch_bit_identical(talos, monkeypatch):
    """TALOS_HIP_COOP=1 sends the same persistent kernel and grid out through
    hipLaunchCooperativeKernel instead of an ordinary launch: the logits and
    the cache must not change by a bit."""
    from talos_amd import configs
    wl = configs.mistral7b_q4(ctx=256)
    prompt = np.random.default_rng(wl.spec.seed + 13).integers(0, wl.spec.vocab_size, 4).astype(np.uint32)
    print("\n[sync] ordinary launch", flush=True)
    base, kb, vb = _run(talos, wl.spec, prompt)
    monkeypatch.setenv("TALOS_HIP_COOP", "1")
    print("[sync] cooperative launch", flush=True)
    alt, ka, va = _run(talos, wl.spec, prompt)
    for i, ((a, am_a), (b, am_b)) in enumerate(zip(base, alt)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"pos {i}: logits differ"
        assert am_a == am_b
    assert np.array_equal(kb.view(np.uint32), ka.view(np.uint32))
    assert np.array_equal(vb.view(np.uint32), va.view(np.uint32))
