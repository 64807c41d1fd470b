"""The allocation-free sampler (talos_hip_sample_noalloc) against the
workspace sampler it mirrors (talos_hip_sample_dev): the same draws on the
same device logits, over two calls in a row, the second with a smaller
input (the scratch keeps the first call's contents), for greedy,
temperature, top-k and top-p draws; and the size limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_noalloc_sampler_matches_workspace_sampler(talos):
    from tests.hipmem import DeviceBuffer
    b = talos.HipBackend(n_layer=1, n_head=2, n_head_kv=1, n_embd=64, n_ff=128, vocab_size=32, context_length=8)
    rng = np.random.default_rng(77)
    d = DeviceBuffer(131072 * 4)
    out_a, out_b = DeviceBuffer(16), DeviceBuffer(16)
    print("\n[noalloc] two calls per setting, 131072 then 32000 logits", flush=True)
    for temperature, top_k, top_p in ((0.0, None, None), (1.0, None, None), (0.8, 40, None), (1.2, None, 0.9),
                                      (0.7, 1000, 0.5)):
        for n in (131072, 32000):
            lg = (rng.standard_normal(n) * 3).astype(np.float32)
            d.upload(lg)
            u = float(rng.random())
            b.sample_dev(d.ptr, n, out_a.ptr, temperature, top_k, top_p, u)
            b.sample_noalloc(d.ptr, n, out_b.ptr, temperature, top_k, top_p, u)
            b.sync()
            a = int(out_a.download(np.uint32, 1)[0])
            c = int(out_b.download(np.uint32, 1)[0])
            assert a == c, f"T {temperature} k {top_k} p {top_p} n {n}: workspace {a} allocation-free {c}"
            assert 0 <= c < n
    with pytest.raises(talos.TalosError) as e:
        b.sample_noalloc(d.ptr, 131073, out_b.ptr, 1.0)
    assert e.value.status == "ERR_SHAPE"
    d.free()
    out_a.free()
    out_b.free()
    b.close()
