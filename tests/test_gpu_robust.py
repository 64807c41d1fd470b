"""Failure handling of the persistent kernel, forced from the host.

Every cross-workgroup wait in the persistent decode kernel is bounded.  With
the poll limit cut to one poll (talos_hip_set_spin_limit) the waits give up
at once: the kernel records the error, skips its later barriers, every
workgroup runs to the end, and the step returns TALOS_ERR_HIP.  The next
step with the default limit must start clean: its logits equal, bit for
bit, those of a fresh context at the same position and cache state.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_bounded_waits_give_up_and_recover(talos):
    from talos_amd import configs
    wl = configs.gqa_q8()
    print("\n[robust] gqa_q8: a step with a one-poll wait limit, then recovery", flush=True)
    m = talos.Model.synth(wl.spec)
    m.forward_token(5, 0)
    assert m.path() == "persistent"
    m.set_spin_limit(1)
    with pytest.raises(talos.TalosError) as e:
        m.forward_token(9, 1)
    assert e.value.status == "ERR_HIP"
    with pytest.raises(talos.TalosError) as e:  # a greedy run fails the same way, and drains
        m.decode_greedy(9, 1, 3)
    assert e.value.status == "ERR_HIP"
    m.set_spin_limit(0)
    got = [m.forward_token(t, p)[0] for p, t in ((1, 9), (2, 4), (3, 7))]
    fresh = talos.Model.synth(wl.spec)
    fresh.forward_token(5, 0)
    want = [fresh.forward_token(t, p)[0] for p, t in ((1, 9), (2, 4), (3, 7))]
    for p, (a, b) in enumerate(zip(got, want)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {p + 1} after recovery differs"
    fresh.close()
    m.close()
