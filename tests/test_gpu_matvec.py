"""GPU fused dequant-matvec vs the oracle's CPU matvec.

Mirrors the reference's kernel tests (src/math/metal/mod.rs:533-685): random
weights uniform in [-1, 1) quantized with the reference's test quantizers,
Q6_K as random valid super-blocks, the same odd shapes, plus the 4096x4096
and 7B projection shapes.  Bar: |gpu - cpu| <= 1e-4 * max(|cpu|, 1) for F32
and 1e-3 * max(|cpu|, 1) for the block formats (the reference's `close`
uses 1e-3 for all; fp32 accumulation in a different order).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [(64, 128), (200, 256), (1, 64), (129, 32), (333, 32), (3, 768)]


def _close(gpu, cpu, tol):
    err = np.abs(gpu - cpu) / np.maximum(np.abs(cpu), 1.0)
    return float(err.max()) if err.size else 0.0


@pytest.fixture(scope="module")
def backend(talos):
    # The matvec API needs only a context; the model dims are placeholders.
    b = talos.HipBackend(n_layer=1, n_head=1, n_head_kv=1, n_embd=64, n_ff=64, vocab_size=64,
                         context_length=8)
    yield b
    b.close()


def _case(kind, rows, cols):
    print(f"\n[matvec] {kind} rows={rows} cols={cols}", flush=True)


@pytest.mark.parametrize("rows,cols", SHAPES + [(200, 257), (4096, 4096)])
def test_matvec_f32(backend, oracle, rows, cols):
    _case("F32", rows, cols)
    rng = np.random.default_rng(rows * 7919 + cols)
    w = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    gpu = backend.matvec(f"f32.{rows}x{cols}", w, 0, rows, cols, x)
    cpu = oracle.matvec(oracle.F32, w, x, rows, cols)
    assert _close(gpu, cpu, 1e-4) <= 1e-4


@pytest.mark.parametrize("t", ["Q8_0", "Q4_0"])
@pytest.mark.parametrize("rows,cols", [(64, 128), (200, 256), (1, 64), (129, 32), (333, 1376),
                                       (4096, 4096), (1024, 4096), (4096, 14336)])
def test_matvec_q(backend, oracle, t, rows, cols):
    _case(t, rows, cols)
    tag = {"Q8_0": oracle.Q8_0, "Q4_0": oracle.Q4_0}[t]
    rng = np.random.default_rng(rows * 31 + cols + tag)
    w = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    q = oracle.quantize(tag, w)
    gpu = backend.matvec(f"{t}.{rows}x{cols}", q, tag, rows, cols, x)
    cpu = oracle.matvec(tag, q, x, rows, cols, nthreads=8)
    assert _close(gpu, cpu, 1e-3) <= 1e-3


def _random_q6k(rng, rows, cols):
    nsb = rows * cols // 256
    raw = rng.integers(0, 256, (nsb, 210), dtype=np.uint8)
    d = rng.uniform(-0.05, 0.05, nsb).astype(np.float16).view(np.uint16)
    raw[:, 208] = (d & 0xFF).astype(np.uint8)
    raw[:, 209] = (d >> 8).astype(np.uint8)
    return raw.reshape(-1)


@pytest.mark.parametrize("rows,cols", [(64, 256), (200, 512), (1, 256), (3, 768), (32000, 4096)])
def test_matvec_q6k(backend, oracle, rows, cols):
    _case("Q6_K", rows, cols)
    rng = np.random.default_rng(rows + cols)
    raw = _random_q6k(rng, rows, cols)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    gpu = backend.matvec(f"q6k.{rows}x{cols}", raw, oracle.Q6_K, rows, cols, x)
    cpu = oracle.matvec(oracle.Q6_K, raw, x, rows, cols, nthreads=8)
    assert _close(gpu, cpu, 1e-3) <= 1e-3


def test_resident_weight_is_cached(backend, oracle):
    """src/math/metal/mod.rs:602-625: a second upload under the same name and
    byte length must keep serving the first tensor."""
    _case("cache", 64, 128)
    rng = np.random.default_rng(5)
    wa = rng.uniform(-1, 1, (64, 128)).astype(np.float32)
    wb = rng.uniform(-1, 1, (64, 128)).astype(np.float32)
    x = rng.uniform(-1, 1, 128).astype(np.float32)
    cpu_a = oracle.matvec(oracle.F32, wa, x, 64, 128)
    g1 = backend.matvec("cache.key", wa, 0, 64, 128, x)
    g2 = backend.matvec("cache.key", wb, 0, 64, 128, x)
    assert _close(g1, cpu_a, 1e-4) <= 1e-4
    assert _close(g2, cpu_a, 1e-4) <= 1e-4
    # a different byte length under the same name replaces the tensor
    wc = rng.uniform(-1, 1, (32, 128)).astype(np.float32)
    g3 = backend.matvec("cache.key", wc, 0, 32, 128, x)
    assert _close(g3, oracle.matvec(oracle.F32, wc, x, 32, 128), 1e-4) <= 1e-4


def test_matvec_bit_identical_reruns(backend, oracle):
    _case("determinism Q4_0", 4096, 4096)
    rng = np.random.default_rng(11)
    q = oracle.quantize(oracle.Q4_0, rng.normal(0, 0.02, (4096, 4096)).astype(np.float32))
    x = rng.normal(0, 1, 4096).astype(np.float32)
    a = backend.matvec("det.q4", q, oracle.Q4_0, 4096, 4096, x)
    b = backend.matvec("det.q4", q, oracle.Q4_0, 4096, 4096, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_matvec_errors(backend, talos):
    x = np.zeros(64, np.float32)
    with pytest.raises(talos.TalosError) as e:
        backend.matvec("bad.type", np.zeros(64 * 4, np.uint8), 3, 1, 64, x)
    assert e.value.status == "ERR_DTYPE"
    with pytest.raises(talos.TalosError) as e:
        backend.matvec("bad.len", np.zeros(10, np.uint8), 8, 1, 64, x)
    assert e.value.status == "ERR_SHAPE"
    with pytest.raises(talos.TalosError) as e:
        backend.matvec("bad.cols", np.zeros(18, np.uint8), 2, 1, 33, x)
    assert e.value.status == "ERR_SHAPE"
