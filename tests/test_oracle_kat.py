"""Known-answer checks that pin the oracle (the CPU restatement of the
reference forward) before it is trusted as the checker.

Sources of the expected values, per test: the reference's own unit tests
(src/math/ops.rs tests, src/math/matmul.rs tests, src/gguf/dtype.rs tests,
src/sample.rs tests, src/math/metal/mod.rs tests), IEEE/f16 facts, closed
forms, and single-element probes of the published GGML block layouts.  Each
is chosen so that a plausible slip (dropped term, swapped index, transposed
nibble order, wrong rounding) fails.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def close(a, b, tol=1e-5):
    assert abs(float(a) - float(b)) < tol, f"expected {b}, got {a}"


# ---- src/math/ops.rs tests ------------------------------------------------

def test_rmsnorm_hand():
    out = O.rmsnorm([1.0, 2.0, 3.0], [1.0, 1.0, 1.0], 0.0)
    s = 1.0 / math.sqrt(14.0 / 3.0)
    for o, x in zip(out, [1.0, 2.0, 3.0]):
        close(o, x * s)


def test_rmsnorm_weighted():
    out = O.rmsnorm([2.0, 0.0], [3.0, 5.0], 0.0)
    close(out[0], 2.0 / math.sqrt(2.0) * 3.0)
    close(out[1], 0.0)


def test_rmsnorm_eps_enters_under_the_root():
    # mean(x^2) = 1; eps = 3 -> scale = 1/sqrt(4) = 0.5 (eps added to the mean,
    # not to the root or the sum).
    out = O.rmsnorm([1.0, -1.0], [1.0, 1.0], 3.0)
    close(out[0], 0.5)
    close(out[1], -0.5)


def test_softmax_known_and_sum():
    x = O.softmax([1.0, 2.0, 3.0])
    close(x.sum(), 1.0)
    den = math.exp(-2) + math.exp(-1) + 1.0
    close(x[0], math.exp(-2) / den)
    close(x[1], math.exp(-1) / den)
    close(x[2], 1.0 / den)


def test_softmax_uniform_and_shift_invariant():
    for v in O.softmax([5.0] * 4):
        close(v, 0.25)
    a = O.softmax([1.0, 2.0, 3.0])
    b = O.softmax([1001.0, 1002.0, 1003.0])  # max-shifted: no overflow
    np.testing.assert_allclose(a, b, atol=1e-6)


def test_silu_and_swiglu():
    close(O.silu(0.0), 0.0)
    close(O.silu(2.0), 2.0 / (1.0 + math.exp(-2.0)))
    close(O.silu(-30.0), -30.0 / (1.0 + math.exp(30.0)), 1e-9)
    out = O.swiglu([0.0, 2.0], [10.0, 3.0])
    close(out[0], 0.0)
    close(out[1], O.silu(2.0) * 3.0)


def test_rope_preserves_pair_norm():
    v = np.arange(8, dtype=np.float32) + 1.0
    r = O.rope(v, 7, 2, 4, 10000.0)
    for h in range(2):
        for i in range(2):
            b = h * 4
            close(r[b + 2 * i] ** 2 + r[b + 2 * i + 1] ** 2, v[b + 2 * i] ** 2 + v[b + 2 * i + 1] ** 2, 1e-4)


def test_rope_pos_zero_identity():
    v = np.arange(18, dtype=np.float32) * 0.5 - 1.0
    np.testing.assert_allclose(O.rope(v, 0, 3, 6, 10000.0), v, atol=1e-6)


def test_rope_closed_form_adjacent_pairs():
    # Pair (2i, 2i+1) of every head turns by pos * base^(-2i/head_dim);
    # elements of other pairs do not move (adjacent-pair convention, not
    # the split-half one).
    hd, pos, base = 8, 5, 10000.0
    for i in range(hd // 2):
        v = np.zeros(2 * hd, np.float32)
        v[hd + 2 * i] = 1.0  # head 1, pair i, x-component
        r = O.rope(v, pos, 2, hd, base)
        ang = pos * base ** (-2.0 * i / hd)
        exp = np.zeros_like(v)
        exp[hd + 2 * i] = math.cos(ang)
        exp[hd + 2 * i + 1] = math.sin(ang)
        np.testing.assert_allclose(r, exp, atol=2e-6)


# ---- src/math/matmul.rs tests ---------------------------------------------

def test_matvec_hand():
    w = np.array([1, 2, 3, 4, 5, 6], np.float32)
    assert O.matvec(O.F32, w, np.array([1, 1], np.float32), 3, 2).tolist() == [3.0, 7.0, 11.0]


@pytest.mark.parametrize("rows,cols", [(8, 8), (5, 13), (13, 5), (7, 100)])
def test_matvec_vs_naive(rows, cols):
    rng = np.random.default_rng(rows * 100 + cols)
    w = rng.uniform(-1, 1, rows * cols).astype(np.float32)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    ref = (w.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64))
    np.testing.assert_allclose(O.matvec(O.F32, w, x, rows, cols), ref, atol=1e-5)
    np.testing.assert_array_equal(O.matvec(O.F32, w, x, rows, cols, nthreads=3),
                                  O.matvec(O.F32, w, x, rows, cols))


# ---- src/sample.rs tests (argmax over f32::total_cmp, ties -> last) --------

def test_argmax_known():
    assert O.argmax([0.1, 9.0, -3.0, 2.0]) == 1


def test_argmax_ties_take_last_index():
    # Iterator::max_by returns the last of equal maxima.
    assert O.argmax([1.0, 3.0, 3.0, 0.0]) == 2
    assert O.argmax([7.0] * 5) == 4


def test_argmax_total_order():
    # total_cmp: -0.0 < +0.0 and NaN (positive) above +inf.
    assert O.argmax([0.0, -0.0]) == 0
    assert O.argmax([-0.0, 0.0]) == 1
    assert O.argmax([np.inf, np.nan, 1.0]) == 1
    assert O.argmax([-np.inf, -1e30]) == 1


# ---- f16 (the `half` crate) -------------------------------------------------

@pytest.mark.parametrize("bits,val", [(0x3C00, 1.0), (0xC000, -2.0), (0x7BFF, 65504.0), (0x0001, 2.0 ** -24),
                                      (0x0400, 2.0 ** -14), (0x3555, 0.333251953125), (0x8000, -0.0)])
def test_f16_known_values(bits, val):
    assert O.f16_to_f32(bits) == val
    assert O.f32_to_f16(val) == bits


def test_f16_special_and_rounding():
    assert math.isinf(O.f16_to_f32(0x7C00)) and O.f16_to_f32(0x7C00) > 0
    assert math.isnan(O.f16_to_f32(0x7E00))
    # round to nearest, ties to even
    assert O.f32_to_f16(1.0 + 2.0 ** -11) == 0x3C00        # tie -> even (down)
    assert O.f32_to_f16(1.0 + 3 * 2.0 ** -11) == 0x3C02    # tie -> even (up)
    assert O.f32_to_f16(1.0 + 2.0 ** -11 + 2.0 ** -20) == 0x3C01
    assert O.f32_to_f16(65520.0) == 0x7C00                  # rounds to inf
    assert O.f32_to_f16(2.0 ** -25) == 0x0000               # tie -> even (zero)
    assert O.f32_to_f16(3 * 2.0 ** -26) == 0x0001


def test_f16_exhaustive_round_trip():
    vals = np.arange(0, 1 << 16, dtype=np.uint32)
    for b in vals[::37]:
        f = O.f16_to_f32(int(b))
        if math.isnan(f):
            continue
        assert O.f32_to_f16(f) == b
        assert f == float(np.uint16(b).view(np.float16))


# ---- src/gguf/dtype.rs tests: dequantize ------------------------------------

def sample_block():
    return np.array([(i - 16.0) * 0.37 + 0.1 for i in range(32)], np.float32)


def test_q8_0_round_trip_dtype_test():
    x = sample_block()
    d = np.float32(np.abs(x).max() / 127.0)
    raw = np.frombuffer(np.float16(d).tobytes(), np.uint8).tolist()
    raw += [int(np.int8(min(max(round_away(np.float32(v / d)), -128), 127))) & 0xFF for v in x]
    out = O.dequantize(O.Q8_0, np.array(raw, np.uint8), 32)
    assert np.all(np.abs(out - x) <= d + 1e-3)


def test_q4_0_round_trip_dtype_test():
    x = sample_block()
    mx = x[np.argmax(np.abs(x))]
    d = np.float32(mx / -8.0)
    idv = np.float32(1.0) / d
    raw = np.frombuffer(np.float16(d).tobytes(), np.uint8).tolist()
    for j in range(16):
        a = min(int(np.float32(x[j] * idv + np.float32(8.5))), 15)
        b = min(int(np.float32(x[j + 16] * idv + np.float32(8.5))), 15)
        raw.append(a | (b << 4))
    out = O.dequantize(O.Q4_0, np.array(raw, np.uint8), 32)
    assert np.all(np.abs(out - x) <= abs(d) + 1e-3)


def test_q8_0_exact_values():
    # d = 0.5 (f16 0x3800); quant bytes are two's complement int8.
    q = np.array([-128, -1, 0, 1, 127] + [3] * 27, np.int8)
    raw = np.concatenate([np.array([0x00, 0x38], np.uint8), q.view(np.uint8)])
    out = O.dequantize(O.Q8_0, raw, 32)
    np.testing.assert_array_equal(out, 0.5 * q.astype(np.float32))


def test_q4_0_nibble_layout():
    # byte j: low nibble -> element j, high nibble -> element j + 16; value
    # d * (nibble - 8).  d = 2.0 (f16 0x4000).
    for j in range(16):
        for hi in (False, True):
            qs = np.full(16, 0x88, np.uint8)  # all nibbles 8 -> 0.0
            qs[j] = (0x8F if not hi else 0xF8)  # one nibble 15 -> +7
            raw = np.concatenate([np.array([0x00, 0x40], np.uint8), qs])
            out = O.dequantize(O.Q4_0, raw, 32)
            exp = np.zeros(32, np.float32)
            exp[j + (16 if hi else 0)] = 14.0
            np.testing.assert_array_equal(out, exp)


def q6k_bytes(ql, qh, sc, d_bits):
    return np.concatenate([ql, qh, sc.view(np.uint8), np.array([d_bits & 0xFF, d_bits >> 8], np.uint8)])


def test_q6_k_single_element_probes():
    # ggml's published Q6_K layout (dequantize_row_q6_K): for half n, l < 32,
    # element n*128 + l + 32k takes low/high nibble of ql[n*64 + l (+32)],
    # bits 2k..2k+1 of qh[n*32 + l], sub-scale sc[n*8 + l/16 + 2k], and
    # value d * sc * (q - 32).  With qh fields = 2 and ql nibbles = 0 every
    # q is 32, i.e. 0.0; each probe raises one quant to 63 (+31).
    sc = np.arange(1, 17, dtype=np.int8)  # distinct sub-scales
    for n in range(2):
        for l in (0, 5, 16, 31):
            for k in range(4):
                ql = np.zeros(128, np.uint8)
                qh = np.full(64, 0xAA, np.uint8)
                byte = n * 64 + l + (32 if k in (1, 3) else 0)
                ql[byte] |= 0x0F if k in (0, 1) else 0xF0
                qh[n * 32 + l] |= 0x3 << (2 * k)
                raw = q6k_bytes(ql, qh, sc, 0x3800)  # d = 0.5
                out = O.dequantize(O.Q6_K, raw, 256)
                e = n * 128 + l + 32 * k
                s = int(sc[n * 8 + l // 16 + 2 * k])
                assert out[e] == 0.5 * s * 31, (n, l, k)
                out[e] = 0.0
                assert not out.any(), (n, l, k)


def test_q6_k_negative_scale_and_bias():
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)  # every q = 0 -> value d * sc * (-32)
    sc = np.full(16, -3, np.int8)
    out = O.dequantize(O.Q6_K, q6k_bytes(ql, qh, sc, 0x3C00), 256)
    np.testing.assert_array_equal(out, np.full(256, 96.0, np.float32))


# ---- quantizers: the reference test quantizers (src/math/metal/mod.rs
# tests quant_q8_0 / quant_q4_0) byte for byte ------------------------------

def round_away(v):
    """f32::round: halves away from zero."""
    return math.copysign(math.floor(abs(float(v)) + 0.5), float(v))


def ref_test_quant_q8_0(block):
    amax = np.float32(np.abs(block).max())
    d = np.float32(amax / np.float32(127.0))
    raw = list(np.frombuffer(np.float16(d).tobytes(), np.uint8))
    for v in block:
        q = min(max(round_away(np.float32(v / d)), -128), 127) if d != 0 else 0.0
        raw.append(int(np.int8(q)) & 0xFF)
    return raw


def ref_test_quant_q4_0(block):
    mx = np.float32(0.0)
    for v in block:
        if abs(v) > abs(mx):
            mx = np.float32(v)
    d = np.float32(mx / np.float32(-8.0))
    idv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
    raw = list(np.frombuffer(np.float16(d).tobytes(), np.uint8))
    for j in range(16):
        a = int(np.clip(int(np.float32(block[j] * idv + np.float32(8.5))), 0, 15))
        b = int(np.clip(int(np.float32(block[j + 16] * idv + np.float32(8.5))), 0, 15))
        raw.append(a | (b << 4))
    return raw


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantizers_match_reference_test_quantizers(seed):
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, 32 * 24).astype(np.float32)
    x[:32] = 0.0  # an all-zero block
    x[32:64] *= 1e-6
    q8 = O.quantize(O.Q8_0, x)
    q4 = O.quantize(O.Q4_0, x)
    exp8 = sum((ref_test_quant_q8_0(x[i:i + 32]) for i in range(0, x.size, 32)), [])
    exp4 = sum((ref_test_quant_q4_0(x[i:i + 32]) for i in range(0, x.size, 32)), [])
    assert q8.tolist() == exp8
    assert q4.tolist() == exp4


def test_q6_k_quantizer_round_trip_bound():
    rng = np.random.default_rng(5)
    x = rng.normal(0, 0.02, 256 * 8).astype(np.float32)
    raw = O.quantize(O.Q6_K, x)
    assert raw.size == 8 * 210
    y = O.dequantize(O.Q6_K, raw, x.size)
    # per 16-element group the step is |d * sc| <= max|x_group| / 31.5 (plus
    # f16 / int8 scale rounding); the error is at most about one step
    for g in range(0, x.size, 16):
        step = np.abs(x[g:g + 16]).max() / 31.0
        assert np.abs(y[g:g + 16] - x[g:g + 16]).max() <= 1.1 * step + 1e-7


# ---- quantized matvec = dequantize then f32 dot (src/math/quant.rs) -------

@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0, O.Q6_K])
def test_quant_matvec_is_dequant_dot(t):
    rng = np.random.default_rng(11)
    rows, cols = 9, 512
    w = rng.uniform(-1, 1, rows * cols).astype(np.float32)
    raw = O.quantize(t, w)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    got = O.matvec(t, raw, x, rows, cols)
    deq = O.dequantize(t, raw, rows * cols).reshape(rows, cols).astype(np.float64)
    np.testing.assert_allclose(got, deq @ x.astype(np.float64), atol=1e-4)
