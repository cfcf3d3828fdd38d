"""The reference's activation tests (src/test/test_activations.c) for the vector forms this
library exports (silu_inplace, relu_inplace, gelu_inplace, sapphire_geglu; kernels.h
declarations, activations.c:16-156), with the same inputs and bounds. The scalar reference
values come from numpy (SiLU, ReLU) and from the oracle's gelu, which is bit-exact with the
reference's (tests/test_oracle_pin.py)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def f32p(a):
    return a.ctypes.data


def gelu_ref(oracle, v):
    return np.float32(oracle.lib.oracle_gelu(float(v)))


def test_silu_inplace(hip):
    """test_activations.c:44-61 and the large-array test (:239-266)."""
    x = np.array([-2, -1, 0, 1, 2], np.float32)
    hip.silu_inplace(f32p(x), 5)
    v = np.array([-2, -1, 0, 1, 2], np.float32)
    assert np.allclose(x, v / (1 + np.exp(-v)), atol=1e-5)
    n = 10000
    orig = ((np.arange(n) - n // 2) * np.float32(0.01)).astype(np.float32)
    arr = orig.copy()
    hip.silu_inplace(f32p(arr), n)
    assert (np.abs(arr - orig) > 1e-4).sum() > n * 0.6
    assert np.allclose(arr, orig / (1 + np.exp(-orig.astype(np.float64))), rtol=1e-5, atol=1e-6)


def test_relu_inplace(hip):
    """test_activations.c:91-103."""
    x = np.array([-3, -1, 0, 1, 3], np.float32)
    hip.relu_inplace(f32p(x), 5)
    assert np.array_equal(x, np.array([0, 0, 0, 1, 3], np.float32))


def test_gelu_inplace(hip, oracle):
    """test_activations.c:139-155: each element becomes gelu of itself (1e-6)."""
    v = np.array([-2, -1, 0, 1, 2], np.float32)
    x = v.copy()
    hip.gelu_inplace(f32p(x), 5)
    assert abs(x[2]) < 1e-5
    for i in range(5):
        assert abs(x[i] - gelu_ref(oracle, v[i])) < 1e-6


def test_sapphire_geglu(hip, oracle):
    """test_activations.c: basic ([x1 x2 | y1 y2]), against the scalar form over 16 pairs,
    the buffer used as input and output, and 10000 pairs."""
    out = np.zeros(2, np.float32)
    inp = np.array([1, 2, 0, 0.5], np.float32)
    assert hip.sapphire_geglu(f32p(out), f32p(inp), 4) == 0
    assert abs(out[0]) < 1e-4 and abs(out[1] - 2 * gelu_ref(oracle, 0.5)) < 1e-4
    n = 16
    inp = np.concatenate([np.arange(n) * np.float32(0.1), np.arange(n) * np.float32(0.05)]).astype(np.float32)
    out = np.zeros(n, np.float32)
    assert hip.sapphire_geglu(f32p(out), f32p(inp), 2 * n) == 0
    for i in range(n):
        assert abs(out[i] - np.float32(inp[i] * gelu_ref(oracle, inp[n + i]))) < 1e-5
    buf = np.array([1, 2, 0, 0.5], np.float32)
    assert hip.sapphire_geglu(f32p(buf), f32p(buf), 4) == 0
    assert abs(buf[0]) < 1e-4 and abs(buf[1] - 2 * gelu_ref(oracle, 0.5)) < 1e-4
    n = 10000
    g = np.random.default_rng(3)
    inp = g.standard_normal(2 * n).astype(np.float32)
    out = np.zeros(n, np.float32)
    assert hip.sapphire_geglu(f32p(out), f32p(inp), 2 * n) == 0
    ref = np.array([inp[i] * gelu_ref(oracle, inp[n + i]) for i in range(n)], np.float32)
    assert np.all(np.isfinite(out)) and np.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_sapphire_geglu_invalid_inputs(hip):
    """test_activations.c: NULL output or input, size 0 and odd sizes give -1."""
    inp = np.array([1, 2, 3, 4], np.float32)
    out = np.zeros(2, np.float32)
    assert hip.sapphire_geglu(None, f32p(inp), 4) == -1
    assert hip.sapphire_geglu(f32p(out), None, 4) == -1
    assert hip.sapphire_geglu(f32p(out), f32p(inp), 0) == -1
    assert hip.sapphire_geglu(f32p(out), f32p(inp), 3) == -1
