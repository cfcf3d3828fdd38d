"""The reference's own tensor-GEMV tests (src/test/test_tensor_gemv.c), run against this
library: the same tensors, inputs, calls and expected values, through kernels.h / tensor.h
(tensor_gemv_* are the legacy macro names of kernel_*, kernels.h:228-238)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32 = 0


def f32p(a):
    return a.ctypes.data


@pytest.fixture
def ctx(hip):
    c = hip.kernel_ctx_create(0, 1024)
    assert c and hip.kernel_ctx_init(c) == 0
    yield c
    hip.kernel_ctx_destroy(c)


def matrix(hip, rows, cols, values):
    A = hip.tensor_create(2, (C.c_int * 2)(rows, cols), F32)
    assert A
    for i, v in enumerate(values):
        assert hip.tensor_set_f32(A, i, float(v)) == 0
    return A


def test_f32_basic(hip, ctx):
    """test_tensor_gemv.c:17-61: A = [[1..4],[5..8],[9..12]], x = 1 -> [10, 26, 42]."""
    A = matrix(hip, 3, 4, range(1, 13))
    x = np.ones(4, np.float32)
    y = np.zeros(3, np.float32)
    assert hip.kernel_gemv(ctx, f32p(y), A, f32p(x)) == 0
    assert np.allclose(y, [10, 26, 42], atol=1e-5)
    hip.tensor_release(A)


def test_f32_random(hip, ctx):
    """test_tensor_gemv.c:63-108: A[i] = (i % 7) * 0.1, x[j] = (j % 5) * 0.2; row 0 checked
    against the sequential sum the test forms with tensor_get_f32."""
    m, n = 16, 32
    A = matrix(hip, m, n, [np.float32(i % 7) * np.float32(0.1) for i in range(m * n)])
    x = np.array([np.float32(j % 5) * np.float32(0.2) for j in range(n)], np.float32)
    y = np.zeros(m, np.float32)
    assert hip.kernel_gemv(ctx, f32p(y), A, f32p(x)) == 0
    e0 = np.float32(0)
    for j in range(n):
        e0 = np.float32(e0 + np.float32(hip.tensor_get_f32(A, j)) * x[j])
    assert abs(y[0] - e0) < 1e-4
    hip.tensor_release(A)


def test_tensor_wrapper(hip, ctx):
    """test_tensor_gemv.c:113-156: kernel_gemv_tensor with A = 2, x = 1 (4 x 5) -> 10."""
    A = matrix(hip, 4, 5, [2.0] * 20)
    x = hip.tensor_create(1, (C.c_int * 1)(5), F32)
    y = hip.tensor_create(1, (C.c_int * 1)(4), F32)
    for i in range(5):
        hip.tensor_set_f32(x, i, 1.0)
    assert hip.kernel_gemv_tensor(ctx, y, A, x) == 0
    assert all(abs(hip.tensor_get_f32(y, i) - 10.0) < 1e-5 for i in range(4))
    for t in (A, x, y):
        hip.tensor_release(t)


@pytest.mark.parametrize("vals,x,y0,alpha,expect", [
    ([1, 0, 0, 1, 1, 1], [2, 3], [10, 20, 30], 1.0, [12, 23, 35]),   # test_tensor_gemv.c:162-203
    ([1, 1, 1, 1], [2, 2], [0, 0], 0.5, [2, 2]),                      # test_tensor_gemv.c:205-238
], ids=["accumulate", "scaled"])
def test_gemv_add(hip, ctx, vals, x, y0, alpha, expect):
    m = len(y0)
    A = matrix(hip, m, len(x), vals)
    xv = np.array(x, np.float32)
    y = np.array(y0, np.float32)
    assert hip.kernel_gemv_add(ctx, f32p(y), A, f32p(xv), alpha) == 0
    assert np.allclose(y, expect, atol=1e-5)
    hip.tensor_release(A)


def test_gemv_batch(hip, ctx):
    """test_tensor_gemv.c:244-283: A = [[1,2],[3,4]], X = [[1,0],[0,1],[1,1]]."""
    A = matrix(hip, 2, 2, [1, 2, 3, 4])
    X = np.array([1, 0, 0, 1, 1, 1], np.float32)
    Y = np.zeros(6, np.float32)
    assert hip.kernel_gemv_batch(ctx, f32p(Y), A, f32p(X), 3) == 0
    assert np.allclose(Y, [1, 3, 2, 4, 3, 7], atol=1e-5)
    hip.tensor_release(A)


def test_error_handling(hip):
    """test_tensor_gemv.c:289-318: a NULL context works for F32; NULL y, A or x is -1."""
    A = matrix(hip, 3, 4, [0.0] * 12)
    x = np.zeros(4, np.float32)
    y = np.zeros(3, np.float32)
    assert hip.kernel_gemv(None, f32p(y), A, f32p(x)) == 0
    assert hip.kernel_gemv(None, None, A, f32p(x)) == -1
    assert hip.kernel_gemv(None, f32p(y), None, f32p(x)) == -1
    assert hip.kernel_gemv(None, f32p(y), A, None) == -1
    hip.tensor_release(A)


def test_ctx_create_destroy_repeated(hip):
    """test_tensor_gemv.c:324-: contexts created, initialised and destroyed repeatedly."""
    for _ in range(3):
        c = hip.kernel_ctx_create(0, 1024)
        assert c and hip.kernel_ctx_init(c) == 0
        hip.kernel_ctx_destroy(c)


def test_weights_changed_after_a_gemv(hip, ctx, oracle):
    """The reference reads a weight tensor's host data on every call. tensor_set_f32 after a
    GEMV therefore changes the next GEMV's result (the device copy is rebuilt), and a write
    through the raw data pointer does once sapphire_tensor_invalidate has been called."""
    from sapphire_amd import synth
    A = matrix(hip, 4, 8, range(32))
    x = np.ones(8, np.float32)
    y = np.zeros(4, np.float32)
    assert hip.kernel_gemv(ctx, f32p(y), A, f32p(x)) == 0
    assert np.array_equal(y, np.arange(32, dtype=np.float32).reshape(4, 8).sum(1))
    assert hip.tensor_set_f32(A, 9, 100.0) == 0
    assert hip.kernel_gemv(ctx, f32p(y), A, f32p(x)) == 0
    want = np.arange(32, dtype=np.float32).reshape(4, 8)
    want[1, 1] = 100.0
    assert np.array_equal(y, want.sum(1))
    hip.tensor_release(A)
    # a quantized view whose blocks the caller rewrites in place
    for dtype in (synth.Q4_0, synth.Q8_0):
        W = synth.quant_matrix(dtype, 64, 640, 5, dtype)
        xq = synth.normal_f32(640, 5, 1)
        A = hip.tensor_create_view(dtype, 2, (C.c_int * 2)(64, 640), W.ctypes.data)
        yq = np.zeros(64, np.float32)
        assert hip.kernel_gemv(ctx, f32p(yq), A, f32p(xq)) == 0
        assert close_to(yq, oracle.gemv(dtype, W, xq))
        W["scale"] *= 2.0
        assert hip.sapphire_tensor_invalidate(A) == 0
        assert hip.kernel_gemv(ctx, f32p(yq), A, f32p(xq)) == 0
        assert close_to(yq, oracle.gemv(dtype, W, xq))
        hip.tensor_release(A)


def close_to(got, ref):
    from tests.conftest import close
    return close(got, ref)[0]
