"""F32 / BF16 GEMV parity on the GPU against the oracle.

The oracle follows the reference's pooled-row kernels (quantized_gemv_{bf16,f32}_avx2,
bf16_avx.c:57-113, f32_avx.c:43-90) bit for bit. Tolerance for float outputs:
|gpu - ref| <= 1e-4 + 1e-3*|ref|; GEMVs whose every product and partial sum is exact in
fp32 (small integers) are compared bit for bit, and non-finite activations must give the
same NaN / infinity pattern.
"""
import ctypes as C

import numpy as np
import pytest

from sapphire_amd import synth
from tests.conftest import close

pytestmark = pytest.mark.gpu

F32, BF16 = synth.F32, synth.BF16

SHAPES = [
    (262144, 640),  # weight-tied LM head of Gemma-3-270M
    (2048, 640),
    (640, 2048),
    (1000, 640),    # ragged M
    (7, 96),
    (1, 8),
    (333, 1152),
    (96, 6912),
    (4096, 64),
    (5, 100),       # BF16 rows of 200 bytes: the element-strided kernel
    (3, 7),
    (4, 33),
    (17, 16384),    # longest K held in LDS
    (9, 20000),     # longer K: the element-strided kernel
]


def weights(dtype, m, k, seed, std=0.05):
    f = synth.normal_f32((m, k), seed, m + 3 * k, 0.0, std)
    if dtype == F32:
        return f
    return (f.view(np.uint32) >> 16).astype(np.uint16)


def run_gemv_f(dtype, W, x, offset=0):
    from sapphire_amd.device import DeviceArray, check, gemv_f, lib
    m, k = W.shape
    raw = W.view(np.uint8).reshape(-1)
    dw = DeviceArray(raw.nbytes + offset)
    if offset:
        dw.zero()
    check(lib().sapphire_memcpy_h2d(dw.ptr + offset, raw.ctypes.data, raw.nbytes), "h2d")
    dx = DeviceArray.from_numpy(x)
    dy = DeviceArray.empty(m)
    gemv_f(dtype, dw, m, k, dx, dy, offset)
    return dy.numpy()


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_f_matches_oracle(hip, oracle, dtype, shape):
    m, k = shape
    print(f"gemv_f dtype={dtype} shape={shape}", flush=True)
    W = weights(dtype, m, k, 5)
    x = synth.normal_f32(k, 6, k)
    ref = oracle.gemv(dtype, W, x)
    y = run_gemv_f(dtype, W, x)
    ok, err = close(y, ref)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("offset", [2, 4, 16], ids=lambda o: f"off{o}")
def test_gemv_f_unaligned_weights(hip, oracle, dtype, offset):
    """Weights that do not start on a 16-byte boundary take the element-strided kernel;
    a 16-byte offset keeps the chunked one."""
    if dtype == F32 and offset == 2:
        pytest.skip("F32 weights are 4-byte aligned")
    m, k = 300, 640
    print(f"gemv_f unaligned dtype={dtype} offset={offset}", flush=True)
    W = weights(dtype, m, k, 8)
    x = synth.normal_f32(k, 9, 1)
    ref = oracle.gemv(dtype, W, x)
    y = run_gemv_f(dtype, W, x, offset)
    ok, err = close(y, ref)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", [(1000, 640), (64, 2048), (5, 100), (3, 7)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_f_exact_integers(hip, oracle, dtype, shape):
    """Weights in [-3, 3] and activations in [-4, 4]: every product and partial sum is an
    integer below 2^24, so any summation order gives the oracle's bits."""
    m, k = shape
    print(f"gemv_f exact dtype={dtype} shape={shape}", flush=True)
    g = np.random.default_rng(m * 31 + k)
    Wf = g.integers(-3, 4, size=(m, k)).astype(np.float32)
    W = Wf if dtype == F32 else (Wf.view(np.uint32) >> 16).astype(np.uint16)
    x = g.integers(-4, 5, size=k).astype(np.float32)
    ref = oracle.gemv(dtype, W, x)
    assert np.array_equal(ref, Wf.astype(np.float64) @ x.astype(np.float64))
    y = run_gemv_f(dtype, W, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_gemv_f_non_finite(hip, oracle, dtype):
    """An infinite activation gives +-inf in rows whose weight there is nonzero and NaN
    where it is zero (0 * inf), as in the reference."""
    m, k = 64, 640
    print(f"gemv_f non-finite dtype={dtype}", flush=True)
    W = weights(dtype, m, k, 12)
    W[0, 5] = 0
    W[1, 5] = 0
    x = synth.normal_f32(k, 13, 1)
    x[5] = np.inf
    x[600] = -np.inf
    ref = oracle.gemv(dtype, W, x)
    y = run_gemv_f(dtype, W, x)
    nan = np.isnan(ref)
    assert nan[0] and nan[1] and np.isinf(ref).any()
    assert np.array_equal(np.isnan(y), nan)
    assert np.array_equal(y[~nan], ref[~nan])


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("ctx_kind", ["ctx", "null"])
def test_kernel_gemv_f_tensor_api(hip, oracle, dtype, ctx_kind):
    """kernel_gemv and kernel_gemv_batch on host pointers (kernels.h:140,161) for F32 / BF16
    tensors, with a context and (kernel_gemv only) without one; the batch is checked
    against the reference's batched order (kernel_gemm_{f32,bf16}_avx2)."""
    m, k, batch = 2048, 1152, 3
    print(f"kernel_gemv_f dtype={dtype} ctx={ctx_kind}", flush=True)
    W = weights(dtype, m, k, 21)
    X = synth.normal_f32((batch, k), 22, batch)
    ref = np.stack([oracle.gemv(dtype, W, X[b]) for b in range(batch)])
    ctx = None
    if ctx_kind == "ctx":
        ctx = hip.kernel_ctx_create(0, 16)
        assert ctx
        assert hip.kernel_ctx_init(ctx) == 0
    shp = (C.c_int * 2)(m, k)
    A = hip.tensor_create_view(dtype, 2, shp, W.ctypes.data)
    try:
        y = np.zeros(m, np.float32)
        assert hip.kernel_gemv(ctx, y.ctypes.data, A, X[0].ctypes.data) == 0
        ok, err = close(y, ref[0])
        assert ok, f"kernel_gemv: max abs err {err}"
        if ctx is not None:
            Y = np.zeros((batch, m), np.float32)
            assert hip.kernel_gemv_batch(ctx, Y.ctypes.data, A, X.ctypes.data, batch) == 0
            ok, err = close(Y, oracle.gemm_f(dtype, W, X))
            assert ok, f"kernel_gemv_batch: max abs err {err}"
    finally:
        hip.tensor_release(A)
        if ctx is not None:
            hip.kernel_ctx_destroy(ctx)


# ---- the batched BF16 form on the matrix cores (sapphire_gemm_bf16_dev) ----

def run_gemm_bf16(W, X, ldx=None, ldy=None):
    from sapphire_amd.device import DeviceArray, check, lib
    m, k = W.shape
    b = X.shape[0]
    ldx = ldx or k
    ldy = ldy or m
    Xp = np.zeros((b, ldx), np.float32)
    Xp[:, :k] = X
    dw, dx = DeviceArray.from_numpy(W), DeviceArray.from_numpy(Xp)
    dy = DeviceArray.empty(b * ldy)
    dy.zero()
    check(lib().sapphire_gemm_bf16_dev(dw.ptr, m, k, dx.ptr, ldx, b, dy.ptr, ldy, None), "gemm_bf16")
    return dy.numpy().reshape(b, ldy)[:, :m]


@pytest.mark.parametrize("shape,batch", [((262144, 640), 16), ((2048, 640), 3), ((1000, 1152), 16), ((640, 2048), 7),
                                         ((33, 40), 5), ((16, 8), 1), ((4096, 256), 17), ((96, 6912), 16)],
                         ids=["lm_head_b16", "2048x640_b3", "ragged_m_b16", "640x2048_b7", "k40_b5", "16x8_b1",
                              "b17_two_passes", "k6912_b16"])
def test_gemm_bf16_matches_oracle(hip, oracle, shape, batch):
    m, k = shape
    print(f"gemm_bf16 shape={shape} batch={batch}", flush=True)
    W = weights(BF16, m, k, 31)
    X = synth.normal_f32((batch, k), 32, batch)
    ref = oracle.gemm_f(BF16, W, X)
    got = run_gemm_bf16(W, X)
    ok, err = close(got, ref)
    assert ok, f"max abs err {err}"


def test_gemm_bf16_strides_and_exact(hip, oracle):
    """Row strides of X and Y wider than K and M; small integers give the oracle's bits."""
    m, k, batch = 300, 96, 9
    print("gemm_bf16 strides / exact", flush=True)
    g = np.random.default_rng(5)
    Wf = g.integers(-3, 4, size=(m, k)).astype(np.float32)
    W = (Wf.view(np.uint32) >> 16).astype(np.uint16)
    X = g.integers(-4, 5, size=(batch, k)).astype(np.float32)
    ref = oracle.gemm_f(BF16, W, X)
    got = run_gemm_bf16(W, X, ldx=k + 13, ldy=m + 7)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_gemm_bf16_rejects(hip):
    from sapphire_amd.device import DeviceArray, lib
    w, x, y = DeviceArray(4096), DeviceArray(4096), DeviceArray(4096)
    L = lib()
    assert L.sapphire_gemm_bf16_dev(w.ptr, 16, 12, x.ptr, 12, 2, y.ptr, 16, None) == -1     # K % 8
    assert L.sapphire_gemm_bf16_dev(w.ptr + 2, 16, 16, x.ptr, 16, 2, y.ptr, 16, None) == -1  # alignment
    assert L.sapphire_gemm_bf16_dev(w.ptr, 16, 16, x.ptr, 8, 2, y.ptr, 16, None) == -1       # ldx < K
