"""Batched GEMM (a batch of sequences through one Q4_0/Q8_0 weight matrix) on the GPU
against the oracle.

The reference has no quantized batched kernel (pool.c:318-321 rejects it), so the
expected output of sequence b is the oracle's kernel_gemv of that sequence's vector
(dispatch.c:101-156). Tolerance: |gpu - ref| <= 1e-4 + 1e-3*|ref| (north star); the
exactly representable case is compared bit for bit.
"""
import ctypes as C

import numpy as np
import pytest

from sapphire_amd import synth
from tests.conftest import close

pytestmark = pytest.mark.gpu

TILED = 2

# Gemma-3-1B-shaped projections (hidden 1152, 4 q heads x 256, 1 kv head, FFN 6912) and
# ragged / small cases; K % 128 == 0 for the TILED layout.
SHAPES = [
    (1024, 1152),   # q_proj
    (256, 1152),    # k/v_proj
    (1152, 1024),   # o_proj
    (6912, 1152),   # gate/up
    (1152, 6912),   # down (K split over workgroups)
    (333, 1152),    # ragged M
    (17, 128),      # one group of four blocks
    (40, 4608),     # K = 144 blocks: four K chunks
]


def _gemm(hip, qm, X, layout=TILED):
    from sapphire_amd.device import DeviceArray, check
    batch = X.shape[0]
    dX = DeviceArray.from_numpy(np.ascontiguousarray(X, np.float32))
    dY = DeviceArray.empty(batch * qm.M)
    wsb = hip.sapphire_gemm_workspace_bytes(qm.dtype, qm.M, qm.K)
    assert wsb > 0
    ws = DeviceArray(wsb)
    check(hip.sapphire_gemm_q_dev(qm.dtype, layout, qm.ptr(layout), qm.M, qm.K, dX.ptr, batch, dY.ptr, ws.ptr, None))
    return dY.numpy().reshape(batch, qm.M)


def _ref(oracle, dtype, W, X, nthreads=8):
    return np.stack([oracle.gemv(dtype, W, X[b], nthreads=nthreads) for b in range(X.shape[0])])


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("batch", [1, 5, 16, 21])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemm_tiled_matches_oracle(hip, oracle, dtype, batch, shape):
    from sapphire_amd.device import QMatrix
    m, k = shape
    print(f"gemm dtype={dtype} batch={batch} shape={shape}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=31, tensor_id=m * 3 + k)
    X = synth.normal_f32((batch, k), 31, 7 + batch)
    got = _gemm(hip, QMatrix(dtype, W, layout=TILED), X)
    ref = _ref(oracle, dtype, W, X)
    ok, err = close(got, ref)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
def test_gemm_lm_head_1152(hip, oracle, dtype):
    """262144 x 1152 (the Gemma-3-1B LM head) with 16 sequences: every output computed on
    the GPU, every 61st row checked against the oracle for all 16 sequences."""
    from sapphire_amd.device import QMatrix
    m, k = 262144, 1152
    print(f"gemm lm head dtype={dtype}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=32, tensor_id=dtype)
    X = synth.normal_f32((16, k), 32, 1)
    got = _gemm(hip, QMatrix(dtype, W, layout=TILED), X)
    rows = np.arange(0, m, 61)
    ref = _ref(oracle, dtype, np.ascontiguousarray(W[rows]), X)
    ok, err = close(got[:, rows], ref)
    assert ok, f"max abs err {err}"
    assert np.isfinite(got).all()


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("shape", [(3000, 640), (512, 6912)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemm_exact_special_case(hip, oracle, dtype, shape):
    """Scales 2^-e and small-integer x: every product and partial sum is exact in fp32 (and
    x is exact in one fp16 term), so the matrix-core result carries the reference's bits."""
    from sapphire_amd.device import QMatrix
    m, k = shape
    W = synth.quant_matrix(dtype, m, k, seed=33, tensor_id=1)
    g = synth.rng(33, 2)
    W["scale"] = np.ldexp(1.0, -g.integers(1, 8, size=W["scale"].shape)).astype(np.float32)
    X = g.integers(-4, 5, size=(16, k)).astype(np.float32)
    got = _gemm(hip, QMatrix(dtype, W, layout=TILED), X)
    ref = _ref(oracle, dtype, W, X)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
def test_gemm_x_ranges(hip, oracle, dtype):
    """Sequences of very different magnitude in one batch (each gets its own power-of-two
    range scale), an all-zero sequence, denormals and many binades inside one vector."""
    from sapphire_amd.device import QMatrix
    m, k = 1024, 1152
    W = synth.quant_matrix(dtype, m, k, seed=34, tensor_id=1)
    X = synth.normal_f32((16, k), 34, 2)
    X[1] *= np.float32(1e-30)
    X[2] *= np.float32(1e30)
    X[3] = 0.0
    X[4, :] = np.float32(1e-40)
    X[5, 0:32] = np.ldexp(1.0, np.arange(-16, 16)).astype(np.float32)
    X[6, 100] = np.float32(3e4)
    got = _gemm(hip, QMatrix(dtype, W, layout=TILED), X)
    ref = _ref(oracle, dtype, W, X)
    for b in range(16):
        # the tolerance scales with the sequence's magnitude: for b = 2 that is 1e30
        scale = max(1.0, float(np.abs(ref[b]).max()))
        ok, err = close(got[b] / scale, ref[b] / scale)
        assert ok, f"sequence {b}: max abs err {err} (scale {scale})"
    assert np.all(got[3] == 0.0)


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
def test_gemm_vector_layouts(hip, oracle, dtype):
    """AOS and PACKED weights take the vector kernel through the same entry point."""
    from sapphire_amd.device import QMatrix
    m, k = 700, 640
    W = synth.quant_matrix(dtype, m, k, seed=35, tensor_id=1)
    X = synth.normal_f32((6, k), 35, 1)
    ref = _ref(oracle, dtype, W, X)
    for layout in (0, 1):
        got = _gemm(hip, QMatrix(dtype, W, layout=layout), X, layout=layout)
        ok, err = close(got, ref)
        assert ok, f"layout {layout}: max abs err {err}"


def test_gemm_rejects_bad_arguments(hip):
    from sapphire_amd.device import DeviceArray, QMatrix
    W = synth.quant_matrix(synth.Q4_0, 64, 256, seed=36, tensor_id=1)
    qm = QMatrix(synth.Q4_0, W, layout=TILED)
    dX, dY = DeviceArray.empty(4 * 256), DeviceArray.empty(4 * 64)
    ws = DeviceArray(hip.sapphire_gemm_workspace_bytes(synth.Q4_0, 64, 256))
    assert hip.sapphire_gemm_q_dev(synth.Q4_0, TILED, qm.ptr(), 64, 256, dX.ptr, 0, dY.ptr, ws.ptr, None) == -1
    assert hip.sapphire_gemm_q_dev(synth.Q4_0, TILED, qm.ptr(), 64, 256, dX.ptr, 4, dY.ptr, None, None) == -1
    assert hip.sapphire_gemm_q_dev(synth.Q4_0, TILED, qm.ptr(), 64, 256, None, 4, dY.ptr, ws.ptr, None) == -1
    assert hip.sapphire_gemm_q_dev(synth.Q4_0, TILED, qm.ptr(), 64, 224, dX.ptr, 4, dY.ptr, ws.ptr, None) == -1
    assert hip.sapphire_gemm_workspace_bytes(synth.F32, 64, 256) == 0


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("shape,batch", [((1152, 6912), 16), ((6912, 1152), 3), ((300, 672), 4)],
                         ids=["down_b16", "up_b3", "k672_b4"])
def test_kernel_gemm_tensor_api(hip, oracle, dtype, shape, batch):
    """kernel_gemm and kernel_gemv_batch on host pointers (kernels.h:146,161): quantized
    batches run on the matrix cores when K % 128 == 0 (else the vector kernel), and a
    later kernel_gemv on the same tensor still uses its GEMV copy."""
    m, k = shape
    print(f"kernel_gemm dtype={dtype} shape={shape} batch={batch}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=37, tensor_id=m + k)
    X = synth.normal_f32((batch, k), 37, batch)
    ref = _ref(oracle, dtype, W, X)
    ctx = hip.kernel_ctx_create(0, 16)
    assert ctx
    assert hip.kernel_ctx_init(ctx) == 0
    shp = (C.c_int * 2)(m, k)
    A = hip.tensor_create_view(dtype, 2, shp, W.ctypes.data)
    try:
        Y = np.zeros((batch, m), np.float32)
        assert hip.kernel_gemm(ctx, Y.ctypes.data, A, X.ctypes.data, batch, m) == 0
        ok, err = close(Y, ref)
        assert ok, f"kernel_gemm: max abs err {err}"
        Y2 = np.zeros((batch, m), np.float32)
        assert hip.kernel_gemv_batch(ctx, Y2.ctypes.data, A, X.ctypes.data, batch) == 0
        ok, err = close(Y2, ref)
        assert ok, f"kernel_gemv_batch: max abs err {err}"
        y = np.zeros(m, np.float32)
        assert hip.kernel_gemv(ctx, y.ctypes.data, A, X[0].ctypes.data) == 0
        ok, err = close(y, ref[0])
        assert ok, f"kernel_gemv after batch: max abs err {err}"
    finally:
        hip.tensor_release(A)
        hip.kernel_ctx_destroy(ctx)
