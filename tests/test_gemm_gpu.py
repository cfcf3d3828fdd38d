"""Batched GEMM (a batch of sequences through one Q4_0/Q8_0 weight matrix) on the GPU
against the oracle.

The reference has no quantized batched kernel (pool.c:318-321 rejects it), so the
expected output of sequence b is the oracle's kernel_gemv of that sequence's vector
(dispatch.c:101-156). Tolerance: |gpu - ref| <= 1e-4 + 1e-3*|ref| (the parity bar); the
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


# ---- the fused input / output transforms (sapphire_gemm_q_fused_dev) ----

from sapphire_amd._lib import GemmInput as _GemmIn, GemmOutput as _GemmOut  # noqa: E402


def _fused(hip, qm, batch, gin, gout, ws=None):
    from sapphire_amd.device import check
    check(hip.sapphire_gemm_q_fused_dev(qm.dtype, qm.ptr(), qm.M, qm.K, batch, C.byref(gin), C.byref(gout),
                                        ws.ptr if ws is not None else None, None))
    check(hip.sapphire_synchronize())


def _norm_w(n, tid):
    return synth.normal_f32(n, 40, tid, 1.0, 0.1)


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("batch", [16, 5])
def test_gemm_fused_residual_and_norms(hip, oracle, dtype, batch):
    """h = x + rmsnorm_delta(p0 + p1 + p2, w_delta); resid_out = h (bit for bit: the norm sums
    run in the reference's order); y = W . rmsnorm_delta(h, w_norm) against the oracle."""
    from sapphire_amd.device import DeviceArray, QMatrix
    m, k = 1536, 1152
    W = synth.quant_matrix(dtype, m, k, seed=41, tensor_id=1)
    qm = QMatrix(dtype, W, layout=TILED)
    x = synth.normal_f32((batch, k), 41, 2)
    parts = synth.normal_f32((3, 16, k), 41, 3)
    wd, wn = _norm_w(k, 1), _norm_w(k, 2)
    d = ((parts[0, :batch] + parts[1, :batch]) + parts[2, :batch]).astype(np.float32)
    h = np.stack([x[b] + oracle.rmsnorm_delta(d[b], wd) for b in range(batch)]).astype(np.float32)
    xin = np.stack([oracle.rmsnorm_delta(h[b], wn) for b in range(batch)])
    ref = _ref(oracle, dtype, W, xin)
    dx, dp, dwd, dwn = (DeviceArray.from_numpy(a) for a in (x, parts, wd, wn))
    dr, dy = DeviceArray.empty(batch * k), DeviceArray.empty(batch * m)
    gin = _GemmIn(dx.ptr, k, dp.ptr, 3, k, 16 * k, dwd.ptr, dr.ptr, k, dwn.ptr, 1e-6)
    gout = _GemmOut(dy.ptr, m, None, 0)
    _fused(hip, qm, batch, gin, gout)
    assert np.array_equal(dr.numpy().reshape(batch, k).view(np.uint32), h.view(np.uint32))
    ok, err = close(dy.numpy().reshape(batch, m), ref)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("ffn", [6912, 200])
def test_gemm_fused_geglu(hip, oracle, dtype, ffn):
    """Gate and up rows interleaved by eight in one matrix; y = gelu(W_g . x) * (W_u . x)
    (transformer.c:141-157) from the GEMM epilogue. Each projection is held to the GEMV
    tolerance t(v) = 1e-4 + 1e-3|v|; the product to what that propagates to:
    |u| t(g) max|gelu'| + |gelu(g)| t(u) (max|gelu'| < 1.13)."""
    from sapphire_amd.device import DeviceArray, QMatrix
    k, batch = 1152, 16
    Wg = synth.quant_matrix(dtype, ffn, k, seed=42, tensor_id=1)
    Wu = synth.quant_matrix(dtype, ffn, k, seed=42, tensor_id=2)
    st = np.empty((2 * ffn, k // 32), dtype=Wg.dtype)
    st.reshape(ffn // 8, 2, 8, k // 32)[:, 0] = Wg.reshape(ffn // 8, 8, k // 32)
    st.reshape(ffn // 8, 2, 8, k // 32)[:, 1] = Wu.reshape(ffn // 8, 8, k // 32)
    qm = QMatrix(dtype, st, layout=TILED)
    x = synth.normal_f32((batch, k), 42, 3)
    gate, up = _ref(oracle, dtype, Wg, x), _ref(oracle, dtype, Wu, x)
    ref = np.stack([oracle.gelu_mul(gate[b], up[b]) for b in range(batch)])
    dx, dy = DeviceArray.from_numpy(x), DeviceArray.empty(batch * ffn)
    _fused(hip, qm, batch, _GemmIn(dx.ptr, k, None, 0, 0, 0, None, None, 0, None, 1e-6), _GemmOut(dy.ptr, ffn, None, 1))
    got = dy.numpy().reshape(batch, ffn).astype(np.float64)
    g64, u64 = gate.astype(np.float64), up.astype(np.float64)
    gelu = np.stack([oracle.gelu_mul(gate[b], np.ones(ffn, np.float32)) for b in range(batch)]).astype(np.float64)
    t = lambda v: 1e-4 + 1e-3 * np.abs(v)
    bound = 1.13 * t(g64) * np.abs(u64) + np.abs(gelu) * t(u64) + t(ref.astype(np.float64))
    err = np.abs(got - ref)
    assert np.all(err <= bound), f"max abs err {err.max()}, worst excess {(err - bound).max()}"


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
def test_gemm_fused_partials_chain(hip, oracle, dtype):
    """The down projection (K = 6912, six K chunks) leaves partial sums; the next GEMM adds
    them while staging (residual + post-norm + pre-norm), as a decode step chains them."""
    from sapphire_amd.device import DeviceArray, QMatrix
    hdim, ffn, batch = 1152, 6912, 16
    Wd = synth.quant_matrix(dtype, hdim, ffn, seed=43, tensor_id=1)
    W2 = synth.quant_matrix(dtype, 1536, hdim, seed=43, tensor_id=2)
    qd, q2 = QMatrix(dtype, Wd, layout=TILED), QMatrix(dtype, W2, layout=TILED)
    g = synth.normal_f32((batch, ffn), 43, 3)
    x = synth.normal_f32((batch, hdim), 43, 4)
    wd, wn = _norm_w(hdim, 3), _norm_w(hdim, 4)
    ns = hip.sapphire_gemm_splits(ffn)
    assert ns == 6
    dg, dx, dwd, dwn = (DeviceArray.from_numpy(a) for a in (g, x, wd, wn))
    dparts = DeviceArray.empty(ns * batch * hdim)
    _fused(hip, qd, batch, _GemmIn(dg.ptr, ffn, None, 0, 0, 0, None, None, 0, None, 1e-6),
           _GemmOut(None, 0, dparts.ptr, 0))
    dr, dy = DeviceArray.empty(batch * hdim), DeviceArray.empty(batch * 1536)
    _fused(hip, q2, batch, _GemmIn(dx.ptr, hdim, dparts.ptr, ns, hdim, batch * hdim, dwd.ptr, dr.ptr, hdim, dwn.ptr,
                                   1e-6), _GemmOut(dy.ptr, 1536, None, 0))
    d = _ref(oracle, dtype, Wd, g)
    partsum = dparts.numpy().reshape(ns, batch, hdim).sum(axis=0, dtype=np.float64)
    ok, err = close(partsum, d)
    assert ok, f"partial sums: max abs err {err}"
    h = np.stack([x[b] + oracle.rmsnorm_delta(d[b], wd) for b in range(batch)]).astype(np.float32)
    ok, err = close(dr.numpy().reshape(batch, hdim), h)
    assert ok, f"residual: max abs err {err}"
    ref = _ref(oracle, dtype, W2, np.stack([oracle.rmsnorm_delta(h[b], wn) for b in range(batch)]))
    ok, err = close(dy.numpy().reshape(batch, 1536), ref)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
def test_gemm_fused_strided_input(hip, oracle, dtype):
    """Input rows read with a leading dimension larger than K (the first 1024 columns of a
    [batch][1536] buffer) and output rows written with one larger than M."""
    from sapphire_amd.device import DeviceArray, QMatrix
    m, k, batch = 1152, 1024, 7
    W = synth.quant_matrix(dtype, m, k, seed=44, tensor_id=1)
    qm = QMatrix(dtype, W, layout=TILED)
    buf = synth.normal_f32((batch, 1536), 44, 2)
    ref = _ref(oracle, dtype, W, np.ascontiguousarray(buf[:, :k]))
    dx = DeviceArray.from_numpy(buf)
    dy = DeviceArray.from_numpy(np.full((batch, m + 4), 7.0, np.float32))
    _fused(hip, qm, batch, _GemmIn(dx.ptr, 1536, None, 0, 0, 0, None, None, 0, None, 1e-6), _GemmOut(dy.ptr, m + 4, None, 0))
    got = dy.numpy().reshape(batch, m + 4)
    ok, err = close(got[:, :m], ref)
    assert ok, f"max abs err {err}"
    assert np.all(got[:, m:] == 7.0)


def test_gemm_fused_rejects(hip):
    from sapphire_amd.device import DeviceArray, QMatrix
    W = synth.quant_matrix(synth.Q4_0, 64, 6912, seed=45, tensor_id=1)
    qm = QMatrix(synth.Q4_0, W, layout=TILED)
    dx, dy, dw = DeviceArray.empty(4 * 6912), DeviceArray.empty(4 * 64), DeviceArray.empty(6912)
    # a norm over K = 6912 needs whole rows in one K chunk
    gin = _GemmIn(dx.ptr, 6912, None, 0, 0, 0, None, None, 0, dw.ptr, 1e-6)
    assert hip.sapphire_gemm_q_fused_dev(qm.dtype, qm.ptr(), 64, 6912, 4, C.byref(gin),
                                         C.byref(_GemmOut(dy.ptr, 64, None, 0)), None, None) == -1
    gin = _GemmIn(dx.ptr, 6912, None, 0, 0, 0, None, None, 0, None, 1e-6)
    assert hip.sapphire_gemm_q_fused_dev(qm.dtype, qm.ptr(), 64, 6912, 17, C.byref(gin),
                                         C.byref(_GemmOut(dy.ptr, 64, None, 0)), None, None) == -1   # batch > 16


def _block_order_index(b, k):
    """Element k of sequence b in the block order of x_blocked / y_blocked (16 sequence slots)."""
    k = np.asarray(k)
    return (k >> 5) * 512 + ((k >> 3) & 3) * 128 + b * 8 + (k & 7)


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("batch", [16, 5])
def test_gemm_fused_block_order(hip, oracle, dtype, batch):
    """The GeGLU output in block order (y_blocked) holds the row-major output's values, bit for
    bit, at the block-order positions; the down projection reading it (x_blocked) leaves the
    same partial sums, bit for bit, as from the row-major rows. Slots of sequences past the
    batch hold NaN and must not be read."""
    from sapphire_amd.device import DeviceArray, QMatrix
    k, ffn = 1152, 6912
    st = synth.quant_matrix(dtype, 2 * ffn, k, seed=44, tensor_id=1)
    qgu = QMatrix(dtype, st, layout=TILED)
    qd = QMatrix(dtype, synth.quant_matrix(dtype, k, ffn, seed=44, tensor_id=2), layout=TILED)
    x = synth.normal_f32((batch, k), 44, 3)
    dx = DeviceArray.from_numpy(x)
    g_rows, g_blk = DeviceArray.empty(batch * ffn), DeviceArray.from_numpy(np.full(16 * ffn, np.nan, np.float32))
    none_in = dict(parts=None, nparts=0, ldp=0, part_stride=0, w_delta=None, resid_out=None, ldr=0, w_norm=None,
                   eps=1e-6)
    _fused(hip, qgu, batch, _GemmIn(x=dx.ptr, ldx=k, **none_in), _GemmOut(y=g_rows.ptr, ldy=ffn, geglu=1))
    _fused(hip, qgu, batch, _GemmIn(x=dx.ptr, ldx=k, **none_in), _GemmOut(y=g_blk.ptr, geglu=1, y_blocked=1))
    rows = g_rows.numpy().reshape(batch, ffn)
    blk = g_blk.numpy()
    j = np.arange(ffn)
    for b in range(batch):
        assert np.array_equal(blk[_block_order_index(b, j)].view(np.uint32), rows[b].view(np.uint32)), b
    ns = hip.sapphire_gemm_splits(ffn)
    p_rows, p_blk = DeviceArray.empty(ns * batch * k), DeviceArray.empty(ns * batch * k)
    _fused(hip, qd, batch, _GemmIn(x=g_rows.ptr, ldx=ffn, **none_in), _GemmOut(parts=p_rows.ptr))
    _fused(hip, qd, batch, _GemmIn(x=g_blk.ptr, x_blocked=1, **none_in), _GemmOut(parts=p_blk.ptr))
    assert np.array_equal(p_rows.numpy().view(np.uint32), p_blk.numpy().view(np.uint32))
    # and they are the oracle's product (norm-wise per sequence: the GeGLU outputs are heavy-tailed,
    # so outputs near zero are differences of large terms; test_gemm_fused_partials_chain holds
    # the element-wise bound on N(0, 1) inputs)
    d = _ref(oracle, dtype, synth.quant_matrix(dtype, k, ffn, seed=44, tensor_id=2), rows).astype(np.float64)
    got = p_rows.numpy().reshape(ns, batch, k).sum(axis=0, dtype=np.float64)
    assert np.all(np.abs(got - d).max(axis=1) <= 1e-5 * np.abs(d).max(axis=1))
