"""GEMV parity on the GPU against the oracle (which is bit-exact with the reference).

Tolerance for float outputs: |gpu - ref| <= 1e-4 + 1e-3*|ref| (the parity bar). Integer
unpack and dequantised weights are compared bit for bit; so are GEMVs whose every
product and partial sum is exact in fp32 (power-of-two scales, small-integer x).
"""
import numpy as np
import pytest

from sapphire_amd import synth
from tests.conftest import close

pytestmark = pytest.mark.gpu

SHAPES = [
    (2048, 640),    # MLP up/gate (C1/C2)
    (640, 2048),    # MLP down (C2)
    (1024, 640),    # q_proj
    (256, 640),     # k/v_proj
    (640, 1024),    # o_proj
    (1000, 640),    # ragged M
    (7, 96),        # nb = 3
    (1, 32),        # single block
    (333, 1152),    # nb = 36 (row kernel)
    (96, 6912),     # nb = 216 (row kernel)
    (4096, 64),     # nb = 2, 32 rows per wave-step
]


def _gemv(hip, dtype, blocks, x, layout):
    from sapphire_amd.device import DeviceArray, QMatrix, gemv
    qm = QMatrix(dtype, blocks, layout=layout)
    dx = DeviceArray.from_numpy(x)
    dy = DeviceArray.empty(qm.M)
    gemv(qm, dx, dy, layout)
    return dy.numpy()


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("layout", [0, 1], ids=["aos", "packed"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_matches_oracle(hip, oracle, dtype, layout, shape):
    m, k = shape
    print(f"gemv dtype={dtype} layout={layout} shape={shape}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=11, tensor_id=m * 7 + k)
    x = synth.normal_f32(k, 11, 5 + k)
    ref = oracle.gemv(dtype, W, x, nthreads=4)
    got = _gemv(hip, dtype, W, x, layout)
    ok, err = close(got, ref)
    assert ok, f"max abs err {err}"


# On a 256-CU device 43963 and 55997 rows leave tiles after the full rounds of the grid
# stride that are split over a workgroup's waves (Q8_0 at 43963: two tail tiles per
# workgroup, two waves each; Q4_0 at 55997 and 65536: one per workgroup over three waves),
# with the last tile ragged; K = 640 runs the double-buffered walk, K = 1152 the single one.
TILED_SHAPES = [
    (16, 640), (1000, 640), (4099, 1024), (333, 1152), (17, 1152), (65536, 640), (20000, 1152),
    (43963, 640), (55997, 640), (43963, 1152), (55997, 1152),
]


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("shape", TILED_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_tiled_matches_oracle(hip, oracle, dtype, shape):
    """The matrix-core kernel on the TILED layout, ragged row counts included."""
    m, k = shape
    print(f"tiled gemv dtype={dtype} shape={shape}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=12, tensor_id=m * 5 + k)
    x = synth.normal_f32(k, 12, 9 + k)
    ref = oracle.gemv(dtype, W, x, nthreads=8)
    got = _gemv(hip, dtype, W, x, 2)
    ok, err = close(got, ref)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("layout", [1, 2], ids=["packed", "tiled"])
def test_lm_head_full_shape(hip, oracle, dtype, layout):
    """262144 x 640, the LM-head shape, against the oracle on every row."""
    print(f"lm head dtype={dtype} layout={layout}", flush=True)
    W = synth.quant_matrix(dtype, 262144, 640, seed=3, tensor_id=dtype)
    x = synth.normal_f32(640, 3, 77)
    ref = oracle.gemv(dtype, W, x, nthreads=8)
    got = _gemv(hip, dtype, W, x, layout)
    ok, err = close(got, ref)
    assert ok, f"max abs err {err}"
    assert int(np.argmax(got)) == int(np.argmax(ref))


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
def test_gemv_tiled_x_extremes(hip, oracle, dtype):
    """Blocks of x spanning many binades, all-zero blocks and denormals: the per-block
    integer conversion of x must keep the tolerance."""
    m, k = 2048, 640
    W = synth.quant_matrix(dtype, m, k, seed=13, tensor_id=1)
    x = synth.normal_f32(k, 13, 2)
    x[0:32] = 0.0                                   # an all-zero block
    x[32:64] *= np.float32(1e-30)                   # tiny block
    x[64:96] = np.float32(1e-40)                    # denormals
    x[96] = np.float32(3e4)                         # one huge element in a block
    x[128:160] = np.ldexp(1.0, np.arange(-16, 16)).astype(np.float32)   # 32 binades
    ref = oracle.gemv(dtype, W, x)
    got = _gemv(hip, dtype, W, x, 2)
    ok, err = close(got, ref)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("layout", [0, 1, 2], ids=["aos", "packed", "tiled"])
def test_gemv_exact_special_case(hip, oracle, dtype, layout):
    """Scales 2^-e and small-integer x: every product and sum is exact in fp32, so any
    summation order gives the reference's bits."""
    m, k = 3000, 640
    W = synth.quant_matrix(dtype, m, k, seed=5, tensor_id=1)
    g = synth.rng(5, 2)
    W["scale"] = np.ldexp(1.0, -g.integers(1, 8, size=W["scale"].shape)).astype(np.float32)
    x = g.integers(-4, 5, size=k).astype(np.float32)
    ref = oracle.gemv(dtype, W, x)
    got = _gemv(hip, dtype, W, x, layout)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("layout", [0, 1, 2], ids=["aos", "packed", "tiled"])
def test_unpack_and_dequant_bit_exact(hip, oracle, dtype, layout):
    """Every byte value in every quant position; ints and fl(int*scale) bit for bit.
    Rotation offsets b + 13r cover 0..255 for (rows, blocks) = (4, 256) and (52, 20)."""
    from sapphire_amd.device import DeviceArray, QMatrix, check
    rows, nb = (4, 256) if layout != 2 else (52, 20)
    W = np.zeros((rows, nb), dtype=synth.block_dtype(dtype))
    vals = np.arange(256, dtype=np.uint8)
    qb = 16 if dtype == synth.Q4_0 else 32
    for r in range(rows):
        for b in range(nb):
            W["q"][r, b] = np.roll(vals, b + 13 * r)[:qb].view(W["q"].dtype)
    W["scale"] = synth.normal_f32((rows, nb), 9, 9, 0.0, 0.01)
    qm = QMatrix(dtype, W, layout=layout)
    L = hip
    ints = DeviceArray.empty(rows * nb * 32, np.int8)
    deq = DeviceArray.empty(rows * nb * 32, np.float32)
    check(L.sapphire_q_unpack_ints_dev(dtype, layout, qm.ptr(layout), rows, nb * 32, ints.ptr, None))
    check(L.sapphire_q_dequant_dev(dtype, layout, qm.ptr(layout), rows, nb * 32, deq.ptr, None))
    got_i = ints.numpy()
    assert np.array_equal(got_i, oracle.unpack_ints(dtype, W))
    assert np.array_equal(got_i, synth.unpack_ints(dtype, W).reshape(-1))
    assert np.array_equal(deq.numpy().view(np.uint32), oracle.dequant(dtype, W).view(np.uint32))


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("layout", [1, 2], ids=["packed", "tiled"])
@pytest.mark.parametrize("shape", [(262144, 640), (20000, 1152), (1000, 640)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_softmax_fused(hip, oracle, dtype, layout, shape):
    """LM head + softmax + greedy token in one call (the GEMV epilogue leaves the softmax
    partials on the TILED layout): logits against the oracle GEMV, probabilities against
    the oracle softmax of the same logits, argmax against the oracle's (a different index
    is accepted only at a near-tie within the logit tolerance)."""
    from sapphire_amd.device import DeviceArray, QMatrix, check
    m, k = shape
    print(f"gemv+softmax dtype={dtype} layout={layout} shape={shape}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=21, tensor_id=m + k + dtype)
    x = synth.normal_f32(k, 21, 3)
    qm = QMatrix(dtype, W, layout=layout)
    dx = DeviceArray.from_numpy(x)
    logits, probs = DeviceArray.empty(m), DeviceArray.empty(m)
    arg = DeviceArray.empty(1, np.int32)
    check(hip.sapphire_gemv_softmax_dev(dtype, layout, qm.ptr(), m, k, dx.ptr, logits.ptr, probs.ptr, arg.ptr, None))
    got_l, got_p, got_a = logits.numpy(), probs.numpy(), int(arg.numpy()[0])
    ref_l = oracle.gemv(dtype, W, x, nthreads=8)
    ok, err = close(got_l, ref_l)
    assert ok, f"logits: max abs err {err}"
    ok, err = close(got_p, oracle.softmax(got_l), rel=1e-3, abs_=1e-9)
    assert ok, f"probs: max abs err {err}"
    assert got_a == oracle.argmax(got_l)
    ra = oracle.argmax(ref_l)
    if got_a != ra:
        assert abs(float(ref_l[got_a]) - float(ref_l[ra])) <= 1e-4 + 1e-3 * abs(float(ref_l[ra])), "argmax differs"
    # argmax only (probs not written), repeated: each call must see a clean reduction state
    for rep in range(3):
        arg.upload(np.array([-1], np.int32))
        check(hip.sapphire_gemv_softmax_dev(dtype, layout, qm.ptr(), m, k, dx.ptr, logits.ptr, None, arg.ptr, None))
        assert int(arg.numpy()[0]) == got_a, f"repeat {rep}"
    # a different input vector on the same weights
    x2 = synth.normal_f32(k, 22, 4)
    dx2 = DeviceArray.from_numpy(x2)
    check(hip.sapphire_gemv_softmax_dev(dtype, layout, qm.ptr(), m, k, dx2.ptr, logits.ptr, probs.ptr, arg.ptr, None))
    l2 = logits.numpy()
    assert int(arg.numpy()[0]) == oracle.argmax(l2)
    ok, err = close(probs.numpy(), oracle.softmax(l2), rel=1e-3, abs_=1e-9)
    assert ok, f"probs (second input): max abs err {err}"
