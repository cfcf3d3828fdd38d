"""GEMV parity on the GPU against the oracle (which is bit-exact with the reference).

Tolerance for float outputs: |gpu - ref| <= 1e-4 + 1e-3*|ref| (north star). Integer
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
    qm = QMatrix(dtype, blocks, packed=(layout == 1), keep_aos=(layout == 0))
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


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
def test_lm_head_full_shape(hip, oracle, dtype):
    """262144 x 640, the LM-head shape, against the oracle on every row."""
    print(f"lm head dtype={dtype}", flush=True)
    W = synth.quant_matrix(dtype, 262144, 640, seed=3, tensor_id=dtype)
    x = synth.normal_f32(640, 3, 77)
    ref = oracle.gemv(dtype, W, x, nthreads=8)
    got = _gemv(hip, dtype, W, x, 1)
    ok, err = close(got, ref)
    assert ok, f"max abs err {err}"
    assert int(np.argmax(got)) == int(np.argmax(ref))


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("layout", [0, 1], ids=["aos", "packed"])
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
@pytest.mark.parametrize("layout", [0, 1], ids=["aos", "packed"])
def test_unpack_and_dequant_bit_exact(hip, oracle, dtype, layout):
    """Every byte value in every quant position; ints and fl(int*scale) bit for bit."""
    from sapphire_amd.device import DeviceArray, QMatrix, check
    nb = 256
    W = np.zeros((4, nb), dtype=synth.block_dtype(dtype))
    vals = np.arange(256, dtype=np.uint8)
    qb = 16 if dtype == synth.Q4_0 else 32
    for r in range(4):
        for b in range(nb):
            W["q"][r, b] = np.roll(vals, b + 13 * r)[:qb].view(W["q"].dtype)
    W["scale"] = synth.normal_f32((4, nb), 9, 9, 0.0, 0.01)
    qm = QMatrix(dtype, W, packed=(layout == 1), keep_aos=(layout == 0))
    L = hip
    ints = DeviceArray.empty(4 * nb * 32, np.int8)
    deq = DeviceArray.empty(4 * nb * 32, np.float32)
    check(L.sapphire_q_unpack_ints_dev(dtype, layout, qm.ptr(layout), 4, nb * 32, ints.ptr, None))
    check(L.sapphire_q_dequant_dev(dtype, layout, qm.ptr(layout), 4, nb * 32, deq.ptr, None))
    got_i = ints.numpy()
    assert np.array_equal(got_i, oracle.unpack_ints(dtype, W))
    assert np.array_equal(got_i, synth.unpack_ints(dtype, W).reshape(-1))
    assert np.array_equal(deq.numpy().view(np.uint32), oracle.dequant(dtype, W).view(np.uint32))
