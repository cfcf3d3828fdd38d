"""Pins of the oracle's quantizer (oracle_quantize).

The reference has no quantizer; the oracle restates ggml's published reference quantizer
with the reference's fp32 scale and Q4_0 nibble order. What pins it:
* known answers written by hand, including the rounding of ties and the clipping of Q4_0;
* the all-zero block and the first-occurrence rule for the Q4_0 extreme;
* reconstruction bounds and exactness of the extreme element on random rows;
* idempotence on blocks that are exactly representable;
* the layout, through the reference's own row kernels (compiled from its sources when
  available, else the oracle's restatement, which is pinned to them bit for bit): a dot
  product with the produced blocks must equal the dot product with the original weights up
  to the quantization error, which a wrong nibble order or scale would break.
"""
import numpy as np
import pytest

from oracle.oracle import Reference
from sapphire_amd import synth

Q4, Q8, F32, BF16 = synth.Q4_0, synth.Q8_0, synth.F32, synth.BF16


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def block_row(vals):
    x = np.zeros((1, 32), np.float32)
    x[0, :len(vals)] = vals
    return x


def deq(oracle, dtype, blocks):
    return oracle.dequant(dtype, blocks).reshape(blocks.shape[0], -1)


def test_q8_known_answers(oracle):
    # amax 127 -> d = 1, 1/d = 1; roundf rounds ties away from zero
    b = oracle.quantize(Q8, F32, block_row([127, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 0.49, -126.6]))
    assert bits(b["scale"])[0, 0] == bits(1.0)
    assert list(oracle.unpack_ints(Q8, b)[:9]) == [127, 64, -64, 1, -1, 2, -3, 0, -127]
    # amax 2.54 -> d = fl(2.54/127)
    b = oracle.quantize(Q8, F32, block_row([-2.54, 1.27, 0.02]))
    assert b["scale"][0, 0] == np.float32(np.float32(2.54) / np.float32(127))
    assert list(oracle.unpack_ints(Q8, b)[:3]) == [-127, 64, 1]


def test_q4_known_answers(oracle):
    # max 8 -> d = -1, 1/d = -1; q = trunc(x * -1 + 8.5) clipped at 15, value q - 8
    b = oracle.quantize(Q4, F32, block_row([8, -7.5, 0.5, -0.5, 1.5, 2.4, -2.6, 3.5, -8.0 + 1e-6]))
    assert bits(b["scale"])[0, 0] == bits(-1.0)
    assert list(oracle.unpack_ints(Q4, b)[:9]) == [-8, 7, 0, 1, -1, -2, 3, -3, 7]
    # the extreme is the first element of largest |x|: -4 comes before +4, so max = -4, d = 0.5
    b = oracle.quantize(Q4, F32, block_row([1, -4, 2, 4]))
    assert b["scale"][0, 0] == np.float32(0.5)
    assert list(oracle.unpack_ints(Q4, b)[:4]) == [2, -8, 4, 7]   # 4 * 2 = 8 -> clipped to 7
    b = oracle.quantize(Q4, F32, block_row([1, 4, 2, -4]))
    assert b["scale"][0, 0] == np.float32(-0.5)
    assert list(oracle.unpack_ints(Q4, b)[:4]) == [-2, -8, -4, 7]
    # nibble order: element 2j in the low nibble of byte j
    b = oracle.quantize(Q4, F32, block_row([8, 0, -7]))
    assert b["q"][0, 0, 0] == (0 | (8 << 4)) and b["q"][0, 0, 1] & 0x0F == 15


def test_zero_block(oracle):
    z = np.zeros((2, 32), np.float32)
    z[1, 5] = -0.0
    b4 = oracle.quantize(Q4, F32, z)
    assert (bits(b4["scale"]) == 0x80000000).all()      # d = +0 / -8 = -0
    assert (b4["q"] == 0x88).all()
    b8 = oracle.quantize(Q8, F32, z)
    assert (bits(b8["scale"]) == 0).all() and (b8["q"] == 0).all()


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("dist", ["normal", "heavy", "scaled"])
def test_reconstruction_bounds(oracle, dtype, dist):
    g = np.random.default_rng(7 + dtype)
    if dist == "normal":
        x = g.standard_normal((64, 640)).astype(np.float32)
    elif dist == "heavy":
        x = (g.standard_t(2, (64, 640)) * 0.1).astype(np.float32)
    else:
        x = (g.standard_normal((64, 640)) * np.exp2(g.integers(-60, 60, (64, 1)))).astype(np.float32)
    b = oracle.quantize(dtype, F32, x)
    w = deq(oracle, dtype, b).astype(np.float64)
    d = np.repeat(np.abs(b["scale"].astype(np.float64)), 32, axis=1)
    err = np.abs(w - x)
    ints = oracle.unpack_ints(dtype, b).reshape(x.shape).astype(np.int64)
    xb = x.reshape(64, 20, 32)
    amax = np.abs(xb).max(axis=2)
    if dtype == Q8:
        # d = amax/127 to 1 ulp, every element within half a step (plus fp32 rounding)
        assert np.allclose(b["scale"], amax / 127, rtol=2 ** -23, atol=0)
        assert (err <= d * (0.5 + 1e-5)).all()
        assert (np.abs(ints) <= 127).all()
    else:
        # the extreme element reconstructs exactly; the others within half a step, except
        # those clipped at code 15 (within one step)
        first = np.abs(xb).argmax(axis=2)
        ext = np.take_along_axis(xb, first[..., None], axis=2)[..., 0]
        wb = w.reshape(64, 20, 32)
        assert np.array_equal(np.take_along_axis(wb, first[..., None], axis=2)[..., 0], ext.astype(np.float64))
        clipped = ints == 7
        assert (err[~clipped] <= d[~clipped] * (0.5 + 1e-5)).all()
        assert (err <= d * (1 + 1e-5)).all()


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
def test_idempotent_on_representable_blocks(oracle, dtype):
    """Blocks that are exactly ints * 2^-e (with the extreme code present) quantize to
    themselves: scale and every code."""
    g = np.random.default_rng(11)
    m = 50
    if dtype == Q8:
        ints = g.integers(-127, 128, (m, 32))
        ints[np.arange(m), g.integers(0, 32, m)] = 127 * g.choice([-1, 1], m)
        scale = np.exp2(g.integers(-20, 5, (m, 1))).astype(np.float64)
    else:
        ints = g.integers(-7, 8, (m, 32))
        ints[np.arange(m), g.integers(0, 32, m)] = -8
        scale = -np.exp2(g.integers(-20, 5, (m, 1))).astype(np.float64)
    x = (ints * scale).astype(np.float32)
    b = oracle.quantize(dtype, F32, x)
    assert np.array_equal(b["scale"][:, 0], scale[:, 0].astype(np.float32))
    assert np.array_equal(oracle.unpack_ints(dtype, b).reshape(m, 32), ints)


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
def test_bf16_source_is_widened_f32(oracle, dtype):
    w = synth.bf16_normal((33, 96), 3, 4)
    wf = (w.astype(np.uint32) << 16).view(np.float32)
    a, b = oracle.quantize(dtype, BF16, w), oracle.quantize(dtype, F32, wf)
    assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
def test_ragged_k_pads_zeros(oracle, dtype):
    x = synth.normal_f32((9, 100), 5, 6)
    xp = np.zeros((9, 128), np.float32)
    xp[:, :100] = x
    assert oracle.quantize(dtype, F32, x).tobytes() == oracle.quantize(dtype, F32, xp).tobytes()


def test_subnormal_scale_is_defined(oracle):
    """amax/127 below the normal range: 1/d overflows; infinite products saturate, NaN ones
    (0 * inf) give the code of zero."""
    x = block_row([1e-39, -5e-40, 0.0])
    b8 = oracle.quantize(Q8, F32, x)
    assert list(oracle.unpack_ints(Q8, b8)[:3]) == [127, -127, 0]
    b4 = oracle.quantize(Q4, F32, x)
    assert list(oracle.unpack_ints(Q4, b4)[:3]) == [-8, 7, 0]


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
def test_layout_through_reference_row_kernel(oracle, dtype):
    """Quantized rows fed to the reference's own row kernel (quantized_gemv_q{4,8}_0) give
    the dot product of the original weights up to the quantization error."""
    ref = Reference() if Reference.available() else None
    g = np.random.default_rng(21)
    w = g.standard_normal((16, 640)).astype(np.float32)
    x = g.standard_normal(640).astype(np.float32)
    b = oracle.quantize(dtype, F32, w)
    wq = deq(oracle, dtype, b).astype(np.float64)
    bound = np.abs(x.astype(np.float64)) @ np.abs(wq - w).T
    for r in range(16):
        got = ref.row(dtype, b[r], x) if ref is not None else oracle.row(dtype, b[r], x)
        exact_q = float(wq[r] @ x.astype(np.float64))
        assert abs(got - exact_q) <= 1e-4 * (1 + abs(exact_q))        # the kernel reads our layout
        assert abs(exact_q - float(w[r].astype(np.float64) @ x)) <= bound[r] + 1e-9
        # ... and the layout matters: a permuted block (ggml's j, j+16 nibble order) is far off
    if dtype == Q4:
        perm = np.concatenate([np.arange(0, 32, 2), np.arange(1, 32, 2)])
        wp = wq.reshape(16, 20, 32)[:, :, perm].reshape(16, 640)
        exact = w.astype(np.float64) @ x
        assert np.abs(wp @ x - exact).mean() > 5 * np.abs(wq @ x - exact).mean()
