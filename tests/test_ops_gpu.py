"""Primitive kernels on the GPU against the oracle (bit-exact with the reference).

Bit-exact: RMSNorm / RMSNorm-delta (same sum-of-squares order and correctly rounded
sqrt/divide), RoPE (same fused forms), residual add, argmax, vec_dot. Within the
parity tolerance (1e-3 rel / 1e-4 abs): GELU*up and softmax, which use the device
expf/tanhf.
"""
import numpy as np
import pytest

from sapphire_amd import synth
from tests.conftest import close

pytestmark = pytest.mark.gpu


def dev(a):
    from sapphire_amd.device import DeviceArray
    return DeviceArray.from_numpy(np.ascontiguousarray(a))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("dim,batch", [(640, 1), (256, 4), (1152, 1), (7, 3), (1001, 2), (256, 512), (640, 256)])
@pytest.mark.parametrize("delta", [True, False], ids=["delta", "plain"])
def test_rmsnorm_bit_exact(hip, oracle, dim, batch, delta):
    from sapphire_amd.device import DeviceArray, check
    x = synth.normal_f32((batch, dim), 1, dim) * 3
    w = synth.normal_f32(dim, 1, dim + 1, 1.0, 0.1)
    dx, dw, dy = dev(x), dev(w), DeviceArray.empty((batch, dim))
    fn = hip.sapphire_rmsnorm_delta_dev if delta else hip.sapphire_rmsnorm_dev
    check(fn(dy.ptr, dx.ptr, dw.ptr, 1e-6, dim, batch, None))
    got = dy.numpy()
    for b in range(batch):
        ref = oracle.rmsnorm_delta(x[b], w) if delta else oracle.rmsnorm(x[b], w)
        assert np.array_equal(bits(got[b]), bits(ref))


@pytest.mark.parametrize("base", [1e4, 1e6])
def test_rope_bit_exact(hip, oracle, base):
    from sapphire_amd.device import check
    hd, heads, max_ctx = 256, 4, 2048
    c, s = oracle.rope_tables(hd, max_ctx, base)
    dc, ds = dev(c), dev(s)
    x = synth.normal_f32((heads, hd), 2, int(base) % 97)
    for pos in (0, 1, 511, 1024, 2047):
        dx = dev(x)
        check(hip.sapphire_rope_apply_dev(dx.ptr, heads, hd, pos, dc.ptr, ds.ptr, None))
        got = dx.numpy()
        for h in range(heads):
            assert np.array_equal(bits(got[h]), bits(oracle.rope_apply(x[h], pos, c, s)))


def test_gelu_mul(hip, oracle):
    from sapphire_amd.device import check
    n = 6912
    g = synth.normal_f32(n, 3, 1) * 2
    u = synth.normal_f32(n, 3, 2)
    dg, du = dev(g), dev(u)
    check(hip.sapphire_gelu_mul_dev(dg.ptr, du.ptr, n, None))
    ok, err = close(dg.numpy(), oracle.gelu_mul(g, u))
    assert ok, err


def test_norm_residual_bit_exact(hip, oracle):
    from sapphire_amd.device import check
    dim = 640
    h = synth.normal_f32(dim, 4, 1) * 5
    r = synth.normal_f32(dim, 4, 2)
    w = synth.normal_f32(dim, 4, 3, 1.0, 0.1)
    dh, dr, dw = dev(h), dev(r), dev(w)
    check(hip.sapphire_norm_residual_dev(dh.ptr, dr.ptr, dw.ptr, 1e-6, dim, None))
    n = oracle.rmsnorm_delta(h, w)
    ref = (r + n).astype(np.float32)
    assert np.array_equal(bits(dr.numpy()), bits(ref))
    assert np.array_equal(bits(dh.numpy()), bits(ref))


@pytest.mark.parametrize("n", [1, 5, 1000, 65536, 262144, 300001])
def test_softmax_argmax(hip, oracle, n):
    from sapphire_amd.device import DeviceArray, check
    x = synth.normal_f32(n, 5, n % 1000) * 4
    if n > 10:
        x[n // 3] = x[n // 2] = x.max() + 1.0     # a tie: the lower index must win
    dx = dev(x)
    probs = DeviceArray.empty(n)
    arg = DeviceArray.empty(1, np.int32)
    check(hip.sapphire_softmax_argmax_dev(dx.ptr, n, probs.ptr, arg.ptr, None))
    assert int(arg.numpy()[0]) == oracle.argmax(x)
    ok, err = close(probs.numpy(), oracle.softmax(x), rel=1e-3, abs_=1e-6)
    assert ok, err
    # in place, argmax only
    check(hip.sapphire_softmax_argmax_dev(dx.ptr, n, None, arg.ptr, None))
    assert int(arg.numpy()[0]) == oracle.argmax(x)


def test_softmax_all_equal(hip, oracle):
    from sapphire_amd.device import DeviceArray, check
    n = 262144
    x = np.full(n, -3.25, np.float32)
    dx = dev(x)
    probs = DeviceArray.empty(n)
    arg = DeviceArray.empty(1, np.int32)
    check(hip.sapphire_softmax_argmax_dev(dx.ptr, n, probs.ptr, arg.ptr, None))
    assert int(arg.numpy()[0]) == 0
    ok, err = close(probs.numpy(), oracle.softmax(x), rel=1e-3, abs_=1e-9)
    assert ok, err


@pytest.mark.parametrize("fill", [np.nan, -np.inf], ids=["nan", "neg_inf"])
def test_argmax_without_a_finite_logit(hip, oracle, fill):
    """No logit above -inf: the greedy token is 0, as sample_greedy (utils.c:145-156) starts
    there, never an index outside [0, n) (a decode step embeds that token next). Covers the
    standalone softmax/argmax and the LM-head GEMV's fused epilogue."""
    from sapphire_amd.device import DeviceArray, QMatrix, check
    n = 20000
    x = np.full(n, fill, np.float32)
    arg = DeviceArray.empty(1, np.int32)
    arg.upload(np.array([-7], np.int32))
    dx = dev(x)                                   # held until the kernels have run
    check(hip.sapphire_softmax_argmax_dev(dx.ptr, n, None, arg.ptr, None))
    assert int(arg.numpy()[0]) == 0
    assert oracle.argmax(x) == 0
    # the fused epilogue: an activation vector of NaN (or -inf) makes every logit NaN (NaN
    # products, or +-inf terms of both signs), and the token is sample_greedy's 0
    W = synth.quant_matrix(synth.Q8_0, n, 640, seed=9, tensor_id=1)
    qm = QMatrix(synth.Q8_0, W, layout=2)
    xv = np.full(640, fill, np.float32)
    dxv = dev(xv)
    logits = DeviceArray.empty(n)
    arg.upload(np.array([-7], np.int32))
    check(hip.sapphire_gemv_softmax_dev(synth.Q8_0, 2, qm.ptr(), n, 640, dxv.ptr, logits.ptr, None, arg.ptr, None))
    ref = oracle.gemv(synth.Q8_0, W, xv, nthreads=8)
    assert np.isnan(ref).all() and np.isnan(logits.numpy()).all()
    assert int(arg.numpy()[0]) == oracle.argmax(ref) == 0
