"""sapphire_gemv_softmax_noalloc_dev (the LM head with its softmax / greedy epilogue, partials
in a fixed per-device array) against sapphire_gemv_softmax_dev, which allocates its partials:
the same kernels on the same inputs, so logits, probabilities and the greedy token must be
identical bit for bit. Two calls in a row, the second smaller, on each layout."""
import numpy as np
import pytest

from sapphire_amd import synth

pytestmark = pytest.mark.gpu

PACKED, TILED = 1, 2


def _run(hip, fn, dtype, layout, qm, x, with_probs):
    from sapphire_amd.device import DeviceArray, check
    m, k = qm.M, qm.K
    logits = DeviceArray.empty(m)
    probs = DeviceArray.empty(m) if with_probs else None
    arg = DeviceArray.empty(1, np.int32)
    arg.upload(np.array([-1], np.int32))
    check(fn(dtype, layout, qm.ptr(), m, k, x.ptr, logits.ptr, probs.ptr if probs else None, arg.ptr, None))
    check(hip.sapphire_synchronize())
    return logits.numpy(), (probs.numpy() if probs else None), int(arg.numpy()[0])


@pytest.mark.parametrize("layout", [TILED, PACKED], ids=["tiled", "packed"])
def test_noalloc_matches_allocating_entry_point(hip, oracle, layout):
    from sapphire_amd.device import DeviceArray, QMatrix
    fn = hip.sapphire_gemv_softmax_noalloc_dev
    cases = ([(synth.Q8_0, 262144, 640, True), (synth.Q4_0, 20000, 1152, False)] if layout == TILED
             else [(synth.Q4_0, 2048, 640, True), (synth.Q8_0, 1000, 640, True)])
    for i, (dtype, m, k, with_probs) in enumerate(cases):
        print(f"noalloc layout={layout} call={i} dtype={dtype} shape={m}x{k}", flush=True)
        W = synth.quant_matrix(dtype, m, k, seed=51, tensor_id=i)
        x = synth.normal_f32(k, 51, 10 + i)
        qm = QMatrix(dtype, W, layout=layout)
        dx = DeviceArray.from_numpy(x)
        got = _run(hip, fn, dtype, layout, qm, dx, with_probs)
        want = _run(hip, hip.sapphire_gemv_softmax_dev, dtype, layout, qm, dx, with_probs)
        assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
        if with_probs:
            assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32))
        assert got[2] == want[2]
        rows = np.arange(0, m, 97)
        assert got[2] == oracle.argmax(got[0]) and 0 <= got[2] < m
        ref = oracle.gemv(dtype, np.ascontiguousarray(W[rows]), x, nthreads=8)
        assert np.allclose(got[0][rows], ref, rtol=1e-3, atol=1e-4)


def test_noalloc_rejects_bad_arguments(hip):
    fn = hip.sapphire_gemv_softmax_noalloc_dev
    assert fn(synth.Q8_0, TILED, None, 16, 640, None, None, None, None, None) == -1
    assert fn(0, TILED, 256, 16, 640, 256, 256, None, 256, None) == -1            # F32 is not quantized
    assert fn(synth.Q8_0, TILED, 256, 16, 100, 256, 256, None, 256, None) == -1   # K not a multiple of 32
