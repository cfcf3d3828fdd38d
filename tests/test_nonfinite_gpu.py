"""NaN and infinite activations through every quantized GEMV path, against the oracle.

The reference accumulates fl(w * x) with fp32 FMAs (q4_0_avx.c:31-42, q8_0_avx.c:50-64), so
one NaN activation makes every row NaN, and an infinite one makes a row +-inf by the sign of
its weight there, or NaN where that weight is 0 (0 * inf) or where infinities of both signs
meet. The GPU kernels compute the finite part with integer digits, offsets and range scales,
and fold the non-finite elements in separately; these tests require the NaN pattern and every
infinity of the oracle exactly, and the finite rows (none here) to the usual tolerance.
"""
import ctypes as C

import numpy as np
import pytest

from sapphire_amd import synth
from tests.conftest import close

pytestmark = pytest.mark.gpu

AOS, PACKED, TILED = 0, 1, 2


def _zero_weight(dtype, W, rows, k):
    """Sets the integer weight of element k to 0 in the given rows (Q4_0: nibble 8)."""
    b, e = divmod(k, 32)
    for r in rows:
        if dtype == synth.Q8_0:
            W[r, b]["q"][e] = 0
        else:
            byte = int(W[r, b]["q"][e >> 1])
            byte = (byte & 0x0F) | 0x80 if e & 1 else (byte & 0xF0) | 0x08
            W[r, b]["q"][e >> 1] = byte


def _patterns(k, seed):
    """Activation vectors with non-finite elements: one NaN; one +inf; +inf and -inf in
    different blocks; several infinities inside one block with finite neighbours."""
    base = synth.normal_f32(k, seed, 3)
    out = {}
    x = base.copy(); x[k // 3] = np.nan; out["nan"] = x
    x = base.copy(); x[5] = np.inf; out["pinf"] = x
    x = base.copy(); x[5] = np.inf; x[k - 7] = -np.inf; out["both"] = x
    x = base.copy(); x[64:72:2] = np.inf; x[70] = -np.inf; out["block"] = x
    return out


def _same_special(got, ref):
    """Identical NaN positions and identical values elsewhere (infinities included)."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), f"NaN pattern differs at {np.flatnonzero(np.isnan(got) != nan)[:8]}"
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf]), "infinite rows differ"
    fin = ~(nan | inf)
    if fin.any():
        ok, err = close(got[fin], ref[fin])
        assert ok, f"finite rows: max abs err {err}"


def _matrix(dtype, m, k, seed):
    W = synth.quant_matrix(dtype, m, k, seed=seed, tensor_id=m + k)
    _zero_weight(dtype, W, [0, 3], 5)            # 0 * inf -> NaN rows
    _zero_weight(dtype, W, [1], k - 7)
    return W


GEMV_CASES = [
    (AOS, 2048, 640), (PACKED, 2048, 640),       # column kernel
    (PACKED, 640, 2048),
    (AOS, 96, 6912), (PACKED, 96, 6912),         # row kernel
    (TILED, 20000, 640), (TILED, 4099, 1024), (TILED, 333, 1152),   # matrix cores
]


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("case", GEMV_CASES, ids=lambda c: f"{['aos', 'packed', 'tiled'][c[0]]}-{c[1]}x{c[2]}")
def test_gemv_non_finite_activations(hip, oracle, dtype, case):
    from sapphire_amd.device import DeviceArray, QMatrix, gemv
    layout, m, k = case
    W = _matrix(dtype, m, k, 41)
    qm = QMatrix(dtype, W, layout=layout)
    for name, x in _patterns(k, 41).items():
        print(f"gemv non-finite dtype={dtype} layout={layout} shape={m}x{k} pattern={name}", flush=True)
        ref = oracle.gemv(dtype, W, x, nthreads=4)
        dy = DeviceArray.empty(m)
        gemv(qm, DeviceArray.from_numpy(x), dy, layout)
        got = dy.numpy()
        if name == "nan":
            assert np.isnan(ref).all()
        elif name in ("pinf", "both"):                # zero weights under x[5] = +inf
            assert np.isnan(ref[[0, 3]]).all() and np.isinf(ref).any()
        else:
            assert np.isinf(ref).any()
        _same_special(got, ref)


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("layout", [PACKED, TILED], ids=["packed", "tiled"])
def test_gemv_softmax_non_finite(hip, oracle, dtype, layout):
    """The LM head with its fused softmax / greedy epilogue: logits as the oracle's, every
    probability NaN (the reference's sum includes exp(inf - inf) or a NaN), and the greedy
    token of sample_greedy (the first +inf; 0 when logits[0] is NaN)."""
    from sapphire_amd.device import DeviceArray, QMatrix, check
    m, k = 20000, 640
    W = _matrix(dtype, m, k, 42)
    qm = QMatrix(dtype, W, layout=layout)
    for name, x in _patterns(k, 42).items():
        print(f"gemv_softmax non-finite dtype={dtype} layout={layout} pattern={name}", flush=True)
        ref = oracle.gemv(dtype, W, x, nthreads=4)
        ref_p = oracle.softmax(ref)
        logits, probs = DeviceArray.empty(m), DeviceArray.empty(m)
        arg = DeviceArray.empty(1, np.int32)
        dx = DeviceArray.from_numpy(x)              # held until the kernels have run
        check(hip.sapphire_gemv_softmax_dev(dtype, layout, qm.ptr(), m, k, dx.ptr, logits.ptr, probs.ptr, arg.ptr,
                                            None))
        _same_special(logits.numpy(), ref)
        assert np.isnan(ref_p).all() and np.isnan(probs.numpy()).all()
        assert int(arg.numpy()[0]) == oracle.argmax(ref)


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("layout", [TILED, PACKED], ids=["tiled", "packed"])
@pytest.mark.parametrize("shape", [(1536, 1152), (1152, 6912), (20000, 1152)], ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemm_batch16_non_finite(hip, oracle, dtype, layout, shape):
    """sapphire_gemm_q_dev at 16 sequences: sequences with a NaN, a +inf, +inf and -inf in
    different K chunks, several infinities in one block, and finite sequences, in one call."""
    from sapphire_amd.device import DeviceArray, QMatrix, check
    m, k = shape
    W = _matrix(dtype, m, k, 43)
    X = synth.normal_f32((16, k), 43, 5)
    pats = list(_patterns(k, 44).values())
    for i, b in enumerate([1, 4, 9, 15]):
        X[b] = pats[i]
    X[12, k - 1] = -np.inf
    print(f"gemm batch16 non-finite dtype={dtype} layout={layout} shape={shape}", flush=True)
    qm = QMatrix(dtype, W, layout=layout)
    dX = DeviceArray.from_numpy(X)
    dY = DeviceArray.empty(16 * m)
    ws = DeviceArray(max(256, hip.sapphire_gemm_workspace_bytes(dtype, m, k)))
    check(hip.sapphire_gemm_q_dev(dtype, layout, qm.ptr(), m, k, dX.ptr, 16, dY.ptr, ws.ptr, None))
    got = dY.numpy().reshape(16, m)
    for b in range(16):
        ref = oracle.gemv(dtype, W, X[b], nthreads=8)
        if b in (1, 4, 9, 12, 15):
            assert not np.isfinite(ref).any()
        _same_special(got[b], ref)


def test_fused_gemm_non_finite_residual(hip, oracle):
    """The fused batched GEMM input of a decode step (sum of partials + residual, then the
    pre-norm): an infinite residual element turns into NaN through the norm (inf * 0), and
    the NaN reaches every output of that sequence, as in the reference's rmsnorm_delta +
    kernel_gemv. Sequences without one stay finite."""
    from sapphire_amd.device import DeviceArray, QMatrix, check
    from sapphire_amd._lib import GemmInput, GemmOutput
    dtype, m, k, B = synth.Q4_0, 1536, 1152, 16
    W = synth.quant_matrix(dtype, m, k, seed=45, tensor_id=1)
    x = synth.normal_f32((B, k), 45, 2)
    x[3, 10] = np.inf
    wn = (1 + 0.1 * synth.normal_f32(k, 45, 3)).astype(np.float32)
    qm = QMatrix(dtype, W, layout=TILED)
    dx, dwn = DeviceArray.from_numpy(x), DeviceArray.from_numpy(wn)
    dy = DeviceArray.empty(B * m)
    gi = GemmInput(x=dx.ptr, ldx=k, w_norm=dwn.ptr, eps=1e-6)
    go = GemmOutput(y=dy.ptr, ldy=m)
    check(hip.sapphire_gemm_q_fused_dev(dtype, qm.ptr(), m, k, B, C.byref(gi), C.byref(go), None, None))
    got = dy.numpy().reshape(B, m)
    for b in (0, 3, 15):
        normed = oracle.rmsnorm_delta(x[b], wn)
        ref = oracle.gemv(dtype, W, normed, nthreads=8)
        if b == 3:
            assert np.isnan(normed[10]) and np.isnan(ref).all()
        _same_special(got[b], ref)


def test_greedy_token_when_logit_zero_is_nan(hip, oracle):
    """sample_greedy (utils.c:145-156) seeds its best logit with logits[0]; nothing compares
    greater than NaN, so a NaN there makes the token 0 whatever the other logits are. A NaN
    block scale in row 0 of the LM head makes logits[0] NaN through the fused epilogue; the
    standalone argmax is given the same logits."""
    from sapphire_amd.device import DeviceArray, QMatrix, check
    m, k = 20000, 640
    for dtype in (synth.Q4_0, synth.Q8_0):
        W = synth.quant_matrix(dtype, m, k, seed=46, tensor_id=dtype)
        W[0, 2]["scale"] = np.nan
        x = synth.normal_f32(k, 46, 1)
        ref = oracle.gemv(dtype, W, x, nthreads=4)
        assert np.isnan(ref[0]) and np.isfinite(ref[1:]).all()
        assert oracle.argmax(ref) == 0
        qm = QMatrix(dtype, W, layout=TILED)
        logits = DeviceArray.empty(m)
        arg = DeviceArray.empty(1, np.int32)
        arg.upload(np.array([-7], np.int32))
        dx = DeviceArray.from_numpy(x)
        check(hip.sapphire_gemv_softmax_dev(dtype, TILED, qm.ptr(), m, k, dx.ptr, logits.ptr, None, arg.ptr, None))
        got = logits.numpy()
        assert np.isnan(got[0]) and int(arg.numpy()[0]) == 0
        arg.upload(np.array([-7], np.int32))
        dref = DeviceArray.from_numpy(ref)
        check(hip.sapphire_softmax_argmax_dev(dref.ptr, m, None, arg.ptr, None))
        assert int(arg.numpy()[0]) == 0
        # the same logits with a finite logits[0]: the first maximum of the rest
        ref2 = ref.copy()
        ref2[0] = 0.0
        dref2 = DeviceArray.from_numpy(ref2)
        check(hip.sapphire_softmax_argmax_dev(dref2.ptr, m, None, arg.ptr, None))
        assert int(arg.numpy()[0]) == oracle.argmax(ref2) != 0
