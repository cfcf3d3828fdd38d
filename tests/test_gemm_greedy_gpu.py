"""The batched LM head with the greedy pick fused into the GEMM (sapphire_gemm_q_greedy_dev, and
the batched decoder's step when it returns no logits) on the GPU.

The fused form forms every row with the arithmetic of the unfused GEMM (sapphire_gemm_q_dev)
and keeps only the best row per sequence, so its tokens must equal, exactly, the oracle's
greedy pick (sample_greedy, utils.c:145-156, through oracle.sample at temperature 0) over the
rows the unfused GEMM stores: ties go to the first index, NaN rows never win, and a NaN in
row 0 gives token 0.
"""
import numpy as np
import pytest

from sapphire_amd import model as smodel
from sapphire_amd import synth
from tests.test_gemm_gpu import TILED, _gemm

pytestmark = pytest.mark.gpu


def _greedy(hip, qm, X):
    from sapphire_amd.device import DeviceArray, check
    batch = X.shape[0]
    dX = DeviceArray.from_numpy(np.ascontiguousarray(X, np.float32))
    dT = DeviceArray.empty(batch, np.int32)
    ws = DeviceArray(hip.sapphire_gemm_workspace_bytes(qm.dtype, qm.M, qm.K))
    check(hip.sapphire_gemm_q_greedy_dev(qm.dtype, qm.ptr(TILED), qm.M, qm.K, dX.ptr, batch, dT.ptr, ws.ptr, None))
    return dT.numpy()


def _expected(oracle, Y):
    return np.array([oracle.sample(Y[b], 0.0, 0.0)[0] for b in range(Y.shape[0])], np.int32)


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("shape,batch", [((262144, 1152), 16), ((262144, 640), 5), ((333, 1152), 16),
                                         ((1024, 1152), 3), ((17, 128), 16)],
                         ids=["lm_head_1b_b16", "lm_head_270m_b5", "ragged_b16", "1024_b3", "one_group_b16"])
def test_greedy_matches_stored_rows(hip, oracle, dtype, shape, batch):
    """Normal rows, the streaming launch (the LM heads) and the 8-wave one, ragged M."""
    from sapphire_amd.device import QMatrix
    m, k = shape
    print(f"greedy gemm dtype={dtype} shape={shape} batch={batch}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=41, tensor_id=m + k)
    X = synth.normal_f32((batch, k), 41, batch)
    qm = QMatrix(dtype, W, layout=TILED)
    Y = _gemm(hip, qm, X)
    got = _greedy(hip, qm, X)
    assert np.array_equal(got, _expected(oracle, Y)), (got, _expected(oracle, Y))


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("m", [262144, 5000], ids=["streaming", "8_waves"])
def test_greedy_ties_and_special_values(hip, oracle, dtype, m):
    """Rows repeat with period 7 (every maximum is tied across many tiles and workgroups: the
    first index wins); an all-zero sequence (every row 0: token 0); a NaN activation (every
    row NaN: token 0); infinite activations (rows +inf, -inf or NaN by the weight's sign)."""
    from sapphire_amd.device import QMatrix
    k = 1152
    print(f"greedy gemm ties dtype={dtype} m={m}", flush=True)
    base = synth.quant_matrix(dtype, 7, k, seed=42, tensor_id=7)
    W = base[np.arange(m) % 7]
    X = synth.normal_f32((16, k), 42, 3)
    X[1] = 0.0
    X[2, 500] = np.nan
    X[3, 77] = np.inf
    X[4, 900] = -np.inf
    qm = QMatrix(dtype, W, layout=TILED)
    Y = _gemm(hip, qm, X)
    exp = _expected(oracle, Y)
    assert exp[0] < 7 and exp[1] == 0 and exp[2] == 0
    got = _greedy(hip, qm, X)
    assert np.array_equal(got, exp), (got, exp)


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
def test_greedy_nan_row_zero(hip, oracle, dtype):
    """An infinite activation at element 2 where row 0's weight is 0 and every other row's is
    positive: row 0 is NaN (0 * inf) and the others +inf. sample_greedy keeps index 0, as
    nothing compares greater than its starting NaN; without that rule a +inf row would win."""
    from sapphire_amd.device import QMatrix
    m, k = 262144, 1152
    print(f"greedy gemm nan row 0 dtype={dtype}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=43, tensor_id=5)
    if dtype == synth.Q4_0:   # element 2: the low nibble of byte 1, weight = nibble - 8
        W["q"][:, 0, 1] = (W["q"][:, 0, 1] & 0xF0) | (9 + np.arange(m) % 7).astype(np.uint8)
        W["q"][0, 0, 1] = (W["q"][0, 0, 1] & 0xF0) | 8
    else:
        W["q"][:, 0, 2] = (1 + np.arange(m) % 100).astype(np.int8)
        W["q"][0, 0, 2] = 0
    w2 = synth.unpack_ints(dtype, W[:, :1])[:, 2]
    assert w2[0] == 0 and np.all(w2[1:] > 0)
    X = synth.normal_f32((4, k), 43, 1)
    X[0, 2] = np.inf
    qm = QMatrix(dtype, W, layout=TILED)
    Y = _gemm(hip, qm, X)
    assert np.isnan(Y[0, 0]) and np.all(Y[0, 1:] == np.inf)
    exp = _expected(oracle, Y)
    assert exp[0] == 0
    got = _greedy(hip, qm, X)
    assert np.array_equal(got, exp), (got, exp)


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("m,win", [(262144, 16 * 1000 + 5), (5000, 16 * 100 + 5)], ids=["streaming", "8_waves"])
def test_greedy_nan_rows_do_not_block(hip, oracle, dtype, m, win):
    """An infinite activation at element 2: row `win` has a positive weight there (+inf), row 0
    and every 7th row a negative one (-inf), all other rows 0 (NaN), so the first row of the
    winner's tile and most of its lanes are NaN. sample_greedy skips the NaN rows: the token is
    `win`."""
    from sapphire_amd.device import QMatrix
    k = 1152
    print(f"greedy gemm nan rows dtype={dtype} m={m}", flush=True)
    W = synth.quant_matrix(dtype, m, k, seed=45, tensor_id=m)
    w = np.zeros(m, np.int64)
    w[::7] = -1
    w[win] = 1
    if dtype == synth.Q4_0:   # element 2: the low nibble of byte 1, weight = nibble - 8
        W["q"][:, 0, 1] = (W["q"][:, 0, 1] & 0xF0) | (8 + w).astype(np.uint8)
    else:
        W["q"][:, 0, 2] = w.astype(np.int8)
    assert np.array_equal(synth.unpack_ints(dtype, W[:, :1])[:, 2], w)
    X = synth.normal_f32((3, k), 45, 2)
    X[0, 2] = np.inf
    X[2, 2] = -np.inf
    qm = QMatrix(dtype, W, layout=TILED)
    Y = _gemm(hip, qm, X)
    assert np.isnan(Y[0, 16 * (win // 16)]) and Y[0, win] == np.inf
    exp = _expected(oracle, Y)
    assert exp[0] == win
    got = _greedy(hip, qm, X)
    assert np.array_equal(got, exp), (got, exp)


def test_greedy_rejects(hip):
    from sapphire_amd.device import DeviceArray, QMatrix
    W = synth.quant_matrix(synth.Q4_0, 64, 4608, seed=44, tensor_id=1)
    qm = QMatrix(synth.Q4_0, W, layout=TILED)
    X = DeviceArray.empty((2, 4608))
    T = DeviceArray.empty(2, np.int32)
    ws = DeviceArray(hip.sapphire_gemm_workspace_bytes(synth.Q4_0, 64, 4608))
    # K over one chunk, no workspace, batch over 16
    assert hip.sapphire_gemm_q_greedy_dev(synth.Q4_0, qm.ptr(TILED), 64, 4608, X.ptr, 2, T.ptr, ws.ptr, None) == -1
    W2 = synth.quant_matrix(synth.Q4_0, 64, 1152, seed=44, tensor_id=2)
    qm2 = QMatrix(synth.Q4_0, W2, layout=TILED)
    assert hip.sapphire_gemm_q_greedy_dev(synth.Q4_0, qm2.ptr(TILED), 64, 1152, X.ptr, 2, T.ptr, None, None) == -1
    assert hip.sapphire_gemm_q_greedy_dev(synth.Q4_0, qm2.ptr(TILED), 64, 1152, X.ptr, 17, T.ptr, ws.ptr, None) == -1


@pytest.mark.parametrize("cfg,batch,prefill", [(smodel.TINY, 16, 20), (smodel.GEMMA3_1B, 16, 1024)],
                         ids=["tiny_b16", "gemma3_1b_b16"])
def test_decoder_greedy_step_without_logits(cfg, batch, prefill):
    """The batched decoder picks its tokens inside the LM-head GEMM when the caller takes no
    logits: the tokens equal those of the step that stores the logits and picks afterwards."""
    from sapphire_amd.engine import Decoder
    print(f"decoder greedy without logits: vocab {cfg.vocab}, hidden {cfg.hidden}, batch {batch}", flush=True)
    m = smodel.synthetic_model(cfg, 20260107)
    k, v = m.kv_prefill(prefill)
    dec = Decoder(m, batch=batch)
    try:
        toks0 = synth.rng(20260107, 1).integers(0, cfg.vocab, size=batch).astype(np.int32)
        pos = np.full(batch, prefill, np.int32)
        runs = []
        for keep in (True, False, True):
            for b in range(batch):
                dec.set_kv_seq(b, k, v)
            t, _, _ = dec.generate_batch(toks0, pos, 4, keep_logits=keep)
            runs.append(t)
        assert np.array_equal(runs[0], runs[1]) and np.array_equal(runs[0], runs[2])
    finally:
        dec.close()
