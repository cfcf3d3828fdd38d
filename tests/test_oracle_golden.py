"""The oracle against the golden fixtures written by tests/golden/make_golden.py from the
compiled reference (bit for bit), and against the reference's own known answers."""
import hashlib
import json
import os

import numpy as np
import pytest

from sapphire_amd import model as smodel
from sapphire_amd import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
Q4, Q8 = synth.Q4_0, synth.Q8_0


def load_npz(name):
    return np.load(os.path.join(GOLD, name))      # allow_pickle stays False


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_dispatch_known_answer(oracle):
    """test_dispatch.c:6-29 prints -0.08400002 for its 4-block row."""
    ka = json.load(open(os.path.join(GOLD, "known_answers.json")))["dispatch_row"]
    W, x = _dispatch_row()
    got = oracle.row(Q4, W, x)
    assert int(got.view(np.uint32)) == ka["unaligned_bits"] == ka["aligned_bits"]
    assert f"{float(got):.8f}" == ka["printed"]


def _dispatch_row():
    W = np.zeros(4, synth.Q4_BLOCK)
    for b in range(4):
        W[b]["scale"] = np.float32(0.05) * np.float32(1.0 + b)
        W[b]["q"] = [(((i + 1) & 0x0F) << 4) | (i & 0x0F) for i in range(16)]
    x = (np.float32(0.001) * np.arange(1, 129, dtype=np.float32)).astype(np.float32)
    return W, x


def _e2e(rows, bpr):
    r = np.arange(rows)[:, None]
    b = np.arange(bpr)[None, :]
    sc = (np.float32(0.01) * (1.0 + ((r + b) & 7)).astype(np.float32)).astype(np.float32)
    W4 = np.zeros((rows, bpr), synth.Q4_BLOCK)
    W4["scale"] = sc
    i = np.arange(16)[None, None, :]
    W4["q"] = ((((i * 2 + 1 + r[..., None] + b[..., None]) & 0x0F) << 4)
               | ((i * 2 + r[..., None] + b[..., None]) & 0x0F)).astype(np.uint8)
    W8 = np.zeros((rows, bpr), synth.Q8_BLOCK)
    W8["scale"] = sc
    i = np.arange(32)[None, None, :]
    W8["q"] = (((i + r[..., None] + b[..., None]) & 0x1F) - 16).astype(np.int8)
    x = (np.float32(0.001) * np.arange(1, bpr * 32 + 1, dtype=np.float32)).astype(np.float32)
    return W4, W8, x


# sum(y) printed by bench_sapphire_end_to_end (8 decimals), rows/blocks_per_row
E2E_PRINTED = {
    (64, 2): ("-3.10272011", "-3.10272005"), (128, 4): ("-24.20736024", "-24.20736025"),
    (256, 8): ("-191.20128822", "-191.20128024"), (1024, 16): ("-3039.55981445", "-3039.55963898"),
    (8192, 32): ("-96951.33789062", "-96951.33959961"),
}


@pytest.mark.parametrize("case", range(5))
def test_end_to_end_sums(oracle, case):
    ka = json.load(open(os.path.join(GOLD, "known_answers.json")))["e2e_sums"][case]
    rows, bpr = ka["rows"], ka["blocks_per_row"]
    W4, W8, x = _e2e(rows, bpr)
    y4 = oracle.gemv(Q4, W4, x, nthreads=4)
    y8 = oracle.gemv(Q8, W8, x, nthreads=4)
    assert hashlib.sha256(y4.tobytes()).hexdigest() == ka["q4_y_sha256"]
    assert hashlib.sha256(y8.tobytes()).hexdigest() == ka["q8_y_sha256"]
    p4, p8 = E2E_PRINTED[(rows, bpr)]
    assert f"{np.sum(y4.astype(np.float64)):.8f}" == p4
    assert f"{np.sum(y8.astype(np.float64)):.8f}" == p8


def gemv_cases():
    g = load_npz("gemv.npz")
    return sorted({k.rsplit("_", 1)[0] for k in g.files})


@pytest.mark.parametrize("key", gemv_cases())
def test_gemv_fixture(oracle, key):
    g = load_npz("gemv.npz")
    dt = Q4 if key.startswith("Q4_0") else Q8
    m, k = map(int, key.split("_")[-1].split("x"))
    W = g[key + "_w"].view(synth.block_dtype(dt)).reshape(m, -1)
    for nt in (1, 3):
        y = oracle.gemv(dt, W, g[key + "_x"], nthreads=nt)
        assert np.array_equal(bits(y), bits(g[key + "_y"]))


def gemv_f_cases():
    g = load_npz("gemv_f.npz")
    return sorted({k.rsplit("_", 1)[0] for k in g.files})


@pytest.mark.parametrize("key", gemv_f_cases())
def test_gemv_f_fixture(oracle, key):
    """F32 / BF16 rows: the pooled kernel (bf16_avx.c:57-113, f32_avx.c), kernel_gemv without a
    context (dispatch.c:60-85) and the batched kernel (kernel_gemm_*_avx2), against the
    compiled reference's outputs bit for bit."""
    g = load_npz("gemv_f.npz")
    dt = 0 if key.startswith("F32") else 1
    w, x, X = g[key + "_w"], g[key + "_x"], g[key + "_X"]
    for nt in (1, 3):
        assert np.array_equal(bits(oracle.gemv(dt, w, x, nthreads=nt)), bits(g[key + "_y"]))
    assert np.array_equal(bits(oracle.gemv_scalar(dt, w, x)), bits(g[key + "_ynoctx"]))
    assert np.array_equal(bits(oracle.gemm_f(dt, w, X)), bits(g[key + "_Y"]))


@pytest.mark.parametrize("dim", [640, 256, 1152, 7, 1001])
def test_rmsnorm_fixture(oracle, dim):
    pr = load_npz("primitives.npz")
    x, w = pr[f"rms_{dim}_x"], pr[f"rms_{dim}_w"]
    assert np.array_equal(bits(oracle.rmsnorm(x, w)), bits(pr[f"rmsnorm_{dim}_out"]))
    assert np.array_equal(bits(oracle.rmsnorm_delta(x, w)), bits(pr[f"rmsnorm_delta_{dim}_out"]))


@pytest.mark.parametrize("base", [10000, 1000000])
def test_rope_fixture(oracle, base):
    pr = load_npz("primitives.npz")
    c, s = oracle.rope_tables(256, 2048, float(base))
    tag = f"rope_{base}"
    assert hashlib.sha256(c.tobytes()).digest() == pr[tag + "_cos_sha256"].tobytes()
    assert hashlib.sha256(s.tobytes()).digest() == pr[tag + "_sin_sha256"].tobytes()
    pos = pr["rope_pos"]
    assert np.array_equal(bits(c.reshape(2048, 256)[pos]), bits(pr[tag + "_cos_rows"]))
    for j, p in enumerate(pos):
        got = oracle.rope_apply(pr[tag + "_x"][j], int(p), c, s)
        assert np.array_equal(bits(got), bits(pr[tag + "_out"][j]))


def test_gelu_fixture(oracle):
    pr = load_npz("primitives.npz")
    x = pr["gelu_x"]
    got = np.array([oracle.lib.oracle_gelu(float(v)) for v in x], np.float32)
    assert np.array_equal(bits(got), bits(pr["gelu_out"]))
    assert np.array_equal(bits(pr["gelu_out"]), bits(pr["gelu_inplace_out"]))
    gin = pr["geglu_in"]
    n = gin.shape[0] // 2
    geglu = (gin[:n] * np.array([oracle.lib.oracle_gelu(float(v)) for v in gin[n:]], np.float32)).astype(np.float32)
    assert np.array_equal(bits(geglu), bits(pr["geglu_out"]))


@pytest.mark.parametrize("n", [1, 5, 8, 13, 1000, 1087])
def test_softmax_greedy_fixture(oracle, n):
    pr = load_npz("primitives.npz")
    x = pr[f"softmax_{n}_in"]
    assert np.array_equal(bits(oracle.softmax(x)), bits(pr[f"softmax_{n}_out"]))
    assert oracle.argmax(x) == int(pr[f"greedy_{n}"][0])


@pytest.mark.parametrize("n", [256, 255, 7, 640])
def test_vec_dot_fixture(oracle, n):
    pr = load_npz("primitives.npz")
    a, b = pr[f"dot_{n}_a"], pr[f"dot_{n}_b"]       # keep the arrays alive across the call
    got = np.float32(oracle.lib.oracle_vec_dot(a.ctypes.data, b.ctypes.data, n))
    assert got.view(np.uint32) == pr[f"dot_{n}_out"].view(np.uint32)[0]


def test_decode_tiny_fixture(oracle):
    """Greedy decode of the 3-layer model: tokens and every logit bit-identical."""
    from oracle.oracle import oracle_decode
    d = json.load(open(os.path.join(GOLD, "decode_tiny.json")))
    cfg = smodel.TINY
    m = smodel.synthetic_model(cfg, d["seed"])
    k, v = m.kv_prefill(d["prefill"])
    assert smodel.model_digest(m, k, v) == d["input_sha256"], "synthetic generator changed"
    toks, logits = oracle_decode(oracle, m, k, v, d["start_token"], d["prefill"], d["steps"], keep_logits=True)
    assert [int(t) for t in toks] == d["tokens"]
    assert [hashlib.sha256(l.tobytes()).hexdigest() for l in logits] == d["logits_sha256"]
