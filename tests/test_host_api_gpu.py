"""The host-pointer API of kernels.h / rope.h on the GPU, against the oracle, and the reference's
own test and bench programs (compiled against include/ and linked with libsapphire_hip.so
alone by `make -C oracle progs`) run on the GPU.

Bars: bit for bit where the device form is (RMSNorm in the reference's sum order, residual
add/copy/scale, vec_dot in the reference's lane order, BF16 widening, both RoPE rotations);
the GEMV tolerance |gpu - ref| <= 1e-4 + 1e-3 |ref| for dot products summed in another order;
a few ulp for the device tanhf/expf (softcap, softmax).
"""
import ctypes as C
import json
import os
import re
import subprocess

import numpy as np
import pytest

from sapphire_amd import synth
from tests.conftest import close

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROGS = os.path.join(ROOT, "oracle", "_ref", "progs")


def p(a):
    return a.ctypes.data


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---- the reference's own programs ----

def _run(name, timeout=300):
    path = os.path.join(PROGS, name)
    if not os.path.exists(path):
        pytest.skip(f"{name} was not built (make -C oracle progs needs the reference tree)")
    print(f"running reference program {name}", flush=True)
    r = subprocess.run([path], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"{name} exited {r.returncode}:\n{r.stdout[-3000:]}\n{r.stderr[-2000:]}"
    return r.stdout


@pytest.mark.parametrize("name", ["test_tensor_gemv", "test_activations", "test_transformer_invariants"])
def test_reference_test_program_passes(hip, name):
    """src/test/<name>.c, its assertions unchanged, against this library."""
    _run(name)


def test_reference_dispatch_program(hip):
    """src/test/test_dispatch.c prints the row dot it asserts on; the reference prints
    -0.08400002 (the known answer in tests/golden/known_answers.json)."""
    out = _run("test_dispatch")
    vals = [float(v) for v in re.findall(r"=(-?[0-9.]+)", out.splitlines()[0])]
    assert len(vals) == 3 and all(abs(v + 0.08400002) <= 1e-4 + 1e-3 * 0.084 for v in vals), out


@pytest.mark.parametrize("name", ["bench_q4", "bench_q8", "bench_bf16"])
def test_reference_row_bench(hip, name):
    """src/test/bench/<name>.c compares this library's row kernel over 1024 rows with the
    bench's own scalar loop and prints the largest difference."""
    out = _run(name)
    diffs = [float(v) for v in re.findall(r"max_diff=([0-9.eE+-]+)", out)]
    assert diffs and max(diffs) <= 1e-3, out


def test_reference_end_to_end_bench(hip):
    """src/test/bench/bench_sapphire_end_to_end.c: kernel_gemv on five Q4_0 / Q8_0 shapes at
    several thread counts; every printed sum(y) against the reference's own run."""
    with open(os.path.join(ROOT, "tests", "golden", "known_answers.json")) as f:
        known = json.load(f)["e2e_sums"]
    out = _run("bench_sapphire_end_to_end")
    blocks = re.split(r"=== CONFIG: rows=(\d+) blocks_per_row=(\d+) ===", out)
    seen = 0
    for i in range(1, len(blocks), 3):
        rows, bpr, body = int(blocks[i]), int(blocks[i + 1]), blocks[i + 2]
        ka = next(k for k in known if k["rows"] == rows and k["blocks_per_row"] == bpr)
        for label, s, rc in re.findall(r"^(\S.*?)\s+avg=.*?sum=\s*(-?[0-9.]+)\s+rc=\s*(-?\d+)", body, re.M):
            want = ka["q8_sum"] if "Q8" in label.upper() else ka["q4_sum"]
            assert int(rc) == 0, (rows, label)
            assert abs(float(s) - want) <= 1e-5 * abs(want) + 1e-4, (rows, label, s, want)
            seen += 1
    assert seen >= 10, out


# ---- host-pointer primitives against the oracle ----

@pytest.mark.parametrize("dim,batch", [(640, 1), (1152, 1), (256, 4), (1000, 3), (7, 2)])
def test_rmsnorm_host(hip, oracle, dim, batch):
    x = synth.normal_f32((batch, dim), 60, dim) * 3
    w = (1 + 0.1 * synth.normal_f32(dim, 60, 1)).astype(np.float32)
    out = np.empty_like(x)
    for b in range(batch):
        assert hip.rmsnorm_delta(p(out[b]), p(x[b]), p(w), 1e-6, dim) == 0
        assert np.array_equal(bits(out[b]), bits(oracle.rmsnorm_delta(x[b], w)))
        assert hip.rmsnorm(p(out[b]), p(x[b]), p(w), 1e-6, dim) == 0
        assert np.array_equal(bits(out[b]), bits(oracle.rmsnorm(x[b], w)))
    assert hip.rmsnorm_batch(p(out), p(x), p(w), 1e-6, batch, dim) == 0
    for b in range(batch):
        assert np.array_equal(bits(out[b]), bits(oracle.rmsnorm(x[b], w)))
    assert hip.rmsnorm_delta(None, p(x), p(w), 1e-6, dim) == -1
    assert hip.rmsnorm(p(out), p(x), p(w), -1.0, dim) == -1


@pytest.mark.parametrize("n", [1, 17, 1024, 262144])
def test_softmax_host(hip, oracle, n):
    x = synth.normal_f32(n, 61, n) * 4
    got = x.copy()
    hip.softmax(p(got), n)
    # the reference sums exp() left to right in fp32 (utils.c:43-46), good to ~2e-4 relative at
    # 262144 terms; the device sums in a tree
    ok, err = close(got, oracle.softmax(x), rel=1e-3, abs_=1e-9)
    assert ok, err
    assert abs(float(got.astype(np.float64).sum()) - 1.0) < 1e-4


def test_vector_ops_host(hip, oracle):
    n = 1000
    a = synth.normal_f32(n, 62, 1)
    b = synth.normal_f32(n, 62, 2)
    d = a.copy()
    hip.vec_add(p(d), p(b), n)
    want = a.copy()
    oracle.lib.oracle_vec_add(p(want), p(b), n)
    assert np.array_equal(bits(d), bits(want))
    c = np.zeros(n, np.float32)
    hip.vec_copy(p(c), p(b), n)
    assert np.array_equal(bits(c), bits(b))
    s = a.copy()
    hip.vec_scale(p(s), float(np.float32(0.37)), n)
    assert np.array_equal(bits(s), bits(a * np.float32(0.37)))
    s1 = a.copy()
    hip.vec_scale(p(s1), 1.0, n)                       # utils.c:88 returns early for s == 1
    assert np.array_equal(bits(s1), bits(a))
    for m in (n, 8, 13, 1):
        got = hip.vec_dot(p(a), p(b), m)
        assert np.float32(got).view(np.uint32) == np.float32(oracle.lib.oracle_vec_dot(p(a), p(b), m)).view(np.uint32)
    sc = (a * 20).astype(np.float32)
    g = sc.copy()
    hip.vec_softcap(p(g), n, 30.0)
    want = (np.float32(30.0) * np.tanh(sc.astype(np.float64) * np.float64(np.float32(1 / 30.0)))).astype(np.float32)
    assert np.allclose(g, want, rtol=5e-7, atol=1e-6)   # device tanhf: a few ulp
    g2 = sc.copy()
    hip.vec_softcap(p(g2), n, 0.0)                     # cap <= 0: unchanged (utils.c:120)
    assert np.array_equal(bits(g2), bits(sc))


def test_bf16_and_norm_weights_host(hip):
    n = 1000
    src = synth.bf16_normal(n, 63, 1)
    dst = np.zeros(n, np.float32)
    hip.bf16_to_f32_vec(p(dst), p(src), n)
    assert np.array_equal(dst.view(np.uint32), src.astype(np.uint32) << 16)
    # get_norm_weights: BF16 tensors widen into the scratch, F32 tensors return their data
    t = hip.tensor_create_view(synth.BF16, 1, (C.c_int * 1)(n), p(src))
    scratch = np.zeros(n, np.float32)
    r = hip.get_norm_weights(t, p(scratch), n)
    assert r == p(scratch) and np.array_equal(scratch, dst)
    hip.tensor_release(t)
    f = synth.normal_f32(n, 63, 2)
    t = hip.tensor_create_view(synth.F32, 1, (C.c_int * 1)(n), p(f))
    assert hip.get_norm_weights(t, p(scratch), n) == p(f)
    hip.tensor_release(t)
    assert hip.get_norm_weights(None, p(scratch), n) is None


@pytest.mark.parametrize("dtype", [synth.Q4_0, synth.Q8_0], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("nb", [1, 3, 20, 36, 216])
def test_quantized_row_kernels_host(hip, oracle, dtype, nb):
    """quantized_gemv_q{4,8}_0_{aligned,unaligned} (q4_0_avx.c:102-148, q8_0_avx.c:16-136):
    the GEMV tolerance on N(0,1) inputs, bit for bit on the exact special case, 0 for bad
    block sizes and NULL pointers."""
    W = synth.quant_matrix(dtype, 6, nb * 32, 64, nb)
    name = "q4_0" if dtype == synth.Q4_0 else "q8_0"
    fns = [getattr(hip, f"quantized_gemv_{name}_aligned"), getattr(hip, f"quantized_gemv_{name}_unaligned")]
    for r in range(6):
        x = synth.normal_f32(nb * 32, 64, 100 + r)
        want = oracle.row(dtype, W[r], x)
        for fn in fns:
            assert close([fn(p(np.ascontiguousarray(W[r])), p(x), nb, 32)], [want])[0]
    E = W.copy()
    E["scale"] = np.float32(0.25)
    xi = np.arange(nb * 32, dtype=np.float32) % 7 - 3
    for fn in fns:
        got = fn(p(np.ascontiguousarray(E[0])), p(xi), nb, 32)
        assert np.float32(got).view(np.uint32) == np.float32(oracle.row(dtype, E[0], xi)).view(np.uint32)
        assert fn(p(np.ascontiguousarray(E[0])), p(xi), nb, 16) == 0.0
        assert fn(None, p(xi), nb, 32) == 0.0


@pytest.mark.parametrize("dtype", [synth.F32, synth.BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("nb,bs", [(20, 32), (640, 1), (7, 32), (33, 1)])
def test_float_row_kernels_host(hip, oracle, dtype, nb, bs):
    """quantized_gemv_{f32,bf16}_{avx2,scalar} (f32_avx.c:21-83, bf16_avx.c:21-108): cols =
    block_count when block_size is 1, else block_count * block_size."""
    cols = nb if bs == 1 else nb * bs
    g = np.random.default_rng(cols)
    wf = g.standard_normal(cols).astype(np.float32)
    w = wf if dtype == synth.F32 else (wf.view(np.uint32) >> 16).astype(np.uint16)
    x = g.standard_normal(cols).astype(np.float32)
    name = "f32" if dtype == synth.F32 else "bf16"
    for kind, orc in (("avx2", oracle.lib.oracle_f_row), ("scalar", oracle.lib.oracle_f_row_scalar)):
        got = getattr(hip, f"quantized_gemv_{name}_{kind}")(p(w), p(x), nb, bs)
        assert close([got], [orc(dtype, p(w), p(x), cols)])[0]
    xi = (np.arange(cols) % 5 - 2).astype(np.float32)
    wi = ((np.arange(cols) % 3) - 1).astype(np.float32)
    wq = wi if dtype == synth.F32 else (wi.view(np.uint32) >> 16).astype(np.uint16)
    assert hip.quantized_gemv_f32_avx2(p(wi), p(xi), nb, bs) == float(wi.astype(np.float64) @ xi)
    assert getattr(hip, f"quantized_gemv_{name}_scalar")(p(wq), p(xi), nb, bs) == float(wi.astype(np.float64) @ xi)
    assert getattr(hip, f"quantized_gemv_{name}_avx2")(None, p(x), nb, bs) == 0.0


class GemmArgs(C.Structure):
    """gemm_args_t (kernels.h:84-93)."""
    _fields_ = [("w_row", C.c_void_p), ("X", C.c_void_p), ("Y", C.c_void_p), ("batch_size", C.c_int),
                ("d_model", C.c_int), ("out_stride", C.c_int), ("blocks", C.c_int), ("block_size", C.c_int)]


@pytest.mark.parametrize("dtype", [synth.F32, synth.BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("batch,cols,stride", [(1, 640, 1), (8, 640, 3), (13, 1152, 13), (32, 37, 2)])
def test_gemm_row_kernels_host(hip, oracle, dtype, batch, cols, stride):
    """kernel_gemm_{f32,bf16}_avx2 (f32_avx.c:97-135, bf16_avx.c:110-150): one weight row times
    batch_size vectors, Y[b * out_stride]; the other Y entries are untouched."""
    g = np.random.default_rng(batch * cols)
    wf = g.standard_normal(cols).astype(np.float32)
    w = wf if dtype == synth.F32 else (wf.view(np.uint32) >> 16).astype(np.uint16)
    X = g.standard_normal((batch, cols)).astype(np.float32)
    Y = np.full(batch * stride, 7.0, np.float32)
    args = GemmArgs(p(w), p(X), p(Y), batch, cols, stride, 0, 0)
    getattr(hip, "kernel_gemm_f32_avx2" if dtype == synth.F32 else "kernel_gemm_bf16_avx2")(C.byref(args))
    ref = np.empty(batch, np.float32)
    assert oracle.lib.oracle_gemm_f(dtype, p(w), 1, cols, p(X), batch, p(ref), 1) == 0
    ok, err = close(Y[::stride][:batch], ref)
    assert ok, err
    mask = np.ones(batch * stride, bool)
    mask[::stride] = False
    mask[batch * stride:] = False
    assert (Y[mask] == 7.0).all()


@pytest.mark.parametrize("hd,pos,base", [(256, 0, 1e6), (256, 1037, 1e6), (256, 2047, 1e4), (64, 9, 1e4), (7, 300, 1e4)])
def test_rope_host(hip, oracle, hd, pos, base):
    """rope_apply_fast (half-split, rope.c:99-117) and apply_rope / apply_rope_default
    (interleaved pairs, rope.c:17-36) on the GPU, bit for bit with the oracle."""
    cos_t, sin_t = oracle.rope_tables(hd, 2048, base)
    x = synth.normal_f32(hd, 65, hd + pos)
    got = x.copy()
    hip.rope_apply_fast(p(got), pos, hd, p(cos_t), p(sin_t))
    assert np.array_equal(bits(got), bits(oracle.rope_apply(x, pos, cos_t, sin_t)))
    got = x.copy()
    hip.apply_rope(p(got), pos, hd, base)
    assert np.array_equal(bits(got), bits(oracle.apply_rope(x, pos, base)))
    got = x.copy()
    hip.apply_rope_default(p(got), pos, hd)
    assert np.array_equal(bits(got), bits(oracle.apply_rope(x, pos, 1e6)))
    hip.rope_apply_fast(None, pos, hd, p(cos_t), p(sin_t))            # NULL: no-op
