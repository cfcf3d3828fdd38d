"""The C-ABI library on the CPU: it loads, exports every function its headers declare,
and its host-side logic (tensor_t carrier, argument validation, host callback pool)
behaves like the reference's. No GPU work is started here."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import sapphire_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#[^\n]*(\\\n[^\n]*)*", "", text, flags=re.M)
    names = set()
    for stmt in text.split(";"):
        stmt = " ".join(stmt.split())
        if not stmt or stmt.startswith("typedef") or "{" in stmt or "(*" in stmt:
            stmt = stmt.split("}")[-1].strip()
            if not stmt or stmt.startswith("typedef") or "(*" in stmt:
                continue
        m = re.search(r"([A-Za-z_][A-Za-z0-9_]*)\s*\([^()]*\)\s*$", stmt)
        if m and not stmt.startswith("extern \"C\""):
            names.add(m.group(1))
    return names


HEADERS = sorted(f for f in os.listdir(INCLUDE) if f.endswith(".h"))


@pytest.fixture(scope="module")
def lib():
    return sapphire_amd.load()


@pytest.fixture(scope="module")
def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", sapphire_amd.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


# rope.h declares the reference's strategy interface for the engine's own positional_encoding.c,
# which keeps defining it (it is not on the decode path).
ENGINE_SIDE = {"rope.h": {"apply_positional_encoding", "rope_encoding_strategy", "alibi_encoding_strategy"}}


@pytest.mark.parametrize("header", HEADERS)
def test_header_symbols_exported(exported, header):
    names = declared_functions(os.path.join(INCLUDE, header))
    assert names, f"no declarations parsed from {header}"
    engine = ENGINE_SIDE.get(header, set())
    assert engine <= names
    missing = sorted(n for n in names - engine if n not in exported)
    assert not missing, f"{header}: declared but not exported: {missing}"
    assert not (engine & exported), f"{header}: the engine's own functions must not be exported here"


def test_reference_api_names_declared():
    """The names the reference's callers bind (include/kernels.h:56-222, tensor.h)."""
    must = {"kernel_ctx_create", "kernel_ctx_init", "kernel_ctx_destroy", "kernel_parallel_for", "kernel_gemv",
            "kernel_gemm", "kernel_gemv_tensor", "kernel_gemv_add", "kernel_gemv_batch",
            "kernel_get_simd_lane_count", "quantized_gemv_q4_0_aligned", "quantized_gemv_q4_0_unaligned",
            "quantized_gemv_q8_0_aligned", "quantized_gemv_q8_0_unaligned", "rmsnorm", "rmsnorm_delta",
            "rmsnorm_batch", "softmax", "vec_add", "vec_copy", "vec_scale", "vec_dot", "gelu_inplace",
            "sapphire_geglu", "tensor_create", "tensor_create_view", "tensor_release", "tensor_shape"}
    declared = declared_functions(os.path.join(INCLUDE, "kernels.h")) | declared_functions(
        os.path.join(INCLUDE, "tensor.h"))
    assert must <= declared


def shape(*dims):
    return (C.c_int * len(dims))(*dims)


def test_tensor_create_and_quant_sizes(lib):
    """test_tensor.c:16-105: shapes, refcount, element sizes, Q4_0 holds numel/2 bytes."""
    t = lib.tensor_create(3, shape(2, 3, 4), 0)
    assert t and lib.tensor_ref_count(t) == 1 and lib.tensor_ndim(t) == 3
    s = lib.tensor_shape(t)
    assert (s[0], s[1], s[2]) == (2, 3, 4) and lib.tensor_numel(t) == 24 and lib.tensor_nbytes(t) == 96
    lib.tensor_release(t)
    assert lib.dtype_element_size(0) == 4 and lib.dtype_element_size(4) == 1 and lib.dtype_element_size(3) == 1
    assert lib.dtype_name(3) == b"Q4_0" and lib.dtype_name(4) == b"Q8_0"
    q4 = lib.tensor_create(1, shape(100), 3)
    assert lib.tensor_nbytes(q4) == 50
    lib.tensor_release(q4)
    q8 = lib.tensor_create(1, shape(100), 4)
    assert lib.tensor_nbytes(q8) == 100
    lib.tensor_release(q8)
    assert not lib.tensor_create(0, shape(1), 0)
    assert not lib.tensor_create(9, shape(*([1] * 9)), 0)


def test_tensor_views_refcount_and_accessors(lib):
    buf = np.arange(12, dtype=np.float32)
    v = lib.tensor_create_view(0, 2, shape(3, 4), buf.ctypes.data)
    assert lib.tensor_data(v) == buf.ctypes.data and lib.tensor_nbytes(v) == 48
    assert lib.tensor_get_f32(v, 5) == 5.0 and lib.tensor_set_f32(v, 5, 7.5) == 0 and buf[5] == 7.5
    assert lib.tensor_get_f32(v, 12) == 0.0 and lib.tensor_set_f32(v, 12, 1.0) == -1
    lib.tensor_ref_inc(v)
    assert lib.tensor_ref_count(v) == 2
    lib.tensor_release(v)
    assert lib.tensor_ref_count(v) == 1
    lib.tensor_release(v)                      # a view never frees the caller's data
    assert buf[5] == 7.5
    # quantized views: nbytes is numel * 1 (tensor.c:149); element access is not provided
    blocks = np.zeros(8 * 20, np.uint8)
    q = lib.tensor_create_view(3, 2, shape(4, 64), blocks.ctypes.data)
    assert lib.tensor_nbytes(q) == 256 and lib.tensor_get_f32(q, 0) == 0.0 and lib.tensor_set_f32(q, 0, 1.0) == -1
    assert lib.tensor_data_f32(q) is None
    lib.tensor_release(q)


def test_tensor_clone_and_transpose(lib):
    t = lib.tensor_create(2, shape(2, 3), 0)
    for i in range(6):
        lib.tensor_set_f32(t, i, float(i))
    c = lib.tensor_clone(t)
    assert [lib.tensor_get_f32(c, i) for i in range(6)] == [0, 1, 2, 3, 4, 5]
    out = C.c_void_p()
    assert lib.tensor_transpose(t, C.byref(out)) == 0
    s = lib.tensor_shape(out.value)
    assert (s[0], s[1]) == (3, 2)
    assert [lib.tensor_get_f32(out.value, i) for i in range(6)] == [0, 3, 1, 4, 2, 5]
    for x in (t, c, out.value):
        lib.tensor_release(x)


def test_argument_validation_without_device(lib):
    """Errors that the reference reports before any work (dispatch.c:102-142)."""
    A = lib.tensor_create(2, shape(3, 4), 0)
    x = np.ones(4, np.float32)
    y = np.zeros(3, np.float32)
    assert lib.kernel_gemv(None, None, A, x.ctypes.data) == -1
    assert lib.kernel_gemv(None, y.ctypes.data, None, x.ctypes.data) == -1
    assert lib.kernel_gemv(None, y.ctypes.data, A, None) == -1
    v1 = lib.tensor_create(1, shape(4), 0)
    assert lib.kernel_gemv(None, y.ctypes.data, v1, x.ctypes.data) == -1        # ndim != 2
    blocks = np.zeros(3 * 20, np.uint8)
    Q = lib.tensor_create_view(3, 2, shape(3, 32), blocks.ctypes.data)
    assert lib.kernel_gemv(None, y.ctypes.data, Q, x.ctypes.data) == -1         # quantized needs a ctx
    F16 = lib.tensor_create(2, shape(3, 4), 2)
    assert lib.kernel_gemv(None, y.ctypes.data, F16, x.ctypes.data) == -1       # no F16 kernels
    assert lib.kernel_gemm(None, y.ctypes.data, A, x.ctypes.data, 1, 3) == -1  # gemm needs a ctx
    assert lib.kernel_gemm(None, y.ctypes.data, A, x.ctypes.data, 0, 3) == -1
    assert lib.kernel_gemv_batch(None, y.ctypes.data, A, x.ctypes.data, 0) == -1
    assert lib.kernel_ctx_init(None) == -1
    assert lib.sapphire_gemv_q_dev(3, 1, None, 3, 32, None, None, None) == -1
    assert lib.sapphire_gemv_q_dev(0, 1, blocks.ctypes.data, 3, 32, x.ctypes.data, y.ctypes.data, None) == -1
    assert b"Q4_0/Q8_0" in lib.sapphire_last_error()
    assert lib.sapphire_gemv_q_dev(3, 1, blocks.ctypes.data, 3, 33, x.ctypes.data, y.ctypes.data, None) == -1
    assert b"multiple of 32" in lib.sapphire_last_error()
    assert lib.sapphire_rmsnorm_delta_dev(None, None, None, 1e-6, 4, 1, None) == -1
    assert lib.sapphire_rope_apply_dev(x.ctypes.data, 1, 7, 0, x.ctypes.data, x.ctypes.data, None) == -1
    assert lib.sapphire_softmax_argmax_dev(x.ctypes.data, 4, None, None, None) == -1
    for t in (A, v1, Q, F16):
        lib.tensor_release(t)
    lib.kernel_ctx_destroy(None)


def test_simd_lane_count(lib):
    assert [lib.kernel_get_simd_lane_count(d) for d in range(5)] == [8] * 5
    assert lib.kernel_get_simd_lane_count(17) == 1


def test_parallel_for_runs_each_index_once(lib):
    """kernel_parallel_for (pool.c:364-396) is host work: fn(arg, i) for every i once."""
    n = 1000
    hits = np.zeros(n, np.int32)
    CB = C.CFUNCTYPE(None, C.c_void_p, C.c_int)

    @CB
    def fn(arg, i):
        hits[i] += 1

    for nt in (1, 4, 0):
        hits[:] = 0
        ctx = lib.kernel_ctx_create(nt, 16)
        assert ctx
        assert lib.kernel_parallel_for(ctx, fn, None, n) == 0
        assert (hits == 1).all()
        lib.kernel_ctx_destroy(ctx)
    assert lib.kernel_parallel_for(None, fn, None, n) == -1


def test_decoder_argument_validation(lib):
    """The decode engine refuses bad arguments before touching a device."""
    from sapphire_amd.engine import DecoderConfig, _protos
    _protos(lib)
    assert not lib.sapphire_decoder_create(None, None)
    bad = DecoderConfig(0, 640, 4, 1, 256, 2048, 262144, 2048, 512, 0, 256.0, 1e6, 1e4, 1e-6, 3, 3)
    assert not lib.sapphire_decoder_create(C.byref(bad), None)
    cfg = DecoderConfig(18, 640, 4, 1, 256, 2048, 262144, 2048, 512, 0, 256.0, 1e6, 1e4, 1e-6, 0, 3)
    from sapphire_amd.engine import DecoderWeights
    w = DecoderWeights()
    assert not lib.sapphire_decoder_create(C.byref(cfg), C.byref(w))      # F32 projections: not Q4_0/Q8_0
    assert b"Q4_0 or Q8_0" in lib.sapphire_last_error()
    toks = np.zeros(4, np.int32)
    assert lib.sapphire_decoder_generate(None, 0, 0, 4, toks.ctypes.data, None, None) == -1
    assert lib.sapphire_decoder_set_kv(None, None, None) == -1
    lib.sapphire_decoder_destroy(None)
