"""The library as a link-level drop-in for the reference's kernels.h / tensor.h / rope.h, and
its host-arithmetic exports (no GPU needed).

* Every function the reference's kernels.h, tensor.h and rope.h declare is exported, except
  rope.h's strategy interface (apply_positional_encoding, rope_encoding_strategy,
  alibi_encoding_strategy of positional_encoding.c), which is not on the decode path and stays
  in the engine; the library's rope.h declares it for that file.
* The reference's own test and bench programs (src/test, src/test/bench) compile against
  include/ and link with libsapphire_hip.so alone, with no undefined symbol
  (`make -C oracle progs`; the GPU tests run them).
* The scalar activations and rope_precompute_freqs are host arithmetic: bit for bit the oracle's.
"""
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INCLUDE = "/root/reference/include"
LIB = os.path.join(ROOT, "sapphire_amd", "libsapphire_hip.so")
STRATEGY_ONLY = {"apply_positional_encoding", "rope_encoding_strategy", "alibi_encoding_strategy"}
PROGS = ["test_tensor_gemv", "test_activations", "test_dispatch", "test_transformer_invariants",
         "bench_q4", "bench_q8", "bench_bf16", "bench_sapphire_end_to_end"]

needs_reference = pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="the reference tree is not present")


def _declared_functions(path):
    s = open(path).read()
    s = re.sub(r"/\*.*?\*/", "", s, flags=re.S)
    s = re.sub(r"//[^\n]*", "", s)
    s = re.sub(r"#[^\n]*", "", s)
    out = set()
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b([A-Za-z_][A-Za-z0-9_]*)\s*\(([^;{]*?)\)\s*;", s):
        if "typedef" not in m.group(1):
            out.add(m.group(2))
    return out


def _exports():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


@needs_reference
@pytest.mark.parametrize("header", ["kernels.h", "tensor.h", "rope.h"])
def test_exports_cover_reference_headers(header):
    declared = _declared_functions(os.path.join(REF_INCLUDE, header))
    assert len(declared) >= 7
    missing = declared - _exports() - (STRATEGY_ONLY if header == "rope.h" else set())
    assert not missing, f"{header}: not exported: {sorted(missing)}"
    if header == "rope.h":
        assert STRATEGY_ONLY <= declared
        ours = _declared_functions(os.path.join(ROOT, "include", "rope.h"))
        assert declared <= ours, "include/rope.h must declare the reference's whole interface"


@needs_reference
def test_reference_programs_link_against_the_library_alone():
    """make -C oracle progs: each program is linked with -Wl,--no-undefined against
    libsapphire_hip.so and libm only."""
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "progs"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    for p in PROGS:
        path = os.path.join(ROOT, "oracle", "_ref", "progs", p)
        assert os.access(path, os.X_OK), p
        needed = subprocess.run(["readelf", "-d", path], capture_output=True, text=True).stdout
        assert "libsapphire_hip.so" in needed and "libsapphire_ref" not in needed


def test_scalar_activations_match_oracle(oracle):
    """silu / relu / gelu / geglu (activations.c:16-105) bit for bit with the oracle, which is
    pinned to the compiled reference; special values included."""
    from sapphire_amd import load, synth
    L = load()
    xs = np.concatenate([synth.normal_f32(4000, 90, 1) * 6,
                         np.array([0.0, -0.0, 1e-38, -1e-38, 30.0, -30.0, 100.0, -100.0, np.inf, -np.inf, np.nan],
                                  np.float32)])
    ys = synth.normal_f32(xs.size, 90, 2) * 3
    O = oracle.lib
    for x, y in zip(xs.tolist(), ys.tolist()):
        pairs = ((L.silu(x), O.oracle_silu(x)), (L.gelu(x), O.oracle_gelu(x)), (L.geglu(x, y), O.oracle_geglu(x, y)),
                 (L.relu(x), np.float32(x) if x > 0 else np.float32(0.0)))
        for got, want in pairs:
            assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32), (x, y, got, want)


@pytest.mark.parametrize("d_k,max_ctx,base", [(256, 2048, 1e6), (256, 2048, 1e4), (64, 100, 10000.0), (6, 9, 500.0)])
def test_rope_precompute_freqs_matches_oracle(oracle, d_k, max_ctx, base):
    from sapphire_amd import load
    L = load()
    c = np.full(max_ctx * d_k, np.nan, np.float32)
    s = np.full(max_ctx * d_k, np.nan, np.float32)
    assert L.rope_precompute_freqs(c.ctypes.data, s.ctypes.data, d_k, max_ctx, base) == 0
    oc, os_ = oracle.rope_tables(d_k, max_ctx, base)
    assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    assert L.rope_precompute_freqs(None, s.ctypes.data, d_k, max_ctx, base) == -1
