"""The library as a link-level drop-in for the reference's kernels.h / tensor.h / rope.h /
transformer.h, and its host-arithmetic exports (no GPU needed).

* Every function the reference's kernels.h, tensor.h, rope.h and transformer.h declare is
  exported, except
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
@pytest.mark.parametrize("header", ["kernels.h", "tensor.h", "rope.h", "transformer.h"])
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


_LAYOUT_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
int main(void) {
    printf("session %zu %zu %zu %zu %zu %zu %zu\n", sizeof(inference_session_t), offsetof(inference_session_t, kv_cache),
           offsetof(inference_session_t, scratch_size), offsetof(inference_session_t, padded_d_ff),
           offsetof(inference_session_t, rope_freqs_cos_global), offsetof(inference_session_t, gemv_ctx),
           offsetof(inference_session_t, num_layers));
    printf("spec %zu %zu %zu\n", sizeof(struct model_spec), offsetof(struct model_spec, llm_model),
           offsetof(struct model_spec, variant_config));
    printf("cfg %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(gemma3_270m_config_t),
           offsetof(gemma3_270m_config_t, head_dim), offsetof(gemma3_270m_config_t, hidden_size),
           offsetof(gemma3_270m_config_t, intermediate_size), offsetof(gemma3_270m_config_t, layer_types_mask),
           offsetof(gemma3_270m_config_t, num_attention_heads), offsetof(gemma3_270m_config_t, num_hidden_layers),
           offsetof(gemma3_270m_config_t, num_key_value_heads), offsetof(gemma3_270m_config_t, query_pre_attn_scalar),
           offsetof(gemma3_270m_config_t, rope_local_base_freq), offsetof(gemma3_270m_config_t, sliding_window),
           offsetof(gemma3_270m_config_t, vocab_size));
    printf("model %zu %zu %zu %zu\n", sizeof(llm_model_t), offsetof(llm_model_t, norm_final_weight),
           offsetof(llm_model_t, layers), sizeof(model_layer_weights_t));
    printf("layer %zu %zu %zu %zu %zu\n", offsetof(model_layer_weights_t, q_proj_weight),
           offsetof(model_layer_weights_t, q_norm_weight), offsetof(model_layer_weights_t, out_proj_weight),
           offsetof(model_layer_weights_t, up_proj_weight), offsetof(model_layer_weights_t, down_proj_weight));
    printf("bufs %zu %zu %zu ctx %zu %zu %zu\n", sizeof(layer_buffers_t), offsetof(layer_buffers_t, residual),
           offsetof(layer_buffers_t, weight_scratch), sizeof(transformer_layer_ctx_t),
           offsetof(transformer_layer_ctx_t, layer_idx), offsetof(transformer_layer_ctx_t, head_dim));
    printf("rope %zu\n", sizeof(transformer_rope_t));
    return 0;
}
"""


@needs_reference
def test_engine_struct_layouts_match_reference(tmp_path):
    """The engine structs transformer.h's entry points read (csrc/engine_abi.h) have the
    reference's sizes and field offsets (inference.h, model_spec.h, llm_model.h,
    gemma3_270m_config.h, transformer.h), compiled by the same host compiler."""
    ref = tmp_path / "ref.c"
    ref.write_text('#include "inference.h"\n#include "gemma3_270m_config.h"\n#include "llm_model.h"\n'
                   '#include "model_spec.h"\n#include "transformer.h"\n' + _LAYOUT_PROBE)
    ours = tmp_path / "ours.cpp"
    ours.write_text('#include "engine_abi.h"\n' + _LAYOUT_PROBE)
    subprocess.run(["gcc", "-I", "/root/reference/include", "-I", "/root/reference", str(ref), "-o",
                    str(tmp_path / "ref")], check=True)
    subprocess.run(["g++", "-I", os.path.join(ROOT, "sapphire_amd", "csrc"), str(ours), "-o", str(tmp_path / "ours")],
                   check=True)
    a = subprocess.run([str(tmp_path / "ref")], capture_output=True, text=True, check=True).stdout
    b = subprocess.run([str(tmp_path / "ours")], capture_output=True, text=True, check=True).stdout
    assert a == b, f"reference:\n{a}\nlibrary:\n{b}"


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
