"""transformer.h on the GPU: the reference's own engine (inference.c, kv_cache.c, the loaders,
utils.c, ... compiled from its sources by `make -C oracle engine`, linked with
libsapphire_hip.so in place of the kernels, tensor.c, normalization.c, activations.c, rope.c,
transformer.c and attention.c) decoding greedily, against the oracle's decode step.

Two drivers (oracle/ref_decode.c):
* per step sapphire_embed_lookup, sapphire_transformer_layer for every layer, then lm_head
  (tied BF16 head) or the final norm and kernel_gemv (quantized head), sample_greedy;
* the engine's own loop: a prompt through inference_forward_batch in chunks of up to 32
  (sapphire_embed_lookup_batch, sapphire_transformer_layer_batch), then inference_forward
  and sample_greedy per step.

Bar: identical greedy tokens and logits within 2e-3 relative (except after a near-tie, as in
test_decode_gpu), and the K/V rows the steps wrote back into the engine's host cache within
2e-3 relative of the oracle's.
"""
import numpy as np
import pytest

from oracle.oracle import (engine_forward_decode, engine_hip_available, engine_layer_decode, engine_patch_decode,
                           engine_stage_decode, oracle_decode, oracle_prefill, patched_model)
from sapphire_amd import model as smodel
from sapphire_amd import synth
from tests.test_decode_gpu import _compare

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not engine_hip_available(), reason="oracle/_ref/libref_engine_hip.so not built")]

REL = 2e-3
TINY_TIED = smodel.DecodeConfig(**{**smodel.TINY.__dict__, "lm_dtype": synth.BF16})
TINY_Q8 = smodel.DecodeConfig(**{**smodel.TINY.__dict__, "wdtype": synth.Q8_0, "lm_dtype": synth.Q8_0})
G270M_TIED = smodel.DecodeConfig(**{**smodel.GEMMA3_270M.__dict__, "lm_dtype": synth.BF16})


def _kv_close(got_k, got_v, ref_k, ref_v, lo, hi):
    for name, g, r in (("K", got_k, ref_k), ("V", got_v, ref_v)):
        d = np.abs(g[:, :, lo:hi] - r[:, :, lo:hi]).max() / np.abs(r[:, :, lo:hi]).max()
        assert d <= REL, f"{name} cache rows {lo}..{hi} differ: {d:.2e}"
        assert np.array_equal(g[:, :, :lo], r[:, :, :lo])


@pytest.mark.parametrize("cfg,seed,prefill,steps", [
    (smodel.TINY, 71, 40, 12),            # windows slide across the local layers
    (TINY_TIED, 72, 30, 12),              # lm_head (tied BF16)
    (TINY_Q8, 73, 5, 10),                 # Q8_0 projections
    (smodel.GEMMA3_270M, 74, 1024, 64),   # the Gemma-3-270M shape, KV at 1024 of 2048, 64 steps
    (G270M_TIED, 75, 1024, 16),           # ... with the reference's own tied BF16 LM head
], ids=["tiny", "tiny_tied", "tiny_q8", "gemma3_270m", "gemma3_270m_tied"])
def test_engine_layers_match_oracle(oracle, cfg, seed, prefill, steps):
    print(f"engine layers cfg={cfg.n_layers}x{cfg.hidden} lm={cfg.lm_dtype} steps={steps}", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    gk, gv = k.copy(), v.copy()
    got_t, got_l = engine_layer_decode(m, gk, gv, tok, prefill, steps)
    print("engine done; oracle", flush=True)
    ref_t, ref_l = oracle_decode(oracle, m, k, v, tok, prefill, steps, nthreads=8, keep_logits=True)
    n = _compare(ref_t, ref_l, got_t, got_l)
    assert n == steps, f"near-tie at step {n}"
    _kv_close(gk, gv, k, v, prefill, prefill + steps)


@pytest.mark.parametrize("cfg,seed,prefill,prompt_len,steps", [
    (TINY_TIED, 76, 0, 40, 10),           # a 40-token prompt from position 0: chunks of 32 and 8
    (TINY_TIED, 77, 20, 5, 12),
    (G270M_TIED, 78, 300, 70, 8),         # the Gemma-3-270M shape: three prefill chunks
], ids=["tiny_prompt40", "tiny_prompt5", "gemma3_270m_prompt70"])
def test_engine_forward_loop_matches_oracle(oracle, cfg, seed, prefill, prompt_len, steps):
    """inference_forward_batch over the prompt, then inference_forward per step: the engine's
    own loop (inference.c:612-651) with every layer on the GPU."""
    print(f"engine forward loop cfg={cfg.n_layers}x{cfg.hidden} prompt={prompt_len} steps={steps}", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    prompt = synth.rng(seed, 99).integers(0, cfg.vocab, size=prompt_len).astype(np.int32)
    tok = smodel.start_token(cfg, seed)
    gk, gv = k.copy(), v.copy()
    got_t, got_l = engine_forward_decode(m, gk, gv, prompt, tok, prefill, steps)
    print("engine done; oracle", flush=True)
    oracle_prefill(oracle, m, k, v, prompt, prefill, nthreads=8)
    ref_t, ref_l = oracle_decode(oracle, m, k, v, tok, prefill + prompt_len, steps, nthreads=8, keep_logits=True)
    n = _compare(ref_t, ref_l, got_t, got_l)
    assert n == steps, f"near-tie at step {n}"
    _kv_close(gk, gv, k, v, prefill, prefill + prompt_len + steps)


# the 1B widths in two layers: an FFN of 6912 (above the fused kernels' 2048-long inputs, so the
# down projection takes the plain GEMV) behind transformer.h
WIDE_FFN = smodel.DecodeConfig(n_layers=2, hidden=1152, n_heads=4, n_kv_heads=1, head_dim=256, ffn=6912, vocab=8192,
                               max_ctx=96, sliding_window=24, global_layers=(1,), lm_dtype=synth.BF16)


@pytest.mark.parametrize("cfg,seed,prefill,prompt_len,steps", [
    (TINY_TIED, 86, 0, 40, 8),            # a 32-token chunk then 8: every stage at batch 32
    (G270M_TIED, 87, 300, 33, 4),         # the Gemma-3-270M shape
    (WIDE_FFN, 88, 10, 20, 6),            # FFN 6912 through compute_ffn_stage
], ids=["tiny_prompt40", "gemma3_270m_prompt33", "ffn6912"])
def test_engine_stage_functions_match_oracle(oracle, cfg, seed, prefill, prompt_len, steps):
    """The reference engine's loop with each layer composed from the library's stage exports
    (compute_attention_stage -> compute_ffn_stage -> finalize_layer_output, as
    transformer.c:318-345 composes them, on buffers laid out as init_layer_buffers does) against
    the oracle's prefill and decode."""
    print(f"engine stages cfg={cfg.n_layers}x{cfg.hidden} ffn={cfg.ffn} prompt={prompt_len} steps={steps}", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    prompt = synth.rng(seed, 99).integers(0, cfg.vocab, size=prompt_len).astype(np.int32)
    tok = smodel.start_token(cfg, seed)
    gk, gv = k.copy(), v.copy()
    got_t, got_l = engine_stage_decode(m, gk, gv, prompt, tok, prefill, steps)
    print("engine done; oracle", flush=True)
    oracle_prefill(oracle, m, k, v, prompt, prefill, nthreads=8)
    ref_t, ref_l = oracle_decode(oracle, m, k, v, tok, prefill + prompt_len, steps, nthreads=8, keep_logits=True)
    n = _compare(ref_t, ref_l, got_t, got_l, f"stages {cfg.n_layers}x{cfg.hidden}")
    assert n == steps, f"near-tie at step {n}"
    _kv_close(gk, gv, k, v, prefill, prefill + prompt_len + steps)


def test_engine_sessions_do_not_share_state(oracle):
    """Two models decoded one after the other in one process (each its own engine session,
    created and destroyed by the engine): the second must not see the first's device state."""
    for seed in (81, 82, 81):
        m = smodel.synthetic_model(TINY_TIED, seed)
        k, v = m.kv_prefill(25)
        tok = smodel.start_token(TINY_TIED, seed)
        got_t, got_l = engine_layer_decode(m, k.copy(), v.copy(), tok, 25, 6)
        ref_t, ref_l = oracle_decode(oracle, m, k, v, tok, 25, 6, keep_logits=True)
        assert _compare(ref_t, ref_l, got_t, got_l) == 6


@pytest.mark.parametrize("patch", [1, 2], ids=["q_proj_invalidated", "norm_attn_set_f32"])
def test_engine_sees_changed_weights(oracle, patch):
    """The device session derived from an engine session follows changes to the model between
    layer calls: after the first step, layer 0's q_proj block scales are rewritten in the host
    array and sapphire_tensor_invalidate drops its device copy (patch 1), or layer 0's
    norm_attn is changed through tensor_set_f32 (patch 2). The later steps must use the new
    weights (the oracle's steps on patched_model), never the old or freed device copies."""
    cfg, seed, prefill, steps = smodel.TINY, 91, 30, 6
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    gk, gv = k.copy(), v.copy()
    got_t, got_l = engine_patch_decode(m, gk, gv, tok, prefill, steps, patch)
    t0, l0 = oracle_decode(oracle, m, k, v, tok, prefill, 1, keep_logits=True)
    t1, l1 = oracle_decode(oracle, patched_model(m, patch), k, v, int(t0[0]), prefill + 1, steps - 1, keep_logits=True)
    ref_t, ref_l = np.concatenate([t0, t1]), np.concatenate([l0, l1])
    n = _compare(ref_t, ref_l, got_t, got_l, f"patch {patch}")
    assert n == steps, f"near-tie at step {n}"
    _kv_close(gk, gv, k, v, prefill, prefill + steps)
