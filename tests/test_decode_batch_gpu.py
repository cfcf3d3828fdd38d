"""Batched greedy decode (sapphire_decoder_create_batch: sequences in lock step, every
projection one matrix-core GEMM over the batch) against the oracle's decode step run on each
sequence on its own. The reference decodes one sequence per inference_forward call
(inference.c:612-651), so that is the expected result of every sequence.

Parity bar: per sequence and step, logits within 2e-3 relative (and each within
2e-3 |ref| + 1e-4 max |ref|) and identical greedy tokens, except after a near-tie (top-2 gap
inside the tolerance), as in test_decode_gpu.
"""
import numpy as np
import pytest

from oracle.oracle import oracle_decode
from sapphire_amd import model as smodel
from sapphire_amd import synth
from tests.test_decode_gpu import GQA2, MID, NH8, NH8_KV2, _compare

pytestmark = pytest.mark.gpu

REL = 2e-3


def _run(oracle, cfg, seed, batch, prefills, steps, nthreads=4, check_kv=True, kv_seqs=None):
    """kv_seqs: the sequences whose K/V cache rows written during the steps are compared with
    the oracle's (all of them when check_kv and kv_seqs is None)."""
    from sapphire_amd.engine import Decoder
    m = smodel.synthetic_model(cfg, seed)
    rng = synth.rng(seed, 4242)
    toks0 = rng.integers(0, cfg.vocab, size=batch).astype(np.int32)
    kvs = [m.kv_prefill(prefills[b], seed_offset=100 + b) for b in range(batch)]
    dec = Decoder(m, batch=batch)
    for b in range(batch):
        dec.set_kv_seq(b, *kvs[b])
    got_toks, got_logits, _ = dec.generate_batch(toks0, np.asarray(prefills, np.int32), steps, keep_logits=True)
    kv_seqs = set(range(batch) if kv_seqs is None else kv_seqs) if check_kv else set()
    got_kv = {b: dec.get_kv_seq(b) for b in kv_seqs}
    dec.close()
    print("gpu done; oracle", flush=True)
    for b in range(batch):
        k, v = kvs[b]
        ref_toks, ref_logits = oracle_decode(oracle, m, k, v, int(toks0[b]), prefills[b], steps, nthreads=nthreads,
                                             keep_logits=True)
        n = _compare(ref_toks, ref_logits, got_toks[:, b], got_logits[:, b], f"{cfg.n_layers}x{cfg.hidden} seq {b}")
        assert n == steps, f"sequence {b}: near-tie at step {n}"
        print(f"sequence {b}: {steps} steps match", flush=True)
        if b in kv_seqs:
            gk, gv = got_kv[b]
            sl = slice(prefills[b], prefills[b] + steps)
            for name, g, r in (("K", gk, k), ("V", gv, v)):
                d = np.abs(g[:, :, sl] - r[:, :, sl]).max() / np.abs(r[:, :, sl]).max()
                assert d <= REL, f"sequence {b}: {name} cache rows differ: {d:.2e}"
            assert np.array_equal(gk[:, :, :prefills[b]], k[:, :, :prefills[b]])


TINY_Q8 = smodel.DecodeConfig(**{**smodel.TINY.__dict__, "wdtype": synth.Q8_0, "lm_dtype": synth.Q8_0})
# the reference's own LM head: the BF16 embedding table (weight tying, transformer.c:393-408)
TINY_TIED = smodel.DecodeConfig(**{**smodel.TINY.__dict__, "lm_dtype": synth.BF16})


@pytest.mark.parametrize("cfg,seed,batch,prefills,steps", [
    (smodel.TINY, 51, 4, [40, 10, 23, 55], 12),              # windows slide at different steps
    (TINY_Q8, 52, 3, [8, 30, 60], 10),                       # Q8_0 weights
    (smodel.TINY, 53, 16, [5 + 4 * b for b in range(16)], 8),  # a full batch of 16
    (MID, 54, 5, [40, 44, 20, 47, 1], 16),                   # head_dim 128, 48-position window
    (TINY_TIED, 56, 6, [12, 33, 4, 50, 27, 9], 10),         # tied BF16 LM head on the matrix cores
    (GQA2, 57, 4, [40, 12, 30, 55], 10),                     # two K/V heads
    (NH8, 61, 7, [40, 12, 30, 55, 3, 24, 60], 10),           # eight query heads over one K/V head
    (NH8_KV2, 62, 4, [40, 12, 30, 55], 10),                  # eight query heads over two K/V heads of 128
], ids=["tiny_b4", "tiny_q8_b3", "tiny_b16", "mid_b5", "tiny_tied_bf16_b6", "gqa2_b4", "nh8_b7", "nh8_kv2_b4"])
def test_decode_batch_matches_oracle(oracle, cfg, seed, batch, prefills, steps):
    print(f"batched decode cfg={cfg.n_layers}x{cfg.hidden} batch={batch} steps={steps}", flush=True)
    _run(oracle, cfg, seed, batch, prefills, steps)


def test_decode_batch_gemma3_1b(oracle):
    """The Gemma-3-1B-shaped Q4_0 model (26 layers, hidden 1152, FFN 6912, vocab 262144),
    four sequences prefilled to different lengths around 1024 of 2048 positions, 4 steps."""
    print("batched decode gemma3-1b", flush=True)
    _run(oracle, smodel.GEMMA3_1B, 20260101, 4, [1024, 1000, 1031, 515], 4, nthreads=16, check_kv=False)


def test_decode_batch_gemma3_1b_16_sequences(oracle):
    """The configured batched workload: the Gemma-3-1B-shaped Q4_0 model with 16 sequences,
    each with its own 2048-position KV cache prefilled to a different length (all but two
    past the 512 sliding window, some across the global layers' 1024), 16 greedy steps in
    lock step; every sequence's tokens and logits against the oracle's one-sequence decode, and
    the K/V rows the steps write for four of them."""
    print("batched decode gemma3-1b, 16 sequences", flush=True)
    prefills = [1024, 1000, 1031, 515, 1536, 7, 2030, 800, 1023, 511, 1300, 64, 1777, 900, 1100, 1990]
    _run(oracle, smodel.GEMMA3_1B, 20260105, 16, prefills, 16, nthreads=16, kv_seqs=[0, 5, 6, 13])


def test_decode_batch_gemma3_1b_tied_bf16_lm_head(oracle):
    """The Gemma-3-1B shape with the tied BF16 LM head (604 MB table), four sequences, 4 steps."""
    print("batched decode gemma3-1b tied bf16 lm head", flush=True)
    cfg = smodel.DecodeConfig(**{**smodel.GEMMA3_1B.__dict__, "lm_dtype": synth.BF16})
    _run(oracle, cfg, 20260103, 4, [1024, 700, 1031, 300], 4, nthreads=16, check_kv=False)


def test_decode_batch_repeatable_and_rejects(oracle):
    from sapphire_amd.engine import Decoder
    m = smodel.synthetic_model(smodel.TINY, 55)
    dec = Decoder(m, batch=2)
    assert dec.lib.sapphire_decoder_batch(dec.ptr) == 2
    for b in range(2):
        dec.set_kv_seq(b, *m.kv_prefill(20, seed_offset=b))
    t1, _, _ = dec.generate_batch([5, 9], [20, 20], 6)
    for b in range(2):
        dec.set_kv_seq(b, *m.kv_prefill(20, seed_offset=b))
    t2, _, _ = dec.generate_batch([5, 9], [20, 20], 6)
    assert np.array_equal(t1, t2)
    with pytest.raises(RuntimeError):
        dec.generate(5, 20, 2)                                     # one-sequence call on a batch
    with pytest.raises(RuntimeError):
        dec.generate_batch([5, 9], [20, m.cfg.max_ctx - 1], 4)     # positions past max_ctx
    dec.close()
    with pytest.raises(RuntimeError):
        Decoder(m, batch=17)


def test_decode_batch_fused_qkv_attention_matches_unfused(oracle, monkeypatch):
    """The batched step's QKV GEMM and attention run as one launch (the attention workgroups
    poll q | k | v words that the GEMM's workgroups store tagged with the step and layer), or,
    with SAPPHIRE_FUSED_QKV_ATTN=0 at create time, as two. Both forms decode the oracle's
    tokens, and their logits agree to rounding (the fused launch's attention takes its K/V
    rows in rounds of 32 positions instead of 72)."""
    from sapphire_amd.engine import Decoder
    cfg, seed, batch, steps = GQA2, 58, 5, 10
    prefills = [40, 12, 30, 55, 3]
    m = smodel.synthetic_model(cfg, seed)
    toks0 = synth.rng(seed, 4242).integers(0, cfg.vocab, size=batch).astype(np.int32)
    kvs = [m.kv_prefill(prefills[b], seed_offset=100 + b) for b in range(batch)]
    out = {}
    for fused in ("1", "0"):
        monkeypatch.setenv("SAPPHIRE_FUSED_QKV_ATTN", fused)
        dec = Decoder(m, batch=batch)
        try:
            for b in range(batch):
                dec.set_kv_seq(b, *kvs[b])
            out[fused] = dec.generate_batch(toks0, np.asarray(prefills, np.int32), steps, keep_logits=True)[:2]
        finally:
            dec.close()
    (tf, lf), (tu, lu) = out["1"], out["0"]
    assert np.array_equal(tf, tu)
    d = np.abs(lf - lu).max() / np.abs(lu).max()
    print(f"fused vs unfused logits: {d:.2e}", flush=True)
    assert d <= 1e-4
    for b in (0, 4):
        ref_toks, _ = oracle_decode(oracle, m, *kvs[b], int(toks0[b]), prefills[b], steps, nthreads=4)
        assert np.array_equal(tf[:, b], ref_toks), f"sequence {b}"


def test_decode_batch_step_counter_across_the_restart(oracle):
    """The fused launch's tags are (step counter << 6) + layer + 1 in 32 bits: generate starts
    the counter over at 1, clearing every tagged word, before a call would take it to 2^26.
    A first call runs the counter's last values, the second starts over, the third goes on;
    each decodes the oracle's tokens from the same state."""
    from sapphire_amd.engine import Decoder
    cfg, seed, batch, steps = smodel.TINY, 59, 4, 6
    prefills = [30, 9, 41, 22]
    m = smodel.synthetic_model(cfg, seed)
    toks0 = synth.rng(seed, 4242).integers(0, cfg.vocab, size=batch).astype(np.int32)
    kvs = [m.kv_prefill(prefills[b], seed_offset=100 + b) for b in range(batch)]
    refs = [oracle_decode(oracle, m, kvs[b][0].copy(), kvs[b][1].copy(), int(toks0[b]), prefills[b], steps,
                          nthreads=4)[0] for b in range(batch)]
    last = (1 << 26) - 2                 # the largest count set_epoch_count takes
    dec = Decoder(m, batch=batch)
    try:
        assert dec.lib.sapphire_decoder_set_epoch_count(dec.ptr, last - steps - 1) == 0
        for _ in range(3):
            for b in range(batch):
                dec.set_kv_seq(b, *kvs[b])
            got, _, _ = dec.generate_batch(toks0, np.asarray(prefills, np.int32), steps)
            for b in range(batch):
                assert np.array_equal(got[:, b], refs[b]), f"sequence {b}"
        assert dec.lib.sapphire_decoder_set_epoch_count(dec.ptr, last + 1) == -1
    finally:
        dec.close()
