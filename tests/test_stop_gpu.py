"""Stop tokens on the device (sapphire_decoder_set_stop_tokens). The reference's generation
loop samples a token and ends when it is 1 or 106 (inference.c:298-301): the stop token is the
last one picked and no later step runs. Here the step that picks a stop token logs it and marks
its sequence done; every later step of that sequence logs -1 and writes no K/V row.

Each test decodes once without stop tokens, takes as the stop a token that first appears a few
steps in, and decodes again with it: the tokens up to and including the stop match the oracle
(one sequence) or the unconstrained run (a batch, whose unconstrained tokens match the oracle in
test_decode_batch_gpu), later entries are -1, and the KV cache holds exactly the rows of the
steps before the stop.
"""
import numpy as np
import pytest

from oracle.oracle import oracle_decode
from sapphire_amd import model as smodel
from sapphire_amd import synth
from tests.test_decode_gpu import WIDE, TINY_TIED, _compare

pytestmark = pytest.mark.gpu

REL = 2e-3


def _first_new(toks, start):
    """(step, token): the first step >= start whose token has not appeared before it, else step
    0 (a model that repeats one token stops at once)."""
    for s in range(start, len(toks)):
        if toks[s] not in toks[:s]:
            return s, int(toks[s])
    return 0, int(toks[0])


def _unused(toks, vocab):
    return next(t for t in range(vocab - 1, 0, -1) if t not in set(int(x) for x in np.ravel(toks)))


# groups: workgroups of the persistent step (None: the default), 0: the multi-launch step
@pytest.mark.parametrize("cfg,seed,prefill,steps,groups", [
    (smodel.TINY, 71, 40, 14, None),     # persistent layers; LM head, argmax and the advance kernel
    (smodel.TINY, 71, 40, 14, 0),        # the multi-launch step: kernels run, rows are not written
    (WIDE, 72, 30, 12, None),            # TILED LM head: the greedy epilogue advances and stops
    (WIDE, 72, 30, 12, 0),
    (TINY_TIED, 73, 40, 12, None),       # BF16 tied LM head
], ids=["tiny", "tiny_graph", "wide", "wide_graph", "tiny_tied"])
def test_stop_single_sequence(oracle, cfg, seed, prefill, steps, groups):
    from sapphire_amd.engine import Decoder
    print(f"stop cfg={cfg.n_layers}x{cfg.hidden} seed={seed} groups={groups}", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k0, v0 = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    k, v = k0.copy(), v0.copy()
    ref_toks, ref_logits = oracle_decode(oracle, m, k, v, tok, prefill, steps, nthreads=4, keep_logits=True)
    s_stop, t_stop = _first_new(list(ref_toks), 3)
    stops = [_unused(ref_toks, cfg.vocab), t_stop]
    dec = Decoder(m)
    if groups is not None:
        dec.set_workgroups(groups)
    dec.set_stop_tokens(stops)
    dec.set_kv(k0, v0)
    got_toks, got_logits, _ = dec.generate(tok, prefill, steps, keep_logits=True)
    gk, gv = dec.get_kv()
    print(f"stop token {t_stop} at step {s_stop}; tokens {got_toks.tolist()}", flush=True)
    n = _compare(ref_toks[:s_stop + 1], ref_logits[:s_stop + 1], got_toks[:s_stop + 1], got_logits[:s_stop + 1],
                 f"stop groups={groups}")
    assert n == s_stop + 1, f"near-tie at step {n}"
    assert np.all(got_toks[s_stop + 1:] == -1), got_toks
    # rows of the steps up to the stop are the oracle's; the stop token's row and later ones
    # keep the prefill's contents
    sl = slice(prefill, prefill + s_stop + 1)
    for name, g, r in (("K", gk, k), ("V", gv, v)):
        d = np.abs(g[:, :, sl] - r[:, :, sl]).max() / np.abs(r[:, :, sl]).max()
        assert d <= REL, f"{name} cache rows differ: {d:.2e}"
    assert np.array_equal(gk[:, :, prefill + s_stop + 1:], k0[:, :, prefill + s_stop + 1:])
    assert np.array_equal(gv[:, :, prefill + s_stop + 1:], v0[:, :, prefill + s_stop + 1:])
    assert np.array_equal(gk[:, :, :prefill], k0[:, :, :prefill])
    # cleared, the same decoder runs every step again
    dec.set_stop_tokens([])
    dec.set_kv(k0, v0)
    all_toks, _, _ = dec.generate(tok, prefill, steps)
    dec.close()
    assert np.array_equal(all_toks[:n], ref_toks[:n])
    assert np.all(all_toks >= 0)


def test_stop_sampled_sequence():
    """Temperature sampling with stop tokens: up to the stop, the sampled tokens of the
    unconstrained run (whose draws follow sample_temperature, test_sampling_gpu)."""
    from sapphire_amd.engine import Decoder
    cfg, seed, prefill, steps = smodel.TINY, 74, 40, 14
    m = smodel.synthetic_model(cfg, seed)
    k0, v0 = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    draws = synth.rng(seed, 9).random(steps).astype(np.float32)
    dec = Decoder(m)
    dec.set_sampling(0.8, draws)
    dec.set_kv(k0, v0)
    free, _, _ = dec.generate(tok, prefill, steps)
    s_stop, t_stop = _first_new(list(free), 3)
    dec.set_stop_tokens([t_stop])
    dec.set_kv(k0, v0)
    got, _, _ = dec.generate(tok, prefill, steps)
    dec.close()
    print(f"sampled: free {free.tolist()} stopped {got.tolist()}", flush=True)
    assert np.array_equal(got[:s_stop + 1], free[:s_stop + 1])
    assert np.all(got[s_stop + 1:] == -1)


def test_stop_batch():
    """A batch: each sequence stops at its own first stop token; the others run every step."""
    from sapphire_amd.engine import Decoder
    cfg, seed, batch, steps = smodel.TINY, 75, 6, 12
    prefills = [40, 10, 23, 55, 31, 7]
    m = smodel.synthetic_model(cfg, seed)
    rng = synth.rng(seed, 4242)
    toks0 = rng.integers(0, cfg.vocab, size=batch).astype(np.int32)
    kvs = [m.kv_prefill(prefills[b], seed_offset=100 + b) for b in range(batch)]
    dec = Decoder(m, batch=batch)
    for b in range(batch):
        dec.set_kv_seq(b, *kvs[b])
    free, _, _ = dec.generate_batch(toks0, np.asarray(prefills, np.int32), steps)
    # stop sequence 0 at a fresh token of its own, and sequence 3 at step 0 (its first token)
    s0, t0 = _first_new(list(free[:, 0]), 4)
    stops = [t0, int(free[0, 3])]
    for b in range(batch):
        dec.set_kv_seq(b, *kvs[b])
    dec.set_stop_tokens(stops)
    got, _, _ = dec.generate_batch(toks0, np.asarray(prefills, np.int32), steps)
    kv_after = [dec.get_kv_seq(b) for b in range(batch)]
    dec.close()
    print(f"stops {stops}; free seq0 {free[:, 0].tolist()} got seq0 {got[:, 0].tolist()}", flush=True)
    for b in range(batch):
        hit = [s for s in range(steps) if int(free[s, b]) in stops]
        s_b = hit[0] if hit else steps
        assert np.array_equal(got[:s_b + 1, b], free[:s_b + 1, b]), f"sequence {b}"
        assert np.all(got[s_b + 1:, b] == -1), f"sequence {b}: {got[:, b]}"
        # no row at or after the stop token's position is written
        k, v = kvs[b]
        first_unwritten = prefills[b] + min(s_b + 1, steps)
        assert np.array_equal(kv_after[b][0][:, :, first_unwritten:], k[:, :, first_unwritten:]), f"sequence {b}"
        assert np.array_equal(kv_after[b][1][:, :, first_unwritten:], v[:, :, first_unwritten:]), f"sequence {b}"
    assert got[1:, 3].tolist() == [-1] * (steps - 1)


def test_stop_tokens_rejected():
    from sapphire_amd.engine import Decoder
    m = smodel.synthetic_model(smodel.TINY, 76)
    dec = Decoder(m)
    try:
        with pytest.raises(RuntimeError, match="at most"):
            dec.set_stop_tokens(list(range(1, 10)))
        with pytest.raises(RuntimeError, match="outside the vocabulary"):
            dec.set_stop_tokens([smodel.TINY.vocab])
        with pytest.raises(RuntimeError, match="outside the vocabulary"):
            dec.set_stop_tokens([-1])
        dec.set_stop_tokens([1, 106])
    finally:
        dec.close()
