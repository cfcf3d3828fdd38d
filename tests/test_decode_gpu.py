"""Device-resident greedy decode (include/decoder.h) against the oracle's decode step, which
is bit-exact with the compiled reference engine (tests/test_oracle_pin.py).

Parity bar, on every step: logits within 2e-3 relative (max |gpu - ref| over a step /
max |ref|), every logit within 2e-3 |ref| + 1e-4 max |ref|, and identical greedy tokens. A
token may differ only where the oracle's top-2 logit gap is inside that tolerance (a
near-tie); the sequences are then compared up to that step. Each comparison prints the worst
normwise error and the largest fraction of the per-logit bound used (run with -s to see them).
"""
import numpy as np
import pytest

from oracle.oracle import oracle_decode
from sapphire_amd import model as smodel
from sapphire_amd import synth

pytestmark = pytest.mark.gpu

REL = 2e-3


def _compare(ref_toks, ref_logits, got_toks, got_logits, label=""):
    steps = len(ref_toks)
    n, worst, used = steps, 0.0, 0.0
    for s in range(steps):
        r, g = ref_logits[s].astype(np.float64), got_logits[s].astype(np.float64)
        fin = np.isfinite(r)
        assert np.array_equal(np.isnan(g), np.isnan(r)), f"step {s}: NaN logits differ"
        assert np.array_equal(g[~fin & ~np.isnan(r)], r[~fin & ~np.isnan(r)]), f"step {s}: infinite logits differ"
        r, g = r[fin], g[fin]
        scale = np.abs(r).max()
        d = np.abs(g - r)
        err = d.max() / scale
        frac = (d / (REL * np.abs(r) + 1e-4 * scale)).max()
        worst, used = max(worst, err), max(used, frac)
        assert err <= REL, f"step {s}: relative logit error {err:.2e}"
        assert frac <= 1.0, f"step {s}: logit error {d.max():.3e} above 2e-3 |ref| + 1e-4 max|ref| ({frac:.2f} of it)"
        if got_toks[s] != ref_toks[s]:
            top2 = np.sort(r)[-2:]
            gap = top2[1] - top2[0]
            assert gap <= REL * scale, f"step {s}: token {got_toks[s]} != {ref_toks[s]} (gap {gap})"
            n = s          # a near-tie: the sequences diverge from here
            break
    print(f"parity{(' ' + label) if label else ''}: {n} of {steps} steps, worst max|gpu-ref|/max|ref| {worst:.2e}, "
          f"per-logit bound used {used:.3f}", flush=True)
    return n


MID = smodel.DecodeConfig(n_layers=6, hidden=256, n_heads=4, n_kv_heads=1, head_dim=128, ffn=512, vocab=8192,
                          max_ctx=160, sliding_window=48, global_layers=(5,))
TINY_Q8 = smodel.DecodeConfig(**{**smodel.TINY.__dict__, "wdtype": synth.Q8_0, "lm_dtype": synth.Q8_0})
# two K/V heads shared by two query heads each (grouped-query attention, attention.c:131-135)
GQA2 = smodel.DecodeConfig(n_layers=3, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=4096,
                           max_ctx=96, sliding_window=24, global_layers=(2,))
# the reference's own LM head: the BF16 embedding table (weight tying, transformer.c:393-408)
TINY_TIED = smodel.DecodeConfig(**{**smodel.TINY.__dict__, "lm_dtype": synth.BF16})
# the 270M widths (hidden 640, heads of 256) in two layers: a TILED LM head, whose greedy
# epilogue picks the token and advances the step
WIDE = smodel.DecodeConfig(n_layers=2, hidden=640, n_heads=4, n_kv_heads=1, head_dim=256, ffn=1024, vocab=8192,
                           max_ctx=96, sliding_window=24, global_layers=(1,))
# hidden above 1024: the persistent step's eight-element-per-thread vector form
H1280 = smodel.DecodeConfig(n_layers=2, hidden=1280, n_heads=4, n_kv_heads=1, head_dim=256, ffn=2048, vocab=8192,
                            max_ctx=96, sliding_window=24, global_layers=(1,))


# eight query heads: over one K/V head of 64 dims, and over two of 128 (four per K/V head)
NH8 = smodel.DecodeConfig(n_layers=2, hidden=256, n_heads=8, n_kv_heads=1, head_dim=64, ffn=512, vocab=4096,
                          max_ctx=96, sliding_window=24, global_layers=(1,))
NH8_KV2 = smodel.DecodeConfig(n_layers=2, hidden=256, n_heads=8, n_kv_heads=2, head_dim=128, ffn=512, vocab=4096,
                              max_ctx=96, sliding_window=24, global_layers=(1,))


# groups: workgroups of the persistent step (None: the decoder's default), 0: the multi-launch step
@pytest.mark.parametrize("cfg,seed,prefill,steps,groups", [
    (smodel.TINY, 31, 40, 16, None),      # window 24 < positions: local layers slide
    (smodel.TINY, 31, 40, 16, 0),
    (smodel.TINY, 31, 40, 16, 16),        # fewer workgroups than positions: several per slice
    (smodel.TINY, 31, 40, 16, 256),       # more workgroups than positions: empty slices
    (TINY_Q8, 32, 10, 12, None),          # Q8_0 weights, positions inside the window
    (TINY_Q8, 32, 10, 12, 0),
    (MID, 33, 40, 24, None),              # head_dim 128, crosses the 48-position window while decoding
    (MID, 33, 40, 24, 0),
    (MID, 33, 40, 24, 96),
    (TINY_TIED, 37, 40, 12, None),
    (TINY_TIED, 37, 40, 12, 0),
    (GQA2, 41, 40, 12, 0),                # two K/V heads (multi-launch step only)
    (WIDE, 42, 40, 16, None),             # TILED LM head with the greedy-step epilogue
    (WIDE, 42, 40, 16, 0),
    (H1280, 44, 40, 12, None),            # hidden 1280 (eight vector elements per thread)
    (H1280, 44, 40, 12, 0),
    (NH8, 45, 40, 12, None),              # eight query heads (16 slices per head)
    (NH8, 45, 40, 12, 0),
    (NH8_KV2, 46, 40, 12, 0),             # eight query heads over two K/V heads (multi-launch step only)
], ids=["tiny", "tiny_graph", "tiny_g16", "tiny_g256", "tiny_q8", "tiny_q8_graph", "mid_window", "mid_window_graph",
        "mid_window_g96", "tiny_tied_bf16", "tiny_tied_bf16_graph", "gqa2_graph", "wide", "wide_graph", "h1280",
        "h1280_graph", "nh8", "nh8_graph", "nh8_kv2_graph"])
def test_decode_matches_oracle(oracle, cfg, seed, prefill, steps, groups):
    from sapphire_amd.engine import Decoder
    print(f"decode cfg={cfg.n_layers}x{cfg.hidden} seed={seed} prefill={prefill} steps={steps} groups={groups}",
          flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    dec = Decoder(m)
    if groups is None:
        assert dec.workgroups > 0, "the persistent step is the default"
    else:
        dec.set_workgroups(groups)
        assert dec.workgroups == groups
    dec.set_kv(k, v)
    got_toks, got_logits, _ = dec.generate(tok, prefill, steps, keep_logits=True)
    gk, gv = dec.get_kv()
    dec.close()
    ref_toks, ref_logits = oracle_decode(oracle, m, k, v, tok, prefill, steps, nthreads=4, keep_logits=True)
    n = _compare(ref_toks, ref_logits, got_toks, got_logits, f"{cfg.n_layers}x{cfg.hidden} groups={groups}")
    assert n == steps, f"near-tie at step {n}"
    # the KV cache rows written while decoding (K after QK-norm + RoPE, V raw)
    sl = slice(prefill, prefill + steps)
    for name, g, r in (("K", gk, k), ("V", gv, v)):
        d = np.abs(g[:, :, sl] - r[:, :, sl]).max() / np.abs(r[:, :, sl]).max()
        assert d <= REL, f"{name} cache rows differ: {d:.2e}"
    assert np.array_equal(gk[:, :, :prefill], k[:, :, :prefill])


def test_decode_gemma3_270m_64_steps(oracle):
    """The Gemma-3-270M-shaped Q4_0 model, KV prefilled to 1024 of 2048 positions, 64
    greedy steps: identical tokens, logits within 2e-3 on every step, for the persistent step
    at 128 (the default), 64 and 256 workgroups and for the multi-launch step."""
    from sapphire_amd.engine import Decoder
    cfg, seed, prefill, steps = smodel.GEMMA3_270M, 20260101, 1024, 64
    print("decode gemma3-270m 64 steps", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    dec = Decoder(m)
    assert dec.workgroups == 128
    runs = {}
    for groups in (128, 64, 256, 0):
        dec.set_workgroups(groups)
        dec.set_kv(k, v)
        runs[groups] = dec.generate(tok, prefill, steps, keep_logits=True)[:2]
        print(f"gpu done: groups={groups}", flush=True)
    dec.close()
    ref_toks, ref_logits = oracle_decode(oracle, m, k, v, tok, prefill, steps, nthreads=16, keep_logits=True)
    for groups, (got_toks, got_logits) in runs.items():
        n = _compare(ref_toks, ref_logits, got_toks, got_logits, f"gemma3-270m groups={groups}")
        assert n == steps, f"groups={groups}: near-tie at step {n}: tokens agree on steps 0..{n - 1}"


def _bf16_norms(m):
    """The model with every norm weight rounded to a bf16 value (its upper 16 bits), so the
    fp32 oracle and a decoder given the bf16 halves see the same numbers."""
    import copy
    m = copy.deepcopy(m)
    trunc = lambda a: (np.ascontiguousarray(a, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    for n in m.norms:
        m.norms[n] = trunc(m.norms[n])
    m.norm_final = trunc(m.norm_final)
    return m


@pytest.mark.parametrize("cfg,seed,prefill,steps", [
    (smodel.TINY, 61, 40, 12),
    (smodel.GEMMA3_270M, 62, 1024, 16),
], ids=["tiny", "gemma3_270m"])
def test_decode_bf16_norm_weights(oracle, cfg, seed, prefill, steps):
    """Norm weights handed over as bf16 (norm_dtype DTYPE_BF16, as a safetensors checkpoint
    stores them) are widened as get_norm_weights does (utils.c:218-225): the decode matches the
    oracle run on the same values in fp32, in the persistent and the multi-launch step."""
    from sapphire_amd.engine import Decoder
    m = _bf16_norms(smodel.synthetic_model(cfg, seed))
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    ref_toks, ref_logits = oracle_decode(oracle, m, k, v, tok, prefill, steps, nthreads=16, keep_logits=True)
    for groups in (None, 0):
        dec = Decoder(m, norm_bf16=True)
        if groups is not None:
            dec.set_workgroups(groups)
        dec.set_kv(k, v)
        got_toks, got_logits, _ = dec.generate(tok, prefill, steps, keep_logits=True)
        dec.close()
        n = _compare(ref_toks, ref_logits, got_toks, got_logits, f"bf16 norms {cfg.n_layers}x{cfg.hidden} groups={groups}")
        assert n == steps, f"groups={groups}: near-tie at step {n}"


def test_decode_rejects_unknown_norm_dtype():
    """A norm_dtype other than F32 / BF16 is refused at create time, with the reason."""
    from sapphire_amd.engine import Decoder
    m = smodel.synthetic_model(smodel.TINY, 63)
    with pytest.raises(RuntimeError, match="norm_dtype"):
        Decoder(m, norm_dtype=7)


@pytest.mark.parametrize("case", ["tied_pairs", "nan_row0", "nan_winner"])
def test_decode_greedy_epilogue_ties_and_nan(oracle, case):
    """The TILED LM head picks the greedy token in its epilogue (one 64-bit key per row: the
    value's order, then the lower index) under sample_greedy's rules (utils.c:145-156):
    * tied_pairs: LM-head rows 2i and 2i+1 identical, so every step's maximum is a tie that
      the lower (even) index must win;
    * nan_row0: a NaN block scale in row 0 makes logits[0] NaN, and the token is 0 on every
      step (nothing compares greater than NaN);
    * nan_winner: a NaN in the row the first step would pick; a NaN row never wins."""
    from sapphire_amd.engine import Decoder
    cfg, seed, prefill, steps = WIDE, 43, 30, 8
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    if case == "tied_pairs":
        m.lm_head[1::2] = m.lm_head[0::2]
    elif case == "nan_row0":
        m.lm_head[0, 3]["scale"] = np.nan
    else:
        first, _ = oracle_decode(oracle, m, k.copy(), v.copy(), tok, prefill, 1, nthreads=4, keep_logits=True)
        m.lm_head[int(first[0]), 1]["scale"] = np.nan
    ref_toks, ref_logits = oracle_decode(oracle, m, k.copy(), v.copy(), tok, prefill, steps, nthreads=4,
                                         keep_logits=True)
    if case == "tied_pairs":
        assert all(t % 2 == 0 for t in ref_toks)
    if case == "nan_row0":
        assert list(ref_toks) == [0] * steps
    runs = {}
    for groups in (None, 0):
        dec = Decoder(m)
        if groups is not None:
            dec.set_workgroups(groups)
        dec.set_kv(k, v)
        runs[groups] = dec.generate(tok, prefill, steps, keep_logits=True)[:2]
        dec.close()
    for groups, (got_toks, got_logits) in runs.items():
        assert list(got_toks) == list(ref_toks), f"groups={groups}: {list(got_toks)} != {list(ref_toks)}"
        assert _compare(ref_toks, ref_logits, got_toks, got_logits, f"{case} groups={groups}") == steps


def test_decode_gemma3_270m_tied_bf16_lm_head(oracle):
    """Gemma-3-270M shape with the reference's own LM head, the 335 MB BF16 embedding table
    (weight tying): 16 greedy steps from KV 1024, persistent and multi-launch steps."""
    from sapphire_amd.engine import Decoder
    cfg = smodel.DecodeConfig(**{**smodel.GEMMA3_270M.__dict__, "lm_dtype": synth.BF16})
    seed, prefill, steps = 20260102, 1024, 16
    print("decode gemma3-270m tied bf16 lm head", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    dec = Decoder(m)
    runs = {}
    for groups in (128, 0):
        dec.set_workgroups(groups)
        dec.set_kv(k, v)
        runs[groups] = dec.generate(tok, prefill, steps, keep_logits=True)[:2]
        print(f"gpu done: groups={groups}", flush=True)
    dec.close()
    ref_toks, ref_logits = oracle_decode(oracle, m, k, v, tok, prefill, steps, nthreads=16, keep_logits=True)
    for groups, (got_toks, got_logits) in runs.items():
        n = _compare(ref_toks, ref_logits, got_toks, got_logits, f"gemma3-270m tied groups={groups}")
        assert n == steps, f"groups={groups}: near-tie at step {n}"


def test_decode_workgroups_validation():
    """sapphire_decoder_set_workgroups keeps the current form when the count cannot run."""
    from sapphire_amd.engine import Decoder
    m = smodel.synthetic_model(smodel.TINY, 35)
    dec = Decoder(m)
    try:
        g0 = dec.workgroups
        for bad in (-1, 2, 257):          # negative, fewer than the query heads, above the maximum
            with pytest.raises(RuntimeError):
                dec.set_workgroups(bad)
            assert dec.workgroups == g0
    finally:
        dec.close()
    bdec = Decoder(m, batch=2)
    try:
        assert bdec.workgroups == 0
        with pytest.raises(RuntimeError):
            bdec.set_workgroups(64)
    finally:
        bdec.close()


def test_decode_persistent_epochs_across_calls(oracle):
    """Many short generate calls on one decoder: every call's steps get fresh epochs, so no stage
    reads a vector left by an earlier step; each call matches the oracle from the same state."""
    from sapphire_amd.engine import Decoder
    cfg = smodel.TINY
    m = smodel.synthetic_model(cfg, 36)
    k, v = m.kv_prefill(30)
    tok = smodel.start_token(cfg, 36)
    ref_toks, _ = oracle_decode(oracle, m, k.copy(), v.copy(), tok, 30, 3, nthreads=4)
    dec = Decoder(m)
    try:
        for _ in range(20):
            dec.set_kv(k, v)
            got, _, _ = dec.generate(tok, 30, 3)
            assert list(got) == list(ref_toks)
    finally:
        dec.close()


def test_decode_persistent_epochs_across_the_reset(oracle):
    """Epochs just below 2^32: a first call whose stages use the last epochs before the reset,
    then calls whose start clears the exchange words and restarts the epochs. Every call
    decodes the oracle's tokens from the same state."""
    from sapphire_amd.engine import Decoder
    cfg = smodel.TINY
    m = smodel.synthetic_model(cfg, 38)
    k, v = m.kv_prefill(30)
    tok = smodel.start_token(cfg, 38)
    steps = 6
    ref_toks, _ = oracle_decode(oracle, m, k.copy(), v.copy(), tok, 30, steps, nthreads=4)
    per = 8 * (cfg.n_layers + 1)
    last = (1 << 32) // per - 1          # the last step count whose epochs fit
    dec = Decoder(m)
    try:
        assert dec.workgroups > 0
        # steps + 1 more fit: no reset before this call, its epochs end just below 2^32
        assert dec.lib.sapphire_decoder_set_epoch_count(dec.ptr, last - steps - 1) == 0
        for _ in range(3):                  # the second call starts over, the third continues
            dec.set_kv(k, v)
            got, _, _ = dec.generate(tok, 30, steps)
            assert list(got) == list(ref_toks)
        assert dec.lib.sapphire_decoder_set_epoch_count(dec.ptr, last + 1) == -1
    finally:
        dec.close()


@pytest.mark.parametrize("run,stop_at", [(4, None), (3, 7), (5, 4)], ids=["run4", "run3_stop7", "run5_stop4"])
def test_decode_token_slots_across_runs(oracle, monkeypatch, run, stop_at):
    """The persistent step's greedy token goes from the LM head to the next step's layers
    kernel through tagged slots, in runs of at most 2^14 - 1 steps, each ending with a settle
    launch that logs its last token and starts the next run from it. With runs of 3-5 steps
    (SAPPHIRE_TOKEN_SLOT_RUN) a 14-step call crosses several runs: the tokens, logits and K/V
    rows are the oracle's; with a stop token first seen at step stop_at, the call ends there
    (stop at the end of a run, and inside one)."""
    from sapphire_amd.engine import Decoder
    cfg, seed, prefill, steps = smodel.TINY, 39, 30, 14
    monkeypatch.setenv("SAPPHIRE_TOKEN_SLOT_RUN", str(run))
    m = smodel.synthetic_model(cfg, seed)
    k0, v0 = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    k, v = k0.copy(), v0.copy()
    ref_toks, ref_logits = oracle_decode(oracle, m, k, v, tok, prefill, steps, nthreads=4, keep_logits=True)
    stops = []
    if stop_at is not None:
        # a token that first appears at stop_at (the seed is chosen so that one does)
        assert ref_toks[stop_at] not in ref_toks[:stop_at], ref_toks
        stops = [int(ref_toks[stop_at])]
    dec = Decoder(m)
    try:
        assert dec.workgroups > 0
        dec.set_stop_tokens(stops)
        for _ in range(2):                  # the second call starts its runs over
            dec.set_kv(k0, v0)
            got_toks, got_logits, _ = dec.generate(tok, prefill, steps, keep_logits=True)
            n = steps if stop_at is None else stop_at + 1
            print(f"run {run}: tokens {got_toks.tolist()}", flush=True)
            assert _compare(ref_toks[:n], ref_logits[:n], got_toks[:n], got_logits[:n], f"run {run}") == n
            assert np.all(got_toks[n:] == -1)
            gk, gv = dec.get_kv()
            sl = slice(prefill, prefill + n)
            for name, g, r in (("K", gk, k), ("V", gv, v)):
                d = np.abs(g[:, :, sl] - r[:, :, sl]).max() / np.abs(r[:, :, sl]).max()
                assert d <= REL, f"{name} cache rows differ: {d:.2e}"
            assert np.array_equal(gk[:, :, prefill + n:], k0[:, :, prefill + n:])
    finally:
        dec.close()


@pytest.mark.parametrize("run,stop_at", [(None, None), (None, 5), (20, None), (20, 12)],
                         ids=["default_run", "stop5", "run20", "run20_stop12"])
def test_decode_multi_step_graph(oracle, monkeypatch, run, stop_at):
    """A persistent-form call that takes no logits launches its steps sixteen to a graph,
    where the sixteen fit in the call and inside one token-slot run, and the others one at a
    time. A 45-step call (16 + 16 + 13 single steps; with runs of 20 steps, 16 + 4 single per
    run and 5 single at the end) decodes the oracle's tokens and K/V rows, also with a stop token
    inside a sixteen-step launch."""
    from sapphire_amd.engine import Decoder
    cfg, seed, prefill, steps = smodel.TINY, 39, 30, 45
    if run is not None:
        monkeypatch.setenv("SAPPHIRE_TOKEN_SLOT_RUN", str(run))
    m = smodel.synthetic_model(cfg, seed)
    k0, v0 = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    k, v = k0.copy(), v0.copy()
    ref_toks, _ = oracle_decode(oracle, m, k, v, tok, prefill, steps, nthreads=4)
    stops = []
    if stop_at is not None:
        # a token that first appears at stop_at (the seed is chosen so that one does)
        assert ref_toks[stop_at] not in ref_toks[:stop_at], ref_toks
        stops = [int(ref_toks[stop_at])]
    n = steps if stop_at is None else stop_at + 1
    dec = Decoder(m)
    try:
        assert dec.workgroups > 0
        dec.set_stop_tokens(stops)
        for _ in range(2):                  # the second call replays the captured graphs
            dec.set_kv(k0, v0)
            got, _, _ = dec.generate(tok, prefill, steps)
            print(f"run {run}, stop {stop_at}: tokens {got.tolist()}", flush=True)
            assert list(got[:n]) == list(ref_toks[:n])
            assert np.all(got[n:] == -1)
            gk, gv = dec.get_kv()
            sl = slice(prefill, prefill + n)
            for name, g, r in (("K", gk, k), ("V", gv, v)):
                d = np.abs(g[:, :, sl] - r[:, :, sl]).max() / np.abs(r[:, :, sl]).max()
                assert d <= REL, f"{name} cache rows differ: {d:.2e}"
            assert np.array_equal(gk[:, :, prefill + n:], k0[:, :, prefill + n:])
    finally:
        dec.close()


def test_decode_repeatable(oracle):
    """Two generate calls on one decoder (the captured graph is replayed, the state reset)."""
    from sapphire_amd.engine import Decoder
    m = smodel.synthetic_model(smodel.TINY, 34)
    k, v = m.kv_prefill(20)
    dec = Decoder(m)
    dec.set_kv(k, v)
    t1, _, _ = dec.generate(5, 20, 8)
    dec.set_kv(k, v)
    t2, _, _ = dec.generate(5, 20, 8)
    dec.close()
    assert list(t1) == list(t2)
    with pytest.raises(RuntimeError):
        dec2 = Decoder(m)
        try:
            dec2.generate(5, m.cfg.max_ctx - 2, 8)      # positions past max_ctx are refused
        finally:
            dec2.close()


# ---- prefill (sapphire_decoder_prefill) ----

def _kv_close(got, ref, sl, what):
    d = np.abs(got[:, :, sl] - ref[:, :, sl]).max() / max(np.abs(ref[:, :, sl]).max(), 1e-30)
    assert d <= REL, f"{what} cache rows differ: {d:.2e}"


@pytest.mark.parametrize("cfg,seed,kv0,n,steps", [
    (smodel.TINY, 41, 0, 40, 8),       # chunks 16 + 16 + 8, local layers slide while prefilling
    (MID, 42, 20, 37, 10),             # on top of 20 cached positions; chunks 16 + 16 + 5
    (smodel.GEMMA3_270M, 43, 0, 100, 16),
], ids=["tiny", "mid_on_cache", "gemma3_270m"])
def test_prefill_matches_oracle(oracle, cfg, seed, kv0, n, steps):
    """A prompt through sapphire_decoder_prefill, then greedy decode from its last token:
    K/V rows and the decoded tokens and logits against the oracle running the same tokens
    one decode step at a time (the reference's batched prefill computes the same thing:
    every row of a chunk is written before attention reads it)."""
    from oracle.oracle import oracle_prefill
    from sapphire_amd.engine import Decoder
    print(f"prefill cfg={cfg.n_layers}x{cfg.hidden} kv0={kv0} n={n} steps={steps}", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(kv0)
    prompt = synth.rng(seed, 5).integers(0, cfg.vocab, n + 1).astype(np.int32)
    dec = Decoder(m)
    dec.set_kv(k, v)
    dec.prefill(prompt[:n], kv0)
    got_toks, got_logits, _ = dec.generate(int(prompt[n]), kv0 + n, steps, keep_logits=True)
    gk, gv = dec.get_kv()
    dec.close()
    rk, rv = k.copy(), v.copy()
    oracle_prefill(oracle, m, rk, rv, prompt[:n], kv0, nthreads=16)
    pk, pv = rk.copy(), rv.copy()    # after the prompt
    ref_toks, ref_logits = oracle_decode(oracle, m, rk, rv, int(prompt[n]), kv0 + n, steps, nthreads=16,
                                         keep_logits=True)
    assert np.array_equal(gk[:, :, :kv0], k[:, :, :kv0]) and np.array_equal(gv[:, :, :kv0], v[:, :, :kv0])
    _kv_close(gk, pk, slice(kv0, kv0 + n), "K")
    _kv_close(gv, pv, slice(kv0, kv0 + n), "V")
    n_ok = _compare(ref_toks, ref_logits, got_toks, got_logits)
    assert n_ok == steps, f"near-tie at step {n_ok}"


def test_prefill_batched_decoder_sequence(oracle):
    """Prefill of one sequence of a batched decoder fills that sequence's cache only."""
    from oracle.oracle import oracle_prefill
    from sapphire_amd.engine import Decoder
    cfg, seed, n = smodel.TINY, 44, 20
    print("prefill batched decoder", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    prompt = synth.rng(seed, 6).integers(0, cfg.vocab, n).astype(np.int32)
    dec = Decoder(m, batch=4)
    shape = (cfg.n_layers, cfg.n_kv_heads, cfg.max_ctx, cfg.head_dim)
    for b in range(4):
        dec.set_kv_seq(b, np.zeros(shape, np.float32), np.zeros(shape, np.float32))
    dec.prefill(prompt, 0, seq=2)
    caches = [dec.get_kv_seq(b) for b in range(4)]
    dec.close()
    rk, rv = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    oracle_prefill(oracle, m, rk, rv, prompt, 0, nthreads=4)
    for b in (0, 1, 3):
        assert not caches[b][0].any() and not caches[b][1].any()
    _kv_close(caches[2][0], rk, slice(0, n), "K")
    _kv_close(caches[2][1], rv, slice(0, n), "V")
    assert not caches[2][0][:, :, n:].any()


def test_prefill_argument_checks():
    from sapphire_amd.engine import Decoder
    m = smodel.synthetic_model(smodel.TINY, 45)
    dec = Decoder(m)
    try:
        with pytest.raises(RuntimeError):
            dec.prefill([1, 2, 3], smodel.TINY.max_ctx - 2)        # past max_ctx
        with pytest.raises(RuntimeError):
            dec.prefill([1, smodel.TINY.vocab], 0)                 # outside the vocabulary
        with pytest.raises(RuntimeError):
            dec.prefill([1, 2], 0, seq=1)                          # one-sequence decoder
    finally:
        dec.close()
