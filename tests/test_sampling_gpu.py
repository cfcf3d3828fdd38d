"""Temperature sampling on the GPU (sapphire_sample_dev, and the decoders' sampled steps)
against the oracle's draw (oracle_sample: vec_scale by 1/T, then sample_temperature,
utils.c:87-92 and 158-180; pinned to the compiled reference in tests/test_sampling.py).

Bar: the reference's token bit for bit, and the weights left in each row (expf((l/T - max)/T),
glibc's expf) bit for bit, for every row and draw:
* rows of many shapes (flat, peaked, very wide, ties, NaN / +inf / -inf), n from 1 to 262144
  (the Gemma-3 vocabulary), temperatures 0.05..3 and greedy;
* draws placed exactly on the reference's running-sum values and one float above them, across
  a 262144-entry row: these pin the float sum and the float running sum, not just the CDF;
* in the decoders (one sequence in both step forms, and the batched decoder, at TINY and at
  the Gemma-3-270M shape, T = 1.0 and 0.7): every step's token equals the oracle's draw on that
  step's logits, and those logits match the oracle's decode step along the same tokens within
  2e-3 relative. (A draw over 262144 tokens moves with any logit difference, so two decodes
  whose logits agree within tolerance need not draw the same tokens; the sampler itself is
  checked exactly, and the logits to the decode tolerance.)
"""
import numpy as np
import pytest

from oracle.oracle import oracle_decode_forced
from sapphire_amd import model as smodel
from sapphire_amd import synth
from sapphire_amd.device import DeviceArray, check
from tests.test_sampling import _rows, _same

pytestmark = pytest.mark.gpu

REL = 2e-3
PAD = 5


@pytest.fixture(scope="module")
def L():
    from sapphire_amd import load
    lib = load()
    check(lib.sapphire_set_device(0), "set device")
    return lib


def _gpu_sample(L, rows, n, t, draws):
    """rows [B][n + PAD] (padding included) -> (tokens[B], rows afterwards)."""
    B, ld = rows.shape
    rows = np.ascontiguousarray(rows, np.float32)
    d = DeviceArray.from_numpy(rows)
    dr = DeviceArray.from_numpy(np.asarray(draws, np.float32))
    tk = DeviceArray.empty(B, np.int32)
    ws = DeviceArray(max(int(L.sapphire_sample_workspace_bytes(n, B)), 256))
    check(L.sapphire_sample_dev(d.ptr, n, B, ld, float(t), dr.ptr, tk.ptr, ws.ptr, None), "sample")
    return tk.numpy(), d.numpy().reshape(B, ld)


@pytest.mark.parametrize("n", [1, 5, 4095, 4096, 4097, 50001, 262144])
def test_sample_rows_match_oracle(L, oracle, n):
    kinds = _rows(n, 100 + n)
    names = list(kinds)
    base = np.full((len(names), n + PAD), 1e30, np.float32)       # padding must stay untouched
    for j, name in enumerate(names):
        base[j, :n] = kinds[name]
    g = np.random.default_rng(n)
    for t in (1.0, 0.7, 0.05, 3.0, 0.0):
        for rep in range(3):
            draws = g.random(len(names)).astype(np.float32)
            if rep == 1:
                draws[:] = np.float32(0.0)
            if rep == 2:
                draws[::2] = np.float32(1.0)
            toks, out = _gpu_sample(L, base, n, t, draws)
            for j, name in enumerate(names):
                want_t, want_w = oracle.sample(base[j, :n], t, draws[j])
                assert toks[j] == want_t, (name, t, rep, float(draws[j]))
                assert _same(out[j, :n], want_w if t > 0 else base[j, :n]), (name, t, rep)
                assert np.array_equal(out[j, n:], base[j, n:])
        print(f"n={n} T={t}: {len(names)} rows x 3 draws match", flush=True)


@pytest.mark.parametrize("kind,t", [("normal1", 1.0), ("normal4", 0.7), ("wide60", 1.0), ("equal", 0.7)])
def test_sample_draws_on_running_sum_values(L, oracle, kind, t):
    """Draws equal to the reference's float running sum at chosen indices (selects that index
    when the sum rose there) and the next float above (the next index where it rose)."""
    n = 262144
    row = _rows(n, 9)[kind]
    _, w = oracle.sample(row, t, 0.5)
    s = np.add.accumulate(w, dtype=np.float32)[-1]
    cum = np.add.accumulate(w / s, dtype=np.float32)
    idx = sorted({0, 1, 2, 31, 32, 33, 4095, 4096, 4097, 8191, 12288, 65535, 131072, 200001, 262142, n - 1} |
                 set(np.random.default_rng(3).integers(0, n, 40).tolist()))
    draws = []
    for i in idx:
        draws += [cum[i], np.nextafter(cum[i], np.float32(2)), np.nextafter(cum[i], np.float32(-1))]
    draws += [np.float32(1.0), np.float32(0.0)]
    draws = np.array(draws, np.float32)
    rows = np.tile(np.concatenate([row, np.zeros(PAD, np.float32)]), (draws.size, 1))
    toks, out = _gpu_sample(L, rows, n, t, draws)
    for j, r in enumerate(draws):
        hit = np.flatnonzero(cum >= r)
        want = int(hit[0]) if hit.size else n - 1
        assert toks[j] == want, (j, float(r), toks[j], want)
        assert toks[j] == oracle.sample(row, t, r)[0]
    assert _same(out[0, :n], w)
    print(f"{kind} T={t}: {draws.size} draws on running-sum values match", flush=True)


def test_sample_rejects_bad_arguments(L):
    x = DeviceArray.from_numpy(np.zeros(8, np.float32))
    tk = DeviceArray.empty(1, np.int32)
    ws = DeviceArray(4096)
    dr = DeviceArray.from_numpy(np.zeros(1, np.float32))
    assert L.sapphire_sample_dev(x.ptr, 8, 1, 4, 1.0, dr.ptr, tk.ptr, ws.ptr, None) == -1      # ld < n
    assert L.sapphire_sample_dev(x.ptr, 8, 1, 8, 1.0, None, tk.ptr, ws.ptr, None) == -1        # no draws
    assert L.sapphire_sample_dev(x.ptr, (1 << 21) + 1, 1, (1 << 21) + 1, 1.0, dr.ptr, tk.ptr, ws.ptr, None) == -1
    assert L.sapphire_sample_workspace_bytes((1 << 21) + 1, 1) == 0
    assert L.sapphire_sample_dev(x.ptr, 8, 1, 8, 0.0, None, tk.ptr, ws.ptr, None) == 0          # greedy: no draws


G270M = smodel.GEMMA3_270M


def _check_steps(oracle, m, k, v, tok, pos, t, draws, got, got_logits):
    """Every token is the oracle's draw on that step's logits, and the logits match the
    oracle's decode step along the same tokens."""
    for s in range(got.shape[0]):
        assert got[s] == oracle.sample(got_logits[s], t, draws[s])[0], f"step {s}"
    kk, vv = k.copy(), v.copy()
    agree = 0
    for s in range(got.shape[0]):
        want_tok, lg = oracle_decode_forced(oracle, m, kk, vv, tok, pos + s, nthreads=8)
        err = np.abs(got_logits[s].astype(np.float64) - lg).max() / np.abs(lg).max()
        assert err <= REL, f"step {s}: relative logit error {err:.2e}"
        agree += oracle.sample(lg, t, draws[s])[0] == got[s]
        tok = int(got[s])
    return agree


@pytest.mark.parametrize("cfg,seed,prefill,steps,t,groups", [
    (smodel.TINY, 61, 40, 16, 1.0, None),
    (smodel.TINY, 61, 40, 16, 0.7, 0),
    (G270M, 62, 1024, 12, 1.0, None),
    (G270M, 63, 700, 12, 0.7, 0),
], ids=["tiny_t1", "tiny_t07_graph", "gemma3_270m_t1", "gemma3_270m_t07_graph"])
def test_decoder_sampling_matches_oracle(oracle, cfg, seed, prefill, steps, t, groups):
    from sapphire_amd.engine import Decoder
    print(f"sampled decode cfg={cfg.n_layers}x{cfg.hidden} T={t} groups={groups}", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    draws = np.random.default_rng(seed).random(steps).astype(np.float32)
    dec = Decoder(m)
    dec.set_kv(k, v)
    if groups is not None:
        dec.set_workgroups(groups)
    dec.set_sampling(t, draws)
    got, got_logits, _ = dec.generate(tok, prefill, steps, keep_logits=True)
    # greedy again after sampling: the step is captured anew
    dec.set_kv(k, v)
    dec.set_sampling(0.0)
    greedy, _, _ = dec.generate(tok, prefill, 2)
    dec.close()
    agree = _check_steps(oracle, m, k, v, tok, prefill, t, draws, got, got_logits)
    print(f"{steps} sampled steps exact on the device's logits; the oracle's own logits draw the same token "
          f"at {agree} of them", flush=True)
    assert greedy[0] == oracle_decode_forced(oracle, m, k.copy(), v.copy(), tok, prefill, nthreads=8)[0]


def test_decoder_sampling_multi_step_graph():
    """A sampled persistent-form call that takes no logits launches sixteen steps per graph;
    its tokens are, draw for draw, those of the call that takes the logits (one step per launch,
    checked against the oracle above). 35 steps: two sixteen-step launches and three single
    ones."""
    from sapphire_amd.engine import Decoder
    cfg, seed, prefill, steps = smodel.TINY, 66, 40, 35
    m = smodel.synthetic_model(cfg, seed)
    k, v = m.kv_prefill(prefill)
    tok = smodel.start_token(cfg, seed)
    draws = np.random.default_rng(seed).random(steps).astype(np.float32)
    dec = Decoder(m)
    try:
        assert dec.workgroups > 0
        dec.set_sampling(0.9, draws)
        dec.set_kv(k, v)
        with_logits, _, _ = dec.generate(tok, prefill, steps, keep_logits=True)
        dec.set_kv(k, v)
        without, _, _ = dec.generate(tok, prefill, steps)
        print(f"sampled without logits {without.tolist()}", flush=True)
        assert list(without) == list(with_logits)
    finally:
        dec.close()


@pytest.mark.parametrize("cfg,seed,prefills,steps,t", [
    (smodel.TINY, 64, [40, 10, 23, 55], 10, 0.7),
    (G270M, 65, [1024, 300, 900], 6, 1.0),
], ids=["tiny_b4_t07", "gemma3_270m_b3_t1"])
def test_batched_decoder_sampling_matches_oracle(oracle, cfg, seed, prefills, steps, t):
    from sapphire_amd.engine import Decoder
    B = len(prefills)
    print(f"sampled batched decode cfg={cfg.n_layers}x{cfg.hidden} batch={B} T={t}", flush=True)
    m = smodel.synthetic_model(cfg, seed)
    toks0 = synth.rng(seed, 4242).integers(0, cfg.vocab, size=B).astype(np.int32)
    kvs = [m.kv_prefill(prefills[b], seed_offset=100 + b) for b in range(B)]
    draws = np.random.default_rng(seed).random(steps * B).astype(np.float32)
    dec = Decoder(m, batch=B)
    for b in range(B):
        dec.set_kv_seq(b, *kvs[b])
    dec.set_sampling(t, draws)
    got, got_logits, _ = dec.generate_batch(toks0, np.asarray(prefills, np.int32), steps, keep_logits=True)
    dec.close()
    dr = draws.reshape(steps, B)
    for b in range(B):
        agree = _check_steps(oracle, m, *kvs[b], int(toks0[b]), prefills[b], t, dr[:, b], got[:, b],
                             got_logits[:, b])
        print(f"sequence {b}: {steps} sampled steps exact ({agree} agree on the oracle's logits)", flush=True)
