"""The device-resident decode engine (include/decoder.h) from Python.

:class:`Decoder` uploads a :class:`sapphire_amd.model.SyntheticModel` (or any object with
the same fields) once and runs greedy decode steps as HIP graph replays; weights,
activations, the KV cache and the sampled tokens stay in HBM.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np

from . import load
from . import model as smodel
from . import synth

_VPP = C.POINTER(C.c_void_p)
_FPP = C.POINTER(C.POINTER(C.c_float))


class DecoderConfig(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("hidden", C.c_int), ("n_heads", C.c_int), ("n_kv_heads", C.c_int),
        ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int), ("max_ctx", C.c_int),
        ("sliding_window", C.c_int), ("global_mask", C.c_ulonglong),
        ("query_pre_attn_scalar", C.c_float), ("rope_theta", C.c_float), ("rope_local_base", C.c_float),
        ("eps", C.c_float), ("wdtype", C.c_int), ("lm_dtype", C.c_int),
    ]


class DecoderWeights(C.Structure):
    _fields_ = [(n, _VPP) for n in smodel.PROJ] + \
               [(n, _FPP) for n in ("norm_attn", "norm_attn_post", "norm_ffn", "norm_ffn_post", "q_norm", "k_norm")] + \
               [("embed_bf16", C.c_void_p), ("norm_final", C.c_void_p), ("lm_head", C.c_void_p),
                ("norm_dtype", C.c_int)]


def _protos(L):
    L.sapphire_decoder_create.restype = C.c_void_p
    L.sapphire_decoder_create.argtypes = [C.POINTER(DecoderConfig), C.POINTER(DecoderWeights)]
    L.sapphire_decoder_destroy.restype = None
    L.sapphire_decoder_destroy.argtypes = [C.c_void_p]
    L.sapphire_decoder_set_kv.restype = C.c_int
    L.sapphire_decoder_set_kv.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
    L.sapphire_decoder_get_kv.restype = C.c_int
    L.sapphire_decoder_get_kv.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
    L.sapphire_decoder_generate.restype = C.c_int
    L.sapphire_decoder_generate.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                            C.POINTER(C.c_float)]
    L.sapphire_decoder_create_batch.restype = C.c_void_p
    L.sapphire_decoder_create_batch.argtypes = [C.POINTER(DecoderConfig), C.POINTER(DecoderWeights), C.c_int]
    L.sapphire_decoder_batch.restype = C.c_int
    L.sapphire_decoder_batch.argtypes = [C.c_void_p]
    for n in ("sapphire_decoder_set_kv_seq", "sapphire_decoder_get_kv_seq"):
        getattr(L, n).restype = C.c_int
        getattr(L, n).argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
    L.sapphire_decoder_set_workgroups.restype = C.c_int
    L.sapphire_decoder_set_workgroups.argtypes = [C.c_void_p, C.c_int]
    L.sapphire_decoder_workgroups.restype = C.c_int
    L.sapphire_decoder_workgroups.argtypes = [C.c_void_p]
    L.sapphire_decoder_set_epoch_count.restype = C.c_int
    L.sapphire_decoder_set_epoch_count.argtypes = [C.c_void_p, C.c_uint32]
    L.sapphire_decoder_set_sampling.restype = C.c_int
    L.sapphire_decoder_set_sampling.argtypes = [C.c_void_p, C.c_float, C.c_void_p, C.c_int]
    L.sapphire_decoder_set_stop_tokens.restype = C.c_int
    L.sapphire_decoder_set_stop_tokens.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    L.sapphire_decoder_prefill.restype = C.c_int
    L.sapphire_decoder_prefill.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_float)]
    L.sapphire_decoder_generate_batch.restype = C.c_int
    L.sapphire_decoder_generate_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                                  C.c_void_p, C.POINTER(C.c_float)]


class Decoder:
    """batch = 1: the one-sequence decoder (sapphire_decoder_create); batch 2..16: the
    batched decoder (sapphire_decoder_create_batch), sequences decoded in lock step."""

    def __init__(self, m: "smodel.SyntheticModel", batch: int = 1, norm_bf16: bool = False, norm_dtype=None):
        """norm_bf16: hand the norm weights over as bf16 (their fp32 values' upper halves, exact
        when the model's norms are bf16-representable), as a safetensors checkpoint holds them.
        norm_dtype: overrides the norm_dtype field handed to the library (argument checks)."""
        self.lib = L = load()
        _protos(L)
        cfg = m.cfg
        self.cfg = cfg
        self._keep = []
        c = DecoderConfig(cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab,
                          cfg.max_ctx, cfg.sliding_window, cfg.global_mask, cfg.query_pre_attn_scalar,
                          cfg.rope_theta, cfg.rope_local_base, cfg.eps, cfg.wdtype, cfg.lm_dtype)
        w = DecoderWeights()
        for n in smodel.PROJ:
            arrs = [np.ascontiguousarray(m.weights[n][l]) for l in range(cfg.n_layers)]
            self._keep.append(arrs)
            setattr(w, n, (C.c_void_p * cfg.n_layers)(*[a.ctypes.data for a in arrs]))
        def norm_array(a):
            a = np.ascontiguousarray(a, np.float32)
            return np.ascontiguousarray(a.view(np.uint32) >> 16).astype(np.uint16) if norm_bf16 else a
        for n in ("norm_attn", "norm_attn_post", "norm_ffn", "norm_ffn_post", "q_norm", "k_norm"):
            arrs = [norm_array(m.norms[n][l]) for l in range(cfg.n_layers)]
            self._keep.append(arrs)
            setattr(w, n, (C.POINTER(C.c_float) * cfg.n_layers)(
                *[C.cast(a.ctypes.data, C.POINTER(C.c_float)) for a in arrs]))
        for n, a in (("embed_bf16", m.embed_bf16), ("norm_final", norm_array(m.norm_final)), ("lm_head", m.lm_head)):
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            setattr(w, n, a.ctypes.data)
        w.norm_dtype = (synth.BF16 if norm_bf16 else 0) if norm_dtype is None else int(norm_dtype)
        self.batch = batch
        if batch == 1:
            self.ptr = L.sapphire_decoder_create(C.byref(c), C.byref(w))
        else:
            self.ptr = L.sapphire_decoder_create_batch(C.byref(c), C.byref(w), int(batch))
        self._keep = None      # the library copied the weights
        if not self.ptr:
            raise RuntimeError("sapphire_decoder_create: " + L.sapphire_last_error().decode())

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: " + self.lib.sapphire_last_error().decode())

    def set_kv(self, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self._check(self.lib.sapphire_decoder_set_kv(self.ptr, k.ctypes.data, v.ctypes.data), "set_kv")

    def get_kv(self):
        c = self.cfg
        shape = (c.n_layers, c.n_kv_heads, c.max_ctx, c.head_dim)
        k, v = np.empty(shape, np.float32), np.empty(shape, np.float32)
        self._check(self.lib.sapphire_decoder_get_kv(self.ptr, k.ctypes.data, v.ctypes.data), "get_kv")
        return k, v

    def set_kv_seq(self, seq: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self._check(self.lib.sapphire_decoder_set_kv_seq(self.ptr, int(seq), k.ctypes.data, v.ctypes.data),
                    "set_kv_seq")

    def get_kv_seq(self, seq: int):
        c = self.cfg
        shape = (c.n_layers, c.n_kv_heads, c.max_ctx, c.head_dim)
        k, v = np.empty(shape, np.float32), np.empty(shape, np.float32)
        self._check(self.lib.sapphire_decoder_get_kv_seq(self.ptr, int(seq), k.ctypes.data, v.ctypes.data),
                    "get_kv_seq")
        return k, v

    @property
    def workgroups(self) -> int:
        """Workgroups of the persistent step; 0 = the multi-launch step."""
        return int(self.lib.sapphire_decoder_workgroups(self.ptr))

    def set_workgroups(self, groups: int) -> None:
        self._check(self.lib.sapphire_decoder_set_workgroups(self.ptr, int(groups)), "set_workgroups")

    def set_sampling(self, temperature: float, draws=None) -> None:
        """temperature > 0: later generate calls draw tokens as sample_temperature does, with
        draws[s * batch + b] for step s of a call and sequence b; <= 0: greedy."""
        d = np.ascontiguousarray(draws if draws is not None else [], np.float32)
        self._check(self.lib.sapphire_decoder_set_sampling(self.ptr, float(temperature),
                                                           d.ctypes.data if d.size else None, int(d.size)),
                    "set_sampling")

    def set_stop_tokens(self, ids) -> None:
        """Later generate calls stop a sequence at the first of these tokens (logged; every later
        step logs -1), as the reference's loop stops on 1 and 106 (inference.c:298-301)."""
        t = np.ascontiguousarray(list(ids), np.int32)
        self._check(self.lib.sapphire_decoder_set_stop_tokens(self.ptr, t.ctypes.data if t.size else None,
                                                               int(t.size)), "set_stop_tokens")

    def generate_batch(self, tokens, pos, steps: int, keep_logits: bool = False):
        """(tokens[steps, batch], logits[steps, batch, vocab] or None, device milliseconds)."""
        tk = np.ascontiguousarray(tokens, np.int32)
        ps = np.ascontiguousarray(pos, np.int32)
        assert tk.shape == (self.batch,) and ps.shape == (self.batch,)
        toks = np.empty((steps, self.batch), np.int32)
        logits = np.empty((steps, self.batch, self.cfg.vocab), np.float32) if keep_logits else None
        ms = C.c_float(0.0)
        self._check(self.lib.sapphire_decoder_generate_batch(self.ptr, tk.ctypes.data, ps.ctypes.data, int(steps),
                                                             toks.ctypes.data,
                                                             logits.ctypes.data if logits is not None else None,
                                                             C.byref(ms)), "generate_batch")
        return toks, logits, float(ms.value)

    def prefill(self, tokens, pos: int, seq: int = 0) -> float:
        """Runs tokens at positions pos.. of sequence `seq` through the layers (their K/V rows
        into the cache, no logits); returns the device milliseconds."""
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        ms = C.c_float(0.0)
        self._check(self.lib.sapphire_decoder_prefill(self.ptr, int(seq), t.ctypes.data, int(t.shape[0]), int(pos),
                                                      C.byref(ms)), "prefill")
        return float(ms.value)

    def generate(self, token: int, pos: int, steps: int, keep_logits: bool = False):
        """(tokens[steps], logits[steps, vocab] or None, device milliseconds)."""
        toks = np.empty(steps, np.int32)
        logits = np.empty((steps, self.cfg.vocab), np.float32) if keep_logits else None
        ms = C.c_float(0.0)
        self._check(self.lib.sapphire_decoder_generate(self.ptr, int(token), int(pos), int(steps), toks.ctypes.data,
                                                       logits.ctypes.data if logits is not None else None,
                                                       C.byref(ms)), "generate")
        return toks, logits, float(ms.value)

    def close(self):
        if getattr(self, "ptr", None):
            self.lib.sapphire_decoder_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        # at interpreter exit the process ends and the runtime reclaims everything: no HIP
        # calls from finalizers then
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


def bench_decode(steps: int = 64, seed: int = 20260101, prefill: int = 1024, reps: int = 3, m=None, kv=None,
                 groups=None):
    """Greedy decode of the Gemma-3-270M-shaped Q4_0 model (KV prefilled to `prefill` of
    2048 positions): tokens/s over `steps` steps, best of `reps` runs after a warm-up.
    `m` / `kv` reuse an already generated model and prefilled caches. `groups`: workgroups of
    the persistent step (0: the multi-launch step; None: the decoder's default)."""
    if m is None:
        m = smodel.synthetic_model(smodel.GEMMA3_270M, seed)
    cfg = m.cfg
    k, v = kv if kv is not None else m.kv_prefill(prefill)
    dec = Decoder(m)
    if groups is not None:
        dec.set_workgroups(groups)
    groups = dec.workgroups
    tok = smodel.start_token(cfg, seed)
    dec.set_kv(k, v)
    dec.generate(tok, prefill, steps)                 # graph capture + warm-up
    best = None
    for _ in range(reps):
        dec.set_kv(k, v)
        toks, _, ms = dec.generate(tok, prefill, steps)
        best = ms if best is None else min(best, ms)
    dec.close()
    layer_bytes = sum(int(m.weights[n][0].nbytes) for n in smodel.PROJ) * cfg.n_layers
    from . import synth
    lm_names = {synth.Q4_0: "Q4_0", synth.Q8_0: "Q8_0", synth.BF16: "BF16 (the embedding table, tied)"}
    w_tok = layer_bytes + int(m.lm_head.nbytes)
    kv_tok = kv_read_bytes(cfg, prefill, steps)
    ms_tok = best / steps
    return {
        "model": f"Gemma-3-270M-shaped, Q4_0 weights (random init), 18 layers, hidden 640, vocab 262144, "
                 f"LM head {lm_names[cfg.lm_dtype]}",
        "steps": steps, "kv_prefill": prefill, "ms_total": round(best, 3), "ms_per_token": round(ms_tok, 4),
        "tok_per_s": round(steps / (best * 1e-3), 1), "first_tokens": [int(t) for t in toks[:8]],
        "weight_bytes_per_token": w_tok, "kv_bytes_per_token": kv_tok,
        "GB_per_s": round((w_tok + kv_tok) / (ms_tok * 1e-3) / 1e9, 1),
        "frac_hbm_peak": round((w_tok + kv_tok) / (ms_tok * 1e-3) / HBM_PEAK, 4),
        "step_form": f"persistent, {groups} workgroups" if groups else "multi-launch graph",
    }


HBM_PEAK = 8.0e12   # MI355X HBM3E, bytes/s


def kv_read_bytes(cfg, prefill: int, steps: int) -> int:
    """K and V bytes one sequence's steps read, averaged per step: step s at position
    prefill + s attends to min(pos + 1, window) rows in a local layer and pos + 1 in a global
    one (attention.c:122-127), each row n_kv_heads * head_dim fp32 for K and for V."""
    win = cfg.sliding_window
    total = 0
    for s in range(steps):
        p = prefill + s
        total += sum((p + 1) if l in cfg.global_layers else min(p + 1, win) for l in range(cfg.n_layers))
    return int(round(total / steps)) * cfg.n_kv_heads * cfg.head_dim * 4 * 2


def bench_decode_batch(steps: int = 32, batch: int = 16, seed: int = 20260101, prefill: int = 1024, reps: int = 2,
                       cfg=None, m=None, kv=None):
    """Batched greedy decode of the Gemma-3-1B-shaped Q4_0 model: `batch` sequences, each with
    its own KV cache prefilled to `prefill` of 2048 positions (the same N(0,1) contents in every
    sequence's cache) and its own seeded start token. tokens/s = batch * steps / time, best of
    `reps` runs after a warm-up (the graph capture)."""
    if m is None:
        m = smodel.synthetic_model(cfg or smodel.GEMMA3_1B, seed)
    cfg = m.cfg
    k, v = kv if kv is not None else m.kv_prefill(prefill)
    dec = Decoder(m, batch=batch)
    for b in range(batch):
        dec.set_kv_seq(b, k, v)
    rng = np.random.default_rng(seed)
    toks0 = rng.integers(0, cfg.vocab, size=batch).astype(np.int32)
    pos = np.full(batch, prefill, np.int32)
    dec.generate_batch(toks0, pos, steps)            # graph capture + warm-up
    best = None
    for _ in range(reps):
        toks, _, ms = dec.generate_batch(toks0, pos, steps)
        best = ms if best is None else min(best, ms)
    dec.close()
    from . import synth
    nq, nk = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim

    def qb(m_, k_, dt):
        return m_ * k_ * 2 if dt == synth.BF16 else m_ * (k_ // 32) * synth.BLOCK_BYTES[dt]
    layer_w = (qb(nq + 2 * nk, cfg.hidden, cfg.wdtype) + qb(cfg.hidden, nq, cfg.wdtype) +
               qb(2 * cfg.ffn, cfg.hidden, cfg.wdtype) + qb(cfg.hidden, cfg.ffn, cfg.wdtype))
    w_step = layer_w * cfg.n_layers + qb(cfg.vocab, cfg.hidden, cfg.lm_dtype)
    kv_step = batch * kv_read_bytes(cfg, prefill, steps)
    ms_step = best / steps
    return {
        "model": "Gemma-3-1B-shaped, Q4_0 weights (random init), 26 layers, hidden 1152, FFN 6912, vocab 262144"
                 + (", LM head = the BF16 embedding table (tied)" if cfg.lm_dtype == synth.BF16 else ""),
        "batch": batch, "steps": steps, "kv_prefill": prefill, "ms_total": round(best, 3),
        "ms_per_step": round(ms_step, 4), "tok_per_s": round(batch * steps / (best * 1e-3), 1),
        "weight_bytes_per_step": w_step, "kv_bytes_per_step": kv_step,
        "GB_per_s": round((w_step + kv_step) / (ms_step * 1e-3) / 1e9, 1),
        "frac_hbm_peak": round((w_step + kv_step) / (ms_step * 1e-3) / HBM_PEAK, 4),
        "first_tokens": [int(t) for t in toks[0]],
    }
