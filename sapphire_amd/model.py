"""Gemma-3-shaped synthetic decode models (random-init weights of the architecture).

The layer composition follows the reference engine: src/inference/inference.c:616-651,
src/transformer/attention.c:311-375, src/transformer/transformer.c:96-283,393-408.
Weights are drawn by :mod:`sapphire_amd.synth`; norm weights are N(1, 0.1) and are
applied as ``(1 + w)`` by rmsnorm_delta (src/transformer/normalization.c:104-117).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import synth


@dataclass(frozen=True)
class DecodeConfig:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_ctx: int
    sliding_window: int = 512
    global_layers: tuple = ()
    query_pre_attn_scalar: float = 256.0
    rope_theta: float = 1e6          # global layers (inference.c:477-483)
    rope_local_base: float = 1e4     # local layers (inference.c:485-491)
    wdtype: int = synth.Q4_0
    lm_dtype: int = synth.Q4_0
    eps: float = 1e-6

    @property
    def global_mask(self) -> int:
        m = 0
        for l in self.global_layers:
            m |= 1 << l
        return m

    def is_global(self, layer: int) -> bool:
        if self.global_layers:
            return layer in self.global_layers
        return (layer + 1) % 6 == 0  # attention.c:110

    @property
    def nq(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def nk(self) -> int:
        return self.n_kv_heads * self.head_dim


# Gemma-3-270M shape: 18 layers, hidden 640, 4 q-heads / 1 kv-head, head_dim 256,
# GeGLU FFN 2048, vocab 262144; every sixth layer global.
GEMMA3_270M = DecodeConfig(n_layers=18, hidden=640, n_heads=4, n_kv_heads=1, head_dim=256,
                           ffn=2048, vocab=262144, max_ctx=2048, sliding_window=512,
                           global_layers=(5, 11, 17))

# Gemma-3-1B shape: 26 layers, hidden 1152, 4 q-heads / 1 kv-head, head_dim 256,
# FFN 6912, vocab 262144.
GEMMA3_1B = DecodeConfig(n_layers=26, hidden=1152, n_heads=4, n_kv_heads=1, head_dim=256,
                         ffn=6912, vocab=262144, max_ctx=2048, sliding_window=512,
                         global_layers=(5, 11, 17, 23))

# A small model with the same structure, for CPU-speed parity tests.
TINY = DecodeConfig(n_layers=3, hidden=128, n_heads=4, n_kv_heads=1, head_dim=64,
                    ffn=256, vocab=4096, max_ctx=96, sliding_window=24, global_layers=(2,))


PROJ = ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")
NORMS = ("norm_attn", "norm_attn_post", "norm_ffn", "norm_ffn_post")


def proj_shape(cfg: DecodeConfig, name: str) -> tuple[int, int]:
    """(rows M, cols K) of each projection, y = W x with W row-major [M, K]."""
    return {
        "wq": (cfg.nq, cfg.hidden), "wk": (cfg.nk, cfg.hidden), "wv": (cfg.nk, cfg.hidden),
        "wo": (cfg.hidden, cfg.nq), "wgate": (cfg.ffn, cfg.hidden), "wup": (cfg.ffn, cfg.hidden),
        "wdown": (cfg.hidden, cfg.ffn),
    }[name]


@dataclass
class SyntheticModel:
    cfg: DecodeConfig
    seed: int
    weights: dict = field(default_factory=dict)   # name -> [n_layers, M, nb] blocks
    norms: dict = field(default_factory=dict)     # name -> [n_layers, len] f32
    embed_bf16: np.ndarray = None                 # [vocab, hidden] uint16
    norm_final: np.ndarray = None                 # [hidden] f32
    lm_head: np.ndarray = None                    # [vocab, nb] blocks, or embed_bf16 (BF16, tied)

    def kv_prefill(self, n_pos: int, seed_offset: int = 0):
        """K/V caches [n_layers, n_kv, max_ctx, hd] with N(0,1) at positions < n_pos."""
        c = self.cfg
        shape = (c.n_layers, c.n_kv_heads, c.max_ctx, c.head_dim)
        k = np.zeros(shape, np.float32)
        v = np.zeros(shape, np.float32)
        k[:, :, :n_pos, :] = synth.normal_f32((c.n_layers, c.n_kv_heads, n_pos, c.head_dim),
                                              self.seed, 900 + seed_offset)
        v[:, :, :n_pos, :] = synth.normal_f32((c.n_layers, c.n_kv_heads, n_pos, c.head_dim),
                                              self.seed, 901 + seed_offset)
        return k, v


def synthetic_model(cfg: DecodeConfig, seed: int) -> SyntheticModel:
    m = SyntheticModel(cfg=cfg, seed=seed)
    tid = 1
    for name in PROJ:
        rows, cols = proj_shape(cfg, name)
        layers = [synth.quant_matrix(cfg.wdtype, rows, cols, seed, tid + 100 * l) for l in range(cfg.n_layers)]
        m.weights[name] = np.stack(layers)
        tid += 1
    for name in NORMS:
        m.norms[name] = synth.normal_f32((cfg.n_layers, cfg.hidden), seed, tid, 1.0, 0.1)
        tid += 1
    m.norms["q_norm"] = synth.normal_f32((cfg.n_layers, cfg.head_dim), seed, tid, 1.0, 0.1)
    m.norms["k_norm"] = synth.normal_f32((cfg.n_layers, cfg.head_dim), seed, tid + 1, 1.0, 0.1)
    m.embed_bf16 = synth.bf16_normal((cfg.vocab, cfg.hidden), seed, tid + 2)
    m.norm_final = synth.normal_f32(cfg.hidden, seed, tid + 3, 1.0, 0.1)
    if cfg.lm_dtype == synth.BF16:
        m.lm_head = m.embed_bf16          # weight tying: lm_head projects through the embedding
    else:
        m.lm_head = synth.quant_matrix(cfg.lm_dtype, cfg.vocab, cfg.hidden, seed, tid + 4)
    return m


def start_token(cfg: DecodeConfig, seed: int) -> int:
    return int(synth.rng(seed, 999).integers(0, cfg.vocab))


def model_digest(m: SyntheticModel, k_cache: np.ndarray = None, v_cache: np.ndarray = None) -> str:
    """sha256 over every input array of a synthetic model (and optional KV caches), to
    detect a change of the generator behind a seed."""
    import hashlib
    h = hashlib.sha256()
    for name in PROJ:
        h.update(np.ascontiguousarray(m.weights[name]).tobytes())
    for name in sorted(m.norms):
        h.update(np.ascontiguousarray(m.norms[name]).tobytes())
    for a in (m.embed_bf16, m.norm_final, m.lm_head, k_cache, v_cache):
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()
