"""Seeded synthetic inputs for the quantized decode path.

Block formats are the reference's own structs (include/kernels.h:29-38):

* Q4_0: ``{float scale; uint8_t q[16];}`` -- 20 bytes per 32 weights, element
  ``2j = q[j] & 0xF``, element ``2j+1 = q[j] >> 4``, value ``(nib - 8) * scale``
  (src/kernels/q4_0_avx.c:61-66).
* Q8_0: ``{float scale; int8_t q[32];}`` -- 36 bytes per 32 weights, value
  ``q * scale`` (src/kernels/q8_0_avx.c:45-59).

Value distributions: per-block scale ``|N(0, 0.01)|`` in fp32; Q8_0 quants uniform in
[-127, 127]; Q4_0 nibbles uniform in 0..15; activations N(0, 1) fp32. Every tensor
draws from its own numpy PCG64 stream seeded with ``(seed, tensor_id)``.
"""
from __future__ import annotations

import numpy as np

Q4_0 = 3
Q8_0 = 4
F32 = 0
BF16 = 1

Q4_BLOCK = np.dtype([("scale", "<f4"), ("q", "u1", (16,))])
Q8_BLOCK = np.dtype([("scale", "<f4"), ("q", "i1", (32,))])
assert Q4_BLOCK.itemsize == 20 and Q8_BLOCK.itemsize == 36

BLOCK_BYTES = {Q4_0: 20, Q8_0: 36}
DTYPE_NAME = {Q4_0: "Q4_0", Q8_0: "Q8_0"}


def block_dtype(dtype: int) -> np.dtype:
    return Q4_BLOCK if dtype == Q4_0 else Q8_BLOCK


def row_bytes(dtype: int, k: int) -> int:
    """Row stride in bytes: ceil(K/32) blocks (src/kernels/pool.c:285,297,301)."""
    return ((k + 31) // 32) * BLOCK_BYTES[dtype]


def rng(seed: int, tensor_id: int) -> np.random.Generator:
    return np.random.default_rng([int(seed) & 0xFFFFFFFF, int(tensor_id) & 0xFFFFFFFF])


def quant_matrix(dtype: int, m: int, k: int, seed: int, tensor_id: int = 0) -> np.ndarray:
    """[m, ceil(k/32)] structured array of blocks, rows contiguous (AoS)."""
    g = rng(seed, tensor_id)
    nb = (k + 31) // 32
    out = np.empty((m, nb), dtype=block_dtype(dtype))
    out["scale"] = np.abs(g.normal(0.0, 0.01, size=(m, nb))).astype(np.float32)
    if dtype == Q4_0:
        # uniform bytes = two independent uniform nibbles per byte
        out["q"] = g.integers(0, 256, size=(m, nb, 16), dtype=np.uint8)
    else:
        out["q"] = g.integers(-127, 128, size=(m, nb, 32), dtype=np.int8)
    return out


def normal_f32(shape, seed: int, tensor_id: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    g = rng(seed, tensor_id)
    return (mean + std * g.standard_normal(size=shape)).astype(np.float32)


def bf16_normal(shape, seed: int, tensor_id: int) -> np.ndarray:
    """N(0,1) values truncated to bf16 bit patterns (uint16)."""
    f = normal_f32(shape, seed, tensor_id)
    return (f.view(np.uint32) >> 16).astype(np.uint16)


def unpack_ints(dtype: int, blocks: np.ndarray) -> np.ndarray:
    """Closed-form integer values of every weight, shape [..., nb*32] int8."""
    if dtype == Q8_0:
        q = blocks["q"].astype(np.int8)
        return q.reshape(q.shape[:-2] + (q.shape[-2] * 32,))
    q = blocks["q"]
    lo = (q & 0x0F).astype(np.int8) - 8
    hi = (q >> 4).astype(np.int8) - 8
    inter = np.stack([lo, hi], axis=-1)  # element 2j = lo_j, 2j+1 = hi_j
    return inter.reshape(q.shape[:-2] + (q.shape[-2] * 32,))


def as_bytes(blocks: np.ndarray) -> np.ndarray:
    """Raw little-endian bytes of a block array (the reference's memory image)."""
    return np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
