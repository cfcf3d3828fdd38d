"""Quantized checkpoints: F32 / BF16 safetensors in, Q4_0 / Q8_0 blocks out.

The reference loads only F32 / BF16 tensors from safetensors
(src/loader/safetensors_reader.c:406-449) and has no quantizer, so its Q4_0 / Q8_0 block
arrays (include/kernels.h:29-38) must come from somewhere else. This module is that
producer for a checkpoint: the seven projections of every layer (the tensor names of
src/loader/gemma3_map.c:5-285) are quantized on the GPU (sapphire_quantize_dev) and written
back as raw block bytes; every other tensor is copied unchanged.

File format: a safetensors file. A quantized tensor is stored as U8 with shape
[M, ceil(K/32) * B_blk] (B_blk 20 for Q4_0, 36 for Q8_0): the reference's block array,
rows contiguous, byte for byte. The file metadata holds, for each quantized tensor,
``"sapphire.q.<name>": "<Q4_0|Q8_0>,<M>,<K>"`` and ``"sapphire.format": "1"``.
"""
from __future__ import annotations

import numpy as np

from . import synth

FORMAT = "1"
# the projections of a Gemma-3 layer (gemma3_map.c): q/k/v/o and gate/up/down
PROJECTIONS = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
               "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")
QNAMES = {synth.Q4_0: "Q4_0", synth.Q8_0: "Q8_0"}
QCODES = {v: k for k, v in QNAMES.items()}


def is_projection(name: str) -> bool:
    return name.startswith("model.layers.") and name.endswith(PROJECTIONS)


def quantize_rows(dtype: int, w: np.ndarray, src_dtype: int) -> np.ndarray:
    """[M, K] float32 (F32) or uint16 bf16 bits (BF16) -> [M, ceil(K/32)] blocks, on the GPU."""
    from .device import DeviceArray, quantize
    m, k = w.shape
    src = DeviceArray.from_numpy(np.ascontiguousarray(w))
    out = DeviceArray(m * ((k + 31) // 32) * synth.BLOCK_BYTES[dtype])
    quantize(dtype, src_dtype, src, m, k, out)
    raw = out.numpy()
    src.free()
    out.free()
    return np.frombuffer(raw.tobytes(), synth.block_dtype(dtype)).reshape(m, (k + 31) // 32)


def blocks_to_bytes(blocks: np.ndarray) -> np.ndarray:
    """[M, nb] blocks -> [M, nb * B_blk] uint8 (the stored form)."""
    m = blocks.shape[0]
    return np.frombuffer(np.ascontiguousarray(blocks).tobytes(), np.uint8).reshape(m, -1)


def bytes_to_blocks(raw: np.ndarray, dtype: int, m: int, k: int) -> np.ndarray:
    nb = (k + 31) // 32
    if raw.shape != (m, nb * synth.BLOCK_BYTES[dtype]):
        raise ValueError(f"stored shape {raw.shape} does not hold {m} x {k} {QNAMES[dtype]} blocks")
    return np.frombuffer(np.ascontiguousarray(raw).tobytes(), synth.block_dtype(dtype)).reshape(m, nb)


def save(path: str, tensors: dict, quantized: dict, metadata: dict | None = None) -> None:
    """Writes plain tensors (numpy arrays or torch tensors) and quantized ones
    ({name: (dtype, blocks [M, nb], K)}) to one safetensors file."""
    import torch
    from safetensors.torch import save_file
    out, meta = {}, {"sapphire.format": FORMAT}
    meta.update(metadata or {})
    for name, t in tensors.items():
        out[name] = t if isinstance(t, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(t))
    for name, (dtype, blocks, k) in quantized.items():
        out[name] = torch.from_numpy(blocks_to_bytes(blocks).copy())
        meta[f"sapphire.q.{name}"] = f"{QNAMES[dtype]},{blocks.shape[0]},{k}"
    save_file(out, path, metadata=meta)


def load(path: str):
    """-> (tensors {name: torch.Tensor}, quantized {name: (dtype, blocks [M, nb], K)})."""
    from safetensors import safe_open
    tensors, quantized = {}, {}
    with safe_open(path, "pt") as f:
        meta = f.metadata() or {}
        for name in f.keys():
            q = meta.get(f"sapphire.q.{name}")
            t = f.get_tensor(name)
            if q is None:
                tensors[name] = t
                continue
            qn, m, k = q.split(",")
            dtype, m, k = QCODES[qn], int(m), int(k)
            quantized[name] = (dtype, bytes_to_blocks(t.numpy(), dtype, m, k), k)
    return tensors, quantized


def quantize_checkpoint(src_path: str, dst_path: str, dtype: int = synth.Q4_0, names=None) -> dict:
    """Quantizes the projections of a F32 / BF16 safetensors checkpoint (or the 2-D tensors
    listed in `names`) on the GPU and writes the result to dst_path. Returns
    {name: (M, K)} of the quantized tensors."""
    import torch
    from safetensors import safe_open
    if dtype not in QNAMES:
        raise ValueError("dtype must be Q4_0 or Q8_0")
    tensors, quantized, done = {}, {}, {}
    with safe_open(src_path, "pt") as f:
        meta = dict(f.metadata() or {})
        for name in f.keys():
            t = f.get_tensor(name)
            want = (name in names) if names is not None else is_projection(name)
            if not want:
                tensors[name] = t
                continue
            if t.ndim != 2 or t.dtype not in (torch.float32, torch.bfloat16):
                raise ValueError(f"{name}: only 2-D F32 / BF16 tensors are quantized (got {t.dtype}, {t.ndim}-D)")
            if t.dtype == torch.bfloat16:
                w, src_dtype = t.contiguous().view(torch.int16).numpy().view(np.uint16), synth.BF16
            else:
                w, src_dtype = t.contiguous().numpy(), synth.F32
            m, k = w.shape
            quantized[name] = (dtype, quantize_rows(dtype, w, src_dtype), k)
            done[name] = (m, k)
    meta.pop("sapphire.format", None)
    save(dst_path, tensors, quantized, {k_: v for k_, v in meta.items() if not k_.startswith("sapphire.q.")})
    return done
