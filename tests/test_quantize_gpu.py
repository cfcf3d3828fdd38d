"""The Q4_0 / Q8_0 producer on the GPU (sapphire_quantize_dev, kernel_quantize) against the
oracle's quantizer, bit for bit (integer codes and fp32 scales), and the blocks it makes
fed to the GPU GEMV."""
import ctypes as C

import numpy as np
import pytest

from sapphire_amd import synth
from tests.conftest import close

pytestmark = pytest.mark.gpu

Q4, Q8, F32, BF16 = synth.Q4_0, synth.Q8_0, synth.F32, synth.BF16

SHAPES = [
    (262144, 640),  # the LM head of Gemma-3-270M
    (2048, 640),
    (640, 2048),
    (7, 96),
    (3, 100),       # ragged K: the last block of a row padded with zeros
    (5, 33),
    (1, 1),
    (64, 6912),
    (9, 1030),      # K % 4 == 2: element loads
]


def source(src_dtype, m, k, seed):
    f = synth.normal_f32((m, k), seed, m + k)
    # blocks of very different magnitudes, exact zeros and ties of |x| of both signs
    f *= np.exp2(np.random.default_rng(seed).integers(-30, 30, (m, 1))).astype(np.float32)
    if m > 2 and k >= 32:
        f[1, :32] = 0.0
        f[2, 3], f[2, 7] = -5.0, 5.0
        f[2, :32] = np.clip(f[2, :32], -4, 4)
        f[2, 3], f[2, 7] = -5.0, 5.0
    if src_dtype == F32:
        return f
    return (f.view(np.uint32) >> 16).astype(np.uint16)


def run_quantize(dtype, src_dtype, src):
    from sapphire_amd.device import DeviceArray, quantize
    m, k = src.shape
    ds = DeviceArray.from_numpy(src)
    out = DeviceArray(m * ((k + 31) // 32) * synth.BLOCK_BYTES[dtype])
    quantize(dtype, src_dtype, ds, m, k, out)
    raw = out.numpy()
    return np.frombuffer(raw.tobytes(), synth.block_dtype(dtype)).reshape(m, (k + 31) // 32)


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("src_dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_quantize_matches_oracle(hip, oracle, dtype, src_dtype, shape):
    m, k = shape
    print(f"quantize dtype={dtype} src={src_dtype} shape={shape}", flush=True)
    src = source(src_dtype, m, k, 3)
    ref = oracle.quantize(dtype, src_dtype, src)
    got = run_quantize(dtype, src_dtype, src)
    assert got.tobytes() == ref.tobytes()


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
def test_quantize_special_blocks(hip, oracle, dtype):
    """Zero blocks (scale -0 for Q4_0), subnormal scales (1/d overflows), the largest
    finite values and exactly representable blocks."""
    print(f"quantize special dtype={dtype}", flush=True)
    x = np.zeros((6, 64), np.float32)
    x[1, :3] = [1e-39, -5e-40, 0.0]
    x[2, :4] = [3.0e38, -3.4e38, 1.0, -1.0]
    x[3] = np.arange(64) - 32
    x[4, 10] = -0.0
    x[5] = np.float32(2.0 ** -126) * (np.arange(64) % 7 - 3)
    ref = oracle.quantize(dtype, F32, x)
    got = run_quantize(dtype, F32, x)
    assert got.tobytes() == ref.tobytes()


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
def test_quantized_blocks_through_gemv(hip, oracle, dtype):
    """Quantize on the GPU, then the GPU GEMV over the produced blocks against the oracle
    GEMV over the oracle's blocks."""
    from sapphire_amd.device import DeviceArray, QMatrix, gemv
    m, k = 4096, 640
    print(f"quantize->gemv dtype={dtype}", flush=True)
    w = synth.bf16_normal((m, k), 8, 1)
    blocks = run_quantize(dtype, BF16, w)
    x = synth.normal_f32(k, 8, 2)
    ref = oracle.gemv(dtype, oracle.quantize(dtype, BF16, w), x)
    qm = QMatrix(dtype, blocks)
    dx, dy = DeviceArray.from_numpy(x), DeviceArray.empty(m)
    gemv(qm, dx, dy)
    ok, err = close(dy.numpy(), ref)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
@pytest.mark.parametrize("src_dtype", [F32, BF16], ids=["f32", "bf16"])
def test_kernel_quantize_host_api(hip, oracle, dtype, src_dtype):
    """kernel_quantize on host pointers, with and without a context, and its argument checks."""
    m, k = 300, 1152
    print(f"kernel_quantize dtype={dtype} src={src_dtype}", flush=True)
    src = source(src_dtype, m, k, 9)
    ref = oracle.quantize(dtype, src_dtype, src)
    shp = (C.c_int * 2)(m, k)
    A = hip.tensor_create_view(src_dtype, 2, shp, src.ctypes.data)
    ctx = hip.kernel_ctx_create(0, 16)
    assert ctx and hip.kernel_ctx_init(ctx) == 0
    try:
        for c in (ctx, None):
            out = np.zeros((m, (k + 31) // 32), synth.block_dtype(dtype))
            assert hip.kernel_quantize(c, out.ctypes.data, dtype, A) == 0
            assert out.tobytes() == ref.tobytes()
        out = np.zeros((m, (k + 31) // 32), synth.block_dtype(dtype))
        assert hip.kernel_quantize(ctx, out.ctypes.data, F32, A) == -1      # not a block dtype
        assert hip.kernel_quantize(ctx, None, dtype, A) == -1
        assert hip.kernel_quantize(ctx, out.ctypes.data, dtype, None) == -1
    finally:
        hip.tensor_release(A)
        hip.kernel_ctx_destroy(ctx)


@pytest.mark.parametrize("dtype", [Q4, Q8], ids=["q4_0", "q8_0"])
def test_quantize_checkpoint(hip, oracle, dtype, tmp_path):
    """A BF16 safetensors checkpoint with Gemma-3 tensor names (two layers of the TINY
    shape): the projections come back as the oracle's blocks, everything else unchanged."""
    import torch
    from safetensors.torch import save_file
    from sapphire_amd import checkpoint
    from sapphire_amd import model as smodel
    print(f"quantize checkpoint dtype={dtype}", flush=True)
    cfg = smodel.TINY
    src = {}
    tid = 0
    for l in range(2):
        for p in checkpoint.PROJECTIONS:
            short = {"q_proj": "wq", "k_proj": "wk", "v_proj": "wv", "o_proj": "wo", "gate_proj": "wgate",
                     "up_proj": "wup", "down_proj": "wdown"}[p.split(".")[1]]
            m, k = smodel.proj_shape(cfg, short)
            tid += 1
            src[f"model.layers.{l}.{p}"] = torch.from_numpy(
                synth.bf16_normal((m, k), 17, tid).view(np.int16)).view(torch.bfloat16)
        src[f"model.layers.{l}.input_layernorm.weight"] = torch.from_numpy(synth.normal_f32(cfg.hidden, 17, 90 + l))
    src["model.embed_tokens.weight"] = torch.from_numpy(
        synth.bf16_normal((cfg.vocab, cfg.hidden), 17, 99).view(np.int16)).view(torch.bfloat16)
    sp, dp = str(tmp_path / "src.safetensors"), str(tmp_path / "q.safetensors")
    save_file(src, sp)
    done = checkpoint.quantize_checkpoint(sp, dp, dtype)
    assert len(done) == 14
    tensors, quantized = checkpoint.load(dp)
    assert set(quantized) == set(done) and set(tensors) == set(src) - set(done)
    for name, (dt, blocks, k) in quantized.items():
        w = src[name].view(torch.int16).numpy().view(np.uint16)
        assert dt == dtype and k == w.shape[1]
        assert blocks.tobytes() == oracle.quantize(dtype, BF16, w).tobytes(), name
    for name, t in tensors.items():
        assert torch.equal(t.view(torch.int16) if t.dtype == torch.bfloat16 else t,
                           src[name].view(torch.int16) if src[name].dtype == torch.bfloat16 else src[name])
