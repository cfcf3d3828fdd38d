"""numpy-facing helpers over the device-pointer API (sapphire_hip.h)."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np

from . import load, synth


def lib():
    return load()


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        err = lib().sapphire_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {err}")


class DeviceArray:
    """Owning device buffer with shape/dtype bookkeeping for numpy round trips."""

    def __init__(self, nbytes: int, shape=None, dtype=np.uint8):
        self.nbytes = int(nbytes)
        self.ptr = lib().sapphire_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise MemoryError(lib().sapphire_last_error().decode())
        self.shape = shape if shape is not None else (self.nbytes,)
        self.dtype = np.dtype(dtype)

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes, a.shape, a.dtype)
        check(lib().sapphire_memcpy_h2d(d.ptr, a.ctypes.data, a.nbytes), "h2d")
        return d

    @classmethod
    def empty(cls, shape, dtype=np.float32) -> "DeviceArray":
        shape = tuple(np.atleast_1d(shape))
        return cls(int(np.prod(shape)) * np.dtype(dtype).itemsize, shape, dtype)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().sapphire_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().sapphire_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes), "h2d")

    def zero(self) -> None:
        check(lib().sapphire_memset(self.ptr, 0, self.nbytes), "memset")

    def free(self) -> None:
        if self.ptr:
            lib().sapphire_free(self.ptr)
            self.ptr = None

    def __del__(self):
        # at interpreter exit the process ends and the runtime reclaims everything: no HIP
        # calls from finalizers then
        if sys.is_finalizing():
            return
        try:
            self.free()
        except Exception:
            pass


class QMatrix:
    """A Q4_0/Q8_0 weight matrix resident on the device in one layout (AOS, PACKED or
    TILED; see sapphire_hip.h), optionally keeping the AOS copy too."""

    def __init__(self, dtype: int, blocks: np.ndarray, packed: bool = True, keep_aos: bool = False,
                 layout: int = None):
        self.dtype = dtype
        self.M, nb = blocks.shape
        self.K = nb * 32
        if layout is None:
            layout = 1 if packed else 0
        self.layout = layout
        aos = DeviceArray.from_numpy(synth.as_bytes(blocks))
        self.aos = aos if keep_aos or layout == 0 else None
        self.conv = None
        if layout != 0:
            L = lib()
            nbytes = L.sapphire_q_layout_bytes(dtype, layout, self.M, self.K)
            if nbytes == 0:
                raise ValueError(f"layout {layout} cannot hold a {self.M}x{self.K} matrix")
            self.conv = DeviceArray(nbytes)
            check(L.sapphire_q_convert_dev(dtype, aos.ptr, self.M, self.K, layout, self.conv.ptr, None), "convert")
            check(L.sapphire_synchronize(), "sync")
            if self.aos is None:
                aos.free()

    @property
    def packed(self):
        return self.conv if self.layout == 1 else None

    def ptr(self, layout: int = None) -> int:
        layout = self.layout if layout is None else layout
        if layout == 0:
            return self.aos.ptr
        assert layout == self.layout, f"matrix is held in layout {self.layout}, not {layout}"
        return self.conv.ptr

    @property
    def algorithmic_bytes(self) -> int:
        """M*ceil(K/32)*B_blk + 4K + 4M: weights + activation + output."""
        return self.M * (self.K // 32) * synth.BLOCK_BYTES[self.dtype] + 4 * self.K + 4 * self.M


def gemv(qm: QMatrix, x: DeviceArray, y: DeviceArray, layout: int = 1, stream=None) -> None:
    check(lib().sapphire_gemv_q_dev(qm.dtype, layout, qm.ptr(layout), qm.M, qm.K, x.ptr, y.ptr, stream), "gemv")


def quantize(dtype: int, src_dtype: int, src: DeviceArray, M: int, K: int, blocks: DeviceArray, stream=None) -> None:
    """F32 / BF16 rows [M][K] on the device -> M * ceil(K/32) Q4_0 / Q8_0 blocks (AOS)."""
    check(lib().sapphire_quantize_dev(dtype, src_dtype, src.ptr, M, K, blocks.ptr, stream), "quantize")


def gemv_f(dtype: int, w: DeviceArray, M: int, K: int, x: DeviceArray, y: DeviceArray, offset: int = 0,
           stream=None) -> None:
    """y = W . x for a row-major F32 / BF16 matrix held at w.ptr + offset bytes."""
    check(lib().sapphire_gemv_f_dev(dtype, w.ptr + offset, M, K, x.ptr, y.ptr, stream), "gemv_f")


class Timer:
    """HIP-event timing on a given stream (None = null stream)."""

    def __init__(self, stream=None):
        L = lib()
        self.stream = stream
        self.a = L.sapphire_event_create()
        self.b = L.sapphire_event_create()

    def start(self):
        check(lib().sapphire_event_record(self.a, self.stream), "event")

    def stop(self) -> float:
        L = lib()
        check(L.sapphire_event_record(self.b, self.stream), "event")
        check(L.sapphire_event_synchronize(self.b), "event sync")
        return float(L.sapphire_event_elapsed_ms(self.a, self.b))

    def __del__(self):
        # at interpreter exit the process ends and the runtime reclaims everything: no HIP
        # calls from finalizers then
        if sys.is_finalizing():
            return
        try:
            L = lib()
            L.sapphire_event_destroy(self.a)
            L.sapphire_event_destroy(self.b)
        except Exception:
            pass
