"""ctypes prototypes of libsapphire_hip.so (include/kernels.h, tensor.h, sapphire_hip.h)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_LIB = None

vp, i32, f32, sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t


class GemmInput(C.Structure):
    """sapphire_gemm_input_t (include/sapphire_hip.h)."""
    _fields_ = [("x", C.c_void_p), ("ldx", C.c_int), ("parts", C.c_void_p), ("nparts", C.c_int), ("ldp", C.c_int),
                ("part_stride", C.c_size_t), ("w_delta", C.c_void_p), ("resid_out", C.c_void_p), ("ldr", C.c_int),
                ("w_norm", C.c_void_p), ("eps", C.c_float), ("x_blocked", C.c_int)]


class GemmOutput(C.Structure):
    """sapphire_gemm_output_t (include/sapphire_hip.h)."""
    _fields_ = [("y", C.c_void_p), ("ldy", C.c_int), ("parts", C.c_void_p), ("geglu", C.c_int), ("y_blocked", C.c_int)]


def _proto(lib, name, res, args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = args


def load_library(path: str):
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m sapphire_amd.build` "
            "(there is no CPU fallback for the HIP path)")
    # RTLD_LOCAL: the library exports the reference's own C API names, so it must not
    # interpose on another library of that API loaded into the same process.
    lib = C.CDLL(path, mode=C.RTLD_LOCAL)
    P = lambda n, r, a: _proto(lib, n, r, a)  # noqa: E731
    # sapphire_hip.h
    P("sapphire_last_error", C.c_char_p, [])
    P("sapphire_version", C.c_char_p, [])
    P("sapphire_device_count", i32, [])
    P("sapphire_set_device", i32, [i32])
    P("sapphire_malloc", vp, [sz])
    P("sapphire_free", i32, [vp])
    P("sapphire_memcpy_h2d", i32, [vp, vp, sz])
    P("sapphire_memcpy_d2h", i32, [vp, vp, sz])
    P("sapphire_memcpy_d2d", i32, [vp, vp, sz, vp])
    P("sapphire_memset", i32, [vp, i32, sz])
    P("sapphire_synchronize", i32, [])
    P("sapphire_stream_create", vp, [])
    P("sapphire_stream_destroy", i32, [vp])
    P("sapphire_stream_synchronize", i32, [vp])
    P("sapphire_event_create", vp, [])
    P("sapphire_event_destroy", i32, [vp])
    P("sapphire_event_record", i32, [vp, vp])
    P("sapphire_event_synchronize", i32, [vp])
    P("sapphire_event_elapsed_ms", f32, [vp, vp])
    P("sapphire_q_aos_bytes", sz, [i32, i32, i32])
    P("sapphire_q_packed_bytes", sz, [i32, i32, i32])
    P("sapphire_q_scales_offset", sz, [i32, i32, i32])
    P("sapphire_q_repack_dev", i32, [i32, vp, i32, i32, vp, vp])
    P("sapphire_q_layout_bytes", sz, [i32, i32, i32, i32])
    P("sapphire_q_convert_dev", i32, [i32, vp, i32, i32, i32, vp, vp])
    P("sapphire_q_unpack_ints_dev", i32, [i32, i32, vp, i32, i32, vp, vp])
    P("sapphire_q_dequant_dev", i32, [i32, i32, vp, i32, i32, vp, vp])
    P("sapphire_gemv_q_dev", i32, [i32, i32, vp, i32, i32, vp, vp, vp])
    P("sapphire_gemv_f_dev", i32, [i32, vp, i32, i32, vp, vp, vp])
    P("sapphire_quantize_dev", i32, [i32, i32, vp, i32, i32, vp, vp])
    P("sapphire_gemm_bf16_dev", i32, [vp, i32, i32, vp, i32, i32, vp, i32, vp])
    P("kernel_quantize", i32, [vp, vp, i32, vp])
    P("sapphire_softmax_argmax_dev", i32, [vp, i32, vp, vp, vp])
    P("sapphire_sample_workspace_bytes", C.c_size_t, [i32, i32])
    P("sapphire_sample_dev", i32, [vp, i32, i32, i32, C.c_float, vp, vp, vp, vp])
    P("sapphire_gemv_softmax_dev", i32, [i32, i32, vp, i32, i32, vp, vp, vp, vp, vp])
    P("sapphire_gemv_softmax_noalloc_dev", i32, [i32, i32, vp, i32, i32, vp, vp, vp, vp, vp])
    P("sapphire_gemm_workspace_bytes", sz, [i32, i32, i32])
    P("sapphire_gemm_q_dev", i32, [i32, i32, vp, i32, i32, vp, i32, vp, vp, vp])
    P("sapphire_gemm_q_greedy_dev", i32, [i32, vp, i32, i32, vp, i32, vp, vp, vp])
    P("sapphire_gemm_splits", i32, [i32])
    P("sapphire_gemm_q_fused_dev", i32, [i32, vp, i32, i32, i32, vp, vp, vp, vp])
    P("sapphire_rmsnorm_delta_dev", i32, [vp, vp, vp, f32, i32, i32, vp])
    P("sapphire_rmsnorm_dev", i32, [vp, vp, vp, f32, i32, i32, vp])
    P("sapphire_rope_apply_dev", i32, [vp, i32, i32, i32, vp, vp, vp])
    P("sapphire_gelu_mul_dev", i32, [vp, vp, i32, vp])
    P("sapphire_norm_residual_dev", i32, [vp, vp, vp, f32, i32, vp])
    P("sapphire_tensor_invalidate", i32, [vp])
    P("sapphire_tensor_device_data", vp, [vp, C.POINTER(i32), vp])
    # tensor.h
    P("tensor_create", vp, [i32, vp, i32])
    P("tensor_create_view", vp, [i32, i32, vp, vp])
    P("tensor_clone", vp, [vp])
    P("tensor_transpose", i32, [vp, C.POINTER(vp)])
    P("tensor_numel", sz, [vp])
    P("dtype_element_size", sz, [i32])
    P("dtype_name", C.c_char_p, [i32])
    P("tensor_get_f32", f32, [vp, sz])
    P("tensor_set_f32", i32, [vp, sz, f32])
    P("tensor_ref_inc", None, [vp])
    P("tensor_release", None, [vp])
    P("tensor_ndim", i32, [vp])
    P("tensor_shape", C.POINTER(i32), [vp])
    P("tensor_data", vp, [vp])
    P("tensor_data_f32", vp, [vp])
    P("tensor_data_mutable", vp, [vp])
    P("tensor_dtype", i32, [vp])
    P("tensor_nbytes", sz, [vp])
    P("tensor_ref_count", i32, [vp])
    # kernels.h
    P("kernel_ctx_create", vp, [i32, i32])
    P("kernel_ctx_init", i32, [vp])
    P("kernel_ctx_destroy", None, [vp])
    P("kernel_parallel_for", i32, [vp, vp, vp, i32])
    for n in ("quantized_gemv_q4_0_aligned", "quantized_gemv_q4_0_unaligned",
              "quantized_gemv_q8_0_aligned", "quantized_gemv_q8_0_unaligned",
              "quantized_gemv_bf16_avx2", "quantized_gemv_bf16_scalar",
              "quantized_gemv_f32_avx2", "quantized_gemv_f32_scalar"):
        P(n, f32, [vp, vp, i32, i32])
    P("kernel_gemm_f32_avx2", None, [vp])
    P("kernel_gemm_bf16_avx2", None, [vp])
    for n in ("silu", "relu", "gelu"):
        P(n, f32, [f32])
    P("geglu", f32, [f32, f32])
    # rope.h
    P("rope_precompute_freqs", i32, [vp, vp, i32, i32, f32])
    P("rope_apply_fast", None, [vp, i32, i32, vp, vp])
    P("apply_rope", None, [vp, i32, i32, f32])
    P("apply_rope_default", None, [vp, i32, i32])
    P("kernel_gemv", i32, [vp, vp, vp, vp])
    P("kernel_gemm", i32, [vp, vp, vp, vp, i32, i32])
    P("kernel_gemv_tensor", i32, [vp, vp, vp, vp])
    P("kernel_gemv_add", i32, [vp, vp, vp, vp, f32])
    P("kernel_gemv_batch", i32, [vp, vp, vp, vp, i32])
    P("kernel_get_simd_lane_count", i32, [i32])
    P("gelu_inplace", None, [vp, i32])
    P("silu_inplace", None, [vp, i32])
    P("relu_inplace", None, [vp, i32])
    P("sapphire_geglu", i32, [vp, vp, sz])
    P("rmsnorm", i32, [vp, vp, vp, f32, i32])
    P("rmsnorm_delta", i32, [vp, vp, vp, f32, i32])
    P("rmsnorm_batch", i32, [vp, vp, vp, f32, i32, i32])
    P("softmax", None, [vp, i32])
    P("vec_softcap", None, [vp, i32, f32])
    P("vec_add", None, [vp, vp, i32])
    P("vec_scale", None, [vp, f32, i32])
    P("vec_copy", None, [vp, vp, i32])
    P("vec_dot", f32, [vp, vp, i32])
    P("bf16_to_f32_vec", None, [vp, vp, i32])
    P("get_norm_weights", vp, [vp, vp, i32])
    _LIB = lib
    return lib


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data
