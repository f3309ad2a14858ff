"""ctypes bindings of the C ABI declared in include/oxforge.h.

This module only describes the ABI (argument and result types) and turns a
non-zero forge_status into ForgeError.  It never falls back to anything: if
liboxforge.so or the gfx950 code object is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_size_t, c_void_p

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(os.path.dirname(PKG_DIR), "lib")
LIB_PATH = os.path.join(LIB_DIR, "liboxforge.so")
KERNELS_PATH = os.path.join(LIB_DIR, "oxforge_kernels.hsaco")

# forge_status
FORGE_OK = 0
FORGE_EINVAL = 1
FORGE_ENOMEM = 2
FORGE_EHIP = 3
FORGE_ENOMODULE = 4
FORGE_ENODEV = 5
FORGE_EIO = 6

# forge_binary_op (BinaryOp, cuda.rs:3-10)
ADD, SUB, MUL, DIV = 0, 1, 2, 3

# forge_map_op
MAP_SCALE, MAP_ADD, MAP_GELU, MAP_GELU_D, MAP_RELU, MAP_RELU_D = 0, 1, 2, 3, 4, 5
MAP_SILU, MAP_SILU_D, MAP_EXP_SHIFT, MAP_HALF_SQ, MAP_IDENTITY = 6, 7, 8, 9, 10

# forge_activation
ACT_IDENTITY, ACT_GELU, ACT_RELU, ACT_SILU = 0, 1, 2, 3


class ForgeError(RuntimeError):
    def __init__(self, status: int, func: str, detail: str):
        super().__init__(f"{func} -> status {status}: {detail}")
        self.status = status
        self.func = func


class Slice(ctypes.Structure):
    """forge_slice {float *ptr; size_t len;} (span.rs:7-11,45-49)."""

    _fields_ = [("ptr", c_void_p), ("len", c_size_t)]


NULL_SLICE = Slice(None, 0)


class SliceU32(ctypes.Structure):
    """forge_slice_u32 {uint32_t *ptr; size_t len;}."""

    _fields_ = [("ptr", c_void_p), ("len", c_size_t)]


class GemmEpilogue(ctypes.Structure):
    """forge_gemm_epilogue."""

    _fields_ = [
        ("alpha", c_float),
        ("bias", Slice),
        ("residual", Slice),
        ("aux_mul", Slice),
        ("pre_out", Slice),
        ("activation", c_int),
        ("update", c_int),
        ("update_scale", c_float),
        ("aux_activation", c_int),
        ("row_parts_in", Slice),
        ("row_parts", c_size_t),
        ("row_n", c_size_t),
        ("row_eps", c_float),
        ("row_div", c_int),
        ("row_sumsq_out", Slice),
        ("col_sums_out", Slice),
        ("col_sums_param", Slice),
        ("col_sums_lr", c_float),
        ("row_sub", Slice),
    ]


class GemmProblem(ctypes.Structure):
    """forge_gemm_problem."""

    _fields_ = [("A", Slice), ("B", Slice), ("C", Slice), ("epilogue", GemmEpilogue)]


RT = c_void_p  # forge_runtime*
ST = c_void_p  # forge_stream*

# name -> argtypes (restype is forge_status unless listed in _RESTYPES)
SIGNATURES = {
    "forge_runtime_create": [c_int, c_char_p, POINTER(c_void_p)],
    "forge_runtime_destroy": [RT],
    "forge_sync": [RT, ST],
    "forge_device_count": [POINTER(c_int)],
    "forge_status_string": [c_int],
    "forge_last_error": [],
    "forge_device_props": [RT, POINTER(c_int), POINTER(c_size_t), POINTER(c_int), c_char_p, c_size_t],
    "forge_streams_create": [RT, c_size_t, POINTER(c_void_p)],
    "forge_streams_fork": [RT, c_size_t, POINTER(c_void_p)],
    "forge_streams_join": [RT, c_size_t, POINTER(c_void_p)],
    "forge_stream_wait": [RT, ST, ST],
    "forge_stream_destroy": [RT, ST],
    "forge_event_create": [RT, POINTER(c_void_p)],
    "forge_event_record": [RT, ST, c_void_p],
    "forge_event_elapsed_ms": [RT, c_void_p, c_void_p, POINTER(c_float)],
    "forge_event_destroy": [RT, c_void_p],
    "forge_alloc": [RT, c_size_t, POINTER(Slice)],
    "forge_alloc_zeroed": [RT, c_size_t, POINTER(Slice)],
    "forge_recycle": [RT, Slice],
    "forge_free": [RT, Slice],
    "forge_reserve": [RT, c_size_t, c_size_t],
    "forge_pool_count": [RT, c_size_t, POINTER(c_size_t)],
    "forge_stream_workspace_floats": [RT, ST, POINTER(c_size_t)],
    "forge_alloc_u32": [RT, c_size_t, POINTER(SliceU32)],
    "forge_free_u32": [RT, SliceU32],
    "forge_memcpy_d2h_u32": [RT, c_void_p, SliceU32, c_size_t],
    "forge_memcpy_h2d": [RT, Slice, c_void_p, c_size_t],
    "forge_memcpy_d2h": [RT, c_void_p, Slice, c_size_t],
    "forge_memcpy_d2d": [RT, ST, Slice, Slice, c_size_t],
    "forge_fill": [RT, ST, Slice, c_float],
    "forge_gemm_f32": [RT, ST, Slice, Slice, Slice, c_size_t, c_size_t, c_size_t],
    "forge_gemm_ex_f32": [RT, ST, c_int, c_int, Slice, Slice, Slice, c_size_t, c_size_t,
                          c_size_t, POINTER(GemmEpilogue)],
    "forge_gemm_sum_f32": [RT, ST, c_int, c_int, c_size_t, POINTER(Slice), POINTER(Slice), Slice,
                           c_size_t, c_size_t, c_size_t, POINTER(GemmEpilogue)],
    "forge_gemm_f32_tile": [RT, ST, c_char_p, Slice, Slice, Slice, c_size_t, c_size_t,
                            c_size_t],
    "forge_gemm_f32_split": [RT, ST, c_char_p, c_int, Slice, Slice, Slice, c_size_t, c_size_t,
                             c_size_t],
    "forge_gemm_ex_f32_tile": [RT, ST, c_char_p, c_int, c_int, Slice, Slice, Slice, c_size_t,
                               c_size_t, c_size_t, POINTER(GemmEpilogue)],
    "forge_gemm_kernel_name": [RT, c_int, c_int, c_size_t, c_size_t, c_size_t, c_int, c_char_p,
                               c_size_t],
    "forge_gemm_batch_f32": [RT, ST, c_int, c_int, c_size_t, c_size_t, c_size_t, c_size_t,
                             POINTER(GemmProblem)],
    "forge_transpose_f32": [RT, ST, Slice, Slice, c_size_t, c_size_t],
    "forge_softmax_rows": [RT, ST, Slice, c_size_t, c_size_t],
    "forge_softmax_rows_bwd": [RT, ST, Slice, Slice, Slice, c_size_t, c_size_t],
    "forge_layer_norm_rows": [RT, ST, Slice, Slice, Slice, c_size_t, c_size_t, c_float],
    "forge_layer_norm_rows_out": [RT, ST, Slice, Slice, Slice, Slice, c_size_t, c_size_t,
                                  c_float],
    "forge_layer_norm_bwd": [RT, ST, Slice, Slice, Slice, Slice, Slice, Slice, c_size_t,
                             c_size_t, c_float],
    "forge_layer_norm_bwd_noalloc": [RT, ST, Slice, Slice, Slice, Slice, Slice, Slice, c_size_t,
                                     c_size_t, c_float],
    "forge_layer_norm_bwd_sgd": [RT, ST, Slice, Slice, Slice, Slice, Slice, Slice, Slice, c_size_t,
                                 c_size_t, c_float, c_float],
    "forge_rms_norm_bwd_sgd": [RT, ST, Slice, Slice, Slice, Slice, Slice, c_size_t, c_size_t,
                               c_float, c_float],
    "forge_layer_norm_bwd_sgd_dot": [RT, ST, Slice, Slice, Slice, Slice, Slice, Slice, Slice,
                                     Slice, Slice, c_size_t, c_size_t, c_float, c_float, c_float],
    "forge_rms_norm_bwd_sgd_dot": [RT, ST, Slice, Slice, Slice, Slice, Slice, Slice, Slice,
                                   c_size_t, c_size_t, c_float, c_float, c_float],
    "forge_sum_cols_sgd": [RT, ST, Slice, c_size_t, c_size_t, Slice, Slice, c_float],
    "forge_rms_norm_rows": [RT, ST, Slice, Slice, c_size_t, c_size_t, c_float],
    "forge_rms_norm_rows_out": [RT, ST, Slice, Slice, Slice, c_size_t, c_size_t, c_float],
    "forge_rms_norm_bwd": [RT, ST, Slice, Slice, Slice, Slice, Slice, c_size_t, c_size_t,
                           c_float],
    "forge_binary": [RT, ST, Slice, Slice, Slice, c_size_t, c_int],
    "forge_binary_assign": [RT, ST, Slice, Slice, c_size_t, c_int],
    "forge_binary_assign_by_rows": [RT, ST, Slice, Slice, c_size_t, c_size_t, c_int],
    "forge_map": [RT, ST, Slice, c_size_t, c_int, c_float],
    "forge_sum_rows": [RT, ST, Slice, Slice, c_size_t, c_size_t],
    "forge_sum_cols": [RT, ST, Slice, Slice, c_size_t, c_size_t],
    "forge_reduce_sum": [RT, ST, Slice, c_size_t, Slice],
    "forge_map_sum": [RT, ST, Slice, c_size_t, c_int, c_float, Slice],
    "forge_reduce_max": [RT, ST, Slice, c_size_t, Slice],
    "forge_fill_seq": [RT, ST, Slice, c_size_t, c_int],
    "forge_causal_mask": [RT, ST, Slice, c_size_t, c_size_t],
    "forge_causal_mask_rows": [RT, ST, Slice, c_size_t, c_size_t, c_size_t],
    "forge_softmax_rows_bwd_scaled": [RT, ST, Slice, Slice, Slice, c_size_t, c_size_t, c_float],
    "forge_activation_backward": [RT, ST, Slice, Slice, Slice, c_size_t, c_int],
    "forge_sgd_update": [RT, ST, Slice, Slice, c_size_t, c_float],
    "forge_fill_random": [RT, ST, Slice, c_size_t, ctypes.c_uint32],
    "forge_compare": [RT, ST, Slice, Slice, c_size_t, Slice],
    "forge_compare_u32": [RT, ST, Slice, Slice, c_size_t, SliceU32],
}

_RESTYPES = {"forge_status_string": c_char_p, "forge_last_error": c_char_p}

_lib = None


def load(path: str | None = None) -> ctypes.CDLL:
    """Loads liboxforge.so (once) and declares every ABI entry point.

    Raises FileNotFoundError if the library has not been built; there is no
    fallback implementation.
    """
    global _lib
    if _lib is not None:
        return _lib
    path = path or os.environ.get("OXFORGE_LIB", LIB_PATH)
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, c_int)
    _lib = lib
    return lib


def check(status: int, func: str) -> None:
    if status != FORGE_OK:
        lib = load()
        detail = lib.forge_last_error().decode(errors="replace")
        raise ForgeError(status, func, detail)


def call(name: str, *args) -> None:
    """Calls an ABI entry point that returns forge_status; raises on error."""
    lib = load()
    check(getattr(lib, name)(*args), name)
